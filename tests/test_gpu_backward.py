"""Backward parity on the GPU: zt_attn_backward / _batched against the CPU
restatement of src/autograd.zig:636-842, max|g - twin| / max|twin| <= 1e-3 per
gradient, plus the row statistics, invariants at full size, determinism and
negative controls."""
import numpy as np
import pytest

from gpuhelp import (BWD_REL, SEED_DO, SEED_K, SEED_Q, SEED_V, THETA, dev_normal, host, max_abs, rel_err)

pytestmark = pytest.mark.gpu


def _alloc(torch, n):
    return torch.full((n,), float("nan"), device="cuda", dtype=torch.float32)


def _run(torch, zt, B, T, H, Hkv, D, sigma=1.0, rope=False, max_tile=64):
    q = dev_normal(torch, zt, B * T * H * D, SEED_Q, sigma)
    k = dev_normal(torch, zt, B * T * Hkv * D, SEED_K, sigma)
    v = dev_normal(torch, zt, B * T * Hkv * D, SEED_V, sigma)
    do = dev_normal(torch, zt, B * T * H * D, SEED_DO, 1.0)
    if rope:
        q2, k2 = torch.empty_like(q), torch.empty_like(k)
        zt.rope(q, q2, B * T, H * D, 0, THETA, D)
        zt.rope(k, k2, B * T, Hkv * D, 0, THETA, D)
        q, k = q2, k2
    dq, dk, dv = _alloc(torch, q.numel()), _alloc(torch, k.numel()), _alloc(torch, k.numel())
    rm, rl, rd = (_alloc(torch, B * T * H) for _ in range(3))
    zt.backward(q, k, v, do, dq, dk, dv, rm, rl, rd, T, H, Hkv, D, max_tile=max_tile, B=B)
    torch.cuda.synchronize()
    ins = [host(x) for x in (q, k, v, do)]
    outs = [host(x) for x in (dq, dk, dv, rm, rl, rd)]
    return ins, outs


CASES = [
    (1, 128, 4, 2, 32),
    (1, 1, 4, 2, 32),
    (1, 7, 2, 2, 34),
    (2, 50, 6, 3, 64),
    (1, 100, 8, 2, 80),
    (1, 77, 4, 1, 128),
    (2, 33, 8, 8, 96),
    (1, 64, 4, 4, 192),
    (1, 90, 4, 2, 256),
    (1, 40, 16, 2, 160),
]


@pytest.mark.parametrize("B,T,H,Hkv,D", CASES)
def test_backward_matches_twin(gpu, zt, oracle, threads, B, T, H, Hkv, D):
    (q, k, v, do), (dq, dk, dv, rm, rl, rd) = _run(gpu, zt, B, T, H, Hkv, D)
    rq, rk, rv = oracle.attention_backward(q, k, v, do, B, T, H, Hkv, D, threads=threads)
    assert rel_err(dq, rq) <= BWD_REL
    assert rel_err(dk, rk) <= BWD_REL
    assert rel_err(dv, rv) <= BWD_REL
    m, l, d = oracle.attention_row_stats(q, k, v, do, B, T, H, Hkv, D)
    assert max_abs(rm, m) <= 1e-4 * max(1.0, np.abs(m).max())
    assert np.max(np.abs(rl - l) / l) <= 1e-4
    assert max_abs(rd, d) <= 1e-4 * max(1.0, np.abs(d).max())


@pytest.mark.parametrize("max_tile", [1, 32, 64])
def test_backward_any_tile_cap(gpu, zt, oracle, max_tile):
    B, T, H, Hkv, D = 1, 70, 4, 2, 64
    (q, k, v, do), (dq, dk, dv, *_) = _run(gpu, zt, B, T, H, Hkv, D, max_tile=max_tile)
    rq, rk, rv = oracle.attention_backward(q, k, v, do, B, T, H, Hkv, D)
    assert max(rel_err(dq, rq), rel_err(dk, rk), rel_err(dv, rv)) <= BWD_REL


_NO_DS = {"ZT_ATTN_DSPLIT": "0"}


@pytest.mark.parametrize("env", [
    {"ZT_ATTN_W8": "1", "ZT_ATTN_PF": "0"}, {"ZT_ATTN_W8": "1", "ZT_ATTN_PF": "1"},
    {"ZT_ATTN_W8": "1", "ZT_ATTN_PF": "1", "ZT_ATTN_BPAIR": "0"},
    {"ZT_ATTN_W8": "0", "ZT_ATTN_DMA": "1", "ZT_ATTN_BPAIR": "0", **_NO_DS},
    {"ZT_ATTN_W8": "0", "ZT_ATTN_DMA": "0", **_NO_DS}, {"ZT_ATTN_W8": "0", "ZT_ATTN_DMA": "1", **_NO_DS},
    {"ZT_ATTN_W8": "0", "ZT_ATTN_DMA": "0", "ZT_ATTN_HS": "4", **_NO_DS},
    {"ZT_ATTN_W8": "0", "ZT_ATTN_DMA": "1", "ZT_ATTN_HS": "4", **_NO_DS},
    {"ZT_ATTN_W8": "0", "ZT_ATTN_DMA": "0", "ZT_ATTN_HS": "1", **_NO_DS},
    {"ZT_ATTN_W8": "0", "ZT_ATTN_DMA": "1", "ZT_ATTN_HS": "1", "ZT_ATTN_RSPLIT": "0", **_NO_DS},
    {"ZT_ATTN_DSPLIT": "1"}, {"ZT_ATTN_DSPLIT": "1", "ZT_ATTN_BPAIR": "0"},
    {"ZT_ATTN_W8": "0", "ZT_ATTN_DMA": "1", "ZT_ATTN_HS": "1", "ZT_ATTN_RSPLIT": "1", **_NO_DS},
    {"ZT_ATTN_W8": "0", "ZT_ATTN_DMA": "1", "ZT_ATTN_HS": "1", "ZT_ATTN_RSPLIT": "1", "ZT_ATTN_BPAIR": "1", **_NO_DS},
    {"ZT_ATTN_W8": "0", "ZT_ATTN_DMA": "1", "ZT_ATTN_HS": "1", "ZT_ATTN_RSPLIT": "0", **_NO_DS},
    {"ZT_ATTN_HS": "1", "ZT_ATTN_DSPLIT": "1"}, {"ZT_ATTN_HS": "1", "ZT_ATTN_DSPLIT": "1", "ZT_ATTN_BPAIR": "1"},
    {"ZT_ATTN_HS": "1", "ZT_ATTN_DMA": "0"}, {"ZT_ATTN_HS": "1", "ZT_ATTN_DMA": "0", "ZT_ATTN_BPAIR": "1"},
])
@pytest.mark.parametrize("B,T,H,Hkv,D", [(1, 200, 8, 2, 128), (2, 75, 4, 1, 64), (1, 100, 8, 2, 256),
                                         (1, 70, 8, 2, 192), (2, 90, 3, 3, 32), (1, 47, 6, 2, 96),
                                         (1, 100, 4, 4, 256), (2, 61, 6, 2, 192)])
def test_backward_every_dkdv_variant(gpu, zt, oracle, threads, tune, env, B, T, H, Hkv, D):
    """Each dk/dv kernel variant (eight-wave, register-staged, asynchronously
    staged, columns split over two waves for d = 192 / 256, rows split over
    two parts for unsplit groups; 1/2/4-way head splits; paired or single key
    tiles per workgroup), forced through the library's tuning variables,
    matches the twin."""
    tune(env)
    (q, k, v, do), (dq, dk, dv, *_) = _run(gpu, zt, B, T, H, Hkv, D)
    rq, rk, rv = oracle.attention_backward(q, k, v, do, B, T, H, Hkv, D, threads=threads)
    assert max(rel_err(dq, rq), rel_err(dk, rk), rel_err(dv, rv)) <= BWD_REL


@pytest.mark.parametrize("env", [
    {"ZT_ATTN_BK": "32", "ZT_ATTN_QPF": "1", "ZT_ATTN_DQ_W": "4"},
    {"ZT_ATTN_BK": "32", "ZT_ATTN_QPF": "1", "ZT_ATTN_DQ_W": "8"},
    {"ZT_ATTN_BK": "32", "ZT_ATTN_QPF": "0", "ZT_ATTN_DQ_W": "8"},
    {"ZT_ATTN_BK": "64", "ZT_ATTN_QPF": "0", "ZT_ATTN_DQ_W": "4"},
    {"ZT_ATTN_BK": "32", "ZT_ATTN_QPF": "1", "ZT_ATTN_DQ_W": "4", "ZT_ATTN_BPAIR": "0"},
])
@pytest.mark.parametrize("B,T,H,Hkv,D", [(1, 200, 8, 2, 128), (2, 75, 4, 1, 64), (1, 61, 6, 3, 66)])
def test_backward_every_dq_variant(gpu, zt, oracle, threads, tune, env, B, T, H, Hkv, D):
    """Each dq kernel variant (four or eight waves, 32- or 64-key tiles, with
    and without register prefetch of the next K/V tile) matches the twin."""
    tune(env)
    (q, k, v, do), (dq, dk, dv, *_) = _run(gpu, zt, B, T, H, Hkv, D)
    rq, rk, rv = oracle.attention_backward(q, k, v, do, B, T, H, Hkv, D, threads=threads)
    assert max(rel_err(dq, rq), rel_err(dk, rk), rel_err(dv, rv)) <= BWD_REL


def test_backward_c2_mha_batch4(gpu, zt, oracle, threads):
    B, T, H, Hkv, D = 4, 1024, 8, 8, 64   # C2
    (q, k, v, do), (dq, dk, dv, *_) = _run(gpu, zt, B, T, H, Hkv, D)
    rq, rk, rv = oracle.attention_backward(q, k, v, do, B, T, H, Hkv, D, threads=threads)
    assert rel_err(dq, rq) <= BWD_REL and rel_err(dk, rk) <= BWD_REL and rel_err(dv, rv) <= BWD_REL


def _invariants(dk, dv, do, B, T, H, Hkv, D):
    # sum_s dk[s] = 0 (rows of dS sum to zero); sum_s dv[s] = sum over the group's heads of all dO rows.
    dk4 = dk.reshape(B, T, Hkv, D).astype(np.float64)
    dv4 = dv.reshape(B, T, Hkv, D).astype(np.float64)
    want = do.reshape(B, T, Hkv, H // Hkv, D).astype(np.float64).sum(axis=(1, 3))
    assert np.max(np.abs(dk4.sum(1))) <= 1e-3 * np.abs(dk4).sum(1).max()
    assert np.max(np.abs(dv4.sum(1) - want)) <= 1e-3 * np.abs(want).max()


@pytest.mark.parametrize("cfg", ["c3", "c5"])
def test_backward_full_size(gpu, zt, oracle, threads, cfg):
    if cfg == "c3":
        B, T, H, Hkv, D, sigma, rope, W = 1, 4096, 32, 8, 128, 1.0, True, 64
    else:
        B, T, H, Hkv, D, sigma, rope, W = 2, 2048, 16, 4, 256, np.sqrt(2.0), False, 32
    (q, k, v, do), (dq, dk, dv, *_) = _run(gpu, zt, B, T, H, Hkv, D, sigma=sigma, rope=rope)
    for g in (dq, dk, dv):
        assert np.all(np.isfinite(g))
    _invariants(dk, dv, do, B, T, H, Hkv, D)
    qs, ks = (B, T, H * D), (B, T, Hkv * D)
    # Last W rows: dq for those rows and dk/dv for key rows >= T - W are exact in the twin.
    rq, rk, rv = oracle.attention_backward(q, k, v, do, B, T, H, Hkv, D, t_begin=T - W, threads=threads)
    assert rel_err(dq.reshape(qs)[:, T - W:], rq.reshape(qs)[:, T - W:]) <= BWD_REL
    assert rel_err(dk.reshape(ks)[:, T - W:], rk.reshape(ks)[:, T - W:]) <= BWD_REL
    assert rel_err(dv.reshape(ks)[:, T - W:], rv.reshape(ks)[:, T - W:]) <= BWD_REL
    # First W rows of dq.
    rq, _, _ = oracle.attention_backward(q, k, v, do, B, T, H, Hkv, D, t_begin=0, t_end=W, threads=threads)
    assert rel_err(dq.reshape(qs)[:, :W], rq.reshape(qs)[:, :W]) <= BWD_REL


@pytest.mark.parametrize("B,T,H,Hkv,D", [(1, 32768, 2, 1, 64), (1, 20000, 4, 4, 128)])
def test_backward_long_sequences(gpu, zt, oracle, threads, B, T, H, Hkv, D):
    """The reference entry point's backward at 5-8x C3's length (2^29 causal
    pairs per head at T = 32768): invariants at full size, the last and first
    rows against the twin."""
    W = 64
    (q, k, v, do), (dq, dk, dv, *_) = _run(gpu, zt, B, T, H, Hkv, D)
    for g in (dq, dk, dv):
        assert np.all(np.isfinite(g))
    _invariants(dk, dv, do, B, T, H, Hkv, D)
    qs, ks = (B, T, H * D), (B, T, Hkv * D)
    rq, rk, rv = oracle.attention_backward(q, k, v, do, B, T, H, Hkv, D, t_begin=T - W, threads=threads)
    assert rel_err(dq.reshape(qs)[:, T - W:], rq.reshape(qs)[:, T - W:]) <= BWD_REL
    assert rel_err(dk.reshape(ks)[:, T - W:], rk.reshape(ks)[:, T - W:]) <= BWD_REL
    assert rel_err(dv.reshape(ks)[:, T - W:], rv.reshape(ks)[:, T - W:]) <= BWD_REL
    rq, _, _ = oracle.attention_backward(q, k, v, do, B, T, H, Hkv, D, t_begin=0, t_end=W, threads=threads)
    assert rel_err(dq.reshape(qs)[:, :W], rq.reshape(qs)[:, :W]) <= BWD_REL


def test_backward_is_deterministic(gpu, zt):
    B, T, H, Hkv, D = 1, 300, 8, 2, 128
    _, a = _run(gpu, zt, B, T, H, Hkv, D)
    _, b = _run(gpu, zt, B, T, H, Hkv, D)
    for x, y in zip(a, b):
        assert np.array_equal(x.view(np.uint32), y.view(np.uint32))


def test_backward_gate_catches_broken_references(gpu, zt, oracle):
    """The reference's backward BROKEN variants (attn_kernels.cu:573-627), planted in
    a float64 CPU reference: each must fail the 1e-3 relative gate on some
    gradient, while the correct reference passes it."""
    from npref import attention_backward_f64
    B, T, H, Hkv, D = 1, 64, 4, 2, 32
    (q, k, v, do), (dq, dk, dv, *_) = _run(gpu, zt, B, T, H, Hkv, D)

    def worst(grads):
        return max(rel_err(dq, grads[0]), rel_err(dk, grads[1]), rel_err(dv, grads[2]))

    assert worst(attention_backward_f64(q, k, v, do, T, H, Hkv, D)) <= BWD_REL
    for variant in ("suffix_to_prefix", "gqa_collapsed", "no_jacobian", "no_scale"):
        assert worst(attention_backward_f64(q, k, v, do, T, H, Hkv, D, variant)) > BWD_REL, variant
    # no_jacobian leaves dv untouched, as the reference's variant 3 does.
    assert rel_err(dv, attention_backward_f64(q, k, v, do, T, H, Hkv, D, "no_jacobian")[2]) <= BWD_REL


@pytest.mark.parametrize("T,H,Hkv,D", [(96, 8, 2, 64), (40, 4, 4, 128), (17, 6, 3, 34)])
def test_block_backward_through_rope_on_the_device(gpu, zt, oracle, threads, T, H, Hkv, D):
    # blockBackward's attention segment (src/autograd.zig:559-569): attention
    # backward on the rotated q, k, then ropeBackward at position 0 takes dq, dk
    # back to the unrotated projections.  Both halves run on the device here.
    (q, k, v, do), (dq, dk, dv, _, _, _) = _run(gpu, zt, 1, T, H, Hkv, D, rope=True)
    dq_in, dk_in = gpu.empty(T * H * D, device="cuda"), gpu.empty(T * Hkv * D, device="cuda")
    zt.rope_backward(gpu.from_numpy(dq).cuda(), dq_in, T, H * D, 0, THETA, D)
    zt.rope_backward(gpu.from_numpy(dk).cuda(), dk_in, T, Hkv * D, 0, THETA, D)
    gpu.cuda.synchronize()
    rq, rk, rv = oracle.attention_backward(q, k, v, do, 1, T, H, Hkv, D, threads=threads)
    want_q = oracle.rope_backward(rq, T, H * D, 0, THETA, D)
    want_k = oracle.rope_backward(rk, T, Hkv * D, 0, THETA, D)
    assert rel_err(host(dq_in), want_q) <= BWD_REL
    assert rel_err(host(dk_in), want_k) <= BWD_REL
    assert rel_err(dv, rv) <= BWD_REL
    # The gradient before ropeBackward is not the answer (rows t > 0 rotate).
    assert rel_err(dq, want_q) > 10 * BWD_REL


def test_plan_names_the_column_split_kernel(gpu, zt, tune):
    """Heads of 192 or 256 take the eight-wave kernel that splits the columns
    over two waves: two head halves of four key blocks for an even head group,
    one part of four key blocks for MHA and odd groups, which also take it at
    64 and 128 where the DMA kernel is not chosen; ZT_ATTN_DSPLIT=0 turns it off."""
    assert zt.plan(1, 256, 8, 2, 256)[2] == "zt_bwd_dkdv8pd_d256_hs2"
    assert zt.plan(1, 256, 8, 2, 192)[2] == "zt_bwd_dkdv8pd_d192_hs2"
    assert zt.plan(1, 256, 8, 8, 256)[2] == "zt_bwd_dkdv8pd_d256_hs1"
    assert zt.plan(1, 256, 6, 2, 192)[2] == "zt_bwd_dkdv8pd_d192_hs1"
    assert zt.plan(2, 2048, 16, 16, 128)[2] == "zt_bwd_dkdv8pd_d128_hs1"   # MHA, grid past the DMA kernel's
    assert zt.plan(8, 1024, 32, 32, 64)[2] == "zt_bwd_dkdv8pd_d64_hs1"
    assert zt.plan(4, 1024, 8, 8, 64)[2] == "zt_bwd_dkdv_dmar_d64"        # C2: the row-split DMA kernel
    assert "8pd" not in zt.plan(1, 256, 8, 2, 160)[2] and "8pd" not in zt.plan(1, 256, 8, 8, 250)[2]
    tune({"ZT_ATTN_DSPLIT": "0"})
    assert "8pd" not in zt.plan(1, 256, 8, 2, 256)[2] and "8pd" not in zt.plan(1, 256, 8, 8, 256)[2]
