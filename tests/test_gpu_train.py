"""The training path with saved statistics (zt_attn_forward_train +
zt_attn_backward_train): the forward also writes each row's log-sum-exp and
the backward uses it instead of rebuilding the softmax.  Gates as for the
reference entry points: out max |diff| <= 1e-4; dq/dk/dv max|g - twin| /
max|twin| <= 1e-3 against the CPU restatement of src/autograd.zig:636-842;
lse and delta (= sum_d out * dO) against the twin's row statistics
(autograd.zig:723-797)."""
import numpy as np
import pytest

from gpuhelp import (BWD_REL, FWD_TOL, SEED_DO, SEED_K, SEED_Q, SEED_V, THETA, dev_normal, host, max_abs,
                     rel_err)

pytestmark = pytest.mark.gpu


def _nan(torch, n):
    return torch.full((n,), float("nan"), device="cuda", dtype=torch.float32)


def _inputs(torch, zt, B, T, H, Hkv, D, sigma=1.0, rope=False):
    q = dev_normal(torch, zt, B * T * H * D, SEED_Q, sigma)
    k = dev_normal(torch, zt, B * T * Hkv * D, SEED_K, sigma)
    v = dev_normal(torch, zt, B * T * Hkv * D, SEED_V, sigma)
    do = dev_normal(torch, zt, B * T * H * D, SEED_DO, 1.0)
    if rope:
        zt.rope_qk(q, k, q, k, B, T, H, Hkv, D, 0, THETA)
    return q, k, v, do


def _train(torch, zt, q, k, v, do, B, T, H, Hkv, D, lse_shift=0.0, ws=False):
    """ws: False = the dq kernel; "ds" (or True) = dq from the stored dS;
    "scores" = that, with the forward's scores read back by the dk/dv kernel."""
    out, lse = _nan(torch, q.numel()), _nan(torch, B * T * H)
    # The workspace starts as NaN so that an unwritten score or dS tile shows.
    work = _nan(torch, zt.backward_train_workspace_bytes(B, T, H, Hkv, D) // 4) if ws else None
    if ws == "scores":
        zt.forward_train_ws(q, k, v, out, lse, work, T, H, Hkv, D, B=B)
    else:
        zt.forward_train(q, k, v, out, lse, T, H, Hkv, D, B=B)
    if lse_shift:
        lse += lse_shift
    dq, dk, dv, delta = _nan(torch, q.numel()), _nan(torch, k.numel()), _nan(torch, k.numel()), _nan(torch, B * T * H)
    if ws:
        stage = 3 | (zt.ZT_WS_SCORES if ws == "scores" else 0)
        zt.backward_train_ws(q, k, v, out, do, lse, dq, dk, dv, work, T, H, Hkv, D, B=B, stage=stage)
        delta = work[:B * T * H]
    else:
        zt.backward_train(q, k, v, out, do, lse, dq, dk, dv, delta, T, H, Hkv, D, B=B)
    torch.cuda.synchronize()
    return [host(x) for x in (out, lse, dq, dk, dv, delta)]


CASES = [
    (1, 128, 4, 2, 32), (1, 1, 4, 2, 32), (1, 7, 2, 2, 34), (2, 50, 6, 3, 64), (1, 100, 8, 2, 80),
    (1, 77, 4, 1, 128), (2, 33, 8, 8, 96), (1, 64, 4, 4, 192), (1, 90, 4, 2, 256), (1, 40, 16, 2, 160),
]


MODES = [False, "ds", "scores"]
MODE_IDS = ["dq-kernel", "dq-from-ds", "scores"]


@pytest.mark.parametrize("ws", MODES, ids=MODE_IDS)
@pytest.mark.parametrize("B,T,H,Hkv,D", CASES)
def test_train_path_matches_twin(gpu, zt, oracle, threads, B, T, H, Hkv, D, ws):
    q, k, v, do = _inputs(gpu, zt, B, T, H, Hkv, D)
    out, lse, dq, dk, dv, delta = _train(gpu, zt, q, k, v, do, B, T, H, Hkv, D, ws=ws)
    qh, kh, vh, dh = (host(x) for x in (q, k, v, do))
    assert max_abs(out, oracle.attention_forward(qh, kh, vh, B, T, H, Hkv, D, threads=threads)) <= FWD_TOL
    m, l, d = oracle.attention_row_stats(qh, kh, vh, dh, B, T, H, Hkv, D)
    want_lse = m + np.log(l)
    assert max_abs(lse, want_lse) <= 1e-5 * max(1.0, np.abs(want_lse).max())
    assert max_abs(delta, d) <= 1e-4 * max(1.0, np.abs(d).max())
    rq, rk, rv = oracle.attention_backward(qh, kh, vh, dh, B, T, H, Hkv, D, threads=threads)
    assert rel_err(dq, rq) <= BWD_REL
    assert rel_err(dk, rk) <= BWD_REL
    assert rel_err(dv, rv) <= BWD_REL


@pytest.mark.parametrize("ws", MODES, ids=MODE_IDS)
@pytest.mark.parametrize("cfg", ["c3", "c5"])
def test_train_path_full_size(gpu, zt, oracle, threads, cfg, ws):
    if cfg == "c3":
        B, T, H, Hkv, D, sigma, rope, W = 1, 4096, 32, 8, 128, 1.0, True, 64
    else:
        B, T, H, Hkv, D, sigma, rope, W = 2, 2048, 16, 4, 256, np.sqrt(2.0), False, 32
    q, k, v, do = _inputs(gpu, zt, B, T, H, Hkv, D, sigma, rope)
    out, lse, dq, dk, dv, delta = _train(gpu, zt, q, k, v, do, B, T, H, Hkv, D, ws=ws)
    for g in (out, lse, dq, dk, dv, delta):
        assert np.all(np.isfinite(g))
    qh, kh, vh, dh = (host(x) for x in (q, k, v, do))
    qs, ks = (B, T, H * D), (B, T, Hkv * D)
    # Invariants over all rows: sum_s dk = 0 per (batch, kv head, d); sum_s dv = sum of dO over the group.
    dk4 = dk.reshape(B, T, Hkv, D).astype(np.float64)
    dv4 = dv.reshape(B, T, Hkv, D).astype(np.float64)
    want = dh.reshape(B, T, Hkv, H // Hkv, D).astype(np.float64).sum(axis=(1, 3))
    assert np.max(np.abs(dk4.sum(1))) <= 1e-3 * np.abs(dk4).sum(1).max()
    assert np.max(np.abs(dv4.sum(1) - want)) <= 1e-3 * np.abs(want).max()
    # Last W rows exact in the twin (dq rows, and dk/dv rows >= T - W); the forward's last rows too.
    rq, rk, rv = oracle.attention_backward(qh, kh, vh, dh, B, T, H, Hkv, D, t_begin=T - W, threads=threads)
    assert rel_err(dq.reshape(qs)[:, T - W:], rq.reshape(qs)[:, T - W:]) <= BWD_REL
    assert rel_err(dk.reshape(ks)[:, T - W:], rk.reshape(ks)[:, T - W:]) <= BWD_REL
    assert rel_err(dv.reshape(ks)[:, T - W:], rv.reshape(ks)[:, T - W:]) <= BWD_REL
    ro = oracle.attention_forward(qh, kh, vh, B, T, H, Hkv, D, t_begin=T - W, threads=threads)
    assert max_abs(out.reshape(qs)[:, T - W:], ro.reshape(qs)[:, T - W:]) <= FWD_TOL


@pytest.mark.parametrize("ws", [False, "scores"], ids=["dq-kernel", "scores"])
@pytest.mark.parametrize("B,T,H,Hkv,D", [(1, 32768, 2, 1, 64), (1, 32768, 1, 1, 64), (1, 20000, 4, 4, 128)])
def test_train_path_long_sequences(gpu, zt, oracle, threads, B, T, H, Hkv, D, ws):
    """Sequences 5-8x C3's length, where score / dS tile offsets in the
    workspace run past 2^31 bytes (4.3 GB of tiles at T = 32768 with two
    heads, 2.1 GB with one): every
    path's kernels (the score-reading head-split and row-split dk/dv kernels,
    and the column-split one past one workgroup per CU) against the twin on
    the first and last rows, plus the full-size column-sum invariants."""
    W = 64
    q, k, v, do = _inputs(gpu, zt, B, T, H, Hkv, D)
    out, lse, dq, dk, dv, delta = _train(gpu, zt, q, k, v, do, B, T, H, Hkv, D, ws=ws)
    for g in (out, lse, dq, dk, dv):
        assert np.all(np.isfinite(g))
    qh, kh, vh, dh = (host(x) for x in (q, k, v, do))
    qs, ks = (B, T, H * D), (B, T, Hkv * D)
    dk4 = dk.reshape(B, T, Hkv, D).astype(np.float64)
    dv4 = dv.reshape(B, T, Hkv, D).astype(np.float64)
    want = dh.reshape(B, T, Hkv, H // Hkv, D).astype(np.float64).sum(axis=(1, 3))
    assert np.max(np.abs(dk4.sum(1))) <= 1e-3 * np.abs(dk4).sum(1).max()
    assert np.max(np.abs(dv4.sum(1) - want)) <= 1e-3 * np.abs(want).max()
    rq, rk, rv = oracle.attention_backward(qh, kh, vh, dh, B, T, H, Hkv, D, t_begin=T - W, threads=threads)
    assert rel_err(dq.reshape(qs)[:, T - W:], rq.reshape(qs)[:, T - W:]) <= BWD_REL
    assert rel_err(dk.reshape(ks)[:, T - W:], rk.reshape(ks)[:, T - W:]) <= BWD_REL
    assert rel_err(dv.reshape(ks)[:, T - W:], rv.reshape(ks)[:, T - W:]) <= BWD_REL
    rq, _, _ = oracle.attention_backward(qh, kh, vh, dh, B, T, H, Hkv, D, t_begin=0, t_end=W, threads=threads)
    assert rel_err(dq.reshape(qs)[:, :W], rq.reshape(qs)[:, :W]) <= BWD_REL
    for t0 in (0, T // 2, T - W):
        ro = oracle.attention_forward(qh, kh, vh, B, T, H, Hkv, D, t_begin=t0, t_end=t0 + W, threads=threads)
        assert max_abs(out.reshape(qs)[:, t0:t0 + W], ro.reshape(qs)[:, t0:t0 + W]) <= FWD_TOL, t0


def test_train_stages_equal_the_whole_and_repeat_bit_for_bit(gpu, zt):
    B, T, H, Hkv, D = 1, 300, 8, 2, 128
    q, k, v, do = _inputs(gpu, zt, B, T, H, Hkv, D)
    a = _train(gpu, zt, q, k, v, do, B, T, H, Hkv, D)
    b = _train(gpu, zt, q, k, v, do, B, T, H, Hkv, D)
    for x, y in zip(a, b):
        assert np.array_equal(x.view(np.uint32), y.view(np.uint32))
    out, lse = gpu.from_numpy(a[0]).cuda(), gpu.from_numpy(a[1]).cuda()
    dq, dk, dv, delta = (_nan(gpu, n) for n in (q.numel(), k.numel(), k.numel(), B * T * H))
    zt.bwd_dq_train(q, k, v, out, do, lse, dq, delta, T, H, Hkv, D, B=B)
    zt.bwd_dkdv_train(q, k, v, out, do, lse, delta, dk, dv, T, H, Hkv, D, B=B)
    gpu.cuda.synchronize()
    for x, y in zip((dq, dk, dv, delta), a[2:]):
        assert np.array_equal(host(x).view(np.uint32), y.view(np.uint32))


def test_train_gate_sees_the_saved_statistics(gpu, zt, oracle):
    # A log-sum-exp off by 0.01 scales every p by e^-0.01: the gate must fail.
    B, T, H, Hkv, D = 1, 64, 4, 2, 64
    q, k, v, do = _inputs(gpu, zt, B, T, H, Hkv, D)
    _, _, dq, dk, dv, _ = _train(gpu, zt, q, k, v, do, B, T, H, Hkv, D, lse_shift=0.01)
    rq, rk, rv = oracle.attention_backward(*(host(x) for x in (q, k, v, do)), B, T, H, Hkv, D)
    assert max(rel_err(dq, rq), rel_err(dk, rk), rel_err(dv, rv)) > BWD_REL


def test_train_ws_stages_and_repeats(gpu, zt):
    """The workspace path is bit-reproducible, its two stages equal the whole,
    and it agrees with the dq-kernel path (dk/dv identically; dq to rounding)."""
    B, T, H, Hkv, D = 2, 130, 8, 2, 64
    q, k, v, do = _inputs(gpu, zt, B, T, H, Hkv, D)
    a = _train(gpu, zt, q, k, v, do, B, T, H, Hkv, D, ws="ds")
    b = _train(gpu, zt, q, k, v, do, B, T, H, Hkv, D, ws="ds")
    for x, y in zip(a, b):
        assert np.array_equal(x.view(np.uint32), y.view(np.uint32))
    c = _train(gpu, zt, q, k, v, do, B, T, H, Hkv, D, ws=False)
    assert rel_err(a[2], c[2]) <= 1e-5 and rel_err(a[3], c[3]) <= 1e-5 and rel_err(a[4], c[4]) <= 1e-5
    out, lse = gpu.from_numpy(a[0]).cuda(), gpu.from_numpy(a[1]).cuda()
    work = _nan(gpu, zt.backward_train_workspace_bytes(B, T, H, Hkv, D) // 4)
    dq, dk, dv = (_nan(gpu, n) for n in (q.numel(), k.numel(), k.numel()))
    zt.backward_train_ws(q, k, v, out, do, lse, dq, dk, dv, work, T, H, Hkv, D, B=B, stage=1)
    zt.backward_train_ws(q, k, v, out, do, lse, dq, dk, dv, work, T, H, Hkv, D, B=B, stage=2)
    gpu.cuda.synchronize()
    for x, y in zip((dq, dk, dv), a[2:5]):
        assert np.array_equal(host(x).view(np.uint32), y.view(np.uint32))
    with pytest.raises(zt.ZtRefused):
        zt.backward_train_ws(q, k, v, out, do, lse, dq, dk, dv, work[:16], T, H, Hkv, D, B=B)


@pytest.mark.parametrize("B,T,H,Hkv,D", [(2, 130, 8, 2, 64), (1, 333, 8, 2, 128), (1, 45, 4, 2, 66),
                                         (2, 77, 8, 2, 256), (1, 100, 4, 2, 160), (1, 90, 8, 2, 192),
                                         (1, 333, 4, 4, 64), (2, 200, 6, 2, 128)])
def test_train_scores_stages_and_repeats(gpu, zt, B, T, H, Hkv, D):
    """The forward that keeps its scores gives the same out and lse bit for bit;
    the backward that reads them back repeats bit for bit, its stages equal the
    whole, and it agrees with the backward that recomputes Q K^T to rounding."""
    q, k, v, do = _inputs(gpu, zt, B, T, H, Hkv, D)
    a = _train(gpu, zt, q, k, v, do, B, T, H, Hkv, D, ws="scores")
    b = _train(gpu, zt, q, k, v, do, B, T, H, Hkv, D, ws="scores")
    for x, y in zip(a, b):
        assert np.array_equal(x.view(np.uint32), y.view(np.uint32))
    c = _train(gpu, zt, q, k, v, do, B, T, H, Hkv, D, ws="ds")
    assert np.array_equal(a[0].view(np.uint32), c[0].view(np.uint32))
    assert np.array_equal(a[1].view(np.uint32), c[1].view(np.uint32))
    assert rel_err(a[2], c[2]) <= 1e-5 and rel_err(a[3], c[3]) <= 1e-5 and rel_err(a[4], c[4]) <= 1e-5
    work = _nan(gpu, zt.backward_train_workspace_bytes(B, T, H, Hkv, D) // 4)
    out, lse = _nan(gpu, q.numel()), _nan(gpu, B * T * H)
    zt.forward_train_ws(q, k, v, out, lse, work, T, H, Hkv, D, B=B)
    dq, dk, dv = (_nan(gpu, n) for n in (q.numel(), k.numel(), k.numel()))
    zt.backward_train_ws(q, k, v, out, do, lse, dq, dk, dv, work, T, H, Hkv, D, B=B, stage=1 | zt.ZT_WS_SCORES)
    zt.backward_train_ws(q, k, v, out, do, lse, dq, dk, dv, work, T, H, Hkv, D, B=B, stage=2)
    gpu.cuda.synchronize()
    for x, y in zip((dq, dk, dv), a[2:5]):
        assert np.array_equal(host(x).view(np.uint32), y.view(np.uint32))
    with pytest.raises(zt.ZtRefused):
        zt.forward_train_ws(q, k, v, out, lse, work[:16], T, H, Hkv, D, B=B)


def test_train_scores_plan_names_the_score_reading_kernel(gpu, zt):
    assert zt.plan_train(1, 4096, 32, 8, 128) == ("zt_fwd8ps_d128_k32", "zt_gemm_dqds_128", "zt_bwd_dkdv8s_d128_hs2")
    assert "dkdv8s" not in zt.plan_train(1, 256, 8, 8, 128)[2]   # MHA: no score-reading kernel
    assert zt.plan_train(4, 1024, 8, 8, 64)[2] == "zt_bwd_dkdv_dmars_d64"  # C2: the scores read back, rows split
    assert zt.plan_train(8, 1024, 8, 8, 64)[2] == "zt_bwd_dkdv8pd_d64_hs1"  # past one workgroup per CU: S formed again
    assert zt.plan_train(8, 1024, 8, 8, 64)[0] == "zt_fwdp_d64_k32"   # MHA: four waves, prefetched
    assert zt.plan_train(4, 1024, 8, 8, 64)[0] == "zt_fwdpk_d64_k32"  # C2: one workgroup per CU, keys split
    assert zt.plan_train(1, 300, 4, 4, 66)[0] == "zt_fwd_d96_k32"     # rows not 16-byte chunks: no prefetch
    assert zt.plan_train(1, 256, 8, 2, 256)[2] == "zt_bwd_dkdv8sd_d256_hs2"   # wide heads: columns split
    assert zt.plan_train(1, 256, 8, 2, 192)[2] == "zt_bwd_dkdv8sd_d192_hs2"
    assert zt.plan_train(1, 256, 8, 2, 160)[2] == "zt_bwd_dkdv_dmas_d160_hs2"   # halves not whole 32 columns
    assert "dmas" not in zt.plan_train(1, 256, 8, 2, 250)[2]   # rows not whole 32-float chunks: no scores


@pytest.mark.parametrize("B,T,H,Hkv,D", [(1, 333, 4, 4, 32), (2, 130, 8, 8, 64), (1, 200, 6, 2, 96),
                                         (1, 150, 3, 1, 128), (1, 16, 2, 2, 64)])
def test_train_row_split_kernel_reads_the_scores(gpu, zt, oracle, tune, B, T, H, Hkv, D):
    """Head groups that cannot be halved (MHA, odd groups) on small grids: the
    row-split dk/dv kernel reading the forward's scores and the same kernel
    forming S again (ZT_ATTN_RSCORES=0) give dq, dk, dv equal to rounding and
    both hold the oracle's gate; out and lse are bit-identical."""
    q, k, v, do = _inputs(gpu, zt, B, T, H, Hkv, D)
    dp = (D + 31) // 32 * 32
    assert zt.plan_train(B, T, H, Hkv, D)[2] == f"zt_bwd_dkdv_dmars_d{dp}"
    a = _train(gpu, zt, q, k, v, do, B, T, H, Hkv, D, ws="scores")
    tune({"ZT_ATTN_RSCORES": 0})
    assert zt.plan_train(B, T, H, Hkv, D)[2] == f"zt_bwd_dkdv_dmar_d{dp}"
    b = _train(gpu, zt, q, k, v, do, B, T, H, Hkv, D, ws="scores")
    for x, y in zip(a[:2], b[:2]):
        assert np.array_equal(x.view(np.uint32), y.view(np.uint32))
    for x, y in zip(a[2:5], b[2:5]):
        assert rel_err(x, y) <= 1e-5
    rq, rk, rv = oracle.attention_backward(*(host(x) for x in (q, k, v, do)), B, T, H, Hkv, D)
    assert max(rel_err(a[2], rq), rel_err(a[3], rk), rel_err(a[4], rv)) <= BWD_REL


@pytest.mark.parametrize("B,T,H,Hkv,D", [(2, 77, 8, 2, 256), (1, 90, 8, 2, 192)])
def test_train_scores_wide_kernels_agree(gpu, zt, oracle, tune, B, T, H, Hkv, D):
    """The column-split kernel and the asynchronously staged one (ZT_ATTN_DSPLIT=0)
    give the same dS, dq, dk and dv to rounding, and both hold the oracle's gate."""
    q, k, v, do = _inputs(gpu, zt, B, T, H, Hkv, D)
    tune({"ZT_ATTN_DSPLIT": "1"})
    assert "dkdv8sd" in zt.plan_train(B, T, H, Hkv, D)[2]
    a = _train(gpu, zt, q, k, v, do, B, T, H, Hkv, D, ws="scores")
    tune({"ZT_ATTN_DSPLIT": "0"})
    assert "dkdv_dmas" in zt.plan_train(B, T, H, Hkv, D)[2]
    b = _train(gpu, zt, q, k, v, do, B, T, H, Hkv, D, ws="scores")
    for x, y in zip(a[2:5], b[2:5]):
        assert rel_err(x, y) <= 1e-5
    rq, rk, rv = oracle.attention_backward(*(host(x) for x in (q, k, v, do)), B, T, H, Hkv, D)
    assert max(rel_err(a[2], rq), rel_err(a[3], rk), rel_err(a[4], rv)) <= BWD_REL


@pytest.mark.parametrize("B,T,H,Hkv,D", [(1, 100, 8, 2, 80), (2, 45, 4, 2, 32), (1, 333, 8, 2, 128),
                                         (1, 70, 8, 2, 256), (1, 61, 8, 2, 192), (1, 333, 4, 4, 64),
                                         (1, 100, 6, 2, 96)])
def test_train_scores_write_nothing_past_the_workspace(gpu, zt, oracle, B, T, H, Hkv, D):
    """Ragged T: the score-reading dk/dv kernel stages 32 rows, so a stage can
    end past the last row; no score or dS tile may be written outside the
    workspace (a guard band after it keeps its fill) and the gradients hold."""
    q, k, v, do = _inputs(gpu, zt, B, T, H, Hkv, D)
    need = zt.backward_train_workspace_bytes(B, T, H, Hkv, D) // 4
    guard = 1 << 16
    whole = gpu.full((need + guard,), 12345.0, device="cuda", dtype=gpu.float32)
    work = whole[:need]
    out, lse = _nan(gpu, q.numel()), _nan(gpu, B * T * H)
    dq, dk, dv = (_nan(gpu, n) for n in (q.numel(), k.numel(), k.numel()))
    zt.forward_train_ws(q, k, v, out, lse, work, T, H, Hkv, D, B=B)
    zt.backward_train_ws(q, k, v, out, do, lse, dq, dk, dv, work, T, H, Hkv, D, B=B, stage=3 | zt.ZT_WS_SCORES)
    gpu.cuda.synchronize()
    assert np.all(host(whole[need:]) == 12345.0)
    rq, rk, rv = oracle.attention_backward(*(host(x) for x in (q, k, v, do)), B, T, H, Hkv, D)
    assert max(rel_err(host(dq), rq), rel_err(host(dk), rk), rel_err(host(dv), rv)) <= BWD_REL


@pytest.mark.parametrize("ws", ["ds", "scores"])
@pytest.mark.parametrize("B,T,H,Hkv,D", [(1, 333, 8, 2, 128), (2, 130, 8, 2, 64), (1, 200, 4, 2, 256),
                                         (1, 150, 8, 2, 96), (1, 77, 4, 1, 128)])
def test_train_paired_tiles_and_128_products_at_small_shapes(gpu, zt, oracle, threads, tune, B, T, H, Hkv, D, ws):
    """The headline path's kernel choices -- paired forward row tiles, paired
    dk/dv key tiles and the 128 x 128 dq-from-dS product -- are made by the
    shape rules only on C3/C5-sized grids; forced here on ragged small shapes
    and graded in full against the twin."""
    tune({"ZT_ATTN_FPAIR": 1, "ZT_ATTN_BPAIR": 1, "ZT_DQDS_TILE": 128, "ZT_DQDS_K": 1})
    assert zt.plan_train(B, T, H, Hkv, D)[1] == "zt_gemm_dqds_128"
    q, k, v, do = _inputs(gpu, zt, B, T, H, Hkv, D)
    out, lse, dq, dk, dv, delta = _train(gpu, zt, q, k, v, do, B, T, H, Hkv, D, ws=ws)
    qh, kh, vh, dh = (host(x) for x in (q, k, v, do))
    assert max_abs(out, oracle.attention_forward(qh, kh, vh, B, T, H, Hkv, D, threads=threads)) <= FWD_TOL
    rq, rk, rv = oracle.attention_backward(qh, kh, vh, dh, B, T, H, Hkv, D, threads=threads)
    assert rel_err(dq, rq) <= BWD_REL
    assert rel_err(dk, rk) <= BWD_REL
    assert rel_err(dv, rv) <= BWD_REL




@pytest.mark.parametrize("B,T,H,Hkv,D", [(1, 333, 8, 2, 128), (1, 90, 8, 2, 256)])
def test_stale_scores_are_refused_not_read(gpu, zt, oracle, capfd, B, T, H, Hkv, D):
    """ZT_WS_SCORES is single use and tied to the forward's q, k and shape: a
    second stage 1 after one forward, a stage 1 for other q or another shape,
    and one after a stage 1 that overwrote the tiles with dS are each refused
    (return 1, reason on stderr) instead of reading tiles that do not hold
    these scores; the call that matches still grades against the twin."""
    q, k, v, do = _inputs(gpu, zt, B, T, H, Hkv, D)
    work = _nan(gpu, zt.backward_train_workspace_bytes(B, T, H, Hkv, D) // 4)
    out, lse = _nan(gpu, q.numel()), _nan(gpu, B * T * H)
    dq, dk, dv = (_nan(gpu, n) for n in (q.numel(), k.numel(), k.numel()))
    scores1 = 1 | zt.ZT_WS_SCORES

    def bwd(qq, stage, T_=T):
        return zt.lib().zt_attn_backward_train_ws(*(zt._ptr(x) for x in (qq, k, v, out, do, lse, dq, dk, dv, work)),
                                                  work.numel() * 4, B, T_, H, Hkv, D, stage, None)

    zt.forward_train_ws(q, k, v, out, lse, work, T, H, Hkv, D, B=B)
    q2 = q.clone()
    capfd.readouterr()
    assert bwd(q2, scores1) == 1                 # other q: refused, the scores stay usable
    assert bwd(q, scores1, T_=T - 1) == 1        # another shape: refused
    assert "ZT_WS_SCORES" in capfd.readouterr().err
    assert bwd(q, scores1) == 0                  # the matching call consumes them
    assert bwd(q, 2) == 0
    gpu.cuda.synchronize()
    rq, rk, rv = oracle.attention_backward(*(host(x) for x in (q, k, v, do)), B, T, H, Hkv, D)
    assert max(rel_err(host(dq), rq), rel_err(host(dk), rk), rel_err(host(dv), rv)) <= BWD_REL
    assert bwd(q, scores1) == 1                  # consumed: the tiles now hold dS
    zt.forward_train_ws(q, k, v, out, lse, work, T, H, Hkv, D, B=B)
    assert bwd(q, 1) == 0                        # a stage 1 that forms S again overwrites them
    assert bwd(q, scores1) == 1
    zt.forward_train(q, k, v, out, lse, T, H, Hkv, D, B=B)
    assert bwd(q, scores1) == 1                  # a forward that stores no scores stamps nothing
    gpu.cuda.synchronize()


@pytest.mark.parametrize("ws", MODES, ids=MODE_IDS)
def test_train_c2_in_full(gpu, zt, oracle, threads, ws):
    """C2 (B=4, T=1024, 8/8 heads, d=64) graded in full on every training path
    (the key-split forward; with ZT_WS_SCORES it keeps its scores and the
    row-split dk/dv kernel reads them back instead of forming S again)."""
    B, T, H, Hkv, D = 4, 1024, 8, 8, 64
    assert zt.plan_train(B, T, H, Hkv, D) == ("zt_fwdpk_d64_k32", "zt_gemm_dqds2_64", "zt_bwd_dkdv_dmars_d64")
    q, k, v, do = _inputs(gpu, zt, B, T, H, Hkv, D)
    out, lse, dq, dk, dv, delta = _train(gpu, zt, q, k, v, do, B, T, H, Hkv, D, ws=ws)
    qh, kh, vh, dh = (host(x) for x in (q, k, v, do))
    assert max_abs(out, oracle.attention_forward(qh, kh, vh, B, T, H, Hkv, D, threads=threads)) <= FWD_TOL
    rq, rk, rv = oracle.attention_backward(qh, kh, vh, dh, B, T, H, Hkv, D, threads=threads)
    assert rel_err(dq, rq) <= BWD_REL
    assert rel_err(dk, rk) <= BWD_REL
    assert rel_err(dv, rv) <= BWD_REL


@pytest.mark.parametrize("parts", [1, 2])
@pytest.mark.parametrize("tile", [64, 128])
@pytest.mark.parametrize("B,T,H,Hkv,D", [(2, 130, 8, 2, 64), (1, 333, 8, 2, 128), (1, 200, 4, 2, 256),
                                         (1, 40, 4, 4, 96), (1, 17, 2, 2, 32)])
def test_train_dq_product_key_parts(gpu, zt, oracle, tune, parts, tile, B, T, H, Hkv, D):
    """The dq-from-dS product with one or two key parts (two four-wave parts
    taking alternate key slabs, their tiles added at the end), on either tile,
    ragged T (a part without a slab in the last step), graded in full."""
    tune({"ZT_DQDS_K": parts, "ZT_DQDS_TILE": tile})
    assert zt.plan_train(B, T, H, Hkv, D)[1] == (f"zt_gemm_dqds2_{tile}" if parts == 2 else f"zt_gemm_dqds_{tile}")
    q, k, v, do = _inputs(gpu, zt, B, T, H, Hkv, D)
    out, lse, dq, dk, dv, delta = _train(gpu, zt, q, k, v, do, B, T, H, Hkv, D, ws="ds")
    rq, rk, rv = oracle.attention_backward(*(host(x) for x in (q, k, v, do)), B, T, H, Hkv, D)
    assert rel_err(dq, rq) <= BWD_REL
