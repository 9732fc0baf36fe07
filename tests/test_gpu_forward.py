"""Forward parity on the GPU: zt_attn_forward / zt_attn_forward_batched against
the CPU restatement of src/attention.zig:60-153, max |diff| <= 1e-4."""
import numpy as np
import pytest

from gpuhelp import (FWD_TOL, SEED_K, SEED_Q, SEED_V, THETA, dev_normal, host, max_abs)

pytestmark = pytest.mark.gpu


def _inputs(torch, zt, B, T, H, Hkv, D, sigma=1.0, n_keys=None):
    n_keys = T if n_keys is None else n_keys
    q = dev_normal(torch, zt, B * T * H * D, SEED_Q, sigma)
    k = dev_normal(torch, zt, B * n_keys * Hkv * D, SEED_K, sigma)
    v = dev_normal(torch, zt, B * n_keys * Hkv * D, SEED_V, sigma)
    return q, k, v


def _run(torch, zt, q, k, v, B, T, H, Hkv, D, **kw):
    out = torch.full((B * T * H * D,), float("nan"), device="cuda", dtype=torch.float32)
    zt.forward(q, k, v, out, T, H, Hkv, D, B=B, **kw)
    torch.cuda.synchronize()
    return host(out)


# C1 of BASELINE.json, then ragged T, odd widths and every group shape.
CASES = [
    (1, 128, 4, 2, 32),      # C1: GPT-mini geometry
    (1, 1, 1, 1, 32),
    (1, 2, 2, 1, 32),
    (1, 37, 6, 3, 34),
    (2, 100, 8, 2, 80),
    (1, 200, 4, 4, 96),
    (1, 64, 16, 2, 200),
    (1, 130, 2, 1, 256),
    (3, 17, 8, 8, 64),
    (1, 300, 12, 4, 128),
    (2, 65, 5, 5, 250),
    (1, 96, 8, 1, 160),
]


@pytest.mark.parametrize("B,T,H,Hkv,D", CASES)
def test_forward_matches_twin(gpu, zt, oracle, threads, B, T, H, Hkv, D):
    q, k, v = _inputs(gpu, zt, B, T, H, Hkv, D)
    out = _run(gpu, zt, q, k, v, B, T, H, Hkv, D)
    ref = oracle.attention_forward(host(q), host(k), host(v), B, T, H, Hkv, D, threads=threads)
    assert max_abs(out, ref) <= FWD_TOL


@pytest.mark.parametrize("bk", ["32", "64"])
@pytest.mark.parametrize("B,T,H,Hkv,D", [(1, 150, 8, 2, 128), (2, 70, 4, 4, 256), (1, 99, 6, 3, 66)])
def test_forward_both_key_tiles(gpu, zt, oracle, tune, bk, B, T, H, Hkv, D):
    tune({"ZT_ATTN_BK": bk})
    q, k, v = _inputs(gpu, zt, B, T, H, Hkv, D)
    out = _run(gpu, zt, q, k, v, B, T, H, Hkv, D)
    ref = oracle.attention_forward(host(q), host(k), host(v), B, T, H, Hkv, D)
    assert max_abs(out, ref) <= FWD_TOL


@pytest.mark.parametrize("env", [{"ZT_ATTN_FPF": "1", "ZT_ATTN_FWD_W": "4"}, {"ZT_ATTN_FPF": "1", "ZT_ATTN_FWD_W": "8"},
                                 {"ZT_ATTN_FPF": "0", "ZT_ATTN_FWD_W": "4"}, {"ZT_ATTN_FPF": "0", "ZT_ATTN_FWD_W": "8"},
                                 {"ZT_ATTN_FPF": "1", "ZT_ATTN_FWD_W": "8", "ZT_ATTN_FPAIR": "0"},
                                 {"ZT_ATTN_FPF": "0", "ZT_ATTN_FWD_W": "4", "ZT_ATTN_FPAIR": "0"}])
@pytest.mark.parametrize("B,T,H,Hkv,D", [(1, 150, 8, 2, 128), (2, 70, 4, 4, 256), (1, 99, 6, 3, 66), (1, 45, 4, 1, 32)])
def test_forward_every_variant(gpu, zt, oracle, tune, env, B, T, H, Hkv, D):
    """Four- and eight-wave workgroups, with and without register prefetch of
    the next K/V tile, paired or single row tiles per workgroup, forced through
    the library's tuning variables."""
    tune({"ZT_ATTN_BK": "32"})
    tune(env)
    q, k, v = _inputs(gpu, zt, B, T, H, Hkv, D)
    out = _run(gpu, zt, q, k, v, B, T, H, Hkv, D)
    ref = oracle.attention_forward(host(q), host(k), host(v), B, T, H, Hkv, D)
    assert max_abs(out, ref) <= FWD_TOL


@pytest.mark.parametrize("max_tile", [1, 32, 64, 1024])
def test_forward_any_tile_cap(gpu, zt, oracle, max_tile):
    B, T, H, Hkv, D = 1, 77, 4, 2, 64
    q, k, v = _inputs(gpu, zt, B, T, H, Hkv, D)
    out = _run(gpu, zt, q, k, v, B, T, H, Hkv, D, max_tile=max_tile)
    ref = oracle.attention_forward(host(q), host(k), host(v), B, T, H, Hkv, D)
    assert max_abs(out, ref) <= FWD_TOL


def test_forward_c2_mha_batch4(gpu, zt, oracle, threads):
    B, T, H, Hkv, D = 4, 1024, 8, 8, 64   # C2
    q, k, v = _inputs(gpu, zt, B, T, H, Hkv, D)
    out = _run(gpu, zt, q, k, v, B, T, H, Hkv, D)
    ref = oracle.attention_forward(host(q), host(k), host(v), B, T, H, Hkv, D, threads=threads)
    assert max_abs(out, ref) <= FWD_TOL


def _rope(gpu, zt, x, T, H, D):
    y = gpu.empty_like(x)
    zt.rope(x, y, T, H * D, 0, THETA, D)
    return y


def test_forward_c3_llama3_rope(gpu, zt, oracle, threads):
    B, T, H, Hkv, D = 1, 4096, 32, 8, 128   # C3, RoPE pre-applied to Q and K
    q, k, v = _inputs(gpu, zt, B, T, H, Hkv, D)
    q, k = _rope(gpu, zt, q, T, H, D), _rope(gpu, zt, k, T, Hkv, D)
    out = _run(gpu, zt, q, k, v, B, T, H, Hkv, D).reshape(T, H * D)
    qh, kh, vh = host(q), host(k), host(v)
    # Rows are independent: grade the first and last 64 rows (the last see all 4096 keys).
    for t0, t1 in ((0, 64), (T - 64, T)):
        ref = oracle.attention_forward(qh, kh, vh, B, T, H, Hkv, D, t_begin=t0, t_end=t1,
                                       threads=threads).reshape(T, H * D)
        assert max_abs(out[t0:t1], ref[t0:t1]) <= FWD_TOL, (t0, t1)
    assert np.all(np.isfinite(out))


def test_forward_c5_wide_head(gpu, zt, oracle, threads):
    B, T, H, Hkv, D = 2, 2048, 16, 4, 256   # C5, variance 2
    q, k, v = _inputs(gpu, zt, B, T, H, Hkv, D, sigma=np.sqrt(2.0))
    out = _run(gpu, zt, q, k, v, B, T, H, Hkv, D).reshape(B, T, H * D)
    qh, kh, vh = host(q), host(k), host(v)
    for t0, t1 in ((0, 48), (T - 48, T)):
        ref = oracle.attention_forward(qh, kh, vh, B, T, H, Hkv, D, t_begin=t0, t_end=t1,
                                       threads=threads).reshape(B, T, H * D)
        assert max_abs(out[:, t0:t1], ref[:, t0:t1]) <= FWD_TOL, (t0, t1)


@pytest.mark.parametrize("T,q_offset,n_keys", [(1, 0, 1), (1, 99, 100), (5, 20, 25), (16, 100, 116), (33, 0, 33)])
def test_forward_at_offset(gpu, zt, oracle, T, q_offset, n_keys):
    B, H, Hkv, D = 1, 8, 2, 64
    q, k, v = _inputs(gpu, zt, B, T, H, Hkv, D, n_keys=n_keys)
    out = _run(gpu, zt, q, k, v, B, T, H, Hkv, D, q_offset=q_offset, n_keys=n_keys)
    ref = oracle.attention_forward_at(host(q), host(k), host(v), B, T, H, Hkv, D, q_offset, n_keys)
    assert max_abs(out, ref) <= FWD_TOL


def test_forward_batched_cache_rows(gpu, zt, oracle):
    # kv_rows > n_keys: each sequence's cache is a larger buffer, only n_keys rows read.
    B, T, H, Hkv, D, n_keys, kv_rows = 3, 4, 4, 2, 32, 20, 32
    q = dev_normal(gpu, zt, B * T * H * D, SEED_Q)
    k = dev_normal(gpu, zt, B * kv_rows * Hkv * D, SEED_K)
    v = dev_normal(gpu, zt, B * kv_rows * Hkv * D, SEED_V)
    out = _run(gpu, zt, q, k, v, B, T, H, Hkv, D, q_offset=n_keys - T, n_keys=n_keys, kv_rows=kv_rows)
    kh = host(k).reshape(B, kv_rows, -1)[:, :n_keys]
    vh = host(v).reshape(B, kv_rows, -1)[:, :n_keys]
    ref = oracle.attention_forward_at(host(q), kh, vh, B, T, H, Hkv, D, n_keys - T, n_keys)
    assert max_abs(out, ref) <= FWD_TOL


def test_forward_reference_known_answers_on_device(gpu, zt, golden):
    for c in golden["attention"]:
        t = lambda x: gpu.tensor(np.float32(x), device="cuda")
        D, T = c["D"], c["T"]
        if D < 32:   # the device admits widths 32..256: pad the head with zero columns
            pad = 32 - D
            def widen(x, heads):
                a = np.float32(x).reshape(T, heads, D)
                return np.concatenate([a, np.zeros((T, heads, pad), np.float32)], -1).ravel()
            q, k, v = widen(c["q"], c["H"]), widen(c["k"], c["Hkv"]), widen(c["v"], c["Hkv"])
            # zero columns leave q.k unchanged but the scale is 1/sqrt(32): rescale q to keep 1/sqrt(D)
            q = (q * np.float32(np.sqrt(32.0 / D))).astype(np.float32)
        else:
            q, k, v = c["q"], c["k"], c["v"]
        Dp = max(D, 32)
        out = gpu.empty(T * c["H"] * Dp, device="cuda", dtype=gpu.float32)
        zt.forward(t(q), t(k), t(v), out, T, c["H"], c["Hkv"], Dp)
        gpu.cuda.synchronize()
        got = host(out).reshape(T, c["H"], Dp)[:, :, :D].ravel()
        tol = 1e-5 if c["tol"] is None else max(c["tol"], 1e-5)
        assert max_abs(got, c["out"]) <= tol, c["name"]


def test_forward_gate_catches_broken_references(gpu, zt, oracle):
    """Negative controls (the reference's BROKEN variants, attn_kernels.cu:150-158),
    planted in the CPU reference: each wrong answer must fail the 1e-4 gate."""
    B, T, H, Hkv, D = 1, 96, 8, 2, 64
    q, k, v = _inputs(gpu, zt, B, T, H, Hkv, D)
    out = _run(gpu, zt, q, k, v, B, T, H, Hkv, D)
    qh, kh, vh = host(q), host(k), host(v)
    g = H // Hkv
    # 2: every query head reads kv head 0 (GQA collapsed)
    k0 = np.tile(kh.reshape(T, Hkv, D)[:, :1], (1, Hkv, 1)).ravel()
    v0 = np.tile(vh.reshape(T, Hkv, D)[:, :1], (1, Hkv, 1)).ravel()
    assert max_abs(out, oracle.attention_forward(qh, k0, v0, B, T, H, Hkv, D)) > FWD_TOL
    # 4: the 1/sqrt(d) scale dropped
    assert max_abs(out, oracle.attention_forward(qh * np.float32(np.sqrt(D)), kh, vh, B, T, H, Hkv, D)) > FWD_TOL
    # 1: the causal mask dropped (full softmax over all T keys)
    from npref import attention_f64
    from npref import np as _np  # noqa: F401
    full = np.zeros((T, H * D))
    qa, ka, va = qh.reshape(T, H, D), kh.reshape(T, Hkv, D), vh.reshape(T, Hkv, D)
    for h in range(H):
        s = qa[:, h].astype(np.float64) @ ka[:, h // g].T.astype(np.float64) / np.sqrt(D)
        p = np.exp(s - s.max(1, keepdims=True))
        full[:, h * D:(h + 1) * D] = (p / p.sum(1, keepdims=True)) @ va[:, h // g]
    assert max_abs(out, full.ravel()) > FWD_TOL
    assert max_abs(out, attention_f64(qh, kh, vh, T, H, Hkv, D).ravel()) <= FWD_TOL


@pytest.mark.parametrize("fks", ["1", "2"])
@pytest.mark.parametrize("B,T,H,Hkv,D", [(4, 1024, 8, 8, 64), (1, 77, 3, 3, 32), (2, 130, 6, 2, 96), (1, 200, 5, 5, 128),
                                         (1, 16, 2, 2, 64), (3, 65, 4, 4, 128)])
def test_forward_key_split_against_twin(gpu, zt, oracle, tune, threads, fks, B, T, H, Hkv, D):
    """The key-split forward (4 row blocks x 2 key parts, merged at the end)
    forced on and off for one query head per workgroup -- MHA and odd
    groups, ragged T, widths to 128 -- through zt_attn_forward and the
    training forward's lse."""
    tune({"ZT_ATTN_FKS": fks})
    name = zt.plan(B, T, H, Hkv, D)[0]
    assert name.startswith("zt_fwdpk_" if fks == "2" else "zt_fwdp_"), name
    q, k, v = _inputs(gpu, zt, B, T, H, Hkv, D)
    out = _run(gpu, zt, q, k, v, B, T, H, Hkv, D)
    qh, kh, vh = host(q), host(k), host(v)
    ref = oracle.attention_forward(qh, kh, vh, B, T, H, Hkv, D, threads=threads)
    assert max_abs(out, ref) <= FWD_TOL
    out2 = gpu.full((B * T * H * D,), float("nan"), device="cuda")
    lse = gpu.full((B * T * H,), float("nan"), device="cuda")
    zt.forward_train(q, k, v, out2, lse, T, H, Hkv, D, B=B)
    gpu.cuda.synchronize()
    assert max_abs(host(out2), ref) <= FWD_TOL
    m, l, _ = oracle.attention_row_stats(qh, kh, vh, np.zeros_like(qh), B, T, H, Hkv, D)
    want = m + np.log(l)
    assert np.max(np.abs(host(lse) - want)) <= 1e-5 * max(1.0, np.abs(want).max())


@pytest.mark.parametrize("T,q_offset,n_keys", [(5, 20, 25), (16, 100, 116), (70, 30, 100), (33, 0, 33), (40, 90, 130)])
def test_forward_key_split_at_offset(gpu, zt, oracle, tune, T, q_offset, n_keys):
    """Chunked prefill (queries at an offset over a longer key range, so the
    second key part's first tile can lie wholly past a row) on the key-split kernel."""
    tune({"ZT_ATTN_FKS": "2"})
    B, H, Hkv, D = 1, 4, 4, 64
    assert zt.plan(B, T, H, Hkv, D)[0].startswith("zt_fwdpk_")
    q, k, v = _inputs(gpu, zt, B, T, H, Hkv, D, n_keys=n_keys)
    out = _run(gpu, zt, q, k, v, B, T, H, Hkv, D, q_offset=q_offset, n_keys=n_keys)
    ref = oracle.attention_forward_at(host(q), host(k), host(v), B, T, H, Hkv, D, q_offset, n_keys)
    assert max_abs(out, ref) <= FWD_TOL
