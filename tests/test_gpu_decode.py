"""Decode-step parity on the GPU: zt_attn_decode (split-K), the reference's
own decode route (zt_attn_forward with T = 1, q_offset = n_keys - 1,
src/decode.zig:462) and zt_attn_decode_step (RoPE + device cache append +
attention, src/decode.zig:244-270) against the CPU restatement of
src/decode.zig:326-392, max |diff| <= 1e-4."""
import numpy as np
import pytest

from gpuhelp import FWD_TOL, SEED_K, SEED_KC, SEED_Q, SEED_V, SEED_VC, THETA, dev_normal, host, max_abs

pytestmark = pytest.mark.gpu


def _decode(gpu, zt, B, n_ctx, H, Hkv, D, n_keys, sigma=1.0):
    q = dev_normal(gpu, zt, B * H * D, SEED_Q, sigma)
    kc = dev_normal(gpu, zt, B * n_ctx * Hkv * D, SEED_KC, sigma)
    vc = dev_normal(gpu, zt, B * n_ctx * Hkv * D, SEED_VC, sigma)
    out = gpu.full((B * H * D,), float("nan"), device="cuda", dtype=gpu.float32)
    ws = gpu.empty(zt.decode_workspace_bytes(B, n_ctx, H, Hkv, D) // 4 + 1, device="cuda", dtype=gpu.float32)
    zt.decode(q, kc, vc, out, n_keys, B, n_ctx, H, Hkv, D, ws)
    gpu.cuda.synchronize()
    return q, kc, vc, host(out)


def test_decode_c4(gpu, zt, oracle, threads):
    B, n_ctx, H, Hkv, D = 64, 8192, 32, 8, 128   # C4: every sequence at position 8191
    n_keys = [n_ctx] * B
    q, kc, vc, out = _decode(gpu, zt, B, n_ctx, H, Hkv, D, n_keys)
    ref = oracle.attn_step(host(q), host(kc), host(vc), n_keys, B, n_ctx, H, Hkv, D, threads=threads)
    assert max_abs(out, ref) <= FWD_TOL


@pytest.mark.parametrize("wgs", ["256", "512", "2048", "32768"])
def test_decode_any_split(gpu, zt, oracle, threads, tune, wgs):
    """However the key axis is split (the workgroup target, a tuning
    variable), the answer holds: 8 sequences x 8 kv heads of 2000 rows run in
    4, 8 or 32 chunks per sequence (the C4 test runs one chunk per sequence)."""
    tune({"ZT_DEC_WGS": wgs})
    B, n_ctx, H, Hkv, D = 8, 2000, 32, 8, 128
    n_keys = [2000, 1999, 1500, 1024, 1023, 600, 65, 1]
    q, kc, vc, out = _decode(gpu, zt, B, n_ctx, H, Hkv, D, n_keys)
    ref = oracle.attn_step(host(q), host(kc), host(vc), n_keys, B, n_ctx, H, Hkv, D, threads=threads)
    assert max_abs(out, ref) <= FWD_TOL


@pytest.mark.parametrize("B,n_ctx,H,Hkv,D", [
    (5, 300, 32, 8, 128), (3, 1000, 8, 8, 64), (4, 257, 16, 2, 256), (2, 100, 6, 3, 32),
    (7, 50, 4, 4, 80), (1, 1, 4, 2, 32), (70, 40, 8, 2, 128), (2, 999, 16, 1, 96), (3, 64, 12, 4, 34),
])
def test_decode_ragged(gpu, zt, oracle, threads, B, n_ctx, H, Hkv, D):
    rng = np.random.default_rng(B * 1000 + n_ctx)
    n_keys = [int(x) for x in rng.integers(1, n_ctx + 1, size=B)]
    n_keys[0] = n_ctx
    n_keys[-1] = 1
    q, kc, vc, out = _decode(gpu, zt, B, n_ctx, H, Hkv, D, n_keys)
    ref = oracle.attn_step(host(q), host(kc), host(vc), n_keys, B, n_ctx, H, Hkv, D, threads=threads)
    assert max_abs(out, ref) <= FWD_TOL


def test_decode_through_the_reference_entry_point(gpu, zt, oracle):
    # The reference's decode seam: zt_attn_forward(T=1, q_offset=n_keys-1, n_keys).
    n_ctx, H, Hkv, D = 700, 32, 8, 128
    q, kc, vc, out = _decode(gpu, zt, 1, n_ctx, H, Hkv, D, [n_ctx])
    out2 = gpu.full((H * D,), float("nan"), device="cuda", dtype=gpu.float32)
    zt.forward(q, kc, vc, out2, 1, H, Hkv, D, q_offset=n_ctx - 1, n_keys=n_ctx)
    gpu.cuda.synchronize()
    ref = oracle.attn_step(host(q), host(kc), host(vc), [n_ctx], 1, n_ctx, H, Hkv, D)
    assert max_abs(host(out2), ref) <= FWD_TOL
    assert max_abs(out, ref) <= FWD_TOL


@pytest.mark.parametrize("env", [{}, {"ZT_ROW_W": 4}, {"ZT_ROW_W": 8, "ZT_ROW_G": 2}, {"ZT_ROW_W": 4, "ZT_ROW_G": 2},
                                 {"ZT_ROW_G": 4}, {"ZT_ROW_G": 8}])
@pytest.mark.parametrize("B,H,Hkv,D,q_offset,n_keys,kv_rows", [
    (1, 32, 8, 128, 2999, 3000, 3000),   # the reference seam: the last position sees every key
    (1, 32, 8, 128, 1234, 3000, 3000),   # a query mid-cache sees only the first q_offset + 1 keys
    (3, 16, 2, 256, 99, 100, 160),       # batched over a larger preallocated cache
    (1, 6, 3, 34, 40, 41, 41), (2, 8, 8, 64, 0, 1, 5), (1, 4, 1, 96, 77, 78, 78),
    (70, 8, 2, 80, 19, 20, 20),          # more than one launch of 64 sequences
    (1, 16, 2, 250, 500, 600, 600), (2, 10, 5, 160, 63, 64, 64),
])
def test_one_row_forward_takes_the_decode_kernel(gpu, zt, oracle, tune, env, B, H, Hkv, D, q_offset, n_keys,
                                                kv_rows):
    """zt_attn_forward(_batched) with T = 1 runs the decode kernel with one chunk
    per (sequence, kv head, head sub-group) and no workspace: every head
    sub-group size and both wave counts, any width, a query anywhere in the
    cache, caches longer than n_keys."""
    tune(env)
    assert zt.plan(B, 1, H, Hkv, D)[0].startswith(("zt_dec_", "zt_dec8_"))
    q = dev_normal(gpu, zt, B * H * D, SEED_Q)
    kc = dev_normal(gpu, zt, B * kv_rows * Hkv * D, SEED_KC)
    vc = dev_normal(gpu, zt, B * kv_rows * Hkv * D, SEED_VC)
    out = gpu.full((B * H * D,), float("nan"), device="cuda", dtype=gpu.float32)
    zt.forward(q, kc, vc, out, 1, H, Hkv, D, q_offset=q_offset, n_keys=n_keys, B=B, kv_rows=kv_rows)
    gpu.cuda.synchronize()
    ref = oracle.attn_step(host(q), host(kc), host(vc), [q_offset + 1] * B, B, kv_rows, H, Hkv, D)
    assert max_abs(host(out), ref) <= FWD_TOL


def test_decode_over_a_filling_cache(gpu, zt, oracle):
    # src/decode_test.zig:222-330: every position of a filling cache agrees.
    n_ctx, H, Hkv, D = 48, 4, 2, 32
    q = dev_normal(gpu, zt, n_ctx * H * D, SEED_Q)
    kc = dev_normal(gpu, zt, n_ctx * Hkv * D, SEED_KC)
    vc = dev_normal(gpu, zt, n_ctx * Hkv * D, SEED_VC)
    ws = gpu.empty(zt.decode_workspace_bytes(1, n_ctx, H, Hkv, D) // 4 + 1, device="cuda", dtype=gpu.float32)
    qh, kh, vh = host(q).reshape(n_ctx, H * D), host(kc), host(vc)
    for pos in range(n_ctx):
        out = gpu.empty(H * D, device="cuda", dtype=gpu.float32)
        zt.decode(q[pos * H * D:(pos + 1) * H * D], kc, vc, out, [pos + 1], 1, n_ctx, H, Hkv, D, ws)
        gpu.cuda.synchronize()
        ref = oracle.attn_step(qh[pos], kh, vh, [pos + 1], 1, n_ctx, H, Hkv, D)
        assert max_abs(host(out), ref) <= FWD_TOL, pos


def test_decode_refuses_bad_n_keys(gpu, zt):
    B, n_ctx, H, Hkv, D = 2, 16, 4, 2, 32
    q = gpu.zeros(B * H * D, device="cuda")
    kc = gpu.zeros(B * n_ctx * Hkv * D, device="cuda")
    out = gpu.zeros(B * H * D, device="cuda")
    ws = gpu.empty(zt.decode_workspace_bytes(B, n_ctx, H, Hkv, D) // 4 + 1, device="cuda")
    for bad in ([0, 5], [5, 17], [-1, 3]):
        with pytest.raises(zt.ZtRefused):
            zt.decode(q, kc, kc, out, bad, B, n_ctx, H, Hkv, D, ws)


def _step_ws(gpu, zt, B, n_ctx, H, Hkv, D):
    return gpu.empty(zt.decode_step_workspace_bytes(B, n_ctx, H, Hkv, D) // 4 + 1, device="cuda")


def _same_rows(dev, ref, tol):
    # Unwritten rows stay NaN on both sides; written rows agree to tol.
    dev, ref = np.asarray(dev), np.asarray(ref)
    assert np.array_equal(np.isnan(dev), np.isnan(ref))
    ok = ~np.isnan(ref)
    assert max_abs(dev[ok], ref[ok]) <= tol


@pytest.mark.parametrize("B,n_ctx,H,Hkv,D,start,steps", [
    (3, 40, 8, 2, 64, [0, 5, 17], 12),
    (2, 24, 6, 3, 34, [0, 9], 15),
    (1, 16, 4, 1, 256, [3], 13),
    (70, 12, 4, 2, 32, None, 3),
])
def test_decode_step_fills_a_device_cache(gpu, zt, oracle, B, n_ctx, H, Hkv, D, start, steps):
    # Rows below each sequence's start hold an earlier history; rows from the
    # start on are NaN, so a row the step did not write, or one past pos that
    # the attention read, would show.  Sequences sit at ragged positions.
    start = start or [int(x) for x in np.random.default_rng(B).integers(0, n_ctx - steps + 1, size=B)]
    rng = np.random.default_rng(n_ctx * 7 + D)
    kh = np.full((B, n_ctx, Hkv * D), np.nan, np.float32)
    vh = np.full((B, n_ctx, Hkv * D), np.nan, np.float32)
    for b, p0 in enumerate(start):
        kh[b, :p0] = rng.standard_normal((p0, Hkv * D))
        vh[b, :p0] = rng.standard_normal((p0, Hkv * D))
    kh, vh = kh.ravel(), vh.ravel()
    kc, vc = gpu.from_numpy(kh.copy()).cuda(), gpu.from_numpy(vh.copy()).cuda()
    ws = _step_ws(gpu, zt, B, n_ctx, H, Hkv, D)
    for s in range(steps):
        q = dev_normal(gpu, zt, B * H * D, SEED_Q + 0x100 * s)
        k = dev_normal(gpu, zt, B * Hkv * D, SEED_K + 0x100 * s)
        v = dev_normal(gpu, zt, B * Hkv * D, SEED_V + 0x100 * s)
        out = gpu.full((B * H * D,), float("nan"), device="cuda")
        pos = [p + s for p in start]
        zt.decode_step(q, k, v, kc, vc, out, pos, B, n_ctx, H, Hkv, D, ws, THETA)
        gpu.cuda.synchronize()
        ref, kh, vh = oracle.decode_step(host(q), host(k), host(v), kh, vh, pos, B, n_ctx, H, Hkv, D, THETA)
        assert max_abs(host(out), ref) <= FWD_TOL, (s, pos)
    _same_rows(host(kc), kh, 2e-6)
    _same_rows(host(vc), vh, 0.0)


def test_decode_step_at_the_c4_shape(gpu, zt, oracle, threads):
    # C4's cache (n_ctx 8192, 32 heads over 8, d 128) with 16 sequences at
    # ragged positions up to the last row; the expectation composes the pinned
    # restatements: rope on q and k at pos, the append, attnStep over pos + 1.
    B, n_ctx, H, Hkv, D = 16, 8192, 32, 8, 128
    pos = [n_ctx - 1] * 4 + [int(x) for x in np.random.default_rng(4).integers(0, n_ctx, size=B - 4)]
    kc = dev_normal(gpu, zt, B * n_ctx * Hkv * D, SEED_KC)
    vc = dev_normal(gpu, zt, B * n_ctx * Hkv * D, SEED_VC)
    kh, vh = host(kc).reshape(B, n_ctx, Hkv * D), host(vc).reshape(B, n_ctx, Hkv * D)
    q = dev_normal(gpu, zt, B * H * D, SEED_Q)
    k = dev_normal(gpu, zt, B * Hkv * D, SEED_K)
    v = dev_normal(gpu, zt, B * Hkv * D, SEED_V)
    out = gpu.full((B * H * D,), float("nan"), device="cuda")
    zt.decode_step(q, k, v, kc, vc, out, pos, B, n_ctx, H, Hkv, D, _step_ws(gpu, zt, B, n_ctx, H, Hkv, D), THETA)
    gpu.cuda.synchronize()
    qh, knh, vnh = host(q).reshape(B, H * D), host(k).reshape(B, Hkv * D), host(v).reshape(B, Hkv * D)
    qr = np.stack([oracle.rope(qh[b], 1, H * D, pos[b], THETA, D) for b in range(B)])
    for b in range(B):
        kh[b, pos[b]] = oracle.rope(knh[b], 1, Hkv * D, pos[b], THETA, D)
        vh[b, pos[b]] = vnh[b]
    ref = oracle.attn_step(qr, kh, vh, [p + 1 for p in pos], B, n_ctx, H, Hkv, D, threads=threads)
    assert max_abs(host(out), ref) <= FWD_TOL
    assert max_abs(host(kc), kh.ravel()) <= 2e-6
    assert np.array_equal(host(vc), vh.ravel())


def test_decode_step_refuses_a_full_cache_and_writes_nothing(gpu, zt):
    B, n_ctx, H, Hkv, D = 2, 8, 4, 2, 32
    kc = gpu.zeros(B * n_ctx * Hkv * D, device="cuda")
    vc = gpu.zeros(B * n_ctx * Hkv * D, device="cuda")
    q, k = gpu.ones(B * H * D, device="cuda"), gpu.ones(B * Hkv * D, device="cuda")
    out = gpu.zeros(B * H * D, device="cuda")
    with pytest.raises(zt.ZtRefused):
        zt.decode_step(q, k, k, kc, vc, out, [7, 8], B, n_ctx, H, Hkv, D, _step_ws(gpu, zt, B, n_ctx, H, Hkv, D))
    gpu.cuda.synchronize()
    assert float(kc.abs().sum()) == 0.0 and float(vc.abs().sum()) == 0.0 and float(out.abs().sum()) == 0.0
