"""Decode-step parity on the GPU: zt_attn_decode (split-K) and the reference's
own decode route (zt_attn_forward with T = 1, q_offset = n_keys - 1,
src/decode.zig:462) against the CPU restatement of src/decode.zig:326-392,
max |diff| <= 1e-4."""
import numpy as np
import pytest

from gpuhelp import FWD_TOL, SEED_KC, SEED_Q, SEED_VC, dev_normal, host, max_abs

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
