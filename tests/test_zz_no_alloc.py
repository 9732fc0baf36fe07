"""zt_attn_decode_noalloc: zt_attn_decode with the chunk partials in the
library's fixed per-device scratch instead of a caller workspace (no
allocation of any kind).  Graded against zt_attn_decode, the entry point it
varies, on the same inputs -- bit for bit, since both run the same kernels
with the same split -- and against the CPU restatement of src/decode.zig:326-392
(max |diff| <= 1e-4), over consecutive calls whose scratch use differs (the
second smaller than the first), so a result that leaned on the previous
call's partials would show."""
import ctypes

import numpy as np
import pytest

from gpuhelp import FWD_TOL, SEED_KC, SEED_Q, SEED_VC, dev_normal, host, max_abs

pytestmark = pytest.mark.gpu


def _call(gpu, zt, B, n_ctx, H, Hkv, D, n_keys, seed_off):
    q = dev_normal(gpu, zt, B * H * D, SEED_Q + seed_off)
    kc = dev_normal(gpu, zt, B * n_ctx * Hkv * D, SEED_KC + seed_off)
    vc = dev_normal(gpu, zt, B * n_ctx * Hkv * D, SEED_VC + seed_off)
    got = gpu.full((B * H * D,), float("nan"), device="cuda", dtype=gpu.float32)
    arr = (ctypes.c_int * B)(*n_keys)
    stream = ctypes.c_void_p(gpu.cuda.current_stream().cuda_stream)
    print(f"[noalloc] B={B} n_ctx={n_ctx} H={H}/{Hkv} d={D}", flush=True)
    rc = zt.lib().zt_attn_decode_noalloc(ctypes.c_void_p(q.data_ptr()), ctypes.c_void_p(kc.data_ptr()),
                                         ctypes.c_void_p(vc.data_ptr()), ctypes.c_void_p(got.data_ptr()), arr, B,
                                         n_ctx, H, Hkv, D, stream)
    assert rc == 0
    want = gpu.full((B * H * D,), float("nan"), device="cuda", dtype=gpu.float32)
    ws = gpu.empty(zt.decode_workspace_bytes(B, n_ctx, H, Hkv, D) // 4 + 1, device="cuda", dtype=gpu.float32)
    zt.decode(q, kc, vc, want, n_keys, B, n_ctx, H, Hkv, D, ws)
    gpu.cuda.synchronize()
    return q, kc, vc, host(got), host(want)


def test_noalloc_decode_matches_the_workspace_decode_on_consecutive_calls(gpu, zt, oracle, threads):
    # (shape, n_keys): 32 key chunks per sequence, then a smaller call of 24
    # chunks, then one chunk per sequence (no partials at all).
    calls = [((2, 8192, 32, 8, 128), [8192, 5000]),
             ((1, 3000, 8, 2, 64), [2999]),
             ((64, 300, 32, 8, 128), [300 - i for i in range(64)])]
    for i, ((B, n_ctx, H, Hkv, D), n_keys) in enumerate(calls):
        q, kc, vc, got, want = _call(gpu, zt, B, n_ctx, H, Hkv, D, n_keys, 16 * i)
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), (B, n_ctx, H, Hkv, D)
        ref = oracle.attn_step(host(q), host(kc), host(vc), n_keys, B, n_ctx, H, Hkv, D, threads=threads)
        assert max_abs(got, ref) <= FWD_TOL, (B, n_ctx, H, Hkv, D)


def test_noalloc_decode_refuses_beyond_its_scratch(gpu, zt, tune, capfd):
    """A split whose partials exceed the fixed scratch is refused before any
    launch (only a forced split goes past it: the default one fits every shape)."""
    L = zt.lib()
    tune({"ZT_DEC_WGS": 32768})
    B, n_ctx, H, Hkv, D = 1, 1 << 20, 64, 8, 256
    arr = (ctypes.c_int * B)(n_ctx)
    assert L.zt_attn_decode_noalloc(None, None, None, None, arr, B, n_ctx, H, Hkv, D, None) == 1
    assert "beyond the library's fixed" in capfd.readouterr().err


def test_noalloc_decode_allocates_nothing_and_replays_from_a_graph(gpu, zt):
    """After one warm-up call (the library's set-up on the device), a call
    leaves the device's free memory unchanged, and the call captured into a
    HIP graph replays to zt_attn_decode's result bit for bit, replay after
    replay, with eager calls on other inputs (which reuse the same scratch)
    and synchronisations between the replays."""
    B, n_ctx, H, Hkv, D = 2, 8192, 32, 8, 128      # keys split into chunks: the partials use the scratch
    n_keys = [8192, 5000]
    arr = (ctypes.c_int * B)(*n_keys)
    L = zt.lib()

    def tensors(off):
        return (dev_normal(gpu, zt, B * H * D, SEED_Q + off), dev_normal(gpu, zt, B * n_ctx * Hkv * D, SEED_KC + off),
                dev_normal(gpu, zt, B * n_ctx * Hkv * D, SEED_VC + off))

    def call(q, kc, vc, out, stream):
        return L.zt_attn_decode_noalloc(ctypes.c_void_p(q.data_ptr()), ctypes.c_void_p(kc.data_ptr()),
                                        ctypes.c_void_p(vc.data_ptr()), ctypes.c_void_p(out.data_ptr()), arr, B,
                                        n_ctx, H, Hkv, D, ctypes.c_void_p(stream.cuda_stream))

    print(f"[noalloc graph] B={B} n_ctx={n_ctx} H={H}/{Hkv} d={D}", flush=True)
    q, kc, vc = tensors(0)
    q2, kc2, vc2 = tensors(32)
    got = gpu.full((B * H * D,), float("nan"), device="cuda", dtype=gpu.float32)
    other = gpu.empty_like(got)
    cur = gpu.cuda.current_stream()
    assert call(q, kc, vc, got, cur) == 0          # warm-up
    gpu.cuda.synchronize()
    free0 = gpu.cuda.mem_get_info()[0]
    assert call(q, kc, vc, got, cur) == 0
    gpu.cuda.synchronize()
    assert gpu.cuda.mem_get_info()[0] == free0

    want = gpu.empty_like(got)
    ws = gpu.empty(zt.decode_workspace_bytes(B, n_ctx, H, Hkv, D) // 4 + 1, device="cuda", dtype=gpu.float32)
    zt.decode(q, kc, vc, want, n_keys, B, n_ctx, H, Hkv, D, ws)
    gpu.cuda.synchronize()
    want_h = host(want)

    graph = gpu.cuda.CUDAGraph()
    got.fill_(float("nan"))
    gpu.cuda.synchronize()
    with gpu.cuda.graph(graph):
        assert call(q, kc, vc, got, gpu.cuda.current_stream()) == 0
    for i in range(4):
        got.fill_(float("nan"))
        graph.replay()
        gpu.cuda.synchronize()
        assert np.array_equal(host(got).view(np.uint32), want_h.view(np.uint32)), i
        assert call(q2, kc2, vc2, other, cur) == 0     # eager use of the same scratch between replays
        gpu.cuda.synchronize()
        assert np.all(np.isfinite(host(other)))
    del graph
