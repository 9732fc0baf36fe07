"""The holder (include/zt_holder.h, the C++ restatement of src/cuda/device.zig's
Attn) driven end to end on the GPU: the model seam (src/model.zig:467-516) and
the decode seam (src/decode.zig:405-473) with their relative 1e-4 gate
(src/train.zig:682-693)."""
import ctypes

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def _holder(zt, t, h, kvh, d):
    p = ctypes.c_void_p()
    assert zt.lib().zt_holder_init(t, h, kvh, d, ctypes.byref(p)) == 0
    return p


def _up(zt, p, which, arr):
    a = np.ascontiguousarray(arr, np.float32)
    return zt.lib().zt_holder_upload(p, which, a.ctypes.data_as(ctypes.c_void_p), a.size)


def _down(zt, p, which, n):
    a = np.empty(n, np.float32)
    assert zt.lib().zt_holder_download(p, a.ctypes.data_as(ctypes.c_void_p), which, n) == 0
    return a


def _rel(a, b):
    return np.max(np.abs(a - b)) / max(np.max(np.abs(b)), 1e-30)


def test_holder_model_seam_forward_and_backward(gpu, zt, oracle):
    T, H, Hkv, D = 256, 4, 2, 32   # the shipped GPT-mini shape (src/model.zig:92-102)
    p = _holder(zt, T, H, Hkv, D)
    try:
        assert zt.lib().zt_holder_total_bytes(p) == 798720
        rng = np.random.default_rng(11)
        q, k, v, do = (rng.standard_normal(n).astype(np.float32) for n in (T * H * D, T * Hkv * D, T * Hkv * D,
                                                                          T * H * D))
        for which, a in ((zt.ZT_BUF_Q, q), (zt.ZT_BUF_K, k), (zt.ZT_BUF_V, v), (zt.ZT_BUF_DOUT, do)):
            assert _up(zt, p, which, a) == 0
        assert zt.lib().zt_holder_forward(p, 1, 64) == 0
        out = _down(zt, p, zt.ZT_BUF_OUT, T * H * D)
        assert _rel(out, oracle.attention_forward(q, k, v, 1, T, H, Hkv, D)) <= 1e-4
        assert zt.lib().zt_holder_backward(p, 64) == 0
        rq, rk, rv = oracle.attention_backward(q, k, v, do, 1, T, H, Hkv, D)
        assert _rel(_down(zt, p, zt.ZT_BUF_DQ, q.size), rq) <= 1e-3
        assert _rel(_down(zt, p, zt.ZT_BUF_DK, k.size), rk) <= 1e-3
        assert _rel(_down(zt, p, zt.ZT_BUF_DV, v.size), rv) <= 1e-3
        # upload is bounds-checked against the buffer it targets
        assert _up(zt, p, zt.ZT_BUF_K, np.zeros(T * H * D)) == zt.ZT_SHAPE_TOO_LARGE
        assert zt.lib().zt_holder_forward_at(p, 1, 64, 0, T + 1, 1) == zt.ZT_SHAPE_TOO_LARGE
        assert zt.lib().zt_holder_forward(p, 0, 64) == zt.ZT_CONFIG_REFUSED
    finally:
        zt.lib().zt_holder_deinit(p)


def test_holder_decode_seam_over_a_filling_cache(gpu, zt, oracle):
    n_ctx, H, Hkv, D = 64, 4, 2, 32
    p = _holder(zt, n_ctx, H, Hkv, D)
    try:
        rng = np.random.default_rng(12)
        kc = rng.standard_normal((n_ctx, Hkv * D)).astype(np.float32)
        vc = rng.standard_normal((n_ctx, Hkv * D)).astype(np.float32)
        qs = rng.standard_normal((n_ctx, H * D)).astype(np.float32)
        for pos in range(n_ctx):
            n_keys = pos + 1
            assert _up(zt, p, zt.ZT_BUF_Q, qs[pos]) == 0
            assert _up(zt, p, zt.ZT_BUF_K, kc[:n_keys]) == 0
            assert _up(zt, p, zt.ZT_BUF_V, vc[:n_keys]) == 0
            assert zt.lib().zt_holder_forward_at(p, 1, 64, n_keys - 1, n_keys, 1) == 0
            out = _down(zt, p, zt.ZT_BUF_OUT, H * D)
            ref = oracle.attn_step(qs[pos], kc, vc, [n_keys], 1, n_ctx, H, Hkv, D)
            assert _rel(out, ref) <= 1e-4, pos
    finally:
        zt.lib().zt_holder_deinit(p)
