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


def _fill(zt, p, which, n, seed, sigma=1.0):
    assert zt.lib().zt_fill_normal(zt.lib().zt_holder_buffer(p, which), n, seed, 0.0, sigma, None) == 0


def _inputs(zt, p, T, H, Hkv, D, rope=False):
    from gpuhelp import SEED_DO, SEED_K, SEED_Q, SEED_V, THETA
    L = zt.lib()
    _fill(zt, p, zt.ZT_BUF_Q, T * H * D, SEED_Q)
    _fill(zt, p, zt.ZT_BUF_K, T * Hkv * D, SEED_K)
    _fill(zt, p, zt.ZT_BUF_V, T * Hkv * D, SEED_V)
    _fill(zt, p, zt.ZT_BUF_DOUT, T * H * D, SEED_DO)
    if rope:
        qb, kb = L.zt_holder_buffer(p, zt.ZT_BUF_Q), L.zt_holder_buffer(p, zt.ZT_BUF_K)
        assert L.zt_rope_qk_forward(qb, kb, qb, kb, 1, T, H, Hkv, D, 0, THETA, None) == 0
    # Written through the raw pointers: drop any saved state, as zt_holder_buffer's contract asks.
    L.zt_holder_forget(p)
    return [_down(zt, p, w, n) for w, n in ((zt.ZT_BUF_Q, T * H * D), (zt.ZT_BUF_K, T * Hkv * D),
                                           (zt.ZT_BUF_V, T * Hkv * D), (zt.ZT_BUF_DOUT, T * H * D))]


def _grads(zt, p, T, H, Hkv, D):
    return [_down(zt, p, w, n) for w, n in ((zt.ZT_BUF_DQ, T * H * D), (zt.ZT_BUF_DK, T * Hkv * D),
                                           (zt.ZT_BUF_DV, T * Hkv * D))]


@pytest.mark.parametrize("exact", [False, True], ids=["saved-statistics", "exact"])
def test_holder_scratch_contract_in_both_modes(gpu, zt, oracle, exact):
    """After forward + backward the row buffers satisfy the reference's scratch
    contract p = exp(s - row_max) / row_den with row_del = delta: the exact
    holder holds the max and the denominator, the default holder the
    log-sum-exp and 1.0 (the same p)."""
    T, H, Hkv, D = 200, 8, 2, 64
    p = ctypes.c_void_p()
    init = zt.lib().zt_holder_init_exact if exact else zt.lib().zt_holder_init
    assert init(T, H, Hkv, D, ctypes.byref(p)) == 0
    try:
        dec_ws = zt.decode_workspace_bytes(1, T, H, Hkv, D)
        assert zt.lib().zt_holder_workspace_bytes(p) == (0 if exact else dec_ws)
        q, k, v, do = _inputs(zt, p, T, H, Hkv, D)
        assert zt.lib().zt_holder_forward(p, 1, 64) == 0
        # the first whole-shape forward takes the score workspace
        assert zt.lib().zt_holder_workspace_bytes(p) == (
            0 if exact else dec_ws + zt.backward_train_workspace_bytes(1, T, H, Hkv, D))
        assert zt.lib().zt_holder_backward(p, 64) == 0
        m, l, d = oracle.attention_row_stats(q, k, v, do, 1, T, H, Hkv, D)
        rm, rl, rd = (_down(zt, p, w, T * H) for w in (zt.ZT_BUF_ROW_MAX, zt.ZT_BUF_ROW_DEN, zt.ZT_BUF_ROW_DEL))
        if exact:
            assert np.max(np.abs(rm - m)) <= 1e-4 * max(1.0, np.abs(m).max())
            assert np.max(np.abs(rl - l) / l) <= 1e-4
        else:
            lse = m + np.log(l)
            assert np.max(np.abs(rm - lse)) <= 1e-5 * max(1.0, np.abs(lse).max())
            assert np.all(rl == 1.0)
        assert np.max(np.abs(rd - d)) <= 1e-4 * max(1.0, np.abs(d).max())
        rq, rk, rv = oracle.attention_backward(q, k, v, do, 1, T, H, Hkv, D)
        for got, want in zip(_grads(zt, p, T, H, Hkv, D), (rq, rk, rv)):
            assert _rel(got, want) <= 1e-3
    finally:
        zt.lib().zt_holder_deinit(p)


@pytest.mark.parametrize("T,H,Hkv,D", [(150, 4, 2, 128), (150, 4, 4, 64), (120, 6, 2, 96)],
                         ids=["head-split-scores", "mha-row-split-scores", "group3-row-split-scores"])
def test_holder_backward_follows_what_the_buffers_hold(gpu, zt, oracle, T, H, Hkv, D):
    """The saved state is used only while it describes the buffers: a second
    backward, a backward after new q was uploaded, after a decode-shaped
    forward_at and after zt_holder_forget all give the twin's gradients for
    what the buffers hold; for an even head group and for groups that cannot
    be halved (whose row-split dk/dv kernel reads the scores too)."""
    p = _holder(zt, T, H, Hkv, D)
    L = zt.lib()
    try:
        q, k, v, do = _inputs(zt, p, T, H, Hkv, D)

        def check(qq):
            rq, rk, rv = oracle.attention_backward(qq, k, v, do, 1, T, H, Hkv, D)
            for got, want in zip(_grads(zt, p, T, H, Hkv, D), (rq, rk, rv)):
                assert _rel(got, want) <= 1e-3

        assert L.zt_holder_forward(p, 1, 64) == 0 and L.zt_holder_backward(p, 64) == 0
        check(q)
        assert L.zt_holder_backward(p, 64) == 0      # the score tiles now hold dS: rebuilt from lse
        check(q)
        q2 = (q * np.float32(0.5)).astype(np.float32)
        assert L.zt_holder_forward(p, 1, 64) == 0
        assert _up(zt, p, zt.ZT_BUF_Q, q2) == 0      # new q after the forward: lse and scores are stale
        assert L.zt_holder_backward(p, 64) == 0
        check(q2)
        assert L.zt_holder_forward(p, 1, 64) == 0
        assert L.zt_holder_forward_at(p, 1, 64, T - 1, T, 1) == 0   # a decode step over the same buffers
        assert L.zt_holder_backward(p, 64) == 0
        check(q2)
        assert L.zt_holder_forward(p, 1, 64) == 0
        L.zt_holder_forget(p)
        assert L.zt_holder_backward(p, 64) == 0
        check(q2)
        # A group_q the reference refuses is refused by the fast forward too.
        assert L.zt_holder_forward(p, 65, 64) == zt.ZT_CONFIG_REFUSED
        assert L.zt_holder_forward(p, 1, 0) == zt.ZT_CONFIG_REFUSED
    finally:
        L.zt_holder_deinit(p)


def test_holder_buffer_pointer_drops_the_saved_state_and_the_read_only_one_keeps_it(gpu, zt, oracle):
    """A writable pointer to q (or k, v, out, row_max) may be used to change what
    the forward saw, so asking for one drops the saved state and the next
    backward rebuilds the statistics from the buffers as they now are; the
    read-only accessor leaves it (the saved-statistics backward leaves
    row_den = 1, the rebuilding one the softmax denominators)."""
    T, H, Hkv, D = 150, 4, 2, 128
    p = _holder(zt, T, H, Hkv, D)
    L = zt.lib()
    try:
        q, k, v, do = _inputs(zt, p, T, H, Hkv, D)
        assert L.zt_holder_forward(p, 1, 64) == 0
        inputs = (zt.ZT_BUF_Q, zt.ZT_BUF_K, zt.ZT_BUF_V, zt.ZT_BUF_OUT, zt.ZT_BUF_ROW_MAX)
        for w in inputs:                              # read-only pointers to the forward's inputs
            assert L.zt_holder_buffer_ro(p, w)
        for w in (zt.ZT_BUF_DOUT, zt.ZT_BUF_DQ, zt.ZT_BUF_DK, zt.ZT_BUF_DV, zt.ZT_BUF_ROW_DEN, zt.ZT_BUF_ROW_DEL):
            assert L.zt_holder_buffer(p, w) == L.zt_holder_buffer_ro(p, w)
        assert L.zt_holder_backward(p, 64) == 0     # none of those drops the saved state
        assert np.all(_down(zt, p, zt.ZT_BUF_ROW_DEN, T * H) == 1.0)
        assert L.zt_holder_forward(p, 1, 64) == 0
        qp = L.zt_holder_buffer(p, zt.ZT_BUF_Q)     # writable q: the state is dropped
        assert zt.lib().zt_fill_normal(qp, T * H * D, 0x5EED00AA, 0.0, 1.0, None) == 0
        q2 = _down(zt, p, zt.ZT_BUF_Q, T * H * D)
        assert L.zt_holder_backward(p, 64) == 0
        assert not np.all(_down(zt, p, zt.ZT_BUF_ROW_DEN, T * H) == 1.0)
        rq, rk, rv = oracle.attention_backward(q2, k, v, do, 1, T, H, Hkv, D)
        for got, want in zip(_grads(zt, p, T, H, Hkv, D), (rq, rk, rv)):
            assert _rel(got, want) <= 1e-3
    finally:
        L.zt_holder_deinit(p)


def test_holder_decode_seam_at_the_c4_sequence_shape(gpu, zt, oracle, threads):
    """decode.zig:462's call on one C4 sequence (8192 cached keys, 32 / 8 heads,
    d = 128) through the holder, which splits the keys over the device with
    its own chunk partials: against the twin at the full cache and at partly
    filled ones, and equal to zt_attn_decode bit for bit, call after call."""
    n_ctx, H, Hkv, D = 8192, 32, 8, 128
    p = _holder(zt, n_ctx, H, Hkv, D)
    L = zt.lib()
    try:
        dec_ws = zt.decode_workspace_bytes(1, n_ctx, H, Hkv, D)
        assert L.zt_holder_workspace_bytes(p) == dec_ws   # a decode-only holder takes no score workspace
        _fill(zt, p, zt.ZT_BUF_Q, H * D, 0x5EED0001)
        _fill(zt, p, zt.ZT_BUF_K, n_ctx * Hkv * D, 0x5EED0005)
        _fill(zt, p, zt.ZT_BUF_V, n_ctx * Hkv * D, 0x5EED0006)
        qh = _down(zt, p, zt.ZT_BUF_Q, H * D)
        kc = _down(zt, p, zt.ZT_BUF_K, n_ctx * Hkv * D)
        vc = _down(zt, p, zt.ZT_BUF_V, n_ctx * Hkv * D)
        for n_keys in (n_ctx, 5000, 1, 129, n_ctx):
            assert L.zt_holder_forward_at(p, 1, 64, n_keys - 1, n_keys, 1) == 0
            out = _down(zt, p, zt.ZT_BUF_OUT, H * D)
            ref = oracle.attn_step(qh, kc, vc, [n_keys], 1, n_ctx, H, Hkv, D, threads=threads)
            assert np.max(np.abs(out - ref)) <= 1e-4, n_keys
            want = gpu.empty(H * D, device="cuda")
            ws = gpu.empty(dec_ws // 4 + 1, device="cuda")
            qd, kd, vd = (gpu.from_numpy(x).cuda() for x in (qh, kc, vc))
            zt.decode(qd, kd, vd, want, [n_keys], 1, n_ctx, H, Hkv, D, ws)
            gpu.cuda.synchronize()
            assert np.array_equal(out.view(np.uint32), host_np(want).view(np.uint32)), n_keys
    finally:
        L.zt_holder_deinit(p)


def host_np(t):
    return t.detach().cpu().numpy().ravel()
