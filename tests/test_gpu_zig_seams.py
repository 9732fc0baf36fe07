"""The reference's drop-in seams as integration/zig_mi355x.patch issues them,
replayed call for call through the C ABI (the Zig cannot be compiled in this
image: no Zig toolchain).  `ZigAttn` mirrors the patched src/cuda/device.zig
Attn (init: zt_holder_init then the eleven zt_holder_buffer pointers; upload /
download: the buffer's index in field order, then zt_holder_upload /
zt_holder_download; forward = forwardAt(group_q, max_tile, 0, c_t, c_t);
forwardAt: forwardBounds, then zt_holder_forward_at; backward:
zt_holder_backward), and the three callers mirror their Zig:
  - cuda_forward: model.cudaForward (src/model.zig:467-516): upload q, k, v;
    forward(1, 64); download out;
  - device_attention_backward: the patched autograd deviceAttentionBackward:
    one holder kept across calls (made again for another shape); upload q, k,
    v, dout; forward(1, 64); backward(64); download dq, dk, dv;
  - cuda_attn_step: decode.cudaAttnStep (src/decode.zig:405-473): upload the
    query row and the n_keys cache rows of k and v; forwardAt(1, 64,
    n_keys - 1, n_keys, 1); download the output row.
Graded against the CPU restatement with the north_star gates: C1 in full (two
layers through one cached holder, and a filling cache), and one whole kv group
of C3 (RoPE'd) after a first call on other inputs; and model.zig's
deliberate-corruption control (ATTN_CORRUPT_KEY), which the gate must reject."""
import ctypes

import numpy as np
import pytest

from gpuhelp import BWD_REL, FWD_TOL, SEED_DO, SEED_K, SEED_Q, SEED_V, THETA, dev_normal, host, max_abs, rel_err

pytestmark = pytest.mark.gpu

N_BUFFERS = 11
ERRORS = {1: "DegenerateShape", 2: "ShapeTooLarge", 3: "ConfigRefused", 4: "DeviceAllocFailed"}


class ZigError(Exception):
    pass


def _check(rc):
    """device.zig's holderError: 0 is success, the codes map onto Error."""
    if rc != 0:
        raise ZigError(ERRORS.get(rc, "DeviceTransferFailed"))


class ZigAttn:
    """The patched device.zig Attn, call for call."""

    def __init__(self, L, t, n_heads, n_kv_heads, dim):
        self.L = L
        h = ctypes.c_void_p()
        _check(L.zt_holder_init(t, n_heads, n_kv_heads, dim, ctypes.byref(h)))
        self.h = h
        self.t, self.n_heads, self.n_kv_heads, self.dim = t, n_heads, n_kv_heads, dim
        (self.q, self.k, self.v, self.out, self.dout, self.dq, self.dk, self.dv, self.row_max, self.row_den,
         self.row_del) = (L.zt_holder_buffer(h, i) for i in range(N_BUFFERS))

    def _which(self, p):
        fields = (self.q, self.k, self.v, self.out, self.dout, self.dq, self.dk, self.dv, self.row_max,
                  self.row_den, self.row_del)
        for i, f in enumerate(fields):
            if f == p:
                return i
        raise ZigError("ShapeTooLarge")

    def deinit(self):
        self.L.zt_holder_deinit(self.h)
        self.h = None

    def forward(self, group_q, max_tile):
        self.forward_at(group_q, max_tile, 0, self.t, self.t)

    def forward_at(self, group_q, max_tile, q_offset, n_keys, t):
        if self.L.zt_forward_bounds(self.t, q_offset, n_keys, t) != 0:
            raise ZigError("ShapeTooLarge")
        _check(self.L.zt_holder_forward_at(self.h, group_q, max_tile, q_offset, n_keys, t))

    def backward(self, max_tile):
        _check(self.L.zt_holder_backward(self.h, max_tile))

    def upload(self, dst, src):
        a = np.ascontiguousarray(src, np.float32)
        _check(self.L.zt_holder_upload(self.h, self._which(dst), a.ctypes.data_as(ctypes.c_void_p), a.size))

    def download(self, dst, src):
        _check(self.L.zt_holder_download(self.h, dst.ctypes.data_as(ctypes.c_void_p), self._which(src), dst.size))


class AutogradDevice:
    """The patched autograd.zig: the module-level holder and deviceAttentionBackward."""

    def __init__(self, L):
        self.L = L
        self.bwd_dev = None
        self.inits = 0

    def device_attention_backward(self, q, k, v, dout, T, H, Hkv, D):
        held = self.bwd_dev
        if held is not None and (held.t, held.n_heads, held.n_kv_heads, held.dim) != (T, H, Hkv, D):
            held.deinit()
            self.bwd_dev = None
        if self.bwd_dev is None:
            self.bwd_dev = ZigAttn(self.L, T, H, Hkv, D)
            self.inits += 1
        a = self.bwd_dev
        a.upload(a.q, q)
        a.upload(a.k, k)
        a.upload(a.v, v)
        a.upload(a.dout, dout)
        a.forward(1, 64)
        a.backward(64)
        dq, dk, dv = np.empty(q.size, np.float32), np.empty(k.size, np.float32), np.empty(v.size, np.float32)
        a.download(dq, a.dq)
        a.download(dk, a.dk)
        a.download(dv, a.dv)
        return dq, dk, dv

    def deinit(self):
        if self.bwd_dev is not None:
            self.bwd_dev.deinit()
        self.bwd_dev = None


def cuda_forward(a, q, k, v, H, D, corrupt_key=None):
    """model.cudaForward; corrupt_key is its ATTN_CORRUPT_KEY (model.zig:452-499):
    an offset added to the first element of the uploaded keys only."""
    a.upload(a.q, q)
    if corrupt_key:
        damaged = np.array(k, np.float32, copy=True)
        damaged[0] += corrupt_key
        a.upload(a.k, damaged)
    else:
        a.upload(a.k, k)
    a.upload(a.v, v)
    a.forward(1, 64)
    out = np.empty(q.size, np.float32)
    a.download(out, a.out)
    return out


def cuda_attn_step(a, q_row, kc, vc, n_keys, H, Hkv, D):
    a.upload(a.q, q_row[:H * D])
    a.upload(a.k, kc[:n_keys * Hkv * D])
    a.upload(a.v, vc[:n_keys * Hkv * D])
    a.forward_at(1, 64, n_keys - 1, n_keys, 1)
    out = np.empty(H * D, np.float32)
    a.download(out, a.out)
    return out


def _host_inputs(rng, T, H, Hkv, D):
    return (rng.standard_normal(T * H * D).astype(np.float32), rng.standard_normal(T * Hkv * D).astype(np.float32),
            rng.standard_normal(T * Hkv * D).astype(np.float32), rng.standard_normal(T * H * D).astype(np.float32))


def test_seams_at_c1(gpu, zt, oracle):
    """C1 (T=128, 4/2 heads, d=32): the model forward seam, two layers of the
    device backward through one cached holder (the second layer's inputs
    replace the first's), a third call at another shape (the holder is made
    again), and a decode over a filling cache."""
    L = zt.lib()
    T, H, Hkv, D = 128, 4, 2, 32
    rng = np.random.default_rng(0xC1)
    fwd = ZigAttn(L, T, H, Hkv, D)
    auto = AutogradDevice(L)
    try:
        for layer in range(2):
            q, k, v, do = _host_inputs(rng, T, H, Hkv, D)
            out = cuda_forward(fwd, q, k, v, H, D)
            assert max_abs(out, oracle.attention_forward(q, k, v, 1, T, H, Hkv, D)) <= FWD_TOL, layer
            dq, dk, dv = auto.device_attention_backward(q, k, v, do, T, H, Hkv, D)
            rq, rk, rv = oracle.attention_backward(q, k, v, do, 1, T, H, Hkv, D)
            assert rel_err(dq, rq) <= BWD_REL and rel_err(dk, rk) <= BWD_REL and rel_err(dv, rv) <= BWD_REL, layer
        assert auto.inits == 1
        T2 = 77
        q, k, v, do = _host_inputs(rng, T2, H, Hkv, D)
        dq, dk, dv = auto.device_attention_backward(q, k, v, do, T2, H, Hkv, D)
        rq, rk, rv = oracle.attention_backward(q, k, v, do, 1, T2, H, Hkv, D)
        assert rel_err(dq, rq) <= BWD_REL and rel_err(dk, rk) <= BWD_REL and rel_err(dv, rv) <= BWD_REL
        assert auto.inits == 2
        # decode.zig's holder is built at n_ctx and fed one growing prefix per step
        n_ctx = T
        dec = ZigAttn(L, n_ctx, H, Hkv, D)
        try:
            kc = rng.standard_normal(n_ctx * Hkv * D).astype(np.float32)
            vc = rng.standard_normal(n_ctx * Hkv * D).astype(np.float32)
            qs = rng.standard_normal((n_ctx, H * D)).astype(np.float32)
            for n_keys in (1, 2, 17, 64, 127, 128):
                out = cuda_attn_step(dec, qs[n_keys - 1], kc, vc, n_keys, H, Hkv, D)
                ref = oracle.attn_step(qs[n_keys - 1], kc, vc, [n_keys], 1, n_ctx, H, Hkv, D)
                assert max_abs(out, ref) <= FWD_TOL, n_keys
            with pytest.raises(ZigError, match="ShapeTooLarge"):
                dec.forward_at(1, 64, n_ctx, n_ctx + 1, 1)
            with pytest.raises(ZigError, match="ConfigRefused"):
                dec.forward(0, 64)
        finally:
            dec.deinit()
    finally:
        fwd.deinit()
        auto.deinit()


def test_the_model_seam_gate_rejects_a_corrupted_key(gpu, zt, oracle):
    """model.zig's deliberate-corruption control (ATTN_CORRUPT_KEY=0.05 makes
    `zig build cuda-attn-check` exit 1): one uploaded key element moved by 0.05
    on the device side only must fail the forward gate against the clean twin,
    and only in kv head 0's query heads; the clean upload through the same
    holder passes it again afterwards."""
    L = zt.lib()
    T, H, Hkv, D = 128, 4, 2, 32
    rng = np.random.default_rng(0xBAD)
    q, k, v, _ = _host_inputs(rng, T, H, Hkv, D)
    ref = oracle.attention_forward(q, k, v, 1, T, H, Hkv, D)
    a = ZigAttn(L, T, H, Hkv, D)
    try:
        clean = cuda_forward(a, q, k, v, H, D)
        assert max_abs(clean, ref) <= FWD_TOL
        bad = cuda_forward(a, q, k, v, H, D, corrupt_key=0.05)
        assert max_abs(bad, ref) > FWD_TOL               # the gate fails
        moved = (bad != clean).reshape(T, H, D)
        assert not moved[:, H // Hkv:].any()             # kv head 1's query heads never read kv head 0's keys
        assert not moved[0].any()                        # row 0 sees key 0 alone: its weight stays 1
        again = cuda_forward(a, q, k, v, H, D)
        assert np.array_equal(again.view(np.uint32), clean.view(np.uint32))
    finally:
        a.deinit()


def test_device_backward_seam_on_a_c3_kv_group(gpu, zt, oracle, threads):
    """C3 (T=4096, 32/8 heads, d=128, RoPE'd q/k) through the patched device
    backward, after a first call on other inputs through the same cached
    holder: every row of kv group 5 against the twin."""
    L = zt.lib()
    T, H, Hkv, D, kv = 4096, 32, 8, 128, 5
    q = dev_normal(gpu, zt, T * H * D, SEED_Q)
    k = dev_normal(gpu, zt, T * Hkv * D, SEED_K)
    v = dev_normal(gpu, zt, T * Hkv * D, SEED_V)
    do = dev_normal(gpu, zt, T * H * D, SEED_DO)
    zt.rope_qk(q, k, q, k, 1, T, H, Hkv, D, 0, THETA)
    gpu.cuda.synchronize()
    qh, kh, vh, dh = (host(x) for x in (q, k, v, do))
    del q, k, v, do
    auto = AutogradDevice(L)
    try:
        print("[zig seams] C3 first call on other inputs", flush=True)
        auto.device_attention_backward(vh.repeat(4)[:qh.size] * 0.5, kh[::-1].copy(), vh, dh, T, H, Hkv, D)
        print("[zig seams] C3 graded call", flush=True)
        dq, dk, dv = auto.device_attention_backward(qh, kh, vh, dh, T, H, Hkv, D)
        assert auto.inits == 1
        rq, rk, rv = oracle.attention_backward_groups(qh, kh, vh, dh, 1, T, H, Hkv, D, kv, kv + 1, threads=threads)
        g = H // Hkv
        sq = lambda x: x.reshape(T, H, D)[:, kv * g:(kv + 1) * g]
        sk = lambda x: x.reshape(T, Hkv, D)[:, kv]
        assert rel_err(sq(dq), sq(rq)) <= BWD_REL
        assert rel_err(sk(dk), sk(rk)) <= BWD_REL
        assert rel_err(sk(dv), sk(rv)) <= BWD_REL
    finally:
        auto.deinit()
