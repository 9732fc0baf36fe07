"""Kernel-side negative controls: the parity gates must reject kernels with a
planted defect, on the device.  Each planted-defect library (tests/planted/,
built by tests/planted/build.py with -DZT_PLANT=<n>; the defects are listed in
z-transformer_amd/csrc/kernels/common.h) is the library itself with one code
object replaced by a broken build of the same source; it is called through
the same C ABI, on the same device inputs, as the correct library, and graded
by the same gates against the CPU restatement.  As the reference requires of
its own BROKEN variants (src/cuda/run-attn.sh:121-177): each forward and
RMSNorm variant fails its gate, each backward variant fails the backward gate
with its own signature (four different defects leave four different traces),
and the variant that drops the softmax Jacobian leaves dv bit-identical
(src/cuda/README.md:882-892) while dq and dk fail."""
import ctypes
import os

import numpy as np
import pytest

from gpuhelp import (BWD_REL, FWD_TOL, SEED_DO, SEED_K, SEED_Q, SEED_V, SEED_W, SEED_X, dev_normal, dev_uniform,
                     host, max_abs, rel_err)

pytestmark = pytest.mark.gpu

HERE = os.path.dirname(os.path.abspath(__file__))
FWD_PLANTS = ["fwd_mask", "fwd_gqa", "fwd_rescale", "fwd_scale"]
BWD_PLANTS = ["bwd_mask", "bwd_gqa", "bwd_jacobian", "bwd_scale"]
NORM_PLANTS = ["norm_weight", "norm_mean", "norm_tensor"]
# The negative-control shape: the planted code objects hold its kernels only.
B, T, H, Hkv, D = 1, 64, 4, 2, 32


@pytest.fixture(scope="module")
def planted(gpu, zt):
    libs = {}
    for name in FWD_PLANTS + BWD_PLANTS + NORM_PLANTS:
        path = os.path.join(HERE, "planted", "_build", name, "libzt_attn.so")
        assert os.path.exists(path), f"{path} is not built: run tests/planted/build.py"
        libs[name] = zt.load_library(path)
        assert libs[name].zt_attn_lds_limit() > 0
    return libs


@pytest.fixture(scope="module")
def inputs(gpu, zt):
    q = dev_normal(gpu, zt, B * T * H * D, SEED_Q)
    k = dev_normal(gpu, zt, B * T * Hkv * D, SEED_K)
    v = dev_normal(gpu, zt, B * T * Hkv * D, SEED_V)
    do = dev_normal(gpu, zt, B * T * H * D, SEED_DO)
    gpu.cuda.synchronize()
    return q, k, v, do


def _p(t):
    return ctypes.c_void_p(t.data_ptr())


def _nan(torch, n):
    return torch.full((n,), float("nan"), device="cuda", dtype=torch.float32)


def _forward(torch, L, q, k, v):
    out = _nan(torch, q.numel())
    assert L.zt_attn_forward(_p(q), _p(k), _p(v), _p(out), T, H, Hkv, D, 1, 64, 0, T, None) == 0
    torch.cuda.synchronize()
    return host(out)


def _backward(torch, L, q, k, v, do):
    dq, dk, dv = _nan(torch, q.numel()), _nan(torch, k.numel()), _nan(torch, k.numel())
    rm, rl, rd = (_nan(torch, B * T * H) for _ in range(3))
    assert L.zt_attn_backward(*map(_p, (q, k, v, do, dq, dk, dv, rm, rl, rd)), T, H, Hkv, D, 64, None) == 0
    torch.cuda.synchronize()
    return [host(x) for x in (dq, dk, dv)]


def _backward_train(torch, L, q, k, v, do):
    out, lse, delta = _nan(torch, q.numel()), _nan(torch, B * T * H), _nan(torch, B * T * H)
    dq, dk, dv = _nan(torch, q.numel()), _nan(torch, k.numel()), _nan(torch, k.numel())
    assert L.zt_attn_forward_train(*map(_p, (q, k, v, out, lse)), B, T, H, Hkv, D, None) == 0
    assert L.zt_attn_backward_train(*map(_p, (q, k, v, out, do, lse, dq, dk, dv, delta)), B, T, H, Hkv, D,
                                     None) == 0
    torch.cuda.synchronize()
    return [host(x) for x in (dq, dk, dv)]


def test_the_planted_kernels_are_the_ones_the_shape_launches(gpu, zt):
    assert zt.plan(B, T, H, Hkv, D) == ("zt_fwd8p_d32_k32", "zt_bwd_dqp_d32_k32", "zt_bwd_dkdv8p_d32_hs2")


def test_forward_gate_rejects_every_planted_forward(gpu, zt, oracle, planted, inputs):
    q, k, v, _ = inputs
    ref = oracle.attention_forward(host(q), host(k), host(v), B, T, H, Hkv, D)
    assert max_abs(_forward(gpu, zt.lib(), q, k, v), ref) <= FWD_TOL
    for name in FWD_PLANTS:
        err = max_abs(_forward(gpu, planted[name], q, k, v), ref)
        print(f"[planted] {name}: max |diff| {err:.3e}", flush=True)
        assert err > FWD_TOL, name


def test_backward_gate_rejects_every_planted_backward_with_its_own_signature(gpu, zt, oracle, planted, inputs):
    q, k, v, do = inputs
    want = oracle.attention_backward(*(host(x) for x in (q, k, v, do)), B, T, H, Hkv, D)
    good = _backward(gpu, zt.lib(), q, k, v, do)
    assert max(rel_err(g, w) for g, w in zip(good, want)) <= BWD_REL
    signatures = {}
    for name in BWD_PLANTS:
        got = _backward(gpu, planted[name], q, k, v, do)
        errs = tuple(rel_err(g, w) for g, w in zip(got, want))
        print(f"[planted] {name}: dq/dk/dv relative error {errs[0]:.3e} / {errs[1]:.3e} / {errs[2]:.3e}", flush=True)
        assert max(errs) > BWD_REL, name
        signatures[name] = tuple(f"{e:.2e}" for e in errs)
        if name == "bwd_jacobian":
            # dS = P leaves dV = dO^T P untouched: bit-identical, while dq and dk fail.
            assert np.array_equal(got[2].view(np.uint32), good[2].view(np.uint32))
            assert errs[0] > BWD_REL and errs[1] > BWD_REL
    assert len(set(signatures.values())) == len(BWD_PLANTS), signatures


def test_training_path_gate_rejects_every_planted_backward(gpu, zt, oracle, planted, inputs):
    """The saved-statistics backward (its own dq kernel, the same dk/dv kernel)."""
    q, k, v, do = inputs
    want = oracle.attention_backward(*(host(x) for x in (q, k, v, do)), B, T, H, Hkv, D)
    good = _backward_train(gpu, zt.lib(), q, k, v, do)
    assert max(rel_err(g, w) for g, w in zip(good, want)) <= BWD_REL
    for name in BWD_PLANTS:
        errs = [rel_err(g, w) for g, w in zip(_backward_train(gpu, planted[name], q, k, v, do), want)]
        assert max(errs) > BWD_REL, name


def test_rmsnorm_gate_rejects_every_planted_rmsnorm(gpu, zt, oracle, planted):
    rows, cols = 16, 512
    x = dev_normal(gpu, zt, rows * cols, SEED_X)
    w = dev_uniform(gpu, zt, cols, SEED_W, 0.5, 1.5)
    ref = oracle.rmsnorm(host(x), host(w), rows, cols)

    def norm(L):
        y = _nan(gpu, rows * cols)
        assert L.zt_rmsnorm_forward(_p(x), _p(w), _p(y), rows, cols, 1e-5, None) == 0
        gpu.cuda.synchronize()
        return host(y)

    assert max_abs(norm(zt.lib()), ref) <= 1e-5
    for name in NORM_PLANTS:
        err = max_abs(norm(planted[name]), ref)
        print(f"[planted] {name}: max |diff| {err:.3e}", flush=True)
        assert err > 1e-5, name
