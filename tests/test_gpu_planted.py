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
TRAIN_PLANTS = ["train_fwd_scores", "train_ds_tiles", "train_dq_scale"]
DEC_PLANTS = ["decode_merge"]
# The negative-control shape: the planted code objects hold its kernels only.
B, T, H, Hkv, D = 1, 64, 4, 2, 32
# The training path's negative-control shape: the headline kernels (d = 128, four
# query heads per kv head, as C3), at a size the twin grades in full.
TB, TT, TH, THkv, TD = 1, 256, 8, 2, 128


@pytest.fixture(scope="module")
def planted(gpu, zt):
    libs = {}
    for name in FWD_PLANTS + BWD_PLANTS + NORM_PLANTS + TRAIN_PLANTS + DEC_PLANTS:
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


def _train_scores(torch, zt, L, q, k, v, do):
    """The headline step on library L: zt_attn_forward_train_ws (keeping the
    scores) then zt_attn_backward_train_ws reading them (ZT_WS_SCORES)."""
    n_q, n_k, rows = q.numel(), k.numel(), TB * TT * TH
    out, lse = _nan(torch, n_q), _nan(torch, rows)
    dq, dk, dv = _nan(torch, n_q), _nan(torch, n_k), _nan(torch, n_k)
    wsb = zt.backward_train_workspace_bytes(TB, TT, TH, THkv, TD)
    ws = _nan(torch, wsb // 4)
    assert L.zt_attn_forward_train_ws(*map(_p, (q, k, v, out, lse, ws)), wsb, TB, TT, TH, THkv, TD, None) == 0
    assert L.zt_attn_backward_train_ws(*map(_p, (q, k, v, out, do, lse, dq, dk, dv, ws)), wsb, TB, TT, TH, THkv,
                                        TD, 3 | zt.ZT_WS_SCORES, None) == 0
    torch.cuda.synchronize()
    return [host(x) for x in (out, lse, dq, dk, dv)]


def test_the_planted_training_kernels_are_the_ones_the_shape_launches(gpu, zt):
    assert zt.plan_train(TB, TT, TH, THkv, TD) == ("zt_fwd8ps_d128_k32", "zt_gemm_dqds2_64", "zt_bwd_dkdv8s_d128_hs2")


def test_training_gate_rejects_planted_headline_kernels_with_their_own_signatures(gpu, zt, oracle, planted):
    """A defect in each kernel of the headline step -- the score-keeping
    forward, the score-reading dk/dv kernel and the dq-from-dS product -- is
    rejected by the gate that grades the product step, each with the trace its
    defect must leave: unscaled stored scores leave O and lse bit-identical and
    every gradient wrong; swapped dS slots leave dk and dv bit-identical and dq
    wrong; the dropped product scale leaves dk and dv bit-identical and dq
    exactly sqrt(d) times right."""
    q = dev_normal(gpu, zt, TB * TT * TH * TD, SEED_Q)
    k = dev_normal(gpu, zt, TB * TT * THkv * TD, SEED_K)
    v = dev_normal(gpu, zt, TB * TT * THkv * TD, SEED_V)
    do = dev_normal(gpu, zt, TB * TT * TH * TD, SEED_DO)
    qh, kh, vh, dh = (host(x) for x in (q, k, v, do))
    want = oracle.attention_backward(qh, kh, vh, dh, TB, TT, TH, THkv, TD)
    ref_out = oracle.attention_forward(qh, kh, vh, TB, TT, TH, THkv, TD)
    good = _train_scores(gpu, zt, zt.lib(), q, k, v, do)
    assert max_abs(good[0], ref_out) <= FWD_TOL
    assert max(rel_err(g, w) for g, w in zip(good[2:], want)) <= BWD_REL
    same = lambda a, b: np.array_equal(a.view(np.uint32), b.view(np.uint32))
    signatures = {}
    for name in TRAIN_PLANTS:
        got = _train_scores(gpu, zt, planted[name], q, k, v, do)
        errs = tuple(rel_err(g, w) for g, w in zip(got[2:], want))
        print(f"[planted] {name}: dq/dk/dv relative error {errs[0]:.3e} / {errs[1]:.3e} / {errs[2]:.3e}", flush=True)
        assert max(errs) > BWD_REL, name
        signatures[name] = tuple(f"{e:.2e}" for e in errs)
        if name == "train_fwd_scores":
            assert same(got[0], good[0]) and same(got[1], good[1])     # O and lse untouched
            assert min(errs) > BWD_REL                                  # every gradient reads the scores
        else:
            assert same(got[3], good[3]) and same(got[4], good[4])     # dk, dv formed in registers
            assert errs[0] > BWD_REL
        if name == "train_dq_scale":
            scale = np.float32(1.0 / np.sqrt(TD))
            assert np.allclose(got[2] * scale, good[2], rtol=1e-6, atol=0)
    assert len(set(signatures.values())) == len(TRAIN_PLANTS), signatures


def test_decode_gate_rejects_the_planted_combine(gpu, zt, oracle, planted):
    """The combine that leaves a split sequence's last chunk out is rejected by
    the decode gate wherever the keys are split (one sequence of 8192 keys: 64
    chunks), and is never launched where each sequence is one chunk (C4's
    grid), so there it changes no bit."""
    L = planted["decode_merge"]
    Hq, Hk, Dd = 32, 8, 128
    for Bd, n_ctx, split in ((1, 8192, True), (64, 300, False)):
        q = dev_normal(gpu, zt, Bd * Hq * Dd, SEED_Q)
        kc = dev_normal(gpu, zt, Bd * n_ctx * Hk * Dd, SEED_K)
        vc = dev_normal(gpu, zt, Bd * n_ctx * Hk * Dd, SEED_V)
        n_keys = [n_ctx - (b % 3) for b in range(Bd)]
        wsb = zt.decode_workspace_bytes(Bd, n_ctx, Hq, Hk, Dd)
        ws = _nan(gpu, wsb // 4 + 1)
        arr = (ctypes.c_int * Bd)(*n_keys)

        def run(lib):
            out = _nan(gpu, Bd * Hq * Dd)
            assert lib.zt_attn_decode(*map(_p, (q, kc, vc, out)), arr, Bd, n_ctx, Hq, Hk, Dd, _p(ws), wsb, None) == 0
            gpu.cuda.synchronize()
            return host(out)

        good, bad = run(zt.lib()), run(L)
        ref = oracle.attn_step(host(q), host(kc), host(vc), n_keys, Bd, n_ctx, Hq, Hk, Dd)
        assert max_abs(good, ref) <= FWD_TOL
        if split:
            print(f"[planted] decode_merge: max |diff| {max_abs(bad, ref):.3e}", flush=True)
            assert max_abs(bad, ref) > FWD_TOL
        else:
            assert np.array_equal(bad.view(np.uint32), good.view(np.uint32))
