"""Whole kv groups at full size: every row of O, dq, dk and dv of kv group 0
and kv group Hkv - 1 at C3 (B=1, T=4096, 32/8 heads, d=128, RoPE'd Q/K) and
C5 (B=2, T=2048, 16/4 heads, d=256, N(0, 2)) against the CPU restatement of
src/attention.zig:60-153 and src/autograd.zig:636-842, on each of the four
step paths (the reference entry points, and the training path with the dq
kernel, with dq from the stored dS, and with the forward's scores read back).

A kv group is graded whole because its dk/dv receive terms from its own query
heads only; the oracle's group backward is bit-identical to the serial
restatement (tests/test_oracle.py).  Every row tile and key tile of those heads
is graded, including the middle tiles that paired workgroups place between the
first and last, on the grids the shape rules pick at these sizes.  Gates:
O max |diff| <= 1e-4; dq/dk/dv max|g - twin| / max|twin| <= 1e-3 per
gradient and group."""
import numpy as np
import pytest

from gpuhelp import (BWD_REL, FWD_TOL, SEED_DO, SEED_K, SEED_Q, SEED_V, THETA, dev_normal, host, max_abs,
                     rel_err)

pytestmark = pytest.mark.gpu

CONFIGS = {
    "c3": (1, 4096, 32, 8, 128, 1.0, True),
    "c5": (2, 2048, 16, 4, 256, float(np.sqrt(2.0)), False),
}
PATHS = ["reference_abi", "dq_kernel", "dq_from_ds", "scores"]


@pytest.fixture(scope="module")
def case(gpu, zt, oracle, threads):
    """Device inputs per config and the oracle's O, dq, dk, dv of kv groups 0
    and Hkv - 1, computed once for the four paths."""
    made = {}

    def get(cfg):
        if cfg in made:
            return made[cfg]
        made.clear()  # one config's tensors at a time
        B, T, H, Hkv, D, sigma, rope = CONFIGS[cfg]
        print(f"[groups] {cfg}: inputs and oracle B={B} T={T} H={H}/{Hkv} d={D}", flush=True)
        q = dev_normal(gpu, zt, B * T * H * D, SEED_Q, sigma)
        k = dev_normal(gpu, zt, B * T * Hkv * D, SEED_K, sigma)
        v = dev_normal(gpu, zt, B * T * Hkv * D, SEED_V, sigma)
        do = dev_normal(gpu, zt, B * T * H * D, SEED_DO, 1.0)
        if rope:
            zt.rope_qk(q, k, q, k, B, T, H, Hkv, D, 0, THETA)
        gpu.cuda.synchronize()
        qh, kh, vh, dh = (host(x) for x in (q, k, v, do))
        ref = {}
        for kv in (0, Hkv - 1):
            o = oracle.attention_forward_groups(qh, kh, vh, B, T, H, Hkv, D, kv, kv + 1, threads=threads)
            dq, dk, dv = oracle.attention_backward_groups(qh, kh, vh, dh, B, T, H, Hkv, D, kv, kv + 1,
                                                          threads=threads)
            ref[kv] = (o, dq, dk, dv)
        made[cfg] = (q, k, v, do, ref)
        return made[cfg]

    return get


def _nan(torch, n):
    return torch.full((n,), float("nan"), device="cuda", dtype=torch.float32)


def _run(torch, zt, path, q, k, v, do, B, T, H, Hkv, D):
    out, dq, dk, dv = _nan(torch, q.numel()), _nan(torch, q.numel()), _nan(torch, k.numel()), _nan(torch, k.numel())
    if path == "reference_abi":
        rm, rl, rd = (_nan(torch, B * T * H) for _ in range(3))
        zt.forward(q, k, v, out, T, H, Hkv, D, B=B)
        zt.backward(q, k, v, do, dq, dk, dv, rm, rl, rd, T, H, Hkv, D, B=B)
    else:
        lse, delta = _nan(torch, B * T * H), _nan(torch, B * T * H)
        work = _nan(torch, zt.backward_train_workspace_bytes(B, T, H, Hkv, D) // 4)
        if path == "scores":
            zt.forward_train_ws(q, k, v, out, lse, work, T, H, Hkv, D, B=B)
        else:
            zt.forward_train(q, k, v, out, lse, T, H, Hkv, D, B=B)
        if path == "dq_kernel":
            zt.backward_train(q, k, v, out, do, lse, dq, dk, dv, delta, T, H, Hkv, D, B=B)
        else:
            stage = 3 | (zt.ZT_WS_SCORES if path == "scores" else 0)
            zt.backward_train_ws(q, k, v, out, do, lse, dq, dk, dv, work, T, H, Hkv, D, B=B, stage=stage)
    torch.cuda.synchronize()
    return [host(x) for x in (out, dq, dk, dv)]


@pytest.mark.parametrize("path", PATHS)
@pytest.mark.parametrize("cfg", ["c3", "c5"])
def test_whole_kv_groups_match_twin(gpu, zt, case, cfg, path):
    B, T, H, Hkv, D, _, _ = CONFIGS[cfg]
    print(f"[groups] {cfg} {path}", flush=True)
    q, k, v, do, ref = case(cfg)
    out, dq, dk, dv = _run(gpu, zt, path, q, k, v, do, B, T, H, Hkv, D)
    g = H // Hkv
    for kv, (ro, rq, rk, rv) in ref.items():
        heads = slice(kv * g, (kv + 1) * g)
        sel_q = lambda x: x.reshape(B, T, H, D)[:, :, heads]
        sel_k = lambda x: x.reshape(B, T, Hkv, D)[:, :, kv]
        assert max_abs(sel_q(out), sel_q(ro)) <= FWD_TOL, (kv, "out")
        assert rel_err(sel_q(dq), sel_q(rq)) <= BWD_REL, (kv, "dq")
        assert rel_err(sel_k(dk), sel_k(rk)) <= BWD_REL, (kv, "dk")
        assert rel_err(sel_k(dv), sel_k(rv)) <= BWD_REL, (kv, "dv")
    # The other groups' outputs exist and are finite (they are graded by the
    # full-size invariants in test_gpu_backward.py / test_gpu_train.py).
    for x in (out, dq, dk, dv):
        assert np.all(np.isfinite(x))
