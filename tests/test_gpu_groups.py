"""Every kv group at full size: every row of O, dq, dk and dv of each of the 8
kv groups at C3 (B=1, T=4096, 32/8 heads, d=128, RoPE'd Q/K) and each of the
4 at C5 (B=2, T=2048, 16/4 heads, d=256, N(0, 2)) against the CPU restatement
of src/attention.zig:60-153 and src/autograd.zig:636-842, on each of the four
step paths (the reference entry points, and the training path with the dq
kernel, with dq from the stored dS, and with the forward's scores read back),
and at C3 also through the holder (zt_holder_forward + zt_holder_backward, the
drop-in device.Attn pair).

A kv group is graded whole because its dk/dv receive terms from its own query
heads only; the oracle's group backward is bit-identical to the serial
restatement (tests/test_oracle.py).  So every row tile and key tile of every
head is graded, on the grids and tile pairings the shape rules pick at these
sizes.  Each test grades one group on every path: the device runs each path
once per config (cached), the oracle one group per test.  Gates: O max
|diff| <= 1e-4; dq/dk/dv max|g - twin| / max|twin| <= 1e-3 per gradient and
group."""
import ctypes

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
GROUPS = [("c3", kv) for kv in range(CONFIGS["c3"][3])] + [("c5", kv) for kv in range(CONFIGS["c5"][3])]


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


def _run_holder(zt, qh, kh, vh, dh, T, H, Hkv, D):
    """The holder's model seam as the patched reference drives it: upload
    q, k, v, dout, forward(1, 64), backward(64), download."""
    L = zt.lib()
    p = ctypes.c_void_p()
    assert L.zt_holder_init(T, H, Hkv, D, ctypes.byref(p)) == 0
    try:
        for which, a in ((zt.ZT_BUF_Q, qh), (zt.ZT_BUF_K, kh), (zt.ZT_BUF_V, vh), (zt.ZT_BUF_DOUT, dh)):
            a = np.ascontiguousarray(a, np.float32)
            assert L.zt_holder_upload(p, which, a.ctypes.data_as(ctypes.c_void_p), a.size) == 0
        assert L.zt_holder_forward(p, 1, 64) == 0
        assert L.zt_holder_backward(p, 64) == 0
        res = []
        for which, n in ((zt.ZT_BUF_OUT, qh.size), (zt.ZT_BUF_DQ, qh.size), (zt.ZT_BUF_DK, kh.size),
                         (zt.ZT_BUF_DV, vh.size)):
            a = np.empty(n, np.float32)
            assert L.zt_holder_download(p, a.ctypes.data_as(ctypes.c_void_p), which, n) == 0
            res.append(a)
        return res
    finally:
        L.zt_holder_deinit(p)


@pytest.fixture(scope="module")
def case(gpu, zt, oracle, threads):
    """One config at a time: its device inputs, each path's outputs (run once)
    and the oracle's O, dq, dk, dv per kv group (computed when first asked)."""
    st = {}

    def inputs(cfg):
        if st.get("cfg") == cfg:
            return st
        st.clear()
        B, T, H, Hkv, D, sigma, rope = CONFIGS[cfg]
        print(f"[groups] {cfg}: inputs B={B} T={T} H={H}/{Hkv} d={D}", flush=True)
        q = dev_normal(gpu, zt, B * T * H * D, SEED_Q, sigma)
        k = dev_normal(gpu, zt, B * T * Hkv * D, SEED_K, sigma)
        v = dev_normal(gpu, zt, B * T * Hkv * D, SEED_V, sigma)
        do = dev_normal(gpu, zt, B * T * H * D, SEED_DO, 1.0)
        if rope:
            zt.rope_qk(q, k, q, k, B, T, H, Hkv, D, 0, THETA)
        gpu.cuda.synchronize()
        st.update(cfg=cfg, dev=(q, k, v, do), host=tuple(host(x) for x in (q, k, v, do)), out={}, ref={})
        return st

    def result(cfg, path):
        s = inputs(cfg)
        if path not in s["out"]:
            B, T, H, Hkv, D, _, _ = CONFIGS[cfg]
            print(f"[groups] {cfg} {path}", flush=True)
            if path == "holder":
                s["out"][path] = _run_holder(zt, *s["host"], T, H, Hkv, D)
            else:
                s["out"][path] = _run(gpu, zt, path, *s["dev"], B, T, H, Hkv, D)
        return s["out"][path]

    def ref(cfg, kv):
        s = inputs(cfg)
        if kv not in s["ref"]:
            B, T, H, Hkv, D, _, _ = CONFIGS[cfg]
            print(f"[groups] {cfg} kv group {kv}: oracle", flush=True)
            qh, kh, vh, dh = s["host"]
            o = oracle.attention_forward_groups(qh, kh, vh, B, T, H, Hkv, D, kv, kv + 1, threads=threads)
            dq, dk, dv = oracle.attention_backward_groups(qh, kh, vh, dh, B, T, H, Hkv, D, kv, kv + 1,
                                                          threads=threads)
            s["ref"] = {kv: (o, dq, dk, dv)}   # one group's reference at a time
        return s["ref"][kv]

    return result, ref


@pytest.mark.parametrize("cfg,kv", GROUPS, ids=[f"{c}-kv{k}" for c, k in GROUPS])
def test_every_kv_group_matches_twin_on_every_path(gpu, zt, case, cfg, kv):
    result, ref = case
    B, T, H, Hkv, D, _, _ = CONFIGS[cfg]
    ro, rq, rk, rv = ref(cfg, kv)
    g = H // Hkv
    heads = slice(kv * g, (kv + 1) * g)
    sel_q = lambda x: x.reshape(B, T, H, D)[:, :, heads]
    sel_k = lambda x: x.reshape(B, T, Hkv, D)[:, :, kv]
    for path in PATHS + (["holder"] if cfg == "c3" else []):
        out, dq, dk, dv = result(cfg, path)
        assert max_abs(sel_q(out), sel_q(ro)) <= FWD_TOL, (path, kv, "out")
        assert rel_err(sel_q(dq), sel_q(rq)) <= BWD_REL, (path, kv, "dq")
        assert rel_err(sel_k(dk), sel_k(rk)) <= BWD_REL, (path, kv, "dk")
        assert rel_err(sel_k(dv), sel_k(rv)) <= BWD_REL, (path, kv, "dv")
