#!/usr/bin/env python3
"""Benchmark of the fused causal GQA attention path on one MI355X.

A step is one attention forward plus backward of a training step
(zt_attn_forward_train_ws, which keeps each row's log-sum-exp and its scaled
scores, then zt_attn_backward_train_ws, whose dk/dv kernel reads those scores
instead of forming Q K^T again and overwrites them with dS, so that dq is one
causal product) over BASELINE.json's C3 workload: B=1, T=4096, 32 query / 8 kv heads,
head_dim 128, f32, RoPE (theta 500000) pre-applied to Q and K, all inputs
seeded N(0,1) on the device and resident in HBM before timing.  The headline
value is fwd+bwd TFLOP/s with the causal-pair FLOP count
(fwd 2*B*H*d*T(T+1), bwd 5*B*H*d*T(T+1)).  The reference's own entry points
(zt_attn_forward + zt_attn_backward, whose backward rebuilds the softmax
statistics) are timed on the same inputs under "reference_abi".  The other
training configurations (C2: MHA d 64; C5: d 256) are timed the same two ways
under "other_configs" (secondary figures).  The same line also carries the
decode step (C4: B=64, 8192 cached keys, GB/s of K/V/q/out) and RMSNorm
([64,4096] and [4096,4096], GB/s over rotating buffers larger than the 256 MB
MALL), per-kernel times from HIP events on the launch stream, the roofline of
the dominant kernel, and the CPU restatement timed on a bounded sample.

    python bench.py [--gpus 1] [--steps 10] [--warmup 3] [--cpu-rows 64] [--no-cpu] [--no-other]
"""
import argparse
import ctypes
import importlib.util
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
METRIC = "causal GQA attn fwd+bwd TFLOP/s f32 (T=4096,d=128); decode attn HBM GB/s"
PEAK_MFMA_F32 = 157.3   # TFLOP/s, MI355X dense FP32 matrix
PEAK_HBM = 8000.0       # GB/s, MI355X HBM3E
THETA = 500000.0
SEEDS = {"q": 0x5EED0001, "k": 0x5EED0002, "v": 0x5EED0003, "do": 0x5EED0004, "kc": 0x5EED0005,
         "vc": 0x5EED0006, "x": 0x5EED0007, "w": 0x5EED0008}
# The reference's own attention benchmark shapes (src/cuda/attn_twin.zig:82-111: tag, T, query heads,
# kv heads, head_dim; B = 1) and what it published for them on its RTX 3080 Ti (src/cuda/README.md:
# 516-539: forward kernel_us, backward bwd_us).  Context for the same-shape rows, not a target.
REF_ATTN_SHAPES = [
    ("ctx256", 256, 4, 2, 32, 104.690, 588.80), ("ctx512", 512, 4, 2, 32, 336.031, 1474.56),
    ("ctx1024", 1024, 4, 2, 32, 1160.164, 4727.10), ("ctx2048", 2048, 4, 2, 32, 4576.780, 17725.34),
    ("ctx4096", 4096, 4, 2, 32, 18374.339, 70319.87), ("llama3-T256", 256, 32, 8, 128, 3155.822, 31140.86),
    ("llama3-T512", 512, 32, 8, 128, 11803.331, 115709.92), ("gqa-96-T256", 256, 32, 8, 96, 2468.086, 18982.82),
    ("gqa-96-T512", 512, 32, 8, 96, 9295.332, 69966.66), ("mha-192-T256", 256, 16, 16, 192, 2411.664, 30832.64),
    ("gqa-256-T256", 256, 8, 4, 256, 1656.361, 28313.25),
]
# The reference's RMSNorm shapes and its published gpu / gpu_sync / gpu_e2e microseconds per call
# (src/cuda/README.md:255-266, same card), timed here the same three ways (src/cuda/norm.cu:486-571).
REF_NORM_SHAPES = [
    ("micro", 32, 32, 3.68, 7.51, 16.49), ("small", 32, 128, 3.16, 6.91, 18.95),
    ("mid", 128, 128, 4.53, 8.33, 32.95), ("ship", 256, 128, 7.31, 11.06, 50.45),
    ("tall", 4096, 128, 76.56, 80.35, 541.32), ("r1024c512", 1024, 512, 21.49, 25.31, 498.58),
    ("r256c2048", 256, 2048, 8.60, 12.43, 478.94), ("r1024c2048", 1024, 2048, 28.79, 32.56, 1769.64),
    ("big", 4096, 4096, 232.11, 235.96, 19672.66),
]


def _load(name, rel):
    spec = importlib.util.spec_from_file_location(name, os.path.join(ROOT, rel))
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def event_time(torch, fn, n, reps=3):
    """Average ms per call of fn over n back-to-back calls, HIP events on the
    current stream (the stream every launch here goes to); the minimum of
    `reps` such measurements (the reference harness's statistic)."""
    return min(_event_time_once(torch, fn, n) for _ in range(reps))


def _event_time_once(torch, fn, n):
    s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    s.record()
    for _ in range(n):
        fn()
    e.record()
    e.synchronize()
    return s.elapsed_time(e) / n


def event_time_after(torch, pre, fn, n, reps=3):
    """Average ms of fn alone over n calls, each preceded by pre() on the same
    stream (events around fn only): for a stage that consumes what pre leaves,
    such as the dk/dv stage reading the scores a forward stored.  Minimum of
    `reps` measurements."""
    best = None
    for _ in range(reps):
        ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(n)]
        for s, e in ev:
            pre()
            s.record()
            fn()
            e.record()
        torch.cuda.synchronize()
        t = sum(s.elapsed_time(e) for s, e in ev) / n
        best = t if best is None else min(best, t)
    return best


def _hip():
    """The HIP runtime, for the synchronous copies and device synchronisations
    the reference's end-to-end timings are made of (cudaMemcpy /
    cudaDeviceSynchronize, src/cuda/norm.cu:556-571): the copy of the runtime
    already in the process (by soname; torch and libzt_attn share it), never a
    second one loaded by path."""
    hip = ctypes.CDLL("libamdhip64.so.7")
    hip.hipMemcpy.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int]
    hip.hipMemcpy.restype = ctypes.c_int
    hip.hipDeviceSynchronize.restype = ctypes.c_int
    return hip


def wall_us(fn, n, reps=3):
    """Host wall-clock microseconds per call of a synchronous fn (min of reps)."""
    best = None
    for _ in range(reps):
        t0 = time.perf_counter()
        for _ in range(n):
            fn()
        t = (time.perf_counter() - t0) * 1e6 / n
        best = t if best is None else min(best, t)
    return best


def norm_views(torch, zt, dev):
    """RMSNorm at the reference's shapes, three ways as src/cuda/norm.cu:486-571
    times it: kernel_us (launches back to back, one synchronise), sync_us
    (launch and synchronise on every call) and e2e_us (host-to-device copy of
    x, kernel, device-to-host copy of y, on every call, pageable host memory),
    beside the reference's published figures for the same shapes."""
    import numpy as np
    hip = _hip()
    fn = zt.lib().zt_rmsnorm_forward
    sp = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    rows_out = []
    for tag, rows, cols, r_gpu, r_sync, r_e2e in REF_NORM_SHAPES:
        x = torch.empty(rows * cols, device=dev)
        zt.fill_normal(x, SEEDS["x"], 0.0, 1.0)
        w = torch.empty(cols, device=dev)
        zt.fill_uniform(w, SEEDS["w"], 0.5, 1.5)
        y = torch.empty_like(x)
        hx = x.cpu().numpy()
        hy = np.empty_like(hx)
        nb = rows * cols * 4
        px, pw, py = (ctypes.c_void_p(t.data_ptr()) for t in (x, w, y))

        def launch():
            if fn(px, pw, py, rows, cols, 1e-5, sp):
                raise RuntimeError("zt_rmsnorm_forward refused")

        def synced():
            launch()
            if hip.hipDeviceSynchronize():
                raise RuntimeError("hipDeviceSynchronize failed")

        def e2e():
            if hip.hipMemcpy(px, hx.ctypes.data, nb, 1):
                raise RuntimeError("hipMemcpy H2D failed")
            launch()
            if hip.hipMemcpy(hy.ctypes.data, py, nb, 2):
                raise RuntimeError("hipMemcpy D2H failed")

        iters = 200 if nb <= (1 << 20) else 40
        launch()
        torch.cuda.synchronize()
        k_us = event_time(torch, launch, iters) * 1e3
        s_us = wall_us(synced, iters)
        e_us = wall_us(e2e, max(5, iters // 4))
        rows_out.append({"shape": tag, "rows": rows, "cols": cols, "kernel_us": round(k_us, 2),
                         "sync_us": round(s_us, 2), "e2e_us": round(e_us, 2),
                         "reference_rtx3080ti": {"kernel_us": r_gpu, "sync_us": r_sync, "e2e_us": r_e2e}})
        log(f"RMSNorm {tag} {rows}x{cols}: kernel {k_us:.2f} us, sync {s_us:.2f} us, e2e {e_us:.2f} us "
            f"(reference, its card: {r_gpu} / {r_sync} / {r_e2e})")
        del x, w, y
    return rows_out


def reference_shape_rows(torch, zt, dev):
    """The reference's attention benchmark shapes (B = 1) through its own two
    entry points, as its harness times them (launches back to back; min of 3):
    zt_attn_forward and zt_attn_backward, and beside them the training pair
    (zt_attn_forward_train_ws + zt_attn_backward_train_ws with the forward's
    scores)."""
    L = zt.lib()
    sp = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    out_rows = []
    for tag, T, H, Hkv, D, r_fwd, r_bwd in REF_ATTN_SHAPES:
        q, do = (torch.empty(T * H * D, device=dev) for _ in range(2))
        k, v = (torch.empty(T * Hkv * D, device=dev) for _ in range(2))
        for t, sd in ((q, "q"), (k, "k"), (v, "v"), (do, "do")):
            zt.fill_normal(t, SEEDS[sd], 0.0, 1.0)
        out, dq = torch.empty_like(q), torch.empty_like(q)
        dk, dv = torch.empty_like(k), torch.empty_like(v)
        rm, rl, rd, lse = (torch.empty(T * H, device=dev) for _ in range(4))
        work = torch.empty(zt.backward_train_workspace_bytes(1, T, H, Hkv, D) // 4, device=dev)
        P = lambda t: ctypes.c_void_p(t.data_ptr())
        fargs = (P(q), P(k), P(v), P(out), T, H, Hkv, D, 1, 64, 0, T, sp)
        bargs = (P(q), P(k), P(v), P(do), P(dq), P(dk), P(dv), P(rm), P(rl), P(rd), T, H, Hkv, D, 64, sp)

        def fwd():
            if L.zt_attn_forward(*fargs):
                raise RuntimeError("zt_attn_forward refused")

        def bwd():
            if L.zt_attn_backward(*bargs):
                raise RuntimeError("zt_attn_backward refused")

        def train():
            zt.forward_train_ws(q, k, v, out, lse, work, T, H, Hkv, D)
            zt.backward_train_ws(q, k, v, out, do, lse, dq, dk, dv, work, T, H, Hkv, D, stage=3 | zt.ZT_WS_SCORES)

        n = 50 if T <= 512 else 20
        fwd()
        bwd()
        train()
        torch.cuda.synchronize()
        t_f = event_time(torch, fwd, n) * 1e3
        t_b = event_time(torch, bwd, n) * 1e3
        t_t = event_time(torch, train, n) * 1e3
        fl = 2.0 * H * D * T * (T + 1)      # one causal T x T x d matmul
        out_rows.append({"shape": tag, "T": T, "n_heads": H, "n_kv_heads": Hkv, "head_dim": D,
                         "fwd_us": round(t_f, 2), "bwd_us": round(t_b, 2), "train_step_us": round(t_t, 2),
                         "fwd_TFLOP/s": round(2 * fl / (t_f * 1e-6) / 1e12, 2),
                         "reference_rtx3080ti": {"fwd_us": r_fwd, "bwd_us": r_bwd}})
        log(f"{tag}: zt_attn_forward {t_f:.1f} us, zt_attn_backward {t_b:.1f} us, training pair {t_t:.1f} us "
            f"(reference, its card: {r_fwd} / {r_bwd} us)")
        del q, k, v, do, out, dq, dk, dv, rm, rl, rd, lse, work
    return out_rows


def seam_e2e(torch, zt, dev, T, H, Hkv, D, reps):
    """The drop-in seams as the patched reference issues them through the
    holder (device.Attn), host buffers in and out:
      forward  = model.cudaForward (src/model.zig:467-516): upload q, k, v;
                 forward(1, 64); download out;
      backward = autograd's deviceAttentionBackward (integration patch):
                 upload q, k, v, dout; forward(1, 64); backward(64); download
                 dq, dk, dv;
    each synchronous end to end (pageable host memory, as Zig's slices are),
    beside the same calls on device-resident buffers (no copies)."""
    import numpy as np
    L = zt.lib()
    hp = ctypes.c_void_p()
    if L.zt_holder_init(T, H, Hkv, D, ctypes.byref(hp)) != 0:
        raise RuntimeError("zt_holder_init refused")
    try:
        host = {}
        for which, n, seed in ((zt.ZT_BUF_Q, T * H * D, SEEDS["q"]), (zt.ZT_BUF_K, T * Hkv * D, SEEDS["k"]),
                               (zt.ZT_BUF_V, T * Hkv * D, SEEDS["v"]), (zt.ZT_BUF_DOUT, T * H * D, SEEDS["do"])):
            t = torch.empty(n, device=dev)
            zt.fill_normal(t, seed, 0.0, 1.0)
            host[which] = t.cpu().numpy()
            del t
        outs = {w: np.empty(T * (H if w in (zt.ZT_BUF_OUT, zt.ZT_BUF_DQ) else Hkv) * D, np.float32)
                for w in (zt.ZT_BUF_OUT, zt.ZT_BUF_DQ, zt.ZT_BUF_DK, zt.ZT_BUF_DV)}

        def up(*ws):
            for w in ws:
                a = host[w]
                if L.zt_holder_upload(hp, w, ctypes.c_void_p(a.ctypes.data), a.size):
                    raise RuntimeError("zt_holder_upload refused")

        def down(*ws):
            for w in ws:
                a = outs[w]
                if L.zt_holder_download(hp, ctypes.c_void_p(a.ctypes.data), w, a.size):
                    raise RuntimeError("zt_holder_download refused")

        def fwd_dev():
            if L.zt_holder_forward(hp, 1, 64):
                raise RuntimeError("zt_holder_forward refused")

        def bwd_dev():
            fwd_dev()
            if L.zt_holder_backward(hp, 64):
                raise RuntimeError("zt_holder_backward refused")

        def fwd_e2e():
            up(zt.ZT_BUF_Q, zt.ZT_BUF_K, zt.ZT_BUF_V)
            fwd_dev()
            down(zt.ZT_BUF_OUT)

        def bwd_e2e():
            up(zt.ZT_BUF_Q, zt.ZT_BUF_K, zt.ZT_BUF_V, zt.ZT_BUF_DOUT)
            bwd_dev()
            down(zt.ZT_BUF_DQ, zt.ZT_BUF_DK, zt.ZT_BUF_DV)

        up(zt.ZT_BUF_Q, zt.ZT_BUF_K, zt.ZT_BUF_V, zt.ZT_BUF_DOUT)
        for _ in range(2):
            bwd_e2e()
            fwd_e2e()
        res = {"forward_e2e_us": wall_us(fwd_e2e, reps), "backward_e2e_us": wall_us(bwd_e2e, reps),
               "forward_device_us": event_time(torch, fwd_dev, reps) * 1e3,
               "forward_backward_device_us": event_time(torch, bwd_dev, reps) * 1e3}
        res = {k2: round(v2, 2) for k2, v2 in res.items()}
        res["bytes_up_down"] = {"forward": 4 * T * (2 * H + 2 * Hkv) * D,
                                "backward": 4 * T * (2 * H + 2 * Hkv) * D + 4 * T * (H + 2 * Hkv) * D}
        return res
    finally:
        L.zt_holder_deinit(hp)


def decode_seam_holder(torch, zt, dev, n_ctx, H, Hkv, D, n_holders, calls):
    """decode.zig:462's forwardAt(1, 64, n_keys - 1, n_keys, 1) through the
    holder, which splits the keys over the device: on device-resident caches
    (n_holders sequences, cycled so the caches exceed the 256 MB MALL) in
    microseconds per call, and end to end as src/decode.zig:405-473 issues it
    (upload the query row and the n_keys cache rows of K and V, forwardAt,
    download the output row)."""
    import numpy as np
    L = zt.lib()
    hs = []
    try:
        for _ in range(n_holders):
            hp = ctypes.c_void_p()
            if L.zt_holder_init(n_ctx, H, Hkv, D, ctypes.byref(hp)) != 0:
                raise RuntimeError("zt_holder_init refused")
            hs.append(hp)
        for i, hp in enumerate(hs):
            for which, n, seed in ((zt.ZT_BUF_Q, H * D, SEEDS["q"]), (zt.ZT_BUF_K, n_ctx * Hkv * D, SEEDS["kc"]),
                                   (zt.ZT_BUF_V, n_ctx * Hkv * D, SEEDS["vc"])):
                if L.zt_fill_normal(L.zt_holder_buffer(hp, which), n, seed + 64 * i, 0.0, 1.0, None):
                    raise RuntimeError("zt_fill_normal refused")
        it = [0]

        def call():
            hp = hs[it[0] % n_holders]
            it[0] += 1
            if L.zt_holder_forward_at(hp, 1, 64, n_ctx - 1, n_ctx, 1):
                raise RuntimeError("zt_holder_forward_at refused")

        for _ in range(2 * n_holders):
            call()
        t_call = event_time(torch, call, calls) * 1e3
        hq = np.empty(H * D, np.float32)
        hk = np.empty(n_ctx * Hkv * D, np.float32)
        hv = np.empty_like(hk)
        ho = np.empty(H * D, np.float32)
        hp = hs[0]
        for a, w in ((hq, zt.ZT_BUF_Q), (hk, zt.ZT_BUF_K), (hv, zt.ZT_BUF_V)):
            L.zt_holder_download(hp, ctypes.c_void_p(a.ctypes.data), w, a.size)

        def e2e():
            for a, w in ((hq, zt.ZT_BUF_Q), (hk, zt.ZT_BUF_K), (hv, zt.ZT_BUF_V)):
                if L.zt_holder_upload(hp, w, ctypes.c_void_p(a.ctypes.data), a.size):
                    raise RuntimeError("zt_holder_upload refused")
            if L.zt_holder_forward_at(hp, 1, 64, n_ctx - 1, n_ctx, 1):
                raise RuntimeError("zt_holder_forward_at refused")
            if L.zt_holder_download(hp, ctypes.c_void_p(ho.ctypes.data), zt.ZT_BUF_OUT, ho.size):
                raise RuntimeError("zt_holder_download refused")

        e2e()
        t_e2e = wall_us(e2e, 5)
        return t_call, t_e2e
    finally:
        for hp in hs:
            L.zt_holder_deinit(hp)


def other_configs(torch, zt, dev, args, normal, scores):
    # ---------------- C2, C5: the other training configurations ----------------
    # Secondary figures (C3 is the headline): the same training step -- the
    # forward keeping its scores where the shape allows, then the backward --
    # and the reference's own entry points, on the configurations' inputs
    # (C5: N(0, 2), sigma = sqrt(2)).
    other = {}
    other_cfgs = {"C2": (4, 1024, 8, 8, 64, 1.0), "C5": (2, 2048, 16, 4, 256, 2.0 ** 0.5)}
    for cname, (Bo, To, Ho, Hkvo, Do, sig) in other_cfgs.items():
        qo, do_ = normal(Bo * To * Ho * Do, SEEDS["q"], sig), normal(Bo * To * Ho * Do, SEEDS["do"], sig)
        ko, vo = normal(Bo * To * Hkvo * Do, SEEDS["k"], sig), normal(Bo * To * Hkvo * Do, SEEDS["v"], sig)
        oo, dqo = torch.empty_like(qo), torch.empty_like(qo)
        dko, dvo = torch.empty_like(ko), torch.empty_like(vo)
        lseo, rmo, rlo, rdo = (torch.empty(Bo * To * Ho, device=dev) for _ in range(4))
        wo = torch.empty(zt.backward_train_workspace_bytes(Bo, To, Ho, Hkvo, Do) // 4, device=dev)
        flop_o = 7 * 2 * Do * Bo * Ho * To * (To + 1) / 2

        def train_o():
            zt.forward_train_ws(qo, ko, vo, oo, lseo, wo, To, Ho, Hkvo, Do, B=Bo)
            zt.backward_train_ws(qo, ko, vo, oo, do_, lseo, dqo, dko, dvo, wo, To, Ho, Hkvo, Do, B=Bo, stage=scores)

        def ref_o():
            zt.forward(qo, ko, vo, oo, To, Ho, Hkvo, Do, B=Bo)
            zt.backward(qo, ko, vo, do_, dqo, dko, dvo, rmo, rlo, rdo, To, Ho, Hkvo, Do, B=Bo)

        entry = {"workload": f"{cname} B={Bo} T={To} Hq={Ho} Hkv={Hkvo} d={Do} f32"}
        for tag, fn in (("train", train_o), ("reference_abi", ref_o)):
            for _ in range(args.warmup):
                fn()
            t_o = event_time(torch, fn, max(3, args.steps))
            entry[tag] = {"ms_per_step": round(t_o, 4), "TFLOP/s": round(flop_o / (t_o * 1e-3) / 1e12, 3)}
            log(f"{cname} step ({tag}): {t_o:.3f} ms, {flop_o / (t_o * 1e-3) / 1e12:.2f} TFLOP/s fwd+bwd")
        # Per kernel of the training step, as for C3: the forward, the dk/dv
        # stage (zt_bwd_delta + the dk/dv kernel, after a forward each time
        # when it reads the forward's scores) and the dq product.
        unit_o = flop_o / 7
        n_fwd, n_dq, n_dkdv = zt.plan_train(Bo, To, Ho, Hkvo, Do)
        reads_scores = any(t in n_dkdv for t in ("dkdv8s", "dkdv_dmas", "dkdv_dmars"))
        fwd_o = lambda: zt.forward_train_ws(qo, ko, vo, oo, lseo, wo, To, Ho, Hkvo, Do, B=Bo)
        st1 = 1 | (zt.ZT_WS_SCORES if reads_scores else 0)
        dkdv_o = lambda: zt.backward_train_ws(qo, ko, vo, oo, do_, lseo, dqo, dko, dvo, wo, To, Ho, Hkvo, Do, B=Bo,
                                              stage=st1)
        dq_o = lambda: zt.backward_train_ws(qo, ko, vo, oo, do_, lseo, dqo, dko, dvo, wo, To, Ho, Hkvo, Do, B=Bo,
                                            stage=2)
        nk = max(5, args.steps)
        t_f = event_time(torch, fwd_o, nk)
        t_kv = event_time_after(torch, fwd_o, dkdv_o, nk) if reads_scores else event_time(torch, dkdv_o, nk)
        t_q = event_time(torch, dq_o, nk)
        ks = []
        for kname, t_k, units in ((n_fwd, t_f, 2), (n_dkdv, t_kv, 3 if reads_scores else 4), (n_dq, t_q, 1)):
            tf_k = units * unit_o / (t_k * 1e-3) / 1e12
            ks.append({"kernel": kname, "ms": round(t_k, 4), "flop": units * unit_o, "tflops": round(tf_k, 3),
                       "frac_mfma_f32": round(tf_k / PEAK_MFMA_F32, 4)})
            log(f"  {cname} {kname}: {t_k * 1e3:.1f} us, {tf_k:.2f} TFLOP/s ({100 * tf_k / PEAK_MFMA_F32:.1f}%)")
        entry["train"]["kernels"] = ks
        entry["train"]["launch_gaps_ms"] = round(entry["train"]["ms_per_step"] - t_f - t_kv - t_q, 4)
        other[cname] = entry
        del qo, ko, vo, do_, oo, dqo, dko, dvo, lseo, rmo, rlo, rdo, wo

    return other


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=10)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--cpu-rows", type=int, default=48, help="query rows of the CPU baseline sample")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-other", action="store_true", help="skip the C2 / C5 figures (profiling runs)")
    ap.add_argument("--no-views", action="store_true",
                    help="skip the reference-shape, sync / end-to-end and seam views (profiling runs)")
    ap.add_argument("--only-other", action="store_true",
                    help="run the C2 / C5 section alone and print its figures (profiling runs)")
    args = ap.parse_args()
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print("bench.py measures one GPU: this build's path runs on one MI355X (sharding by kv head or batch "
              "across GPUs, which needs no collective, is not built). Run with --gpus 1.", file=sys.stderr)
        sys.exit(2)

    import torch
    zt = _load("zt_attn", "z-transformer_amd/zt_attn.py")
    torch.cuda.set_device(0)
    dev = "cuda:0"
    assert zt.lib().zt_attn_lds_limit() > 0, "libzt_attn found no usable gfx950 device"

    def normal(n, seed, sigma=1.0):
        t = torch.empty(n, device=dev, dtype=torch.float32)
        zt.fill_normal(t, seed, 0.0, sigma)
        return t

    if args.only_other:
        other = other_configs(torch, zt, dev, args, normal, 3 | zt.ZT_WS_SCORES)
        print(json.dumps({"other_configs": other}), flush=True)
        return

    # ---------------- calibration: what this device sustains ----------------
    cal_src = torch.empty(1 << 30, device=dev)          # 4 GiB streaming-read source
    cal_scratch = torch.empty(2048 * 256, device=dev)
    cal_tflops, cal_gbs = zt.calibrate(cal_src, cal_scratch)
    del cal_src, cal_scratch
    log(f"calibration: FP32 MFMA sustained {cal_tflops:.1f} TFLOP/s, streaming read {cal_gbs:.0f} GB/s")

    # ---------------- C3: fused causal GQA fwd + bwd ----------------
    B, T, H, Hkv, D = 1, 4096, 32, 8, 128
    q0, k0 = normal(B * T * H * D, SEEDS["q"]), normal(B * T * Hkv * D, SEEDS["k"])
    q, k = torch.empty_like(q0), torch.empty_like(k0)

    def rope_qk():  # src/model.zig:372-377: q and k rotated at position 0, one launch
        zt.rope_qk(q0, k0, q, k, B, T, H, Hkv, D, 0, THETA)

    rope_qk()
    t_rope = event_time(torch, rope_qk, 10)
    rope_bytes = 2 * (q.numel() + k.numel()) * 4
    log(f"C3 RoPE q+k: {t_rope * 1e3:.1f} us, {rope_bytes / (t_rope * 1e-3) / 1e9:.0f} GB/s")
    del q0, k0
    v, do = normal(B * T * Hkv * D, SEEDS["v"]), normal(B * T * H * D, SEEDS["do"])
    out, dq = torch.empty_like(q), torch.empty_like(q)
    dk, dv = torch.empty_like(k), torch.empty_like(v)
    rm, rl, rd = (torch.empty(B * T * H, device=dev) for _ in range(3))
    lse, delta = (torch.empty(B * T * H, device=dev) for _ in range(2))
    work_bytes = zt.backward_train_workspace_bytes(B, T, H, Hkv, D)  # delta + the causal dS tiles
    work = torch.empty(work_bytes // 4, device=dev)
    pairs = B * H * T * (T + 1) / 2          # causal (query, key) pairs over all heads
    unit = 2 * D * pairs                      # FLOPs of one T x T x d causal matmul
    fwd_flop, bwd_flop = 2 * unit, 5 * unit

    # The timed step is a training step's attention: the forward keeps each
    # row's log-sum-exp and its scores, and the backward uses them
    # (zt_attn_forward_train_ws / zt_attn_backward_train_ws).  The same pair
    # without the scores, the pair without a workspace, and the reference's
    # own entry points, whose backward rebuilds the statistics, are timed
    # beside it.  dkdv_units: the matmuls the dk/dv kernel executes (the
    # score-reading kernel: dP, dV, dK; the others also S = Q K^T).
    scores = 3 | zt.ZT_WS_SCORES
    paths = {
        "train": dict(
            fwd=lambda: zt.forward_train_ws(q, k, v, out, lse, work, T, H, Hkv, D),
            # The dk/dv stage consumes the scores the forward stored (a second
            # ZT_WS_SCORES stage without a forward between is refused), so it is
            # timed after a forward each time, with events around the stage only.
            dkdv=lambda: zt.backward_train_ws(q, k, v, out, do, lse, dq, dk, dv, work, T, H, Hkv, D,
                                              stage=1 | zt.ZT_WS_SCORES),
            dkdv_after_fwd=True,
            dq=lambda: zt.backward_train_ws(q, k, v, out, do, lse, dq, dk, dv, work, T, H, Hkv, D, stage=2),
            bwd=lambda: zt.backward_train_ws(q, k, v, out, do, lse, dq, dk, dv, work, T, H, Hkv, D, stage=scores),
            names=zt.plan_train(B, T, H, Hkv, D), dkdv_units=3, dq_exec_units=1),
        "train_recompute_scores": dict(
            fwd=lambda: zt.forward_train(q, k, v, out, lse, T, H, Hkv, D),
            dkdv=lambda: zt.backward_train_ws(q, k, v, out, do, lse, dq, dk, dv, work, T, H, Hkv, D, stage=1),
            dq=lambda: zt.backward_train_ws(q, k, v, out, do, lse, dq, dk, dv, work, T, H, Hkv, D, stage=2),
            bwd=lambda: zt.backward_train_ws(q, k, v, out, do, lse, dq, dk, dv, work, T, H, Hkv, D),
            names=(zt.plan(B, T, H, Hkv, D)[0], zt.plan_train(B, T, H, Hkv, D)[1], zt.plan(B, T, H, Hkv, D)[2]),
            dkdv_units=4, dq_exec_units=1),
        "train_dq_kernel": dict(
            fwd=lambda: zt.forward_train(q, k, v, out, lse, T, H, Hkv, D),
            dq=lambda: zt.bwd_dq_train(q, k, v, out, do, lse, dq, delta, T, H, Hkv, D),
            dkdv=lambda: zt.bwd_dkdv_train(q, k, v, out, do, lse, delta, dk, dv, T, H, Hkv, D),
            bwd=lambda: zt.backward_train(q, k, v, out, do, lse, dq, dk, dv, delta, T, H, Hkv, D),
            names=(zt.plan(B, T, H, Hkv, D)[0], "zt_bwd_dql_d%d_k32" % D, zt.plan(B, T, H, Hkv, D)[2]),
            dkdv_units=4, dq_exec_units=3),
        "reference_abi": dict(
            fwd=lambda: zt.forward(q, k, v, out, T, H, Hkv, D),
            dq=lambda: zt.bwd_dq(q, k, v, do, dq, rm, rl, rd, T, H, Hkv, D),
            dkdv=lambda: zt.bwd_dkdv(q, k, v, do, dk, dv, rm, rl, rd, T, H, Hkv, D),
            bwd=lambda: zt.backward(q, k, v, do, dq, dk, dv, rm, rl, rd, T, H, Hkv, D),
            names=zt.plan(B, T, H, Hkv, D), dkdv_units=4, dq_exec_units=4),
    }
    res = {}
    for pname, pth in paths.items():
        def step():
            pth["fwd"]()
            pth["bwd"]()

        for _ in range(args.warmup):
            step()
        torch.cuda.synchronize()
        s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        t_wall = time.perf_counter()
        s.record()
        for _ in range(args.steps):
            step()
        e.record()
        torch.cuda.synchronize()
        wall_ms = (time.perf_counter() - t_wall) * 1e3 / args.steps
        ms_step = s.elapsed_time(e) / args.steps
        val = (fwd_flop + bwd_flop) / (ms_step * 1e-3) / 1e12
        log(f"C3 step ({pname}): {ms_step:.3f} ms (wall {wall_ms:.3f} ms), {val:.2f} TFLOP/s fwd+bwd")

        n_k = max(3, args.steps)
        t_fwd = event_time(torch, pth["fwd"], n_k)
        if pth.get("dkdv_after_fwd"):
            t_dkdv = event_time_after(torch, pth["fwd"], pth["dkdv"], n_k)
        else:
            pth["dkdv"]()
            t_dkdv = event_time(torch, pth["dkdv"], n_k)
        # the dq stage reads what the dk/dv stage last wrote (row statistics or dS)
        t_dq = event_time(torch, pth["dq"], n_k)
        # Algorithmic FLOPs per launch: the forward's two matmuls; of the
        # backward's five (S recompute, dP, dV, dK, dQ) the dk/dv kernel owns
        # the ones it executes (three when it reads the forward's scores, else
        # four) and the dq kernel one -- the dq kernel's own recomputes earn no credit.
        n_fwd, n_dq, n_dkdv = pth["names"]
        kernels = [
            {"kernel": n_fwd, "ms": t_fwd, "flop": fwd_flop},
            {"kernel": n_dq, "ms": t_dq, "flop": unit},
            {"kernel": n_dkdv, "ms": t_dkdv, "flop": pth["dkdv_units"] * unit},
        ]
        for kk in kernels:
            kk["tflops"] = kk["flop"] / (kk["ms"] * 1e-3) / 1e12
            kk["frac_mfma_f32"] = kk["tflops"] / PEAK_MFMA_F32
            log(f"  {kk['kernel']}: {kk['ms']:.3f} ms, {kk['tflops']:.2f} TFLOP/s ({100 * kk['frac_mfma_f32']:.1f}% "
                f"of FP32 MFMA peak)")
        fwd_tflops = fwd_flop / (t_fwd * 1e-3) / 1e12
        bwd_tflops = bwd_flop / ((t_dq + t_dkdv) * 1e-3) / 1e12
        # What the backward's kernels execute (dk/dv's matmuls plus the dq
        # kernel's own, recomputes included): the utilisation figure.  The FA2
        # count above credits 5 units whatever runs, so it is no fraction of peak.
        bwd_exec = (pth["dkdv_units"] + pth["dq_exec_units"]) * unit / ((t_dq + t_dkdv) * 1e-3) / 1e12
        log(f"  forward {fwd_tflops:.2f} TFLOP/s ({100 * fwd_tflops / PEAK_MFMA_F32:.1f}% of FP32 MFMA peak); "
            f"backward {bwd_tflops:.2f} TFLOP/s by the FA2 count, {bwd_exec:.2f} TFLOP/s executed "
            f"({100 * bwd_exec / PEAK_MFMA_F32:.1f}% of peak)")
        res[pname] = dict(ms_step=ms_step, value=val, kernels=kernels, fwd_tflops=fwd_tflops,
                          bwd_tflops=bwd_tflops, bwd_exec_tflops=bwd_exec)
    # The drop-in holder (include/zt_holder.h, device.zig's Attn) on device-resident
    # buffers: zt_holder_forward + zt_holder_backward as device.Attn.forward(1, 64) +
    # backward(64) issue them, on the same C3 inputs (copied into the holder's buffers).
    L = zt.lib()
    hp = ctypes.c_void_p()
    if L.zt_holder_init(T, H, Hkv, D, ctypes.byref(hp)) != 0:
        raise RuntimeError("zt_holder_init refused at C3")
    # The same seeded inputs, generated into the holder's own buffers, q and k rotated in place.
    for which, n, seed in ((zt.ZT_BUF_Q, q.numel(), SEEDS["q"]), (zt.ZT_BUF_K, k.numel(), SEEDS["k"]),
                           (zt.ZT_BUF_V, v.numel(), SEEDS["v"]), (zt.ZT_BUF_DOUT, do.numel(), SEEDS["do"])):
        if L.zt_fill_normal(L.zt_holder_buffer(hp, which), n, seed, 0.0, 1.0, None):
            raise RuntimeError("zt_fill_normal refused")
    hq, hk = L.zt_holder_buffer(hp, zt.ZT_BUF_Q), L.zt_holder_buffer(hp, zt.ZT_BUF_K)
    if L.zt_rope_qk_forward(hq, hk, hq, hk, B, T, H, Hkv, D, 0, THETA, None):
        raise RuntimeError("zt_rope_qk_forward refused")
    L.zt_holder_forget(hp)  # written through the raw pointers

    def holder_step():
        if L.zt_holder_forward(hp, 1, 64) or L.zt_holder_backward(hp, 64):
            raise RuntimeError("holder refused")

    for _ in range(args.warmup):
        holder_step()
    t_holder = event_time(torch, holder_step, max(3, args.steps))
    holder_ws = L.zt_holder_workspace_bytes(hp)
    L.zt_holder_deinit(hp)
    log(f"C3 step (holder: zt_holder_forward + zt_holder_backward): {t_holder:.3f} ms, "
        f"{(fwd_flop + bwd_flop) / (t_holder * 1e-3) / 1e12:.2f} TFLOP/s, workspace {holder_ws / 2 ** 30:.2f} GiB")
    ms_step, value = res["train"]["ms_step"], res["train"]["value"]
    kernels, fwd_tflops, bwd_tflops = res["train"]["kernels"], res["train"]["fwd_tflops"], res["train"]["bwd_tflops"]
    exec_flop = sum(kk["flop"] for kk in kernels)   # the matmuls the step's kernels execute
    dom = max(kernels, key=lambda x: x["ms"])
    traffic = None
    tpath = os.path.join(ROOT, "profiles", "traffic.json")
    if os.path.exists(tpath):
        with open(tpath) as f:
            traffic = json.load(f).get(dom["kernel"])
    roofline = {"bound": "mfma", "achieved": round(dom["tflops"], 3), "peak": PEAK_MFMA_F32, "unit": "TFLOP/s",
                "frac": round(dom["tflops"] / PEAK_MFMA_F32, 4), "traffic": traffic, "kernel": dom["kernel"]}
    del out, dq, dk, dv, do, q, k, v, rm, rl, rd, lse, delta, work

    other = {} if args.no_other else other_configs(torch, zt, dev, args, normal, scores)

    # ---------------- C4: decode step ----------------
    Bd, n_ctx = 64, 8192
    qd = normal(Bd * H * D, SEEDS["q"])
    kc = normal(Bd * n_ctx * Hkv * D, SEEDS["kc"])
    vc = normal(Bd * n_ctx * Hkv * D, SEEDS["vc"])
    od = torch.empty_like(qd)
    ws = torch.empty(zt.decode_workspace_bytes(Bd, n_ctx, H, Hkv, D) // 4 + 1, device=dev)
    n_keys = [n_ctx] * Bd

    def dec():
        zt.decode(qd, kc, vc, od, n_keys, Bd, n_ctx, H, Hkv, D, ws)

    for _ in range(3):
        dec()
    t_dec = event_time(torch, dec, max(10, args.steps))
    dec_bytes = 2 * Bd * n_ctx * Hkv * D * 4 + 2 * Bd * H * D * 4
    dec_gbs = dec_bytes / (t_dec * 1e-3) / 1e9
    log(f"C4 decode: {t_dec * 1e3:.1f} us, {dec_gbs:.0f} GB/s ({100 * dec_gbs / PEAK_HBM:.1f}% of HBM peak)")

    # The device-resident step: RoPE on q and the new k, append at row 8191, attend.
    kn = normal(Bd * Hkv * D, SEEDS["k"])
    vn = normal(Bd * Hkv * D, SEEDS["v"])
    ws2 = torch.empty(zt.decode_step_workspace_bytes(Bd, n_ctx, H, Hkv, D) // 4 + 1, device=dev)
    pos = [n_ctx - 1] * Bd

    def dec_step():
        zt.decode_step(qd, kn, vn, kc, vc, od, pos, Bd, n_ctx, H, Hkv, D, ws2, THETA)

    for _ in range(3):
        dec_step()
    t_step = event_time(torch, dec_step, max(10, args.steps))
    step_gbs = dec_bytes / (t_step * 1e-3) / 1e9
    log(f"C4 decode_step (rope + append + attention): {t_step * 1e3:.1f} us, {step_gbs:.0f} GB/s")

    # The reference's own decode route (src/decode.zig:462): device.Attn.forwardAt(1, 64,
    # n_keys - 1, n_keys, 1), i.e. zt_attn_forward with T = 1 once per sequence over that
    # sequence's cache, called straight through the C entry point with resolved pointers.
    fwd_c = zt.lib().zt_attn_forward
    sp = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    rows = [(ctypes.c_void_p(qd.data_ptr() + b * H * D * 4), ctypes.c_void_p(kc.data_ptr() + b * n_ctx * Hkv * D * 4),
             ctypes.c_void_p(vc.data_ptr() + b * n_ctx * Hkv * D * 4), ctypes.c_void_p(od.data_ptr() + b * H * D * 4))
            for b in range(Bd)]

    def dec_seam():
        for qb, kb, vb, ob in rows:
            if fwd_c(qb, kb, vb, ob, 1, H, Hkv, D, 1, 64, n_ctx - 1, n_ctx, sp):
                raise RuntimeError("zt_attn_forward refused")

    for _ in range(3):
        dec_seam()
    t_seam = event_time(torch, dec_seam, max(5, args.steps // 2))
    seam_gbs = dec_bytes / (t_seam * 1e-3) / 1e9
    log(f"C4 reference decode seam (zt_attn_forward, T=1, one call per sequence): {t_seam * 1e3:.1f} us, "
        f"{seam_gbs:.0f} GB/s")
    del kc, vc, qd, od, ws, kn, vn, ws2
    # The same seam through the holder (device.Attn.forwardAt, which splits the keys).
    t_hcall, t_he2e = decode_seam_holder(torch, zt, dev, n_ctx, H, Hkv, D, n_holders=8, calls=64)
    call_bytes = dec_bytes / Bd
    log(f"C4 decode seam through the holder: {t_hcall:.1f} us per call ({call_bytes / (t_hcall * 1e-6) / 1e9:.0f} "
        f"GB/s), {Bd * t_hcall:.1f} us per 64-sequence step; end to end with the cache upload {t_he2e:.0f} us "
        f"per call")

    # ---------------- dense products (tensor.matmul and its gradients) ----------------
    mm = {}
    for tag, (M, K, N) in (("4096^3", (4096, 4096, 4096)), ("w_down 256x512x128", (256, 512, 128)),
                           ("w_up 256x128x512", (256, 128, 512)), ("head 256x128x456", (256, 128, 456))):
        a, b = normal(M * K, SEEDS["x"]), normal(K * N, SEEDS["w"])
        c = torch.empty(M * N, device=dev)
        zt.matmul(a, b, c, M, K, N)  # checked once through the binding, then timed at the C entry point
        args_mm = (ctypes.c_void_p(a.data_ptr()), ctypes.c_void_p(b.data_ptr()), ctypes.c_void_p(c.data_ptr()),
                   M, K, N, ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
        t_mm = event_time(torch, lambda: zt.lib().zt_matmul(*args_mm), 10)
        tf = 2.0 * M * K * N / (t_mm * 1e-3) / 1e12
        kname = zt.gemm_kernel(M, K, N)
        mm[tag] = {"us": round(t_mm * 1e3, 2), "TFLOP/s": round(tf, 2), "frac_mfma_f32": round(tf / PEAK_MFMA_F32, 4),
                   "kernel": kname}
        log(f"matmul {tag}: {t_mm * 1e3:.1f} us, {tf:.2f} TFLOP/s ({kname})")
        del a, b, c
    # The model shapes sit near the launch floor: empty kernels of the w_down
    # split-K grid (128 workgroups of 16 waves), back to back.
    mm["launch_floor_us"] = {"128 x 1024 threads": round(zt.launch_floor_us(128, 1024), 3)}
    log(f"matmul launch floor: {mm['launch_floor_us']}")

    # ---------------- RMSNorm over rotating buffers ----------------
    norm = {}
    # The launch floor: back-to-back launches of an empty kernel of the RMSNorm
    # grids (one 256-thread workgroup per row), timed in the library itself.
    floor = {"64 x 256 threads": round(zt.launch_floor_us(64, 256), 3),
             "4096 x 256 threads": round(zt.launch_floor_us(4096, 256), 3)}
    log(f"launch floor, 64 workgroups: {floor}")
    for rows, cols, sets in ((64, 4096, 256), (4096, 4096, 4)):
        xs = normal(sets * rows * cols, SEEDS["x"]).view(sets, rows * cols)
        ys = torch.empty_like(xs)
        w = torch.empty(cols, device=dev)
        zt.fill_uniform(w, SEEDS["w"], 0.5, 1.5)
        it = [0]
        # Straight to the C entry point with the pointers resolved once: a
        # native caller pays no Python binding cost, and at 2 MB per call the
        # binding's tensor checks would otherwise be most of what is timed.
        fn = zt.lib().zt_rmsnorm_forward
        px = [ctypes.c_void_p(xs[i].data_ptr()) for i in range(sets)]
        py = [ctypes.c_void_p(ys[i].data_ptr()) for i in range(sets)]
        pw = ctypes.c_void_p(w.data_ptr())
        sp = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)

        def nrm():
            i = it[0] % sets
            it[0] += 1
            if fn(px[i], pw, py[i], rows, cols, 1e-5, sp):
                raise RuntimeError("zt_rmsnorm_forward refused")

        for _ in range(sets):
            nrm()
        t_n = event_time(torch, nrm, 4 * sets)
        # The same launches, one per buffer set, captured once into a HIP
        # graph (kernel nodes only) and replayed: no host launch cost between
        # kernels, so this is the kernel's own time on the device.
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            cap = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
            for i in range(sets):
                if fn(px[i], pw, py[i], rows, cols, 1e-5, cap):
                    raise RuntimeError("zt_rmsnorm_forward refused under capture")
        graph.replay()
        torch.cuda.synchronize()
        t_g = event_time(torch, graph.replay, 4) / sets
        del graph
        nb = (2 * rows * cols + cols) * 4
        gbs = nb / (t_n * 1e-3) / 1e9
        gbs_g = nb / (t_g * 1e-3) / 1e9
        tag = f"{rows}x{cols}"
        norm[tag] = {"us": round(t_n * 1e3, 3), "GB/s": round(gbs, 1), "frac_hbm": round(gbs / PEAK_HBM, 4),
                     "bytes": nb, "rotating_sets": sets,
                     "graph_replay": {"us": round(t_g * 1e3, 3), "GB/s": round(gbs_g, 1),
                                      "frac_hbm": round(gbs_g / PEAK_HBM, 4)}}
        log(f"RMSNorm {tag}: {t_n * 1e3:.2f} us, {gbs:.0f} GB/s; graph replay {t_g * 1e3:.2f} us, "
            f"{gbs_g:.0f} GB/s")
        del xs, ys
    norm["launch_floor_us"] = floor

    # ---------------- Reference point: a plain 1 GiB device copy ----------------
    # The achievable streaming rate on this box, and the known-size kernel that
    # calibrates the FETCH_SIZE / WRITE_SIZE counters in profiles/.
    src = torch.empty(1 << 28, device=dev)
    dst = torch.empty_like(src)
    src.fill_(1.0)
    t_cp = event_time(torch, lambda: dst.copy_(src), 10)
    copy_gbs = 2 * src.numel() * 4 / (t_cp * 1e-3) / 1e9
    log(f"device copy 1 GiB: {t_cp * 1e3:.0f} us, {copy_gbs:.0f} GB/s")
    del src, dst

    # ---------------- The reference's own views: same shapes, sync and end-to-end ----------------
    norm_sync_e2e = ref_shapes = seams = None
    if not args.no_views:
        norm_sync_e2e = norm_views(torch, zt, dev)
        ref_shapes = reference_shape_rows(torch, zt, dev)
        seams = {"GPT-mini T=256 Hq=4 Hkv=2 d=32": seam_e2e(torch, zt, dev, 256, 4, 2, 32, 50),
                 "C3 T=4096 Hq=32 Hkv=8 d=128": seam_e2e(torch, zt, dev, 4096, 32, 8, 128, 5)}
        for tag, r in seams.items():
            log(f"seams {tag}: {r}")

    # ---------------- CPU baseline: the restatement on a bounded sample ----------------
    cpu = None
    if not args.no_cpu:
        import numpy as np
        oracle = _load("zt_oracle", "oracle/zt_oracle.py")
        W = max(1, min(args.cpu_rows, T))
        qh = oracle.fill_normal(B * T * H * D, SEEDS["q"])
        kh = oracle.fill_normal(B * T * Hkv * D, SEEDS["k"])
        qh = oracle.rope(qh, B * T, H * D, 0, THETA, D)
        kh = oracle.rope(kh, B * T, Hkv * D, 0, THETA, D)
        vh = oracle.fill_normal(B * T * Hkv * D, SEEDS["v"])
        dh = oracle.fill_normal(B * T * H * D, SEEDS["do"])
        t0 = time.perf_counter()
        oracle.attention_forward(qh, kh, vh, B, T, H, Hkv, D, t_begin=T - W, threads=1)
        oracle.attention_backward(qh, kh, vh, dh, B, T, H, Hkv, D, t_begin=T - W, threads=1)
        secs = time.perf_counter() - t0
        spairs = B * H * sum(t + 1 for t in range(T - W, T))
        sflop = 14 * D * spairs    # fwd 4d + bwd 10d FLOPs per causal pair, as the GPU figure counts
        cpu_model = "unknown"
        try:
            with open("/proc/cpuinfo") as f:
                cpu_model = next(l.split(":", 1)[1].strip() for l in f if l.startswith("model name"))
        except (OSError, StopIteration):
            pass
        cpu = {"value": round(sflop / secs / 1e12, 6), "unit": "TFLOP/s", "cores": 1, "kind": "port",
               "cpu_model": cpu_model, "host_threads": os.cpu_count(),
               "sample": f"C3 query rows {T - W}..{T - 1} ({W} of {T}, all {H} heads, full causal prefix), "
                         f"forward+backward of the C restatement of attention.zig/autograd.zig, 1 thread, "
                         f"{secs:.1f} s", "seconds": round(secs, 2)}
        log(f"CPU baseline: {cpu['value'] * 1e3:.3f} GFLOP/s on {W} rows ({secs:.1f} s)")
        # The same sample with the restatement's OpenMP variants, which split the
        # work by (sequence, head) / (sequence, kv head) and keep every element's
        # operation order (bit-identical to one thread); 16 threads is one GPU's
        # share of the box's host cores.
        nthr = max(1, min(16, os.cpu_count() or 1))
        t0 = time.perf_counter()
        oracle.attention_forward(qh, kh, vh, B, T, H, Hkv, D, t_begin=T - W, threads=nthr)
        oracle.attention_backward(qh, kh, vh, dh, B, T, H, Hkv, D, t_begin=T - W, threads=nthr)
        tsecs = time.perf_counter() - t0
        cpu["threaded"] = {"value": round(sflop / tsecs / 1e12, 6), "cores": nthr, "seconds": round(tsecs, 2)}
        log(f"CPU baseline, {nthr} threads: {cpu['threaded']['value'] * 1e3:.3f} GFLOP/s ({tsecs:.1f} s)")
        del np

    line = {
        "metric": METRIC, "value": round(value, 3), "unit": "TFLOP/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(ms_step, 4), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "f32",
        "data": "synthetic: splitmix64/Box-Muller N(0,1) generated on the device, RoPE theta=500000 on Q/K",
        "config": {"workload": "C3 causal GQA forward+backward, B=1 T=4096 Hq=32 Hkv=8 d=128 f32",
                   "global_batch": B, "seq_len": T, "n_heads": H, "n_kv_heads": Hkv, "head_dim": D,
                   "parallelism": "none (1 GPU)"},
        "roofline": roofline,
        "cpu_baseline": cpu,
        "fwd_tflops": round(fwd_tflops, 3), "bwd_tflops": round(bwd_tflops, 3),
        "bwd_executed_tflops": round(res["train"]["bwd_exec_tflops"], 3),
        "bwd_executed_frac": round(res["train"]["bwd_exec_tflops"] / PEAK_MFMA_F32, 4),
        "step_path": "zt_attn_forward_train_ws + zt_attn_backward_train_ws with ZT_WS_SCORES (saved log-sum-exp "
                     "and scores; the dk/dv kernel reads the scores and stores dS in their place; dq = dS k)",
        "executed_tflops": round(exec_flop / (ms_step * 1e-3) / 1e12, 3),
        "train_recompute_scores": {"step_path": "zt_attn_forward_train + zt_attn_backward_train_ws (the dk/dv "
                                                "kernel forms Q K^T again)",
                                   "ms_per_step": round(res["train_recompute_scores"]["ms_step"], 4),
                                   "TFLOP/s": round(res["train_recompute_scores"]["value"], 3)},
        "train_dq_kernel": {"step_path": "zt_attn_forward_train + zt_attn_backward_train",
                            "ms_per_step": round(res["train_dq_kernel"]["ms_step"], 4),
                            "TFLOP/s": round(res["train_dq_kernel"]["value"], 3)},
        "workspace_bytes": work_bytes,
        "holder": {"step_path": "zt_holder_forward + zt_holder_backward (device.Attn's forward(1, 64) + backward(64); "
                                "saved log-sum-exp and scores in the holder's own workspace)",
                   "ms_per_step": round(t_holder, 4),
                   "TFLOP/s": round((fwd_flop + bwd_flop) / (t_holder * 1e-3) / 1e12, 3),
                   "workspace_bytes": holder_ws},
        "reference_abi": {"step_path": "zt_attn_forward + zt_attn_backward",
                          "ms_per_step": round(res["reference_abi"]["ms_step"], 4),
                          "TFLOP/s": round(res["reference_abi"]["value"], 3),
                          "kernels": [{k2: (round(v2, 4) if isinstance(v2, float) else v2) for k2, v2 in kk.items()}
                                      for kk in res["reference_abi"]["kernels"]]},
        "kernels": [{k2: (round(v2, 4) if isinstance(v2, float) else v2) for k2, v2 in kk.items()} for kk in kernels],
        "other_configs": other or None,
        "decode": {"workload": "C4 B=64 n_keys=8192 Hq=32 Hkv=8 d=128 f32", "us": round(t_dec * 1e3, 2),
                   "GB/s": round(dec_gbs, 1), "bytes": dec_bytes, "frac_hbm": round(dec_gbs / PEAK_HBM, 4),
                   "step_us": round(t_step * 1e3, 2), "step_GB/s": round(step_gbs, 1),
                   "reference_seam": {"path": "zt_attn_forward(T=1, q_offset=n_keys-1, n_keys) once per sequence, "
                                              "as src/decode.zig:462 issues it",
                                      "us": round(t_seam * 1e3, 2), "GB/s": round(seam_gbs, 1)},
                   "holder_seam": {"path": "zt_holder_forward_at(1, 64, n_keys-1, n_keys, 1) on one sequence's "
                                           "device-resident cache (device.Attn.forwardAt, keys split over the "
                                           "device), 8 holders cycled",
                                   "us_per_call": round(t_hcall, 2), "us_per_64_sequences": round(Bd * t_hcall, 1),
                                   "GB/s": round(call_bytes / (t_hcall * 1e-6) / 1e9, 1),
                                   "e2e_us_per_call": round(t_he2e, 1),
                                   "e2e_path": "src/decode.zig:405-473 as issued: upload the query row and 8192 "
                                               "cache rows of K and V, forwardAt, download the output row"}},
        "rmsnorm": norm,
        "rmsnorm_reference_shapes": norm_sync_e2e,
        "reference_shapes": ref_shapes,
        "seams_e2e": seams,
        "matmul": mm,
        "calibration": {"mfma_f32_tflops": round(cal_tflops, 1), "read_GB/s": round(cal_gbs, 1),
                        "dominant_frac_of_sustained": round(dom["tflops"] / cal_tflops, 4),
                        "decode_frac_of_streaming_read": round(dec_gbs / cal_gbs, 4)},
        "rope_qk": {"workload": "C3 q and k, position 0", "us": round(t_rope * 1e3, 2), "bytes": rope_bytes,
                    "GB/s": round(rope_bytes / (t_rope * 1e-3) / 1e9, 1)},
        "hbm_copy": {"bytes": 2 * (1 << 30), "GB/s": round(copy_gbs, 1), "frac_hbm": round(copy_gbs / PEAK_HBM, 4)},
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
