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


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=10)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--cpu-rows", type=int, default=48, help="query rows of the CPU baseline sample")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-other", action="store_true", help="skip the C2 / C5 figures (profiling runs)")
    args = ap.parse_args()
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print("bench.py measures one GPU: this build's path runs on one MI355X (per-head/batch sharding "
              "across GPUs is described in DESIGN.md and not built). Run with --gpus 1.", file=sys.stderr)
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
            # Repeated on its own, the dk/dv stage reads the dS its previous
            # launch left in place of the scores; its work does not depend on the values.
            dkdv=lambda: zt.backward_train_ws(q, k, v, out, do, lse, dq, dk, dv, work, T, H, Hkv, D,
                                              stage=1 | zt.ZT_WS_SCORES),
            dq=lambda: zt.backward_train_ws(q, k, v, out, do, lse, dq, dk, dv, work, T, H, Hkv, D, stage=2),
            bwd=lambda: zt.backward_train_ws(q, k, v, out, do, lse, dq, dk, dv, work, T, H, Hkv, D, stage=scores),
            names=zt.plan_train(B, T, H, Hkv, D), dkdv_units=3),
        "train_recompute_scores": dict(
            fwd=lambda: zt.forward_train(q, k, v, out, lse, T, H, Hkv, D),
            dkdv=lambda: zt.backward_train_ws(q, k, v, out, do, lse, dq, dk, dv, work, T, H, Hkv, D, stage=1),
            dq=lambda: zt.backward_train_ws(q, k, v, out, do, lse, dq, dk, dv, work, T, H, Hkv, D, stage=2),
            bwd=lambda: zt.backward_train_ws(q, k, v, out, do, lse, dq, dk, dv, work, T, H, Hkv, D),
            names=(zt.plan(B, T, H, Hkv, D)[0], zt.plan_train(B, T, H, Hkv, D)[1], zt.plan(B, T, H, Hkv, D)[2]),
            dkdv_units=4),
        "train_dq_kernel": dict(
            fwd=lambda: zt.forward_train(q, k, v, out, lse, T, H, Hkv, D),
            dq=lambda: zt.bwd_dq_train(q, k, v, out, do, lse, dq, delta, T, H, Hkv, D),
            dkdv=lambda: zt.bwd_dkdv_train(q, k, v, out, do, lse, delta, dk, dv, T, H, Hkv, D),
            bwd=lambda: zt.backward_train(q, k, v, out, do, lse, dq, dk, dv, delta, T, H, Hkv, D),
            names=(zt.plan(B, T, H, Hkv, D)[0], "zt_bwd_dql_d%d_k32" % D, zt.plan(B, T, H, Hkv, D)[2]),
            dkdv_units=4),
        "reference_abi": dict(
            fwd=lambda: zt.forward(q, k, v, out, T, H, Hkv, D),
            dq=lambda: zt.bwd_dq(q, k, v, do, dq, rm, rl, rd, T, H, Hkv, D),
            dkdv=lambda: zt.bwd_dkdv(q, k, v, do, dk, dv, rm, rl, rd, T, H, Hkv, D),
            bwd=lambda: zt.backward(q, k, v, do, dq, dk, dv, rm, rl, rd, T, H, Hkv, D),
            names=zt.plan(B, T, H, Hkv, D), dkdv_units=4),
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
        pth["dkdv"]()  # the dq stage reads what the dk/dv stage wrote (row statistics or dS)
        t_dkdv = event_time(torch, pth["dkdv"], n_k)
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
        log(f"  forward {fwd_tflops:.2f} TFLOP/s ({100 * fwd_tflops / PEAK_MFMA_F32:.1f}%), backward "
            f"{bwd_tflops:.2f} TFLOP/s ({100 * bwd_tflops / PEAK_MFMA_F32:.1f}%)")
        res[pname] = dict(ms_step=ms_step, value=val, kernels=kernels, fwd_tflops=fwd_tflops,
                          bwd_tflops=bwd_tflops)
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

    # ---------------- C2, C5: the other training configurations ----------------
    # Secondary figures (C3 is the headline): the same training step -- the
    # forward keeping its scores where the shape allows, then the backward --
    # and the reference's own entry points, on the configurations' inputs
    # (C5: N(0, 2), sigma = sqrt(2)).
    other = {}
    other_cfgs = {} if args.no_other else {"C2": (4, 1024, 8, 8, 64, 1.0), "C5": (2, 2048, 16, 4, 256, 2.0 ** 0.5)}
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
        entry["train"]["kernels"] = list(zt.plan_train(Bo, To, Ho, Hkvo, Do))
        other[cname] = entry
        del qo, ko, vo, do_, oo, dqo, dko, dvo, lseo, rmo, rlo, rdo, wo

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
                                      "us": round(t_seam * 1e3, 2), "GB/s": round(seam_gbs, 1)}},
        "rmsnorm": norm,
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
