"""The library driven from several host threads at once, each on its own HIP
stream with its own buffers and workspace: the training pair with stored
scores, the reference entry points and the decode step, repeated, must give
bit for bit what the same calls give one after the other on one stream.  The
launcher's shared state -- the per-device kernel handle cache, filled on
first use under a lock, and the record of which workspace holds whose scores
-- is what this exercises (ctypes releases the GIL for the library calls, so
the host code really runs concurrently)."""
import threading

import numpy as np
import pytest

from gpuhelp import SEED_DO, SEED_K, SEED_Q, SEED_V, dev_normal, host

pytestmark = pytest.mark.gpu

SHAPES = [(1, 300, 8, 2, 128), (2, 130, 4, 4, 64), (1, 200, 6, 2, 96), (1, 77, 8, 1, 256), (3, 64, 4, 2, 32),
          (1, 513, 16, 4, 64)]
REPEATS = 4


def _inputs(gpu, zt, B, T, H, Hkv, D, salt):
    return (dev_normal(gpu, zt, B * T * H * D, SEED_Q + salt), dev_normal(gpu, zt, B * T * Hkv * D, SEED_K + salt),
            dev_normal(gpu, zt, B * T * Hkv * D, SEED_V + salt), dev_normal(gpu, zt, B * T * H * D, SEED_DO + salt))


def _run(gpu, zt, shape, ins, stream):
    """The three paths on `stream`; returns the outputs as host arrays."""
    B, T, H, Hkv, D = shape
    q, k, v, do = ins
    with gpu.cuda.stream(stream):
        out, lse = gpu.empty_like(q), gpu.empty(B * T * H, device="cuda")
        work = gpu.empty(zt.backward_train_workspace_bytes(B, T, H, Hkv, D) // 4, device="cuda")
        dq, dk, dv = gpu.empty_like(q), gpu.empty_like(k), gpu.empty_like(v)
        zt.forward_train_ws(q, k, v, out, lse, work, T, H, Hkv, D, B=B, stream=stream)
        zt.backward_train_ws(q, k, v, out, do, lse, dq, dk, dv, work, T, H, Hkv, D, B=B, stage=3 | zt.ZT_WS_SCORES,
                             stream=stream)
        out2 = gpu.empty_like(q)
        zt.forward(q, k, v, out2, T, H, Hkv, D, B=B, stream=stream)
        dq2, dk2, dv2 = gpu.empty_like(q), gpu.empty_like(k), gpu.empty_like(v)
        rm, rl, rd = (gpu.empty(B * T * H, device="cuda") for _ in range(3))
        zt.backward(q, k, v, do, dq2, dk2, dv2, rm, rl, rd, T, H, Hkv, D, B=B, stream=stream)
        n_keys = [T] + [max(1, T // (b + 2)) for b in range(1, B)]
        qd = q.view(B, T, H * D)[:, -1].contiguous()
        od = gpu.empty(B * H * D, device="cuda")
        ws = gpu.empty(zt.decode_workspace_bytes(B, T, H, Hkv, D) // 4 + 1, device="cuda")
        zt.decode(qd, k, v, od, n_keys, B, T, H, Hkv, D, ws, stream=stream)
        stream.synchronize()
    return [host(x) for x in (out, lse, dq, dk, dv, out2, dq2, dk2, dv2, od)]


def test_threads_on_their_own_streams_match_one_stream(gpu, zt):
    inputs = [_inputs(gpu, zt, *s, salt=i) for i, s in enumerate(SHAPES)]
    gpu.cuda.synchronize()
    want = [_run(gpu, zt, s, ins, gpu.cuda.current_stream()) for s, ins in zip(SHAPES, inputs)]
    got = [[None] * REPEATS for _ in SHAPES]
    errors = []
    start = threading.Barrier(len(SHAPES))

    def worker(i):
        try:
            stream = gpu.cuda.Stream()   # default priority
            start.wait()
            for r in range(REPEATS):
                got[i][r] = _run(gpu, zt, SHAPES[i], inputs[i], stream)
        except Exception as e:  # reported below, with the shape
            errors.append((SHAPES[i], repr(e)))

    threads = [threading.Thread(target=worker, args=(i,)) for i in range(len(SHAPES))]
    for t in threads:
        t.start()
    for t in threads:
        t.join(timeout=120)
    assert not any(t.is_alive() for t in threads)
    assert not errors, errors
    for i, s in enumerate(SHAPES):
        for r in range(REPEATS):
            for a, b in zip(got[i][r], want[i]):
                assert np.array_equal(a.view(np.uint32), b.view(np.uint32)), (s, r)
