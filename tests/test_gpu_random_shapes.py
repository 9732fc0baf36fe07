"""A seeded sweep over random shapes: batch, sequence length, head group,
kv heads and head width drawn at random (a fixed seed, so the cases are the
same on every run and print their shape), each graded against the CPU
restatement on every path a caller reaches -- the reference entry points
(zt_attn_forward + zt_attn_backward), the training pair with its stored
scores (zt_attn_forward_train_ws + zt_attn_backward_train_ws with
ZT_WS_SCORES), and the decode step over the same keys as a cache with
ragged n_keys -- with the north_star gates (forward and decode max |diff| <=
1e-4; dq, dk, dv max |diff| / max |twin| <= 1e-3)."""
import numpy as np
import pytest

from gpuhelp import BWD_REL, FWD_TOL, SEED_DO, SEED_K, SEED_Q, SEED_V, dev_normal, host, max_abs, rel_err

pytestmark = pytest.mark.gpu

N_CASES = 24


def _cases():
    rng = np.random.default_rng(20261202)
    out = []
    while len(out) < N_CASES:
        B = int(rng.integers(1, 4))
        T = int(rng.choice([int(rng.integers(1, 64)), int(rng.integers(64, 420))]))
        group = int(rng.choice([1, 1, 2, 3, 4, 5, 8]))
        Hkv = int(rng.integers(1, 5))
        # mostly whole 32-column groups, some other even widths
        D = int(rng.choice([32, 64, 96, 128, 160, 192, 256])) if rng.random() < 0.7 else 2 * int(rng.integers(16, 129))
        if B * T * T * group * Hkv * D > 3.0e8:   # keep the twin's backward to a second or two
            continue
        out.append((B, T, group * Hkv, Hkv, D))
    return out


CASES = _cases()


def _nan(torch, n):
    return torch.full((n,), float("nan"), device="cuda", dtype=torch.float32)


@pytest.mark.parametrize("B,T,H,Hkv,D", CASES, ids=[f"B{b}-T{t}-H{h}-Hkv{k}-D{d}" for b, t, h, k, d in CASES])
def test_random_shape_on_every_path(gpu, zt, oracle, threads, B, T, H, Hkv, D):
    print(f"[random shape] B={B} T={T} H={H} Hkv={Hkv} D={D}", flush=True)
    q = dev_normal(gpu, zt, B * T * H * D, SEED_Q + T)
    k = dev_normal(gpu, zt, B * T * Hkv * D, SEED_K + T)
    v = dev_normal(gpu, zt, B * T * Hkv * D, SEED_V + T)
    do = dev_normal(gpu, zt, B * T * H * D, SEED_DO + T)
    qh, kh, vh, dh = (host(x) for x in (q, k, v, do))
    ref_out = oracle.attention_forward(qh, kh, vh, B, T, H, Hkv, D, threads=threads)
    rq, rk, rv = oracle.attention_backward(qh, kh, vh, dh, B, T, H, Hkv, D, threads=threads)

    # The reference entry points.
    out = _nan(gpu, q.numel())
    zt.forward(q, k, v, out, T, H, Hkv, D, B=B)
    dq, dk, dv = _nan(gpu, q.numel()), _nan(gpu, k.numel()), _nan(gpu, k.numel())
    rm, rl, rd = (_nan(gpu, B * T * H) for _ in range(3))
    zt.backward(q, k, v, do, dq, dk, dv, rm, rl, rd, T, H, Hkv, D, B=B)
    gpu.cuda.synchronize()
    assert max_abs(host(out), ref_out) <= FWD_TOL
    assert rel_err(host(dq), rq) <= BWD_REL
    assert rel_err(host(dk), rk) <= BWD_REL
    assert rel_err(host(dv), rv) <= BWD_REL

    # The training pair with the stored scores.
    out2, lse = _nan(gpu, q.numel()), _nan(gpu, B * T * H)
    work = _nan(gpu, zt.backward_train_workspace_bytes(B, T, H, Hkv, D) // 4)
    zt.forward_train_ws(q, k, v, out2, lse, work, T, H, Hkv, D, B=B)
    dq2, dk2, dv2 = _nan(gpu, q.numel()), _nan(gpu, k.numel()), _nan(gpu, k.numel())
    zt.backward_train_ws(q, k, v, out2, do, lse, dq2, dk2, dv2, work, T, H, Hkv, D, B=B, stage=3 | zt.ZT_WS_SCORES)
    gpu.cuda.synchronize()
    assert max_abs(host(out2), ref_out) <= FWD_TOL
    assert rel_err(host(dq2), rq) <= BWD_REL
    assert rel_err(host(dk2), rk) <= BWD_REL
    assert rel_err(host(dv2), rv) <= BWD_REL

    # Decode: the same keys as a cache of n_ctx = T rows per sequence, the
    # query of each sequence its own row n_keys - 1 of q.
    rng = np.random.default_rng(T * 131 + D)
    n_keys = [int(x) for x in rng.integers(1, T + 1, size=B)]
    n_keys[0] = T
    qrow = np.stack([qh.reshape(B, T, H * D)[b, n_keys[b] - 1] for b in range(B)]).astype(np.float32)
    qd = gpu.from_numpy(np.ascontiguousarray(qrow).ravel()).cuda()
    od = _nan(gpu, B * H * D)
    ws = gpu.empty(zt.decode_workspace_bytes(B, T, H, Hkv, D) // 4 + 1, device="cuda", dtype=gpu.float32)
    zt.decode(qd, k, v, od, n_keys, B, T, H, Hkv, D, ws)
    gpu.cuda.synchronize()
    ref_dec = oracle.attn_step(qrow.ravel(), kh, vh, n_keys, B, T, H, Hkv, D)
    assert max_abs(host(od), ref_dec) <= FWD_TOL
