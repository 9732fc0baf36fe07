"""Online-softmax bookkeeping under scores that climb along the keys.

The forward and the statistics-building dq kernel move a row's exponent base
only when the row meets a tile maximum more than 2^8 above it (lazy
rescaling).  Synthetic inputs rarely do that after the first tile; here q and
k share a direction and k grows with the key index, so every row's maximum
climbs by several log2 units per 32-key tile and the base moves again and
again (and, for the heads whose ramp runs the other way, never after the
first tile).  Both must still match the CPU restatement: O, lse, dq, dk, dv,
and the reference's row statistics, whose row_max is the true maximum
(src/cuda/attn_kernels.cu:508-517 scratch contract)."""
import numpy as np
import pytest

from gpuhelp import BWD_REL, FWD_TOL, host, max_abs, rel_err

B, T, H, Hkv, D = 1, 384, 4, 2, 64


def _ramp_inputs(rng):
    """Heads of kv group 0 see scores rising with the key (about +6 log2 units
    per 32 keys), kv group 1 falling."""
    q = rng.normal(0.0, 0.1, (B, T, H, D)) + 1.0
    k = rng.normal(0.0, 0.1, (B, T, Hkv, D))
    ramp = np.arange(T, dtype=np.float64)[None, :, None] * (8.0 * 4.2 / 32.0) / D
    k[:, :, 0, :] += ramp
    k[:, :, 1, :] -= ramp
    v = rng.normal(0.0, 1.0, (B, T, Hkv, D))
    do = rng.normal(0.0, 1.0, (B, T, H, D))
    return [np.ascontiguousarray(x, dtype=np.float32).ravel() for x in (q, k, v, do)]


def _dev(gpu, x):
    return gpu.from_numpy(x).cuda()


def test_scores_span_many_rescales():
    q, k, *_ = _ramp_inputs(np.random.default_rng(7))
    qh = q.reshape(T, H, D)[:, 0].astype(np.float64)
    kh = k.reshape(T, Hkv, D)[:, 0].astype(np.float64)
    s = (qh @ kh.T) / np.sqrt(D) * np.log2(np.e)   # log2 units, row t sees keys <= t
    climb = s[T - 1, 32:T:32] - s[T - 1, 0:T - 32:32]
    assert np.all(climb > 4.0) and s[T - 1, T - 1] - s[T - 1, 0] > 8.0 * 8  # at least eight base moves


@pytest.mark.gpu
@pytest.mark.parametrize("path", ["reference_abi", "train", "train_scores"])
def test_forward_under_climbing_scores(gpu, zt, oracle, path):
    q, k, v, _ = _ramp_inputs(np.random.default_rng(7))
    dq_, dk_, dv_ = _dev(gpu, q), _dev(gpu, k), _dev(gpu, v)
    out = gpu.full((q.size,), float("nan"), device="cuda")
    lse = gpu.full((B * T * H,), float("nan"), device="cuda")
    if path == "reference_abi":
        zt.forward(dq_, dk_, dv_, out, T, H, Hkv, D)
    elif path == "train":
        zt.forward_train(dq_, dk_, dv_, out, lse, T, H, Hkv, D)
    else:
        ws = gpu.empty(zt.backward_train_workspace_bytes(B, T, H, Hkv, D) // 4, device="cuda")
        zt.forward_train_ws(dq_, dk_, dv_, out, lse, ws, T, H, Hkv, D)
    gpu.cuda.synchronize()
    ref = oracle.attention_forward(q, k, v, B, T, H, Hkv, D)
    assert max_abs(host(out), ref) <= FWD_TOL
    if path != "reference_abi":
        m, l, _ = oracle.attention_row_stats(q, k, v, np.zeros_like(q), B, T, H, Hkv, D)
        assert max_abs(host(lse), m + np.log(l)) <= 1e-4 * max(1.0, float(np.abs(m).max()))


@pytest.mark.gpu
def test_reference_backward_under_climbing_scores(gpu, zt, oracle):
    q, k, v, do = _ramp_inputs(np.random.default_rng(7))
    t = [_dev(gpu, x) for x in (q, k, v, do)]
    dq, dk, dv = (gpu.full((x.numel(),), float("nan"), device="cuda") for x in (t[0], t[1], t[1]))
    rm, rl, rd = (gpu.full((B * T * H,), float("nan"), device="cuda") for _ in range(3))
    zt.backward(*t, dq, dk, dv, rm, rl, rd, T, H, Hkv, D)
    gpu.cuda.synchronize()
    rq, rk, rv = oracle.attention_backward(q, k, v, do, B, T, H, Hkv, D)
    assert rel_err(host(dq), rq) <= BWD_REL
    assert rel_err(host(dk), rk) <= BWD_REL
    assert rel_err(host(dv), rv) <= BWD_REL
    m, l, d = oracle.attention_row_stats(q, k, v, do, B, T, H, Hkv, D)
    assert max_abs(host(rm), m) <= 1e-4 * max(1.0, np.abs(m).max())
    assert np.max(np.abs(host(rl) - l) / l) <= 1e-4
    assert max_abs(host(rd), d) <= 1e-4 * max(1.0, np.abs(d).max())
