"""RMSNorm (src/norm.zig:18-47), RoPE (src/rope.zig:21-55) and its backward
(src/autograd.zig:851-872) on the GPU against the CPU restatement.  RMSNorm gate: the reference kernel's 1e-5
absolute (src/cuda/norm.cu:56); the f64 sum of squares differs from the
reference's sequential sum only in association, so nearly every element is
bit-identical."""
import numpy as np
import pytest

from gpuhelp import SEED_W, SEED_X, THETA, dev_normal, dev_uniform, host, max_abs

pytestmark = pytest.mark.gpu


def _norm(gpu, zt, x, w, rows, cols, eps=1e-5):
    y = gpu.full((rows * cols,), float("nan"), device="cuda", dtype=gpu.float32)
    zt.rmsnorm(x, w, y, rows, cols, eps)
    gpu.cuda.synchronize()
    return host(y)


@pytest.mark.parametrize("rows,cols", [(64, 4096), (4096, 4096), (1, 1), (3, 3), (5, 4), (7, 100), (9, 1023),
                                       (2, 4097), (4, 16384), (3, 20000), (256, 128), (1000, 2)])
def test_rmsnorm_matches_twin(gpu, zt, oracle, rows, cols):
    x = dev_normal(gpu, zt, rows * cols, SEED_X)
    w = dev_uniform(gpu, zt, cols, SEED_W, 0.5, 1.5)
    y = _norm(gpu, zt, x, w, rows, cols)
    ref = oracle.rmsnorm(host(x), host(w), rows, cols)
    assert max_abs(y, ref) <= 1e-5
    assert np.mean(y.view(np.uint32) == ref.view(np.uint32)) >= 0.999


def test_rmsnorm_reference_known_answers(gpu, zt, golden):
    for c in golden["rmsnorm"]:
        x = gpu.tensor(np.float32(c["x"]), device="cuda")
        w = gpu.tensor(np.float32(c["w"]), device="cuda")
        y = _norm(gpu, zt, x, w, c["rows"], c["cols"])
        tol = 0.0 if c["tol"] is None else c["tol"]
        assert max_abs(y, c["y"]) <= tol, c["src"]
    c = golden["rmsnorm_f64_row"]
    x = gpu.full((c["cols"],), np.float32(c["x"]).item(), device="cuda", dtype=gpu.float32)
    y = _norm(gpu, zt, x, gpu.ones(c["cols"], device="cuda"), 1, c["cols"])
    assert abs(float(y[0]) - c["exact"]) <= c["tol"]


def test_rmsnorm_zero_rows_and_zero_values(gpu, zt):
    w = gpu.ones(8, device="cuda")
    y = gpu.empty(0, device="cuda")
    zt.rmsnorm(gpu.empty(0, device="cuda"), w, y, 0, 8)
    x = gpu.zeros(16, device="cuda")
    out = _norm(gpu, zt, x, w, 2, 8)
    assert np.all(out == 0)


def test_rmsnorm_gate_catches_broken_references(gpu, zt, oracle):
    # src/cuda/norm.cu:58-86 variants: weight + 1e-3, mean instead of mean of squares.
    rows, cols = 16, 512
    x = dev_normal(gpu, zt, rows * cols, SEED_X)
    w = dev_uniform(gpu, zt, cols, SEED_W, 0.5, 1.5)
    y = _norm(gpu, zt, x, w, rows, cols)
    xh, wh = host(x), host(w)
    assert max_abs(y, oracle.rmsnorm(xh, wh + np.float32(1e-3), rows, cols)) > 1e-5
    xr = xh.reshape(rows, cols).astype(np.float64)
    mean_not_sq = (xr / np.float32(np.sqrt(np.abs(xr.mean(1, keepdims=True)) + 1e-5)) * wh).ravel()
    assert max_abs(y, mean_not_sq) > 1e-5


@pytest.mark.parametrize("rows,heads,hd,pos", [(4096, 32, 128, 0), (17, 3, 6, 5), (8, 2, 256, 1000), (1, 1, 2, 1)])
def test_rope_matches_twin(gpu, zt, oracle, rows, heads, hd, pos):
    cols = heads * hd
    x = dev_normal(gpu, zt, rows * cols, SEED_X)
    y = gpu.empty_like(x)
    zt.rope(x, y, rows, cols, pos, THETA, hd)
    gpu.cuda.synchronize()
    ref = oracle.rope(host(x), rows, cols, pos, THETA, hd)
    assert max_abs(host(y), ref) <= 2e-6


@pytest.mark.parametrize("rows,heads,hd,pos", [(1, 32, 128, 8191), (64, 8, 64, 0), (33, 3, 34, 17), (7, 2, 256, 1000)])
def test_rope_backward_matches_twin(gpu, zt, oracle, rows, heads, hd, pos):
    # src/autograd.zig:851-872 on the device.
    cols = heads * hd
    x = dev_normal(gpu, zt, rows * cols, SEED_X)
    y = gpu.full((rows * cols,), float("nan"), device="cuda")
    zt.rope_backward(x, y, rows, cols, pos, THETA, hd)
    gpu.cuda.synchronize()
    ref = oracle.rope_backward(host(x), rows, cols, pos, THETA, hd)
    assert max_abs(host(y), ref) <= 2e-6
    if pos + rows > 1:  # the forward rotation is not the answer
        assert max_abs(host(y), oracle.rope(host(x), rows, cols, pos, THETA, hd)) > 1e-3


@pytest.mark.parametrize("B,T,H,Hkv,hd,pos", [(1, 4096, 32, 8, 128, 0), (3, 50, 6, 2, 34, 7), (2, 9, 4, 4, 256, 100)])
@pytest.mark.parametrize("backward", [False, True])
def test_rope_qk_matches_twin(gpu, zt, oracle, B, T, H, Hkv, hd, pos, backward):
    # q and k in one launch; every sequence restarts at pos (src/model.zig:372-377).
    q = dev_normal(gpu, zt, B * T * H * hd, SEED_X)
    k = dev_normal(gpu, zt, B * T * Hkv * hd, SEED_W)
    qh, kh = host(q).reshape(B, T * H * hd), host(k).reshape(B, T * Hkv * hd)
    qo, ko = gpu.full_like(q, float("nan")), gpu.full_like(k, float("nan"))
    zt.rope_qk(q, k, qo, ko, B, T, H, Hkv, hd, pos, THETA, backward=backward)
    zt.rope_qk(q, k, q, k, B, T, H, Hkv, hd, pos, THETA, backward=backward)  # in place
    gpu.cuda.synchronize()
    fn = oracle.rope_backward if backward else oracle.rope
    want_q = np.concatenate([fn(qh[b], T, H * hd, pos, THETA, hd) for b in range(B)])
    want_k = np.concatenate([fn(kh[b], T, Hkv * hd, pos, THETA, hd) for b in range(B)])
    for got_q, got_k in ((qo, ko), (q, k)):
        assert max_abs(host(got_q), want_q) <= 2e-6
        assert max_abs(host(got_k), want_k) <= 2e-6
    assert np.mean(host(qo) == want_q) >= 0.999  # separate f64 roundings, as the reference


def test_rope_reference_known_answers(gpu, zt, golden):
    for c in golden["rope"]:
        x = gpu.tensor(np.float32(c["x"]), device="cuda")
        y = gpu.empty_like(x)
        zt.rope(x, y, c["rows"], c["cols"], c["pos"], THETA, c["head_dim"])
        gpu.cuda.synchronize()
        tol = 0.0 if c["tol"] is None else c["tol"]
        assert max_abs(host(y), c["y"]) <= tol, c["src"]


def test_device_fill_matches_host_generator(gpu, zt, oracle):
    t = dev_normal(gpu, zt, 100_000, SEED_X)
    ref = oracle.fill_normal(100_000, SEED_X)
    assert max_abs(host(t), ref) <= 1e-6
    u = dev_uniform(gpu, zt, 10_000, SEED_W, 0.5, 1.5)
    assert max_abs(host(u), oracle.fill_uniform(10_000, SEED_W, 0.5, 1.5)) <= 1e-7


def test_calibration_probes_report_plausible_rates(gpu, zt):
    # Sustained FP32 MFMA below the 157.3 TFLOP/s datasheet peak but near it;
    # a streaming read below the 8 TB/s HBM peak.
    src = gpu.empty(1 << 28, device="cuda")
    scratch = gpu.empty(2048 * 256, device="cuda")
    tf, gbs = zt.calibrate(src, scratch)
    assert 100.0 < tf < 160.0, tf
    assert 2000.0 < gbs < 8200.0, gbs
    with pytest.raises(zt.ZtRefused):
        zt.calibrate(src, gpu.empty(16, device="cuda"))
