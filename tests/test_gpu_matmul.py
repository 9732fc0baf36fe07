"""The model's dense products on the GPU (zt_matmul = tensor.matmul,
src/tensor.zig:78-106; zt_weight_grad / zt_input_grad = autograd.zig's
weightGrad :958-972 and inputGrad :999-1022) against the reference's known
answers and its own accumulator gate (src/tensor_test.zig:185-273):
|got - f32(exact)| / sum|products| must stay below (K-1) * eps_f32 (an f32
reduction) and, for a long reduction, above (K-1) * eps_f64 (not a wider one)."""
import numpy as np
import pytest

from gpuhelp import host

pytestmark = pytest.mark.gpu

EPS32, EPS64 = np.finfo(np.float32).eps, np.finfo(np.float64).eps


def _dev(gpu, x):
    return gpu.from_numpy(np.ascontiguousarray(x, dtype=np.float32).ravel()).cuda()


def _divergence(got, exact, abs_sum, base=None):
    wide = exact.astype(np.float32).astype(np.float64)
    scale = abs_sum if base is None else abs_sum + np.abs(base)
    scale = np.where(scale == 0, 1.0, scale)
    return float(np.max(np.abs(got.astype(np.float64) - wide) / scale)) if got.size else 0.0


def test_matmul_reference_known_answers(gpu, zt, golden):
    for c in golden["matmul"]:
        M, K, N = c["M"], c["K"], c["N"]
        a = _dev(gpu, np.float32(c["a"]) if c["a"] else np.zeros(M * K))
        b = _dev(gpu, np.float32(c["b"]) if c["b"] else np.full(K * N, 2.0))
        out = gpu.full((M * N,), float("nan"), device="cuda")
        zt.matmul(a, b, out, M, K, N)
        gpu.cuda.synchronize()
        assert np.array_equal(host(out), np.float32(c["out"])), c["src"]


@pytest.mark.parametrize("M,K,N", [(256, 512, 128), (1000, 777, 333), (2048, 2048, 2048), (5, 3, 7), (130, 30, 6)])
def test_matmul_passes_the_reference_accumulator_gate(gpu, zt, oracle, M, K, N):
    rng = np.random.default_rng(M + K + N)
    a = rng.uniform(-0.02, 0.02, (M, K)).astype(np.float32)
    b = rng.uniform(-0.02, 0.02, (K, N)).astype(np.float32)
    out = gpu.full((M * N,), float("nan"), device="cuda")
    zt.matmul(_dev(gpu, a), _dev(gpu, b), out, M, K, N)
    gpu.cuda.synchronize()
    a64, b64 = a.astype(np.float64), b.astype(np.float64)
    exact, abs_sum = a64 @ b64, np.abs(a64) @ np.abs(b64)
    worst = _divergence(host(out).reshape(M, N), exact, abs_sum)
    assert worst < (K - 1) * EPS32
    if K >= 64:
        assert worst > (K - 1) * EPS64
    if M * K * N <= 256 * 512 * 128:  # no less accurate than the reference's own f32 sum, within 4x
        ref = _divergence(oracle.matmul(a, b, M, K, N).reshape(M, N), exact, abs_sum)
        assert worst <= 4 * ref + EPS32


@pytest.mark.parametrize("T,I,J", [(256, 128, 512), (256, 512, 128), (300, 456, 128), (7, 5, 9), (64, 130, 66)])
def test_weight_grad_accumulates_input_t_dout(gpu, zt, oracle, T, I, J):
    rng = np.random.default_rng(T * 7 + I)
    inp = rng.uniform(-1, 1, (T, I)).astype(np.float32)
    dout = rng.uniform(-1, 1, (T, J)).astype(np.float32)
    w0 = rng.uniform(-1, 1, (I, J)).astype(np.float32)
    w = _dev(gpu, w0)
    zt.weight_grad(w, _dev(gpu, inp), _dev(gpu, dout), T, I, J)
    gpu.cuda.synchronize()
    i64, d64 = inp.astype(np.float64), dout.astype(np.float64)
    exact = w0.astype(np.float64) + i64.T @ d64
    abs_sum = np.abs(i64).T @ np.abs(d64)
    assert _divergence(host(w).reshape(I, J), exact, abs_sum, w0) < T * EPS32
    ref = oracle.weight_grad(w0, inp, dout, T, I, J).reshape(I, J)
    assert np.max(np.abs(host(w).reshape(I, J) - ref)) <= 2 * T * EPS32 * max(1.0, float(np.max(abs_sum)))


@pytest.mark.parametrize("T,J,I", [(256, 512, 128), (256, 128, 512), (300, 128, 456), (7, 9, 5), (64, 66, 130)])
def test_input_grad_accumulates_dout_w_t(gpu, zt, oracle, T, J, I):
    rng = np.random.default_rng(T * 11 + J)
    dout = rng.uniform(-1, 1, (T, J)).astype(np.float32)
    w = rng.uniform(-1, 1, (I, J)).astype(np.float32)
    d0 = rng.uniform(-1, 1, (T, I)).astype(np.float32)
    din = _dev(gpu, d0)
    zt.input_grad(din, _dev(gpu, dout), _dev(gpu, w), T, J, I)
    gpu.cuda.synchronize()
    d64, w64 = dout.astype(np.float64), w.astype(np.float64)
    exact = d0.astype(np.float64) + d64 @ w64.T
    abs_sum = np.abs(d64) @ np.abs(w64).T
    assert _divergence(host(din).reshape(T, I), exact, abs_sum, d0) < J * EPS32
    ref = oracle.input_grad(d0, dout, w, T, J, I).reshape(T, I)
    assert np.max(np.abs(host(din).reshape(T, I) - ref)) <= 2 * J * EPS32 * max(1.0, float(np.max(abs_sum)))


def test_products_gate_catches_a_transposed_operand(gpu, zt):
    # Negative control: the gate fails for the product with an operand transposed.
    rng = np.random.default_rng(3)
    M = K = N = 64
    a = rng.uniform(-1, 1, (M, K)).astype(np.float32)
    b = rng.uniform(-1, 1, (K, N)).astype(np.float32)
    out = gpu.empty(M * N, device="cuda")
    zt.matmul(_dev(gpu, a), _dev(gpu, b), out, M, K, N)
    gpu.cuda.synchronize()
    a64, b64 = a.astype(np.float64), b.astype(np.float64)
    wrong = a64 @ b64.T
    assert _divergence(host(out).reshape(M, N), wrong, np.abs(a64) @ np.abs(b64)) > (K - 1) * EPS32


def test_matmul_refusals(gpu, zt):
    a, b, out = (gpu.zeros(6, device="cuda") for _ in range(3))
    with pytest.raises(zt.DimensionMismatch):
        zt.matmul(a, b, out, 2, 3, 3)
    assert zt.lib().zt_matmul(None, None, None, -1, 2, 2, None) == 1


@pytest.mark.parametrize("tile", ["128", "64", "32"])
@pytest.mark.parametrize("M,K,N", [(200, 70, 150), (33, 129, 65), (128, 64, 256), (256, 96, 384), (384, 160, 128)])
def test_every_tile_size_passes_the_gate(gpu, zt, tune, tile, M, K, N):
    """Each workgroup tile (forced through ZT_GEMM_TILE), for all three
    products, on ragged shapes and on whole tiles (M, N multiples of every
    tile, K of the 32-deep slab: the unconditional-load path)."""
    tune({"ZT_GEMM_TILE": tile})
    rng = np.random.default_rng(M * K + N)
    a = rng.uniform(-1, 1, (M, K)).astype(np.float32)
    b = rng.uniform(-1, 1, (K, N)).astype(np.float32)
    a64, b64 = a.astype(np.float64), b.astype(np.float64)
    out = gpu.full((M * N,), float("nan"), device="cuda")
    zt.matmul(_dev(gpu, a), _dev(gpu, b), out, M, K, N)
    c0 = rng.uniform(-1, 1, (M, N)).astype(np.float32)
    wg = _dev(gpu, c0)   # w[M,N] += (a^T as stored K x M)^T b: weightGrad with T = K, I = M, J = N
    zt.weight_grad(wg, _dev(gpu, np.ascontiguousarray(a.T)), _dev(gpu, b), K, M, N)
    ig = _dev(gpu, c0)   # din[M,N] += a (b^T as stored N x K)^T: inputGrad with T = M, J = K, I = N
    zt.input_grad(ig, _dev(gpu, a), _dev(gpu, np.ascontiguousarray(b.T)), M, K, N)
    gpu.cuda.synchronize()
    exact, abs_sum = a64 @ b64, np.abs(a64) @ np.abs(b64)
    assert _divergence(host(out).reshape(M, N), exact, abs_sum) < (K - 1) * EPS32
    for g in (wg, ig):
        assert _divergence(host(g).reshape(M, N), c0.astype(np.float64) + exact, abs_sum, c0) < K * EPS32


@pytest.mark.parametrize("split,tile", [("4", "16"), ("8", "32"), ("16", "16"), ("16", "32")])
@pytest.mark.parametrize("M,K,N", [(200, 70, 150), (33, 129, 65), (256, 512, 128), (5, 3, 7), (64, 1000, 48)])
def test_every_split_k_variant_passes_the_gate(gpu, zt, tune, split, tile, M, K, N):
    """The split-K kernels (forced through ZT_GEMM_SK / ZT_GEMM_SK_TILE), for
    all three products, on ragged shapes: K not a multiple of 16, fewer
    16-deep blocks than waves, and more than two blocks per wave."""
    tune({"ZT_GEMM_SK": split, "ZT_GEMM_SK_TILE": tile})
    rng = np.random.default_rng(M * K + N + int(split))
    a = rng.uniform(-1, 1, (M, K)).astype(np.float32)
    b = rng.uniform(-1, 1, (K, N)).astype(np.float32)
    a64, b64 = a.astype(np.float64), b.astype(np.float64)
    out = gpu.full((M * N,), float("nan"), device="cuda")
    zt.matmul(_dev(gpu, a), _dev(gpu, b), out, M, K, N)
    c0 = rng.uniform(-1, 1, (M, N)).astype(np.float32)
    wg = _dev(gpu, c0)
    zt.weight_grad(wg, _dev(gpu, np.ascontiguousarray(a.T)), _dev(gpu, b), K, M, N)
    ig = _dev(gpu, c0)
    zt.input_grad(ig, _dev(gpu, a), _dev(gpu, np.ascontiguousarray(b.T)), M, K, N)
    gpu.cuda.synchronize()
    exact, abs_sum = a64 @ b64, np.abs(a64) @ np.abs(b64)
    assert _divergence(host(out).reshape(M, N), exact, abs_sum) < max(K - 1, 1) * EPS32
    for g in (wg, ig):
        assert _divergence(host(g).reshape(M, N), c0.astype(np.float64) + exact, abs_sum, c0) < K * EPS32


def test_split_k_is_deterministic_and_chosen_for_the_model_shapes(gpu, zt):
    """The model's products take the split-K kernel by the shape rule, and two
    runs agree bit for bit (the partial tiles are summed in wave order)."""
    for M, K, N in ((256, 512, 128), (256, 128, 512), (256, 128, 456)):
        rng = np.random.default_rng(M + K + N)
        a = _dev(gpu, rng.uniform(-1, 1, (M, K)))
        b = _dev(gpu, rng.uniform(-1, 1, (K, N)))
        outs = []
        for _ in range(2):
            out = gpu.full((M * N,), float("nan"), device="cuda")
            zt.matmul(a, b, out, M, K, N)
            gpu.cuda.synchronize()
            outs.append(host(out).view(np.uint32))
        assert np.array_equal(outs[0], outs[1])
    assert zt.gemm_kernel(256, 512, 128) == "zt_gemm_nn_sk16"
    assert zt.gemm_kernel(4096, 4096, 4096) == "zt_gemm_nn_128"
