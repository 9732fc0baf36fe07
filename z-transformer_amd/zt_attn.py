"""ctypes binding of libzt_attn.so (include/zt_attn.h, include/zt_holder.h).

Plumbing for tests and the benchmark: device memory and streams come from
torch tensors, every computation runs in the HIP library.  There is no
fallback: `lib()` raises when the library has not been built, and every
wrapper raises `ZtRefused` when the C side returns non-zero.
"""
import ctypes
import os

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "_build", "libzt_attn.so")

_lib = None

# The reference C ABI's six symbols, then the extensions (include/zt_attn.h),
# then the holder's C face (include/zt_holder.h).
ABI_SYMBOLS = [
    "zt_attn_dim_ok", "zt_attn_forward_shmem", "zt_attn_bwd_dq_shmem", "zt_attn_bwd_dkdv_shmem",
    "zt_attn_forward", "zt_attn_backward",
    "zt_attn_forward_batched", "zt_attn_backward_batched", "zt_attn_bwd_dq", "zt_attn_bwd_dkdv",
    "zt_attn_decode_workspace", "zt_attn_decode", "zt_attn_decode_step_workspace", "zt_attn_decode_step",
    "zt_rmsnorm_forward", "zt_rope_forward", "zt_rope_backward", "zt_rope_qk_forward",
    "zt_rope_qk_backward", "zt_fill_normal", "zt_fill_uniform", "zt_attn_version",
    "zt_attn_lds_limit", "zt_attn_plan", "zt_attn_forward_train", "zt_attn_backward_train",
    "zt_attn_bwd_dq_train", "zt_attn_bwd_dkdv_train", "zt_attn_plan_train", "zt_calibrate",
    "zt_matmul", "zt_weight_grad", "zt_input_grad", "zt_attn_backward_train_workspace",
    "zt_attn_backward_train_ws", "zt_attn_forward_train_ws", "zt_attn_set_tuning", "zt_attn_get_tuning",
    "zt_calibrate_launch", "zt_attn_decode_noalloc", "zt_matmul_plan",
]
HOLDER_SYMBOLS = [
    "zt_bytes_for", "zt_to_cint", "zt_forward_bounds", "zt_holder_init", "zt_holder_deinit",
    "zt_holder_total_bytes", "zt_holder_buffer", "zt_holder_forward", "zt_holder_forward_at",
    "zt_holder_backward", "zt_holder_upload", "zt_holder_download", "zt_holder_init_exact",
    "zt_holder_workspace_bytes", "zt_holder_forget", "zt_holder_buffer_ro",
]

# include/zt_holder.h enum zt_error
ZT_OK, ZT_DEGENERATE_SHAPE, ZT_SHAPE_TOO_LARGE, ZT_CONFIG_REFUSED, ZT_DEVICE_ALLOC_FAILED, \
    ZT_DEVICE_TRANSFER_FAILED = range(6)
ZT_QUERY_HEADED, ZT_KV_HEADED, ZT_PER_ROW = range(3)
(ZT_BUF_Q, ZT_BUF_K, ZT_BUF_V, ZT_BUF_OUT, ZT_BUF_DOUT, ZT_BUF_DQ, ZT_BUF_DK, ZT_BUF_DV, ZT_BUF_ROW_MAX,
 ZT_BUF_ROW_DEN, ZT_BUF_ROW_DEL) = range(11)


class ZtRefused(RuntimeError):
    """The C side refused a call (it printed the reason on stderr)."""


def lib():
    """The library built in-tree (z-transformer_amd/_build/libzt_attn.so), bound once."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise FileNotFoundError(
                f"{LIB_PATH} is not built; run `python z-transformer_amd/build.py` (or __graft_entry__.build())")
        _lib = load_library(LIB_PATH)
    return _lib


def load_library(path):
    """Another build of the library (the tests' planted-defect builds) with the
    same C ABI, bound like lib() and kept separate from it."""
    L = ctypes.CDLL(path, mode=os.RTLD_LOCAL)
    P, I, Z, D, U64 = ctypes.c_void_p, ctypes.c_int, ctypes.c_size_t, ctypes.c_double, ctypes.c_uint64
    sig = {
        "zt_attn_dim_ok": (I, [I]),
        "zt_attn_forward_shmem": (Z, [I, I, I]),
        "zt_attn_bwd_dq_shmem": (Z, [I, I]),
        "zt_attn_bwd_dkdv_shmem": (Z, [I]),
        "zt_attn_forward": (I, [P, P, P, P, I, I, I, I, I, I, I, I, P]),
        "zt_attn_backward": (I, [P, P, P, P, P, P, P, P, P, P, I, I, I, I, I, P]),
        "zt_attn_forward_batched": (I, [P, P, P, P, I, I, I, I, I, I, I, I, I, I, P]),
        "zt_attn_backward_batched": (I, [P, P, P, P, P, P, P, P, P, P, I, I, I, I, I, I, P]),
        "zt_attn_bwd_dq": (I, [P] * 8 + [I] * 6 + [P]),
        "zt_attn_bwd_dkdv": (I, [P] * 9 + [I] * 5 + [P]),
        "zt_attn_decode_workspace": (Z, [I, I, I, I, I]),
        "zt_attn_decode": (I, [P, P, P, P, P, I, I, I, I, I, P, Z, P]),
        "zt_attn_decode_noalloc": (I, [P, P, P, P, P, I, I, I, I, I, P]),
        "zt_attn_decode_step_workspace": (Z, [I, I, I, I, I]),
        "zt_attn_decode_step": (I, [P] * 7 + [I] * 5 + [D, P, Z, P]),
        "zt_rmsnorm_forward": (I, [P, P, P, I, I, D, P]),
        "zt_attn_forward_train": (I, [P] * 5 + [I] * 5 + [P]),
        "zt_attn_backward_train": (I, [P] * 10 + [I] * 5 + [P]),
        "zt_attn_bwd_dq_train": (I, [P] * 8 + [I] * 5 + [P]),
        "zt_attn_bwd_dkdv_train": (I, [P] * 9 + [I] * 5 + [P]),
        "zt_attn_plan_train": (I, [I] * 5 + [P, P, P, Z]),
        "zt_attn_backward_train_workspace": (Z, [I] * 5),
        "zt_attn_backward_train_ws": (I, [P] * 10 + [Z] + [I] * 6 + [P]),
        "zt_attn_forward_train_ws": (I, [P] * 6 + [Z] + [I] * 5 + [P]),
        "zt_matmul": (I, [P, P, P, I, I, I, P]),
        "zt_weight_grad": (I, [P, P, P, I, I, I, P]),
        "zt_input_grad": (I, [P, P, P, I, I, I, P]),
        "zt_matmul_plan": (I, [I, I, I, P, I]),
        "zt_calibrate": (I, [P, Z, P, Z, P, P, P]),
        "zt_calibrate_launch": (I, [ctypes.c_uint, ctypes.c_uint, I, P, P]),
        "zt_rope_forward": (I, [P, P, I, I, I, D, I, P]),
        "zt_rope_backward": (I, [P, P, I, I, I, D, I, P]),
        "zt_rope_qk_forward": (I, [P, P, P, P, I, I, I, I, I, I, D, P]),
        "zt_rope_qk_backward": (I, [P, P, P, P, I, I, I, I, I, I, D, P]),
        "zt_fill_normal": (I, [P, Z, U64, D, D, P]),
        "zt_fill_uniform": (I, [P, Z, U64, D, D, P]),
        "zt_attn_version": (ctypes.c_char_p, []),
        "zt_attn_lds_limit": (Z, []),
        "zt_attn_set_tuning": (I, [ctypes.c_char_p, I]),
        "zt_attn_get_tuning": (I, [ctypes.c_char_p]),
        "zt_attn_plan": (I, [I, I, I, I, I, I, ctypes.c_char_p, ctypes.c_char_p, ctypes.c_char_p, Z]),
        "zt_bytes_for": (I, [I, Z, Z, Z, Z, ctypes.POINTER(Z)]),
        "zt_to_cint": (I, [Z, ctypes.POINTER(I)]),
        "zt_forward_bounds": (I, [I, I, I, I]),
        "zt_holder_init": (I, [Z, Z, Z, Z, ctypes.POINTER(P)]),
        "zt_holder_init_exact": (I, [Z, Z, Z, Z, ctypes.POINTER(P)]),
        "zt_holder_workspace_bytes": (Z, [P]),
        "zt_holder_forget": (None, [P]),
        "zt_holder_deinit": (None, [P]),
        "zt_holder_total_bytes": (Z, [P]),
        "zt_holder_buffer": (P, [P, I]),
        "zt_holder_buffer_ro": (P, [P, I]),
        "zt_holder_forward": (I, [P, I, I]),
        "zt_holder_forward_at": (I, [P, I, I, I, I, I]),
        "zt_holder_backward": (I, [P, I]),
        "zt_holder_upload": (I, [P, I, P, Z]),
        "zt_holder_download": (I, [P, P, I, Z]),
    }
    for name, (res, args) in sig.items():
        fn = getattr(L, name)
        fn.restype = res
        fn.argtypes = args
    return L


def set_tuning(name, value):
    """Force a kernel variant (include/zt_attn.h, zt_attn_set_tuning); -1 restores the shape rule."""
    _check(lib().zt_attn_set_tuning(name.encode(), int(value)), f"zt_attn_set_tuning({name}, {value})")


def get_tuning(name):
    return lib().zt_attn_get_tuning(name.encode())


def _ptr(t):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def _stream(stream):
    if stream is None:
        import torch
        stream = torch.cuda.current_stream()
    return ctypes.c_void_p(stream.cuda_stream)


def _check(rc, what):
    if rc != 0:
        raise ZtRefused(f"{what} refused (rc={rc})")


def _f32_cuda(*ts):
    import torch
    for t in ts:
        if t.dtype != torch.float32 or not t.is_cuda or not t.is_contiguous():
            raise ValueError("tensors must be contiguous float32 on the GPU")


def forward(q, k, v, out, T, n_heads, n_kv_heads, dim, group_q=1, max_tile=64, q_offset=0, n_keys=None,
            B=1, kv_rows=None, stream=None):
    """zt_attn_forward (B == 1, kv_rows == n_keys) or zt_attn_forward_batched."""
    _f32_cuda(q, k, v, out)
    n_keys = T if n_keys is None else n_keys
    if B == 1 and (kv_rows is None or kv_rows == n_keys):
        rc = lib().zt_attn_forward(_ptr(q), _ptr(k), _ptr(v), _ptr(out), T, n_heads, n_kv_heads, dim, group_q,
                                   max_tile, q_offset, n_keys, _stream(stream))
    else:
        kv_rows = n_keys if kv_rows is None else kv_rows
        rc = lib().zt_attn_forward_batched(_ptr(q), _ptr(k), _ptr(v), _ptr(out), B, T, n_heads, n_kv_heads, dim,
                                           group_q, max_tile, q_offset, n_keys, kv_rows, _stream(stream))
    _check(rc, "zt_attn_forward")


def backward(q, k, v, dout, dq, dk, dv, row_max, row_den, row_del, T, n_heads, n_kv_heads, dim, max_tile=64, B=1,
             stream=None):
    _f32_cuda(q, k, v, dout, dq, dk, dv, row_max, row_den, row_del)
    if B == 1:
        rc = lib().zt_attn_backward(*map(_ptr, (q, k, v, dout, dq, dk, dv, row_max, row_den, row_del)), T, n_heads,
                                    n_kv_heads, dim, max_tile, _stream(stream))
    else:
        rc = lib().zt_attn_backward_batched(*map(_ptr, (q, k, v, dout, dq, dk, dv, row_max, row_den, row_del)), B,
                                            T, n_heads, n_kv_heads, dim, max_tile, _stream(stream))
    _check(rc, "zt_attn_backward")


def bwd_dq(q, k, v, dout, dq, row_max, row_den, row_del, T, n_heads, n_kv_heads, dim, max_tile=64, B=1,
           stream=None):
    _f32_cuda(q, k, v, dout, dq, row_max, row_den, row_del)
    _check(lib().zt_attn_bwd_dq(*map(_ptr, (q, k, v, dout, dq, row_max, row_den, row_del)), B, T, n_heads,
                                n_kv_heads, dim, max_tile, _stream(stream)), "zt_attn_bwd_dq")


def bwd_dkdv(q, k, v, dout, dk, dv, row_max, row_den, row_del, T, n_heads, n_kv_heads, dim, B=1, stream=None):
    _f32_cuda(q, k, v, dout, dk, dv, row_max, row_den, row_del)
    _check(lib().zt_attn_bwd_dkdv(*map(_ptr, (q, k, v, dout, dk, dv, row_max, row_den, row_del)), B, T, n_heads,
                                  n_kv_heads, dim, _stream(stream)), "zt_attn_bwd_dkdv")


def forward_train(q, k, v, out, lse, T, n_heads, n_kv_heads, dim, B=1, stream=None):
    _f32_cuda(q, k, v, out, lse)
    _check(lib().zt_attn_forward_train(_ptr(q), _ptr(k), _ptr(v), _ptr(out), _ptr(lse), B, T, n_heads, n_kv_heads,
                                       dim, _stream(stream)), "zt_attn_forward_train")


# include/zt_attn.h: stage flag of zt_attn_backward_train_ws, the workspace holds the forward's scores
ZT_WS_SCORES = 4


def forward_train_ws(q, k, v, out, lse, workspace, T, n_heads, n_kv_heads, dim, B=1, stream=None):
    _f32_cuda(q, k, v, out, lse, workspace)
    nbytes = workspace.numel() * workspace.element_size()
    _check(lib().zt_attn_forward_train_ws(_ptr(q), _ptr(k), _ptr(v), _ptr(out), _ptr(lse), _ptr(workspace), nbytes,
                                          B, T, n_heads, n_kv_heads, dim, _stream(stream)),
           "zt_attn_forward_train_ws")


def backward_train(q, k, v, out, dout, lse, dq, dk, dv, delta, T, n_heads, n_kv_heads, dim, B=1, stream=None):
    _f32_cuda(q, k, v, out, dout, lse, dq, dk, dv, delta)
    _check(lib().zt_attn_backward_train(_ptr(q), _ptr(k), _ptr(v), _ptr(out), _ptr(dout), _ptr(lse), _ptr(dq),
                                        _ptr(dk), _ptr(dv), _ptr(delta), B, T, n_heads, n_kv_heads, dim,
                                        _stream(stream)), "zt_attn_backward_train")


def bwd_dq_train(q, k, v, out, dout, lse, dq, delta, T, n_heads, n_kv_heads, dim, B=1, stream=None):
    _f32_cuda(q, k, v, out, dout, lse, dq, delta)
    _check(lib().zt_attn_bwd_dq_train(_ptr(q), _ptr(k), _ptr(v), _ptr(out), _ptr(dout), _ptr(lse), _ptr(dq),
                                      _ptr(delta), B, T, n_heads, n_kv_heads, dim, _stream(stream)),
           "zt_attn_bwd_dq_train")


def bwd_dkdv_train(q, k, v, out, dout, lse, delta, dk, dv, T, n_heads, n_kv_heads, dim, B=1, stream=None):
    _f32_cuda(q, k, v, out, dout, lse, delta, dk, dv)
    _check(lib().zt_attn_bwd_dkdv_train(_ptr(q), _ptr(k), _ptr(v), _ptr(out), _ptr(dout), _ptr(lse), _ptr(delta),
                                        _ptr(dk), _ptr(dv), B, T, n_heads, n_kv_heads, dim, _stream(stream)),
           "zt_attn_bwd_dkdv_train")


def backward_train_workspace_bytes(B, T, n_heads, n_kv_heads, dim):
    return lib().zt_attn_backward_train_workspace(B, T, n_heads, n_kv_heads, dim)


def backward_train_ws(q, k, v, out, dout, lse, dq, dk, dv, workspace, T, n_heads, n_kv_heads, dim, B=1, stage=3,
                      stream=None):
    _f32_cuda(q, k, v, out, dout, lse, dq, dk, dv, workspace)
    nbytes = workspace.numel() * workspace.element_size()
    _check(lib().zt_attn_backward_train_ws(_ptr(q), _ptr(k), _ptr(v), _ptr(out), _ptr(dout), _ptr(lse), _ptr(dq),
                                           _ptr(dk), _ptr(dv), _ptr(workspace), nbytes, B, T, n_heads, n_kv_heads,
                                           dim, stage, _stream(stream)), "zt_attn_backward_train_ws")


def plan_train(B, T, n_heads, n_kv_heads, dim):
    bufs = [ctypes.create_string_buffer(64) for _ in range(3)]
    _check(lib().zt_attn_plan_train(B, T, n_heads, n_kv_heads, dim, *bufs, 64), "zt_attn_plan_train")
    return tuple(b.value.decode() for b in bufs)


def decode_workspace_bytes(B, n_ctx, n_heads, n_kv_heads, dim):
    return lib().zt_attn_decode_workspace(B, n_ctx, n_heads, n_kv_heads, dim)


def decode(q, k_cache, v_cache, out, n_keys, B, n_ctx, n_heads, n_kv_heads, dim, workspace, stream=None):
    """n_keys: a sequence of B ints (host)."""
    _f32_cuda(q, k_cache, v_cache, out)
    arr = (ctypes.c_int * B)(*[int(x) for x in n_keys])
    nbytes = workspace.numel() * workspace.element_size()
    rc = lib().zt_attn_decode(_ptr(q), _ptr(k_cache), _ptr(v_cache), _ptr(out), arr, B, n_ctx, n_heads, n_kv_heads,
                              dim, _ptr(workspace), nbytes, _stream(stream))
    _check(rc, "zt_attn_decode")


def decode_step_workspace_bytes(B, n_ctx, n_heads, n_kv_heads, dim):
    return lib().zt_attn_decode_step_workspace(B, n_ctx, n_heads, n_kv_heads, dim)


def decode_step(q, k_new, v_new, k_cache, v_cache, out, pos, B, n_ctx, n_heads, n_kv_heads, dim, workspace,
                theta=500000.0, stream=None):
    """pos: a sequence of B ints (host), the position each sequence appends at."""
    _f32_cuda(q, k_new, v_new, k_cache, v_cache, out)
    arr = (ctypes.c_int * B)(*[int(x) for x in pos])
    nbytes = workspace.numel() * workspace.element_size()
    rc = lib().zt_attn_decode_step(_ptr(q), _ptr(k_new), _ptr(v_new), _ptr(k_cache), _ptr(v_cache), _ptr(out), arr,
                                   B, n_ctx, n_heads, n_kv_heads, dim, theta, _ptr(workspace), nbytes,
                                   _stream(stream))
    _check(rc, "zt_attn_decode_step")


def rmsnorm(x, w, y, rows, cols, eps=1e-5, stream=None):
    _f32_cuda(x, w, y)
    _check(lib().zt_rmsnorm_forward(_ptr(x), _ptr(w), _ptr(y), rows, cols, eps, _stream(stream)), "zt_rmsnorm_forward")


def rope(x, y, rows, cols, pos, theta, head_dim, stream=None):
    _f32_cuda(x, y)
    _check(lib().zt_rope_forward(_ptr(x), _ptr(y), rows, cols, pos, theta, head_dim, _stream(stream)),
           "zt_rope_forward")


def plan(B, T, n_heads, n_kv_heads, dim, max_tile=64):
    """(forward, dq, dk/dv) kernel names the library launches at this shape."""
    bufs = [ctypes.create_string_buffer(64) for _ in range(3)]
    _check(lib().zt_attn_plan(B, T, n_heads, n_kv_heads, dim, max_tile, *bufs, 64), "zt_attn_plan")
    return tuple(b.value.decode() for b in bufs)


def rope_backward(dout, din, rows, cols, pos, theta, head_dim, stream=None):
    _f32_cuda(dout, din)
    _check(lib().zt_rope_backward(_ptr(dout), _ptr(din), rows, cols, pos, theta, head_dim, _stream(stream)),
           "zt_rope_backward")


def rope_qk(q, k, q_out, k_out, B, T, n_heads, n_kv_heads, head_dim, pos=0, theta=500000.0, backward=False,
            stream=None):
    _f32_cuda(q, k, q_out, k_out)
    fn = lib().zt_rope_qk_backward if backward else lib().zt_rope_qk_forward
    _check(fn(_ptr(q), _ptr(k), _ptr(q_out), _ptr(k_out), B, T, n_heads, n_kv_heads, head_dim, pos, theta,
              _stream(stream)), "zt_rope_qk")


class DimensionMismatch(ValueError):
    """src/tensor.zig:79: a.cols != b.rows."""


def matmul(a, b, out, M, K, N, stream=None):
    """out[M,N] = a[M,K] b[K,N] (src/tensor.zig:78-106)."""
    _f32_cuda(a, b, out)
    if a.numel() != M * K or b.numel() != K * N or out.numel() != M * N:
        raise DimensionMismatch(f"{M}x{K} @ {K}x{N} into {out.numel()} elements")
    _check(lib().zt_matmul(_ptr(a), _ptr(b), _ptr(out), M, K, N, _stream(stream)), "zt_matmul")


def gemm_kernel(M, K, N):
    """The kernel zt_matmul launches for an M x K x N product."""
    buf = ctypes.create_string_buffer(64)
    _check(lib().zt_matmul_plan(M, K, N, buf, 64), "zt_matmul_plan")
    return buf.value.decode()


def weight_grad(w, inp, dout, T, I, J, stream=None):
    """w[I,J] += inp[T,I]^T dout[T,J] (src/autograd.zig:958-972)."""
    _f32_cuda(w, inp, dout)
    _check(lib().zt_weight_grad(_ptr(w), _ptr(inp), _ptr(dout), T, I, J, _stream(stream)), "zt_weight_grad")


def input_grad(din, dout, w, T, J, I, stream=None):
    """din[T,I] += dout[T,J] w[I,J]^T (src/autograd.zig:999-1022)."""
    _f32_cuda(din, dout, w)
    _check(lib().zt_input_grad(_ptr(din), _ptr(dout), _ptr(w), T, J, I, _stream(stream)), "zt_input_grad")


def calibrate(src, scratch, stream=None):
    """(sustained FP32 MFMA TFLOP/s, streaming-read GB/s) measured on this device."""
    _f32_cuda(src, scratch)
    tf, gb = ctypes.c_double(0.0), ctypes.c_double(0.0)
    _check(lib().zt_calibrate(_ptr(src), src.numel() * 4, _ptr(scratch), scratch.numel() * 4, ctypes.addressof(tf),
                              ctypes.addressof(gb), _stream(stream)), "zt_calibrate")
    return tf.value, gb.value


def launch_floor_us(blocks, threads, launches=256, stream=None):
    """Average microseconds per back-to-back launch of an empty kernel of this grid."""
    us = ctypes.c_double(0.0)
    _check(lib().zt_calibrate_launch(blocks, threads, launches, ctypes.addressof(us), _stream(stream)),
           "zt_calibrate_launch")
    return us.value


def fill_normal(t, seed, mean=0.0, sigma=1.0, stream=None):
    _f32_cuda(t)
    _check(lib().zt_fill_normal(_ptr(t), t.numel(), seed, mean, sigma, _stream(stream)), "zt_fill_normal")


def fill_uniform(t, seed, lo=0.0, hi=1.0, stream=None):
    _f32_cuda(t)
    _check(lib().zt_fill_uniform(_ptr(t), t.numel(), seed, lo, hi, _stream(stream)), "zt_fill_uniform")
