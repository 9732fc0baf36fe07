"""numpy face of the CPU restatement (oracle/zt_oracle.c).

TEST INFRASTRUCTURE ONLY: the parity checker and the CPU baseline.  Only
tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may import
this module; the shipped library never does.  Build with `make -C oracle`.
"""
import ctypes
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "_build", "libzt_oracle.so")
_lib = None


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise FileNotFoundError(f"{LIB_PATH} is not built; run `make -C oracle`")
        L = ctypes.CDLL(LIB_PATH)
        P, I, D, Z, U = ctypes.c_void_p, ctypes.c_int, ctypes.c_double, ctypes.c_size_t, ctypes.c_uint64
        sig = {
            "zto_attention_forward": (I, [P, P, P, P] + [I] * 7),
            "zto_attention_forward_mt": (I, [P, P, P, P] + [I] * 8),
            "zto_attention_forward_at": (I, [P, P, P, P] + [I] * 7),
            "zto_attention_backward": (I, [P] * 7 + [I] * 7),
            "zto_attention_backward_mt": (I, [P] * 7 + [I] * 8),
            "zto_attention_row_stats": (I, [P] * 7 + [I] * 5),
            "zto_attention_backward_groups": (I, [P] * 7 + [I] * 8),
            "zto_attention_forward_groups": (I, [P] * 4 + [I] * 8),
            "zto_attn_step": (I, [P] * 5 + [I] * 5),
            "zto_attn_step_mt": (I, [P] * 5 + [I] * 6),
            "zto_rmsnorm": (None, [P, P, P, I, I, D]),
            "zto_rope": (I, [P, P, I, I, I, D, I]),
            "zto_rope_backward": (I, [P, P, I, I, I, D, I]),
            "zto_decode_step": (I, [P] * 7 + [I] * 5 + [D]),
            "zto_matmul": (None, [P, P, P, I, I, I]),
            "zto_weight_grad": (None, [P, P, P, I, I, I]),
            "zto_input_grad": (None, [P, P, P, I, I, I]),
            "zto_fill_normal": (None, [P, Z, U, D, D]),
            "zto_fill_uniform": (None, [P, Z, U, D, D]),
            "zto_splitmix64": (U, [U, U]),
        }
        for n, (r, a) in sig.items():
            f = getattr(L, n)
            f.restype = r
            f.argtypes = a
        _lib = L
    return _lib


def _p(a):
    return a.ctypes.data_as(ctypes.c_void_p)


def _f32(a):
    a = np.ascontiguousarray(a, dtype=np.float32)
    return a


class OracleRefused(ValueError):
    pass


def attention_forward(q, k, v, B, T, H, Hkv, D, t_begin=0, t_end=None, threads=1, out=None):
    """src/attention.zig:60-153 over B sequences; rows [t_begin, t_end)."""
    q, k, v = _f32(q), _f32(k), _f32(v)
    t_end = T if t_end is None else t_end
    out = np.zeros(B * T * H * D, np.float32) if out is None else out
    rc = lib().zto_attention_forward_mt(_p(q), _p(k), _p(v), _p(out), B, T, H, Hkv, D, t_begin, t_end, threads)
    if rc:
        raise OracleRefused(f"InvalidHeadConfig/shape rc={rc}")
    return out


def attention_forward_at(q, k, v, B, T, H, Hkv, D, q_offset, n_keys):
    q, k, v = _f32(q), _f32(k), _f32(v)
    out = np.zeros(B * T * H * D, np.float32)
    rc = lib().zto_attention_forward_at(_p(q), _p(k), _p(v), _p(out), B, T, H, Hkv, D, q_offset, n_keys)
    if rc:
        raise OracleRefused(f"rc={rc}")
    return out


def attention_backward(q, k, v, dout, B, T, H, Hkv, D, t_begin=0, t_end=None, threads=1):
    """src/autograd.zig:636-842; returns (dq, dk, dv) as flat f32 arrays."""
    q, k, v, dout = _f32(q), _f32(k), _f32(v), _f32(dout)
    t_end = T if t_end is None else t_end
    dq = np.zeros(B * T * H * D, np.float32)
    dk = np.zeros(B * T * Hkv * D, np.float32)
    dv = np.zeros(B * T * Hkv * D, np.float32)
    rc = lib().zto_attention_backward_mt(_p(q), _p(k), _p(v), _p(dout), _p(dq), _p(dk), _p(dv), B, T, H, Hkv, D,
                                         t_begin, t_end, threads)
    if rc:
        raise OracleRefused(f"rc={rc}")
    return dq, dk, dv


def attention_forward_groups(q, k, v, B, T, H, Hkv, D, kv_begin, kv_end, threads=16, out=None):
    """attention.forward for every row of the heads of kv groups [kv_begin, kv_end);
    the other heads' columns of `out` are left as given (zeros by default)."""
    q, k, v = _f32(q), _f32(k), _f32(v)
    out = np.zeros(B * T * H * D, np.float32) if out is None else out
    rc = lib().zto_attention_forward_groups(_p(q), _p(k), _p(v), _p(out), B, T, H, Hkv, D, kv_begin, kv_end, threads)
    if rc:
        raise OracleRefused(f"rc={rc}")
    return out


def attention_backward_groups(q, k, v, dout, B, T, H, Hkv, D, kv_begin, kv_end, threads=16):
    """attentionBackward over whole kv groups [kv_begin, kv_end), bit-identical to
    attention_backward there; returns (dq, dk, dv), zero outside those groups."""
    q, k, v, dout = _f32(q), _f32(k), _f32(v), _f32(dout)
    dq = np.zeros(B * T * H * D, np.float32)
    dk = np.zeros(B * T * Hkv * D, np.float32)
    dv = np.zeros(B * T * Hkv * D, np.float32)
    rc = lib().zto_attention_backward_groups(_p(q), _p(k), _p(v), _p(dout), _p(dq), _p(dk), _p(dv), B, T, H, Hkv, D,
                                             kv_begin, kv_end, threads)
    if rc:
        raise OracleRefused(f"rc={rc}")
    return dq, dk, dv


def attention_row_stats(q, k, v, dout, B, T, H, Hkv, D):
    q, k, v, dout = _f32(q), _f32(k), _f32(v), _f32(dout)
    m = np.zeros(B * T * H)
    l = np.zeros(B * T * H)
    d = np.zeros(B * T * H)
    rc = lib().zto_attention_row_stats(_p(q), _p(k), _p(v), _p(dout), _p(m), _p(l), _p(d), B, T, H, Hkv, D)
    if rc:
        raise OracleRefused(f"rc={rc}")
    return m, l, d


def attn_step(q, kc, vc, n_keys, B, n_ctx, H, Hkv, D, threads=1):
    """src/decode.zig:326-392 per sequence."""
    q, kc, vc = _f32(q), _f32(kc), _f32(vc)
    nk = np.ascontiguousarray(n_keys, dtype=np.int32)
    out = np.zeros(B * H * D, np.float32)
    rc = lib().zto_attn_step_mt(_p(q), _p(kc), _p(vc), _p(out), _p(nk), B, n_ctx, H, Hkv, D, threads)
    if rc:
        raise OracleRefused(f"rc={rc}")
    return out


def rmsnorm(x, w, rows, cols, eps=1e-5):
    """src/norm.zig:18-47."""
    x, w = _f32(x), _f32(w)
    y = np.zeros(rows * cols, np.float32)
    lib().zto_rmsnorm(_p(x), _p(w), _p(y), rows, cols, eps)
    return y


def rope(x, rows, cols, pos, theta, head_dim):
    """src/rope.zig:21-55.  Raises OracleRefused(1=OddHeadDim, 2=DimensionMismatch)."""
    x = _f32(x)
    y = np.zeros(rows * cols, np.float32)
    rc = lib().zto_rope(_p(x), _p(y), rows, cols, pos, theta, head_dim)
    if rc:
        raise OracleRefused(rc)
    return y


def rope_backward(dout, rows, cols, pos, theta, head_dim):
    """src/autograd.zig:851-872."""
    dout = _f32(dout)
    din = np.zeros(rows * cols, np.float32)
    rc = lib().zto_rope_backward(_p(dout), _p(din), rows, cols, pos, theta, head_dim)
    if rc:
        raise OracleRefused(rc)
    return din


def decode_step(q, k_new, v_new, k_cache, v_cache, pos, B, n_ctx, H, Hkv, D, theta=500000.0):
    """src/decode.zig:244-270; returns (out, k_cache, v_cache) with the caches updated."""
    q, k_new, v_new = _f32(q), _f32(k_new), _f32(v_new)
    kc = np.array(k_cache, dtype=np.float32, copy=True).ravel()
    vc = np.array(v_cache, dtype=np.float32, copy=True).ravel()
    p = np.ascontiguousarray(pos, dtype=np.int32)
    out = np.zeros(B * H * D, np.float32)
    rc = lib().zto_decode_step(_p(q), _p(k_new), _p(v_new), _p(kc), _p(vc), _p(out), _p(p), B, n_ctx, H, Hkv, D,
                               theta)
    if rc:
        raise OracleRefused(rc)
    return out, kc, vc


def matmul(a, b, M, K, N):
    """src/tensor.zig:78-106."""
    a, b = _f32(a), _f32(b)
    out = np.zeros(M * N, np.float32)
    lib().zto_matmul(_p(a), _p(b), _p(out), M, K, N)
    return out


def weight_grad(w, inp, dout, T, I, J):
    """src/autograd.zig:958-972; returns w + input^T dout (w is not modified)."""
    w = np.array(w, dtype=np.float32, copy=True).ravel()
    inp, dout = _f32(inp), _f32(dout)
    lib().zto_weight_grad(_p(w), _p(inp), _p(dout), T, I, J)
    return w


def input_grad(out, dout, w, T, J, I):
    """src/autograd.zig:999-1022; returns out + dout w^T (out is not modified)."""
    out = np.array(out, dtype=np.float32, copy=True).ravel()
    dout, w = _f32(dout), _f32(w)
    lib().zto_input_grad(_p(out), _p(dout), _p(w), T, J, I)
    return out


def fill_normal(n, seed, mean=0.0, sigma=1.0):
    out = np.zeros(n, np.float32)
    lib().zto_fill_normal(_p(out), n, seed, mean, sigma)
    return out


def fill_uniform(n, seed, lo=0.0, hi=1.0):
    out = np.zeros(n, np.float32)
    lib().zto_fill_uniform(_p(out), n, seed, lo, hi)
    return out


def splitmix64(seed, counter):
    return lib().zto_splitmix64(seed, counter)
