"""The C ABI without a GPU: the library loads, exports every function the
headers declare, and refuses bad calls in the reference's order before any
device call (src/cuda/attn_kernels.cu:833-1036).  With no device present a
well-formed call is refused at the LDS-ceiling step, which is what the
reference does for a device whose ceiling cannot be read (:910-915)."""
import ctypes
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
NULL = None


def _declared(header):
    src = open(os.path.join(ROOT, "include", header)).read()
    src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
    return sorted(set(re.findall(r"\b(zt_[a-z0-9_]+)\s*\(", src)))


def test_library_exports_every_declared_symbol(zt):
    L = zt.lib()
    declared = _declared("zt_attn.h") + _declared("zt_holder.h")
    assert len(declared) >= 28
    for name in declared:
        assert hasattr(L, name), name
    assert set(zt.ABI_SYMBOLS + zt.HOLDER_SYMBOLS) == set(declared)


def test_reference_six_symbols_present(zt):
    for name in ["zt_attn_dim_ok", "zt_attn_forward_shmem", "zt_attn_bwd_dq_shmem", "zt_attn_bwd_dkdv_shmem",
                 "zt_attn_forward", "zt_attn_backward"]:
        assert hasattr(zt.lib(), name)


def test_dim_ok_admits_exactly_the_even_widths_32_to_256(zt, golden):
    L = zt.lib()
    for d in range(-40, 600):
        assert L.zt_attn_dim_ok(d) == (1 if (32 <= d <= 256 and d % 2 == 0) else 0), d
    for d in golden["dim_ok_table"]["refused_examples"]:
        assert L.zt_attn_dim_ok(d) == 0


def test_dim_ok_is_silent(zt, capfd):
    zt.lib().zt_attn_dim_ok(7)
    assert capfd.readouterr().err == ""


def test_shmem_counts(zt):
    L = zt.lib()
    for d in range(32, 257, 2):
        f64, f32 = L.zt_attn_forward_shmem(d, 64, 1), L.zt_attn_forward_shmem(d, 32, 1)
        assert 0 < f32 <= f64 <= 160 * 1024
        assert 0 < L.zt_attn_bwd_dq_shmem(d, 32) <= L.zt_attn_bwd_dq_shmem(d, 64) <= 160 * 1024
        assert 0 < L.zt_attn_bwd_dkdv_shmem(d) <= 160 * 1024
    assert L.zt_attn_forward_shmem(33, 64, 1) == 0 and L.zt_attn_bwd_dkdv_shmem(300) == 0


def _fwd(L, T=8, H=4, Hkv=2, dim=32, group_q=1, max_tile=64, q_offset=0, n_keys=8):
    return L.zt_attn_forward(NULL, NULL, NULL, NULL, T, H, Hkv, dim, group_q, max_tile, q_offset, n_keys, NULL)


def _bwd(L, T=8, H=4, Hkv=2, dim=32, max_tile=64):
    return L.zt_attn_backward(*([NULL] * 10), T, H, Hkv, dim, max_tile, NULL)


@pytest.mark.parametrize("kw,msg", [
    (dict(T=0), "T 0 is not launchable"),
    (dict(T=-1), "T -1 is not launchable"),
    (dict(dim=33), "head_dim 33 is refused"),
    (dict(dim=258), "head_dim 258 is refused"),
    (dict(H=3, Hkv=2), "3 heads over 2 kv heads is not a group"),
    (dict(H=4, Hkv=0), "4 heads over 0 kv heads"),
    (dict(H=65536, Hkv=1), "exceeds the 65535"),
    (dict(group_q=0), "group_q 0"),
    (dict(group_q=65), "group_q 65"),
    (dict(dim=256, group_q=8), "group_q 8 at head_dim 256"),
    (dict(q_offset=-1), "q_offset -1"),
    (dict(n_keys=0), "n_keys 0"),
    (dict(T=2, q_offset=7, n_keys=8), "q_offset 7, n_keys 8"),
    (dict(T=1, q_offset=2147483647, n_keys=1), "q_offset 2147483647"),
    (dict(max_tile=0), "max_tile 0"),
])
def test_forward_refusals_in_reference_order(zt, capfd, kw, msg):
    assert _fwd(zt.lib(), **kw) == 1
    assert msg in capfd.readouterr().err


def test_refusal_order_T_before_width_before_group(zt, capfd):
    L = zt.lib()
    assert _fwd(L, T=0, dim=33, H=3) == 1
    err = capfd.readouterr().err
    assert "T 0" in err and "head_dim" not in err
    assert _fwd(L, dim=33, H=3) == 1
    err = capfd.readouterr().err
    assert "head_dim 33" in err and "not a group" not in err


@pytest.mark.parametrize("kw,msg", [
    (dict(T=0), "T 0 is not launchable"),
    (dict(dim=31), "head_dim 31 is refused"),
    (dict(H=5, Hkv=2), "not a group"),
    (dict(H=70000, Hkv=2), "exceeds the 65535"),
    (dict(max_tile=-3), "max_tile -3"),
])
def test_backward_refusals_in_reference_order(zt, capfd, kw, msg):
    assert _bwd(zt.lib(), **kw) == 1
    assert msg in capfd.readouterr().err


def test_no_device_means_refusal_not_a_crash(zt, capfd):
    import torch
    if torch.cuda.is_available():
        pytest.skip("a GPU is present")
    L = zt.lib()
    assert L.zt_attn_lds_limit() == 0
    assert _fwd(L) == 1 and "LDS ceiling could not be read" in capfd.readouterr().err
    assert _bwd(L) == 1 and "LDS ceiling could not be read" in capfd.readouterr().err
    assert L.zt_rmsnorm_forward(NULL, NULL, NULL, 0, 8, 1e-5, NULL) == 0  # zero rows: nothing to launch
    assert L.zt_rmsnorm_forward(NULL, NULL, NULL, 2, 0, 1e-5, NULL) == 1


def test_decode_refusals(zt, capfd):
    L = zt.lib()
    nk = (ctypes.c_int * 2)(5, 9)
    ws = L.zt_attn_decode_workspace(2, 8, 4, 2, 32)
    assert ws > 0
    assert L.zt_attn_decode(NULL, NULL, NULL, NULL, nk, 0, 8, 4, 2, 32, NULL, 0, NULL) == 1
    assert L.zt_attn_decode(NULL, NULL, NULL, NULL, nk, 2, 8, 4, 2, 30, NULL, 0, NULL) == 1
    assert L.zt_attn_decode(NULL, NULL, NULL, NULL, nk, 2, 8, 3, 2, 32, NULL, 0, NULL) == 1
    assert L.zt_attn_decode(NULL, NULL, NULL, NULL, nk, 2, 8, 4, 2, 32, NULL, ws, NULL) == 1
    assert "n_keys 9, outside [1, 8]" in capfd.readouterr().err
    nk2 = (ctypes.c_int * 2)(5, 8)
    assert L.zt_attn_decode(NULL, NULL, NULL, NULL, nk2, 2, 8, 4, 2, 32, NULL, ws - 1, NULL) == 1
    assert "workspace" in capfd.readouterr().err
    assert L.zt_attn_decode(NULL, NULL, NULL, NULL, nk2, 2, 8, 4, 2, 32, 0x10004, ws, NULL) == 1
    assert "not 16-byte aligned" in capfd.readouterr().err
    assert L.zt_attn_decode_workspace(0, 8, 4, 2, 32) == 0


def test_train_path_refusals(zt, capfd):
    L = zt.lib()
    p = 0x10000
    assert L.zt_attn_forward_train(p, p, p, p, NULL, 1, 8, 4, 2, 32, NULL) == 1
    assert "lse" in capfd.readouterr().err
    assert L.zt_attn_forward_train(p, p, p, p, p, 1, 0, 4, 2, 32, NULL) == 1
    assert "T 0" in capfd.readouterr().err
    assert L.zt_attn_backward_train(p, p, p, p, p, p, p, p, p, NULL, 1, 8, 4, 2, 32, NULL) == 1
    assert "delta" in capfd.readouterr().err
    assert L.zt_attn_bwd_dkdv_train(p, p, p, p, p, NULL, p, p, p, 1, 8, 4, 2, 32, NULL) == 1
    assert L.zt_attn_backward_train(p, p, p, p, p, p, p, p, p, p, 1, 8, 3, 2, 32, NULL) == 1
    assert "not a group" in capfd.readouterr().err
    need = L.zt_attn_backward_train_workspace(1, 8, 4, 2, 32)
    assert need > 0
    assert L.zt_attn_forward_train_ws(p, p, p, p, p, p, need - 1, 1, 8, 4, 2, 32, NULL) == 1
    assert "workspace" in capfd.readouterr().err
    assert L.zt_attn_forward_train_ws(p, p, p, p, NULL, p, need, 1, 8, 4, 2, 32, NULL) == 1
    assert "lse" in capfd.readouterr().err
    assert L.zt_attn_backward_train_ws(p, p, p, p, p, p, p, p, p, p, need, 1, 8, 4, 2, 32, 4, NULL) == 1
    assert "stage" in capfd.readouterr().err   # ZT_WS_SCORES alone names no stage
    # Workspaces hold 16-byte vectors: a base that is not 16-byte aligned is refused.
    assert L.zt_attn_forward_train_ws(p, p, p, p, p, p + 4, need, 1, 8, 4, 2, 32, NULL) == 1
    assert "not 16-byte aligned" in capfd.readouterr().err
    assert L.zt_attn_backward_train_ws(p, p, p, p, p, p, p, p, p, p + 8, need, 1, 8, 4, 2, 32, 3, NULL) == 1
    assert "not 16-byte aligned" in capfd.readouterr().err


def test_dense_product_refusals(zt, capfd):
    L = zt.lib()
    assert L.zt_matmul(NULL, NULL, NULL, -1, 2, 2, NULL) == 1 and "not launchable" in capfd.readouterr().err
    assert L.zt_matmul(NULL, NULL, NULL, 0, 5, 7, NULL) == 0   # no rows: nothing to write
    assert L.zt_matmul(NULL, NULL, NULL, 3, 5, 0, NULL) == 0
    assert L.zt_matmul(NULL, NULL, NULL, 3, 5, 2, NULL) == 1 and "null" in capfd.readouterr().err
    assert L.zt_weight_grad(NULL, NULL, NULL, 4, -2, 3, NULL) == 1
    assert L.zt_input_grad(NULL, NULL, NULL, 4, 3, 0, NULL) == 0


def test_decode_refuses_misaligned_rows(zt, capfd):
    # dim % 4 == 0 rows are read 16 bytes at a time; dim % 4 == 2 rows 8 at a time.
    L = zt.lib()
    nk = (ctypes.c_int * 2)(5, 8)
    ws = L.zt_attn_decode_workspace(2, 8, 4, 2, 32)
    good, off8 = 0x10000, 0x10008
    assert L.zt_attn_decode(good, off8, good, good, nk, 2, 8, 4, 2, 32, good, ws, NULL) == 1
    assert "not 16-byte aligned" in capfd.readouterr().err
    ws34 = L.zt_attn_decode_workspace(2, 8, 4, 2, 34)
    assert L.zt_attn_decode(good, good, good, 0x10004, nk, 2, 8, 4, 2, 34, good, ws34, NULL) == 1
    assert "not 8-byte aligned" in capfd.readouterr().err


def test_decode_step_refusals(zt, capfd):
    L = zt.lib()
    B, n_ctx, H, Hkv, D = 2, 8, 4, 2, 32
    ws = L.zt_attn_decode_step_workspace(B, n_ctx, H, Hkv, D)
    assert ws >= L.zt_attn_decode_workspace(B, n_ctx, H, Hkv, D) + B * H * D * 4
    p = 0x10000

    def step(pos, theta=5e5, wsb=ws, kc=p, dim=D):
        arr = (ctypes.c_int * B)(*pos)
        return L.zt_attn_decode_step(p, p, p, kc, p, p, arr, B, n_ctx, H, Hkv, dim, ctypes.c_double(theta), p, wsb,
                                     NULL)

    assert step([3, 8]) == 1 and "position 8, outside the 8-row cache" in capfd.readouterr().err
    assert step([-1, 0]) == 1 and "position -1" in capfd.readouterr().err
    assert step([1, 2], theta=0.0) == 1 and "theta" in capfd.readouterr().err
    assert step([1, 2], wsb=ws - 1) == 1 and "workspace" in capfd.readouterr().err
    assert step([1, 2], kc=p + 8) == 1 and "aligned" in capfd.readouterr().err
    assert step([1, 2], dim=31) == 1 and "head_dim 31" in capfd.readouterr().err
    assert L.zt_attn_decode_step_workspace(0, n_ctx, H, Hkv, D) == 0


@pytest.mark.parametrize("fn", ["zt_rope_qk_forward", "zt_rope_qk_backward"])
def test_rope_qk_refusals(zt, capfd, fn):
    f = getattr(zt.lib(), fn)
    p = 0x10000
    assert f(p, p, p, p, 1, 4, 4, 2, 3, 0, ctypes.c_double(5e5), NULL) == 1
    assert "head_dim 3" in capfd.readouterr().err
    assert f(p, p, p, p, -1, 4, 4, 2, 8, 0, ctypes.c_double(5e5), NULL) == 1
    assert f(p, p, p, p, 1, 4, 4, 2, 8, -2, ctypes.c_double(5e5), NULL) == 1
    assert f(p, p, p, p, 1, 4, 4, 2, 8, 0, ctypes.c_double(0.0), NULL) == 1
    assert "theta" in capfd.readouterr().err
    assert f(p, NULL, p, p, 1, 4, 4, 2, 8, 0, ctypes.c_double(5e5), NULL) == 1
    assert "null" in capfd.readouterr().err
    assert f(NULL, NULL, NULL, NULL, 0, 4, 4, 2, 8, 0, ctypes.c_double(5e5), NULL) == 0  # no rows


@pytest.mark.parametrize("fn", ["zt_rope_forward", "zt_rope_backward"])
def test_rope_refusals(zt, fn):
    f = getattr(zt.lib(), fn)
    assert f(NULL, NULL, 1, 3, 0, 5e5, 3, NULL) == 1
    assert f(NULL, NULL, 1, 6, 0, 5e5, 4, NULL) == 1
    assert f(NULL, NULL, 1, 0, 0, 5e5, 0, NULL) == 1
    assert f(NULL, NULL, 0, 8, 0, 5e5, 4, NULL) == 0  # zero rows: nothing to launch


# ------------------------------------------- holder (src/cuda/device.zig) --

def _bytes_for(zt, kind, *shape):
    out = ctypes.c_size_t(0)
    rc = zt.lib().zt_bytes_for(kind, *shape, ctypes.byref(out))
    return rc, out.value


def test_holder_sizes_at_the_shipped_shape(zt, golden):
    g = golden["holder_bytes"]
    t, h, kvh, d = g["shape"]
    assert _bytes_for(zt, zt.ZT_QUERY_HEADED, t, h, kvh, d) == (0, g["query_headed"])
    assert _bytes_for(zt, zt.ZT_KV_HEADED, t, h, kvh, d) == (0, g["kv_headed"])
    assert _bytes_for(zt, zt.ZT_PER_ROW, t, h, kvh, d) == (0, g["per_row"])
    assert 4 * g["query_headed"] + 4 * g["kv_headed"] + 3 * g["per_row"] == g["total"]
    # dk and dv across the four layers equal the KV cache scale.zig costs (device.zig:509-530)
    assert 2 * 4 * g["kv_headed"] == g["kv_cache_total"]


def test_holder_degenerate_and_overflow(zt):
    for shape in [(0, 4, 2, 32), (256, 0, 2, 32), (256, 4, 2, 0), (256, 4, 0, 32)]:
        assert _bytes_for(zt, zt.ZT_PER_ROW if shape[2] == 0 else zt.ZT_QUERY_HEADED, *shape)[0] == \
            zt.ZT_DEGENERATE_SHAPE
    big = 2 ** 64 - 1
    assert _bytes_for(zt, zt.ZT_QUERY_HEADED, big, 4, 2, 32)[0] == zt.ZT_SHAPE_TOO_LARGE
    assert _bytes_for(zt, zt.ZT_QUERY_HEADED, 1 << 40, 1 << 40, 1, 1)[0] == zt.ZT_SHAPE_TOO_LARGE
    assert _bytes_for(zt, zt.ZT_KV_HEADED, big, 4, 2, 32)[0] == zt.ZT_SHAPE_TOO_LARGE
    v = ctypes.c_int(0)
    assert zt.lib().zt_to_cint(1 << 31, ctypes.byref(v)) == zt.ZT_SHAPE_TOO_LARGE
    assert zt.lib().zt_to_cint(256, ctypes.byref(v)) == 0 and v.value == 256
    assert zt.lib().zt_to_cint(2 ** 31 - 1, ctypes.byref(v)) == 0 and v.value == 2 ** 31 - 1


def test_holder_forward_bounds(zt, golden):
    g = golden["forward_bounds"]
    for q_offset, n_keys, t in g["accept"]:
        assert zt.lib().zt_forward_bounds(g["c_t"], q_offset, n_keys, t) == 0
    for q_offset, n_keys, t in g["refuse"]:
        assert zt.lib().zt_forward_bounds(g["c_t"], q_offset, n_keys, t) == zt.ZT_SHAPE_TOO_LARGE


def test_holder_init_refuses_before_allocating(zt):
    h = ctypes.c_void_p()
    L = zt.lib()
    assert L.zt_holder_init(8, 4, 2, 30, ctypes.byref(h)) == zt.ZT_CONFIG_REFUSED   # width
    assert L.zt_holder_init(8, 3, 2, 32, ctypes.byref(h)) == zt.ZT_CONFIG_REFUSED   # group
    assert L.zt_holder_init(8, 65536, 1, 32, ctypes.byref(h)) == zt.ZT_CONFIG_REFUSED
    assert L.zt_holder_init(1 << 31, 4, 2, 32, ctypes.byref(h)) == zt.ZT_SHAPE_TOO_LARGE
    assert h.value is None


def test_tuning_variables_are_set_only_through_the_setter(zt, capfd):
    """Kernel variants follow the shape unless zt_attn_set_tuning forces one;
    unknown names and values outside a variable's admitted set are refused,
    and -1 returns a variable to its shape rule."""
    L = zt.lib()
    assert L.zt_attn_get_tuning(b"ZT_ATTN_BPAIR") == -1
    assert L.zt_attn_set_tuning(b"ZT_ATTN_BPAIR", 0) == 0
    assert L.zt_attn_get_tuning(b"ZT_ATTN_BPAIR") == 0
    assert L.zt_attn_set_tuning(b"ZT_ATTN_BPAIR", 2) == 1
    assert "not a value of the tuning variable ZT_ATTN_BPAIR" in capfd.readouterr().err
    assert L.zt_attn_get_tuning(b"ZT_ATTN_BPAIR") == 0
    assert L.zt_attn_set_tuning(b"ZT_ATTN_BPAIR", -1) == 0
    assert L.zt_attn_get_tuning(b"ZT_ATTN_BPAIR") == -1
    assert L.zt_attn_set_tuning(b"ZT_NO_SUCH_KNOB", 1) == 1
    assert "is not a tuning variable" in capfd.readouterr().err
    assert L.zt_attn_get_tuning(b"ZT_NO_SUCH_KNOB") == -2
    assert L.zt_attn_set_tuning(None, 1) == 1
    assert L.zt_attn_set_tuning(b"ZT_DEC_WGS", 32768) == 0 and L.zt_attn_get_tuning(b"ZT_DEC_WGS") == 32768
    assert L.zt_attn_set_tuning(b"ZT_DEC_WGS", -1) == 0


def test_library_reads_no_environment_variable(zt):
    """No getenv reaches a launch: the shared object does not import it."""
    import subprocess
    out = subprocess.run(["nm", "-D", "--undefined-only", zt.LIB_PATH], capture_output=True, text=True,
                         check=True).stdout
    assert "getenv" not in out


def test_train_workspace_holds_only_the_causal_tiles(zt):
    """B * H * nt (nt + 1) / 2 tiles of 16 x 16 after delta (1.0 GiB at C3, not 2)."""
    for B, T, H, Hkv, D in ((1, 4096, 32, 8, 128), (2, 2048, 16, 4, 256), (1, 33, 4, 2, 32)):
        nt = (T + 15) // 16
        delta = (B * T * H * 4 + 255) // 256 * 256
        assert zt.backward_train_workspace_bytes(B, T, H, Hkv, D) == delta + B * H * nt * (nt + 1) // 2 * 1024
    assert zt.backward_train_workspace_bytes(1, 4096, 32, 8, 128) < 1.1 * 2 ** 30
