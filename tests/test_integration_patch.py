"""The reference-side binding (integration/zig_mi355x.patch) against the
reference tree: it applies (`git apply --check` on a copy of the four files it
touches); device.zig's Attn keeps its API and Error set and forwards every call
to the holder's C ABI (include/zt_holder.h), with no CUDA runtime call and no
direct call of the stateless pair left; every extern the patched device.zig
declares is declared in include/ and exported by libzt_attn.so; autograd.zig's
device backward keeps one holder across calls and runs the holder's forward
then backward.  Needs the reference tree (read only, copied to a temporary
directory); skipped where it is absent.  The Zig itself cannot be compiled
here (no Zig toolchain in this image); tests/test_gpu_zig_seams.py replays the
exact C calls the patched code issues, on the GPU."""
import ctypes
import os
import re
import shutil
import subprocess

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
REPO = os.path.dirname(HERE)
PATCH = os.path.join(REPO, "integration", "zig_mi355x.patch")
REFERENCE = "/root/reference"
FILES = ["build.zig", "src/cuda/device.zig", "src/model.zig", "src/autograd.zig"]
LIB = os.path.join(REPO, "z-transformer_amd", "_build", "libzt_attn.so")

needs_reference = pytest.mark.skipif(not os.path.isdir(REFERENCE) or shutil.which("git") is None,
                                     reason="the reference tree or git is absent")


def _patched_files(patch_text):
    return sorted(set(re.findall(r"^\+\+\+ b/(\S+)$", patch_text, re.M)))


def _code(text):
    """Zig source without // comments (a comment may name what the code no longer does)."""
    return "\n".join(line.split("//")[0] for line in text.splitlines())


def _block(text, opener):
    """The body of the container that starts at `opener`, up to its closing `};` at column 0."""
    i = text.index(opener)
    j = text.index("\n};\n", i)
    return text[i:j]


def test_the_patch_touches_exactly_the_binding_files():
    text = open(PATCH).read()
    assert _patched_files(text) == sorted(FILES)


@pytest.fixture(scope="module")
def patched(tmp_path_factory):
    if not os.path.isdir(REFERENCE) or shutil.which("git") is None:
        pytest.skip("the reference tree or git is absent")
    d = tmp_path_factory.mktemp("ref")
    for f in FILES:
        dst = d / f
        dst.parent.mkdir(parents=True, exist_ok=True)
        shutil.copyfile(os.path.join(REFERENCE, f), dst)
    r = subprocess.run(["git", "apply", "--check", "-v", PATCH], cwd=d, capture_output=True, text=True)
    assert r.returncode == 0, r.stderr
    subprocess.run(["git", "apply", PATCH], cwd=d, check=True, capture_output=True)
    return {f: (d / f).read_text() for f in FILES}


@needs_reference
def test_device_zig_binds_the_holder_and_keeps_no_runtime_call(patched):
    device = patched["src/cuda/device.zig"]
    code = _code(device)
    assert not re.search(r"\bcuda(Malloc|Free|Memcpy)\s*\(", code)
    assert not re.search(r"\bhip(Malloc|Free|Memcpy)\s*\(", code)   # the holder allocates and copies
    for fn in ("init", "deinit", "buffer", "forward_at", "backward", "upload", "download"):
        assert f"pub extern fn zt_holder_{fn}(" in device
    attn = _code(_block(device, "pub const Attn = struct {"))
    # Every method goes through the holder; none calls the stateless pair.
    assert not re.search(r"\bzt_attn_(forward|backward)\s*\(", attn)
    for call in ("zt_holder_init(", "zt_holder_forward_at(", "zt_holder_backward(", "zt_holder_upload(",
                 "zt_holder_download(", "zt_holder_deinit("):
        assert call in attn, call
    # The API callers use is unchanged: the same public methods, the same Error set.
    for sig in ("pub fn init(t: usize, n_heads: usize, n_kv_heads: usize, dim: usize) Error!Attn",
                "pub fn deinit(self: *Attn) void", "pub fn totalBytes(self: *const Attn) usize",
                "pub fn forward(self: *const Attn, group_q: c_int, max_tile: c_int) Error!void",
                "pub fn backward(self: *const Attn, max_tile: c_int) Error!void",
                "pub fn upload(self: *const Attn, dst: [*]f32, src: []const f32) Error!void",
                "pub fn download(self: *const Attn, dst: []f32, src: [*]f32) Error!void"):
        assert sig in device, sig
    original = open(os.path.join(REFERENCE, "src/cuda/device.zig")).read()
    assert _block(device, "pub const Error = error{") == _block(original, "pub const Error = error{")
    # The holder's zt_error codes map onto Error in its order (include/zt_holder.h).
    hdr = open(os.path.join(REPO, "include", "zt_holder.h")).read()
    codes = dict((n, int(v)) for n, v in re.findall(r"ZT_(\w+) = (\d+)", hdr))
    mapping = dict((int(v), n) for v, n in re.findall(r"(\d) => Error\.(\w+)", device))
    assert mapping == {codes["DEGENERATE_SHAPE"]: "DegenerateShape", codes["SHAPE_TOO_LARGE"]: "ShapeTooLarge",
                       codes["CONFIG_REFUSED"]: "ConfigRefused", codes["DEVICE_ALLOC_FAILED"]: "DeviceAllocFailed"}
    assert "else => Error.DeviceTransferFailed" in device and codes["DEVICE_TRANSFER_FAILED"] == 5


@needs_reference
def test_every_extern_of_the_patched_device_zig_is_declared_and_exported(patched):
    names = set(re.findall(r"pub extern fn (zt_\w+)\(", patched["src/cuda/device.zig"]))
    assert {"zt_attn_forward", "zt_attn_backward", "zt_holder_init", "zt_holder_backward"} <= names
    headers = "".join(open(os.path.join(REPO, "include", h)).read() for h in ("zt_attn.h", "zt_holder.h"))
    for n in names:
        assert re.search(rf"\b{n}\s*\(", headers), n
    if not os.path.exists(LIB):
        pytest.skip("libzt_attn.so is not built")
    lib = ctypes.CDLL(LIB)
    for n in names:
        assert hasattr(lib, n), n


@needs_reference
def test_device_backward_keeps_one_holder_and_runs_its_forward_then_backward(patched):
    auto = patched["src/autograd.zig"]
    fn = _code(auto[auto.index("fn deviceAttentionBackward("):auto.index("pub fn deinitDeviceBackward")])
    assert "var bwd_dev: ?model.device.Attn = null;" in auto
    assert fn.count("Attn.init(") == 1 and "if (bwd_dev == null)" in fn
    order = [fn.index(s) for s in ("a.upload(a.q", "a.upload(a.k", "a.upload(a.v", "a.upload(a.dout",
                                   "a.forward(1, 64)", "a.backward(64)", "a.download(dq.data, a.dq)",
                                   "a.download(dk.data, a.dk)", "a.download(dv.data, a.dv)")]
    assert order == sorted(order)
    block = auto[auto.index("fn blockBackward("):auto.index("pub const AttnGrads")]
    assert "if (comptime model.cuda_attn)\n        try deviceAttentionBackward(" in block


@needs_reference
def test_build_links_the_mi355x_library(patched):
    build = patched["build.zig"]
    assert 'linkSystemLibrary("zt_attn"' in build
    step = build.split("fn cudaAttnObject")[1].split("\n}\n")[0]
    assert "nvcc $flags" not in step and "z-transformer_amd/build.py" in step
    assert "pub const device = @import(\"cuda/device.zig\");" in patched["src/model.zig"]
