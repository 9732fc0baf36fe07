"""The reference-side binding (integration/zig_mi355x.patch) against the
reference tree: it applies (`git apply --check` on a copy of the four files it
touches), it leaves no CUDA runtime call behind in device.zig, and the entry
points it links are the ones this library exports.  Needs the reference tree
(read only, copied to a temporary directory); skipped where it is absent."""
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

needs_reference = pytest.mark.skipif(not os.path.isdir(REFERENCE) or shutil.which("git") is None,
                                     reason="the reference tree or git is absent")


def _patched_files(patch_text):
    return sorted(set(re.findall(r"^\+\+\+ b/(\S+)$", patch_text, re.M)))


def test_the_patch_touches_exactly_the_binding_files():
    text = open(PATCH).read()
    assert _patched_files(text) == sorted(FILES)


@needs_reference
def test_the_patch_applies_to_the_reference_tree(tmp_path):
    for f in FILES:
        dst = tmp_path / f
        dst.parent.mkdir(parents=True, exist_ok=True)
        shutil.copyfile(os.path.join(REFERENCE, f), dst)
    r = subprocess.run(["git", "apply", "--check", "-v", PATCH], cwd=tmp_path, capture_output=True, text=True)
    assert r.returncode == 0, r.stderr
    subprocess.run(["git", "apply", PATCH], cwd=tmp_path, check=True, capture_output=True)
    device = (tmp_path / "src/cuda/device.zig").read_text()
    code = "\n".join(line.split("//")[0] for line in device.splitlines())
    assert not re.search(r"\bcuda(Malloc|Free|Memcpy)\s*\(", code)
    for fn in ("hipMalloc", "hipFree", "hipMemcpy"):
        assert f"pub extern fn {fn}(" in device
    build = (tmp_path / "build.zig").read_text()
    assert 'linkSystemLibrary("zt_attn"' in build and 'linkSystemLibrary("amdhip64"' in build
    step = build.split("fn cudaAttnObject")[1].split("\n}\n")[0]
    assert "nvcc $flags" not in step and "z-transformer_amd/build.py" in step


@needs_reference
def test_every_entry_point_device_zig_binds_is_exported():
    """device.zig's own externs (unchanged by the patch) name symbols of the
    C ABI this library declares."""
    device = open(os.path.join(REFERENCE, "src/cuda/device.zig")).read()
    names = set(re.findall(r"pub extern fn (zt_\w+)\(", device))
    assert names
    header = open(os.path.join(REPO, "include", "zt_attn.h")).read()
    for n in names:
        assert re.search(rf"\b{n}\s*\(", header), n
