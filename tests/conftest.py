"""Shared fixtures.  `gpu`-marked tests need an MI355X; everything else runs on
the CPU.  The HIP binding and the oracle are loaded by path (the package
directory name is not an importable identifier)."""
import importlib.util
import json
import os

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a gfx950 GPU (MI355X)")


def load_module(name, path):
    spec = importlib.util.spec_from_file_location(name, path)
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


@pytest.fixture(scope="session")
def zt():
    return load_module("zt_attn", os.path.join(ROOT, "z-transformer_amd", "zt_attn.py"))


@pytest.fixture(scope="session")
def oracle():
    return load_module("zt_oracle", os.path.join(ROOT, "oracle", "zt_oracle.py"))


@pytest.fixture(scope="session")
def golden():
    with open(os.path.join(ROOT, "tests", "golden", "reference_known_answers.json")) as f:
        return json.load(f)


@pytest.fixture(scope="session")
def gpu(zt):
    """A GPU session: torch on cuda:0 and the HIP library loaded.  Fails (does
    not skip) when a GPU is present but the library is missing."""
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no GPU in this container")
    zt.lib()  # raises if libzt_attn.so is not built
    assert zt.lib().zt_attn_lds_limit() > 0, "libzt_attn found no usable gfx950 device"
    return torch


@pytest.fixture
def tune(zt):
    """Forces kernel variants for one test through the library's tuning
    variables (zt_attn_set_tuning) and returns every one it set to the shape
    rule afterwards.  Call as tune({"ZT_ATTN_BPAIR": 1, ...})."""
    touched = []

    def apply(settings):
        for name, value in settings.items():
            zt.set_tuning(name, int(value))
            touched.append(name)

    yield apply
    for name in touched:
        zt.set_tuning(name, -1)


@pytest.fixture(scope="session")
def threads():
    return min(16, os.cpu_count() or 1)
