"""Builds the planted-defect test libraries (TEST INFRASTRUCTURE ONLY).

Each entry of PLANTS compiles one kernel source with -DZT_PLANT=<n> (the
defect points in z-transformer_amd/csrc/kernels/common.h) -- for the forward
and backward sources only the kernels of the negative-control shapes (d = 32
for the reference entry points, d = 128 for the training path), for the dense
product and decode sources all of them -- and links it with the other,
unmodified code objects and the library's own host objects into
tests/planted/_build/<name>/libzt_attn.so.  tests/test_gpu_planted.py loads
each one and checks that its parity gate rejects it.  Nothing shipped loads
these libraries; the product library is built without ZT_PLANT.  Run after
z-transformer_amd/build.py (it reuses that build's objects).
"""
import importlib.util
import os
import sys
from concurrent.futures import ThreadPoolExecutor

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
OUT = os.path.join(HERE, "_build")

# name -> (ZT_PLANT value, code object it replaces)
PLANTS = {
    "fwd_mask": (1, "fwd"), "fwd_gqa": (2, "fwd"), "fwd_rescale": (3, "fwd"), "fwd_scale": (4, "fwd"),
    "bwd_mask": (11, "bwd"), "bwd_gqa": (12, "bwd"), "bwd_jacobian": (13, "bwd"), "bwd_scale": (14, "bwd"),
    "norm_weight": (21, "misc"), "norm_mean": (22, "misc"), "norm_tensor": (23, "misc"),
    # The training path's headline kernels and the decode combine.
    "train_fwd_scores": (5, "fwd"), "train_ds_tiles": (15, "bwd"), "train_dq_scale": (16, "gemm"),
    "decode_merge": (17, "dec"),
}


def _product_build():
    spec = importlib.util.spec_from_file_location("zt_build", os.path.join(ROOT, "z-transformer_amd", "build.py"))
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def lib_path(name):
    return os.path.join(OUT, name, "libzt_attn.so")


def build(verbose=False):
    pb = _product_build()
    kdir = os.path.join(ROOT, "z-transformer_amd", "csrc", "kernels")
    src_of = dict(pb.KERNELS)
    product = {tag: os.path.join(pb.BUILD, f"{tag}.hsaco") for tag, _ in pb.KERNELS}
    host = [os.path.join(pb.BUILD, o) for o in ("zt_attn.o", "zt_holder.o", "noalloc.o")]
    for path in list(product.values()) + host:
        if not os.path.exists(path):
            raise FileNotFoundError(f"{path} missing: run z-transformer_amd/build.py first")

    def one(item):
        name, (plant, tag) = item
        d = os.path.join(OUT, name)
        os.makedirs(d, exist_ok=True)
        co = pb.genco(os.path.join(kdir, src_of[tag]), os.path.join(d, f"{tag}.hsaco"), [f"ZT_PLANT={plant}"])
        return pb.link(lib_path(name), {**product, tag: co}, host, os.path.join(d, "co_embed.S"))

    with ThreadPoolExecutor(max_workers=min(8, len(PLANTS))) as ex:
        libs = list(ex.map(one, PLANTS.items()))
    if verbose:
        print(f"built {len(libs)} planted-defect test libraries under {OUT}")
    return libs


if __name__ == "__main__":
    build(verbose=True)
    sys.exit(0)
