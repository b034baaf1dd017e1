"""Build recipe for bramha_amd/libbramha_hip.so (gfx950, in-tree).

Every source is compiled with hipcc for gfx950 only, in parallel, then linked into
one shared library that exports the C ABI of include/bramha_hip.h.
Run: python bramha_amd/build.py   (by path: importing the package loads the library).
"""
import os
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
LIB = os.path.join(HERE, "libbramha_hip.so")
OBJ_DIR = os.path.join(ROOT, "_build", "bramha_amd")
SOURCES = [
    "csrc/k_gemv.hip",
    "csrc/k_gemm.hip",
    "csrc/k_prefill.hip",
    "csrc/k_lmhead.hip",
    "csrc/k_attn.hip",
    "csrc/k_attn_o.hip",
    "csrc/k_ops.hip",
    "csrc/k_probe.hip",
    "csrc/bh_host.cpp",
    "csrc/bh_api.cpp",
    "csrc/bh_model.cpp",
    "csrc/bh_loader.cpp",
]
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
FLAGS = [
    "--offload-arch=gfx950",
    "-O3",
    "-fPIC",
    "-std=c++17",
    "-Wall",
    "-Wno-unused-result",
    # packed fp32 VALU ops stay off on this target (the host pass warns that it
    # does not know the feature; that is expected)
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-I" + os.path.join(ROOT, "include"),
]


def _compile(src):
    path = os.path.join(HERE, src)
    obj = os.path.join(OBJ_DIR, os.path.basename(src) + ".o")
    cmd = [HIPCC, "-x", "hip", "-c", path, "-o", obj] + FLAGS
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError("hipcc failed for %s:\n%s" % (src, r.stderr[-6000:]))
    return obj


def build(verbose=False):
    os.makedirs(OBJ_DIR, exist_ok=True)
    with ThreadPoolExecutor(max_workers=min(8, len(SOURCES))) as ex:
        objs = list(ex.map(_compile, SOURCES))
    tmp = LIB + ".tmp"
    cmd = [HIPCC, "-shared", "-o", tmp] + objs + ["--offload-arch=gfx950", "-fPIC"]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError("link failed:\n" + r.stderr[-6000:])
    os.replace(tmp, LIB)
    if verbose:
        print("built", LIB)
    return LIB


if __name__ == "__main__":
    build(verbose=True)
    sys.exit(0)
