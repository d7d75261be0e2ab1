"""Build libtao_hip.so (gfx950) in-tree with hipcc.

Usage: python tao-memory_amd/build.py  (or __graft_entry__.build()).
Compiles every csrc/*.hip to an object and links the shared library into
tao_attention/_lib/, where the Python host loads it with ctypes.
"""

import os
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
OUT_DIR = os.path.join(HERE, "tao_attention", "_lib")
LIB = os.path.join(OUT_DIR, "libtao_hip.so")
OBJ_DIR = os.path.join(HERE, "_build")

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"
FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-fPIC", "-std=c++17",
    # Reproducible fp32 arithmetic: no implicit FMA contraction (kernels
    # call fmaf where they want a fused multiply-add).
    "-ffp-contract=off",
    # Keep the compiler from forming packed fp32 ops.
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Wno-unused-function",
]


def sources():
    return sorted(os.path.join(CSRC, f) for f in os.listdir(CSRC) if f.endswith(".hip"))


def _compile(src):
    obj = os.path.join(OBJ_DIR, os.path.basename(src)[:-4] + ".o")
    cmd = [HIPCC, *FLAGS, "-c", src, "-o", obj]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode:
        raise RuntimeError(f"hipcc failed for {src}:\n{proc.stderr}")
    return obj


FAST_SRC = os.path.join(CSRC, "host", "tao_fast.cpp")


def fast_path():
    import sysconfig
    return os.path.join(OUT_DIR, "_tao_fast" + sysconfig.get_config_var("EXT_SUFFIX"))


def build_fast(verbose=True):
    """Host-only torch extension for the per-token decode call (g++)."""
    import sysconfig
    import torch
    from torch.utils import cpp_extension
    out = fast_path()
    abi = int(torch._C._GLIBCXX_USE_CXX11_ABI)
    cmd = [os.environ.get("CXX", "g++"), "-O2", "-shared", "-fPIC", "-std=c++17",
           f"-D_GLIBCXX_USE_CXX11_ABI={abi}", "-DTORCH_EXTENSION_NAME=_tao_fast",
           "-DTORCH_API_INCLUDE_EXTENSION_H",
           *[f"-I{p}" for p in cpp_extension.include_paths()],
           f"-I{sysconfig.get_paths()['include']}",
           FAST_SRC, "-o", out + ".tmp",
           *[f"-L{p}" for p in cpp_extension.library_paths()],
           "-lc10", "-ltorch", "-ltorch_cpu", "-ltorch_python"]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode:
        raise RuntimeError(f"g++ failed for {FAST_SRC}:\n{proc.stderr[-4000:]}")
    os.replace(out + ".tmp", out)
    if verbose:
        print(f"built {out}")
    return out


def build(verbose=True):
    os.makedirs(OUT_DIR, exist_ok=True)
    os.makedirs(OBJ_DIR, exist_ok=True)
    srcs = sources()
    with ThreadPoolExecutor(max_workers=min(8, len(srcs))) as pool:
        objs = list(pool.map(_compile, srcs))
    tmp = LIB + ".tmp"
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp, *objs]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode:
        raise RuntimeError(f"link failed:\n{proc.stderr}")
    os.replace(tmp, LIB)
    if verbose:
        print(f"built {LIB} from {len(srcs)} sources")
    build_fast(verbose)
    return LIB


if __name__ == "__main__":
    build()
    sys.exit(0)
