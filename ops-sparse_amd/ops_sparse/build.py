"""Compiles libaclsparse_hip.so for gfx950 with hipcc (in-tree, no JIT cache)."""
import os
import subprocess

_HERE = os.path.dirname(os.path.abspath(__file__))
PKG_ROOT = os.path.dirname(_HERE)
REPO_ROOT = os.path.dirname(PKG_ROOT)
CSRC = os.path.join(PKG_ROOT, "csrc")
SOURCES = ["handle_descr.cpp", "spmv_host.cpp", "spmv_kernels.hip", "spmv_op_host.cpp", "spmv_op_kernels.hip",
           "spmm_op_host.cpp", "spmm_op_kernels.hip"]
OUT = os.path.join(PKG_ROOT, "lib", "libaclsparse_hip.so")

HIPCC_FLAGS = [
    "-std=c++17", "-O3", "--offload-arch=gfx950", "-fPIC", "-shared",
    # keep the compiler from forming packed-fp32 instructions
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall",
]


def build_library(verbose=False):
    os.makedirs(os.path.dirname(OUT), exist_ok=True)
    srcs = [os.path.join(CSRC, s) for s in SOURCES if os.path.exists(os.path.join(CSRC, s))]
    cmd = ["hipcc", *HIPCC_FLAGS, "-I" + os.path.join(REPO_ROOT, "include"), *srcs, "-o", OUT + ".tmp"]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError("hipcc failed:\n" + res.stdout + res.stderr)
    os.replace(OUT + ".tmp", OUT)
    if verbose:
        print(" ".join(cmd))
    return OUT


if __name__ == "__main__":
    print(build_library(verbose=True))
