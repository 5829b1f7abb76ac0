"""Compiles libaclsparse_hip.so for gfx950 with hipcc (in-tree, no JIT cache).

The library carries a build id: a SHA-256 over the native sources, the public
header and the compiler flags, exported as ``aclsparseHipBuildId()``.  The
loader (``_lib.lib``) recomputes it from the source tree and refuses a
library built from other sources, so a stale binary cannot be tested or
benchmarked by mistake.
"""
import hashlib
import os
import subprocess

_HERE = os.path.dirname(os.path.abspath(__file__))
PKG_ROOT = os.path.dirname(_HERE)
REPO_ROOT = os.path.dirname(PKG_ROOT)
CSRC = os.path.join(PKG_ROOT, "csrc")
HEADER = os.path.join(REPO_ROOT, "include", "cann_ops_sparse.h")
SOURCES = ["handle_descr.cpp", "spmv_host.cpp", "spmv_kernels.hip", "spmv_staged_kernels.hip", "spmv_op_host.cpp",
           "spmv_op_kernels.hip", "spmm_op_host.cpp", "spmm_op_kernels.hip", "spmv_noalloc.hip"]
OUT = os.path.join(PKG_ROOT, "lib", "libaclsparse_hip.so")
OBJ_DIR = os.path.join(PKG_ROOT, "lib", "obj")

HIPCC_FLAGS = [
    "-std=c++17", "-O3", "--offload-arch=gfx950", "-fPIC", "-shared",
    # keep the compiler from forming packed-fp32 instructions
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall",
]


def _inputs():
    """Every file whose content goes into the library: the csrc tree (sources and
    private headers, sorted by name) and the public header."""
    names = sorted(n for n in os.listdir(CSRC) if n.endswith((".cpp", ".hip", ".h")))
    return [os.path.join(CSRC, n) for n in names] + [HEADER]


def source_hash():
    """Build id of the current source tree: SHA-256 over file names, contents and flags."""
    h = hashlib.sha256()
    for path in _inputs():
        h.update(os.path.basename(path).encode() + b"\0")
        with open(path, "rb") as f:
            h.update(f.read())
        h.update(b"\0")
    h.update(" ".join(HIPCC_FLAGS).encode())
    return h.hexdigest()[:32]


BUILD_ID_PREFIX = b"aclsparse-hip-build-id:"


def file_build_id(path):
    """Build id stored in a library file (None when the file is missing or has none)."""
    if not os.path.exists(path):
        return None
    with open(path, "rb") as f:
        data = f.read()
    i = data.find(BUILD_ID_PREFIX)
    if i < 0:
        return None
    j = i + len(BUILD_ID_PREFIX)
    return data[j:j + 32].decode(errors="replace")


def build_library(verbose=False):
    """Compiles every source to an object in parallel (ops-sparse_amd/lib/obj), then links."""
    from concurrent.futures import ThreadPoolExecutor

    os.makedirs(OBJ_DIR, exist_ok=True)
    bid = source_hash()
    compile_flags = [f for f in HIPCC_FLAGS if f != "-shared"]
    cmds = []
    for src in SOURCES:
        obj = os.path.join(OBJ_DIR, os.path.splitext(src)[0] + ".o")
        cmds.append(["hipcc", *compile_flags, f"-DACLSPARSE_HIP_BUILD_ID=\"{bid}\"",
                     "-I" + os.path.join(REPO_ROOT, "include"), "-c", os.path.join(CSRC, src), "-o", obj])

    def run(cmd):
        res = subprocess.run(cmd, capture_output=True, text=True)
        if res.returncode != 0:
            raise RuntimeError("hipcc failed:\n" + " ".join(cmd) + "\n" + res.stdout + res.stderr)
        return cmd

    with ThreadPoolExecutor(max_workers=min(len(cmds), 8)) as ex:
        for cmd in ex.map(run, cmds):
            if verbose:
                print(" ".join(cmd))
    link = ["hipcc", *HIPCC_FLAGS, *[c[-1] for c in cmds], "-o", OUT + ".tmp"]
    run(link)
    os.replace(OUT + ".tmp", OUT)
    if verbose:
        print(" ".join(link))
    return OUT


if __name__ == "__main__":
    print(build_library(verbose=True))
