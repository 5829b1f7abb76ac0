"""aclsparseSpMVNoAlloc (the entry point that allocates nothing) against aclsparseSpMV, through the C ABI.

The no-alloc entry point runs the same row kernels (or transpose path) on
tables it rebuilds in a static device array, so its result must be bit-identical
to aclsparseSpMV's on the same inputs (matrices here are below the staged
path's size, where aclsparseSpMV runs the same kernels).  Consecutive calls
share the array: each case calls it twice, the second time on a smaller
matrix, and checks both results.
"""
import ctypes

import pytest
import torch

from helpers import assert_close
from ops_sparse import _lib
from ops_sparse._lib import Operation, Status
from ops_sparse.spmv import CsrSpMV
from ops_sparse import workloads as wl

pytestmark = pytest.mark.gpu

MAX_BYTES = 32 * 1024 * 1024
OP = {"N": Operation.NON_TRANSPOSE, "T": Operation.TRANSPOSE, "H": Operation.CONJUGATE_TRANSPOSE}


def no_alloc(plan):
    lib = _lib.lib()
    return Status(lib.aclsparseSpMVNoAlloc(plan.handle.h, int(plan.op), plan.alpha.ptr, plan.mat.d, plan.x.d,
                                           plan.beta.ptr, plan.y.d, int(plan.compute_type), int(plan.alg)))


def both(w, dev):
    """(y from aclsparseSpMV, y from aclsparseSpMVNoAlloc) for workload w, same initial y."""
    w = w.to(dev)
    y_ref = w.y0.to(w.out_dtype).clone()
    y_na = w.y0.to(w.out_dtype).clone()
    ref = CsrSpMV(w.rows, w.cols, w.row_ptr, w.col_ind, w.values, w.x, y_ref, w.alpha, w.beta, op=OP[w.trans])
    ref.run()
    na = CsrSpMV(w.rows, w.cols, w.row_ptr, w.col_ind, w.values, w.x, y_na, w.alpha, w.beta, op=OP[w.trans])
    st = no_alloc(na)
    torch.cuda.synchronize()
    assert st == Status.SUCCESS
    return w, y_ref, y_na


def bits(y):
    return y.view(torch.int16) if y.element_size() == 2 else y.view(torch.int32) if y.element_size() == 4 else y.view(torch.int64)


CASES = [
    # (first workload, second smaller workload)
    ("laplacian_then_uniform", lambda: wl.laplacian_2d(n=1024), lambda: wl.c1_uniform41(rows=3000, cols=5000)),
    ("zipf_then_laplacian", lambda: wl.zipf_rows(rows=1 << 19, mean=16.0, cap=20000),
     lambda: wl.laplacian_2d(n=300)),
    ("transpose_then_smaller", lambda: wl.poisson_transpose(rows=1 << 16),
     lambda: wl.poisson_transpose(rows=1 << 12, seed=7)),
    ("fp16_i64_then_bf16", lambda: wl.uniform_rows_lowp(rows=1 << 18, per_row=32, dtype=torch.float16),
     lambda: wl.uniform_rows_lowp(rows=1 << 12, per_row=7, dtype=torch.bfloat16)),
]


@pytest.mark.parametrize("case", CASES, ids=[c[0] for c in CASES])
def test_no_alloc_matches_spmv_twice(case, dev):
    _, first, second = case
    for make in (first, second):
        w, y_ref, y_na = both(make(), dev)
        assert torch.equal(bits(y_ref), bits(y_na)), f"{w.name}: no-alloc result differs from aclsparseSpMV"
        assert_close(w.to("cpu"), y_na)


def test_no_alloc_rejects_tables_beyond_the_array(dev):
    """Normalised row offsets alone exceed the array: INSUFFICIENT_RESOURCES, y untouched."""
    rows = MAX_BYTES // 4 + 1024
    row_ptr = torch.zeros(rows + 1, dtype=torch.int32, device=dev)
    row_ptr[-1] = 1  # one entry, in the last row
    col = torch.zeros(1, dtype=torch.int32, device=dev)
    val = torch.zeros(1, dtype=torch.float32, device=dev)
    x = torch.ones(16, dtype=torch.float32, device=dev)
    y = torch.full((rows,), 3.0, dtype=torch.float32, device=dev)
    plan = CsrSpMV(rows, 16, row_ptr, col, val, x, y, 1.0, 0.0)
    assert no_alloc(plan) == Status.INSUFFICIENT_RESOURCES
    torch.cuda.synchronize()
    assert bool((y == 3.0).all())


def test_no_alloc_zero_rows_and_after_rejection(dev):
    """An empty matrix is a no-op; a normal call after a rejected one still matches aclsparseSpMV."""
    row_ptr = torch.zeros(1, dtype=torch.int32, device=dev)
    col = torch.zeros(0, dtype=torch.int32, device=dev)
    val = torch.zeros(0, dtype=torch.float32, device=dev)
    x = torch.ones(8, dtype=torch.float32, device=dev)
    y = torch.zeros(1, dtype=torch.float32, device=dev)
    plan = CsrSpMV(0, 8, row_ptr, col, val, x, y[:0], 1.0, 0.0)
    assert no_alloc(plan) == Status.SUCCESS
    w, y_ref, y_na = both(wl.laplacian_2d(n=64), dev)
    assert torch.equal(bits(y_ref), bits(y_na))


def test_no_alloc_calls_captured_in_a_hip_graph(dev):
    """Two aclsparseSpMVNoAlloc calls (an fp32 Laplacian, then a smaller transpose) captured on a side
    stream into one HIP graph after a warm call: every replay, with eager work and synchronisations
    between the replays, is bit-identical to aclsparseSpMV on the same inputs."""
    w1 = wl.laplacian_2d(n=512).to(dev)
    w2 = wl.poisson_transpose(rows=1 << 14, seed=11).to(dev)
    refs, plans, ys = [], [], []
    for w in (w1, w2):
        _, y_ref, _ = both(w, dev)  # also the warm call of the no-alloc entry point
        refs.append(y_ref)
    s = torch.cuda.Stream()
    torch.cuda.synchronize()
    with torch.cuda.stream(s):
        for w in (w1, w2):
            y = w.y0.to(w.out_dtype).clone()
            plans.append(CsrSpMV(w.rows, w.cols, w.row_ptr, w.col_ind, w.values, w.x, y, w.alpha, w.beta,
                                 op=OP[w.trans]))
            ys.append(y)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        for p in plans:
            assert no_alloc(p) == Status.SUCCESS
    for _ in range(3):
        for w, y in zip((w1, w2), ys):
            y.copy_(w.y0.to(w.out_dtype))
        torch.cuda.synchronize()
        with torch.cuda.stream(s):
            g.replay()
        torch.cuda.synchronize()
        for y, r in zip(ys, refs):
            assert torch.equal(bits(y), bits(r))
        both(wl.laplacian_2d(n=100), dev)  # eager no-alloc work on the same array between replays


_FIRST_CALL_UNDER_CAPTURE = r"""
import sys, torch
sys.path[:0] = {paths!r}
from ops_sparse import _lib
from ops_sparse._lib import Status
from ops_sparse.spmv import CsrSpMV
from ops_sparse import workloads as wl
dev = torch.device("cuda:0")
w = wl.laplacian_2d(n=256).to(dev)
s = torch.cuda.Stream()
y = w.y0.clone()
y_ref = w.y0.clone()
torch.cuda.synchronize()
with torch.cuda.stream(s):
    plan = CsrSpMV(w.rows, w.cols, w.row_ptr, w.col_ind, w.values, w.x, y, w.alpha, w.beta)
    ref = CsrSpMV(w.rows, w.cols, w.row_ptr, w.col_ind, w.values, w.x, y_ref, w.alpha, w.beta)
    ref.run()
torch.cuda.synchronize()
lib = _lib.lib()
g = torch.cuda.CUDAGraph()
with torch.cuda.graph(g, stream=s):  # the process's first no-alloc call: resolves the array's address
    st = lib.aclsparseSpMVNoAlloc(plan.handle.h, 0, plan.alpha.ptr, plan.mat.d, plan.x.d, plan.beta.ptr,
                                  plan.y.d, int(plan.compute_type), int(plan.alg))
assert Status(st) == Status.SUCCESS, st
for _ in range(2):
    y.copy_(w.y0)
    torch.cuda.synchronize()
    with torch.cuda.stream(s):
        g.replay()
    torch.cuda.synchronize()
    assert torch.equal(y.view(torch.int32), y_ref.view(torch.int32))
print("first-call-under-capture ok")
"""


def test_no_alloc_first_call_made_under_capture(dev):
    """A process whose very first aclsparseSpMVNoAlloc call is made while its stream is being captured:
    the address lookup of the static array is a host-side query, legal under capture, and the graph
    replays correctly (run in a fresh process, since this one has already called the entry point)."""
    import os
    import subprocess
    import sys

    here = os.path.dirname(os.path.abspath(__file__))
    repo = os.path.dirname(here)
    paths = [os.path.join(repo, "ops-sparse_amd"), os.path.join(repo, "oracle"), repo]
    code = _FIRST_CALL_UNDER_CAPTURE.replace("{paths!r}", repr(paths))
    r = subprocess.run([sys.executable, "-c", code], capture_output=True, text=True, timeout=240)
    assert r.returncode == 0, r.stdout[-2000:] + r.stderr[-4000:]
    assert "first-call-under-capture ok" in r.stdout
