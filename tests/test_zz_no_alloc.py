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
    ("zipf_then_laplacian", lambda: wl.zipf_rows(rows=1 << 20, mean=16.0, cap=20000),
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
