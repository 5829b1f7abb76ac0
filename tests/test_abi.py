"""CPU checks of the C ABI: the library loads, exports every function the
public header declares, and the host-side entry points (handle, descriptors,
argument validation) return the reference's status codes.  No call here
reaches a kernel launch: every SpMV/SpMVOp call either fails validation or
only sizes a workspace, so the suite runs without a GPU."""
import ctypes
import os
import re

import numpy as np
import pytest

from ops_sparse import _lib
from ops_sparse._lib import (DataType, Format, IndexBase, IndexType, Operation, Order, PointerMode, SpMMOpAlg, SpMVAlg,
                             SpMVOpAlg, Status)

HEADER = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "include", "cann_ops_sparse.h")
N, T, H = int(Operation.NON_TRANSPOSE), int(Operation.TRANSPOSE), int(Operation.CONJUGATE_TRANSPOSE)
F32 = int(DataType.FLOAT)


def declared_functions():
    text = open(HEADER).read()
    return sorted(set(re.findall(r"^\s*(?:aclsparseStatus_t|const char\*)\s+(aclsparse\w+)\s*\(", text, re.M)))


@pytest.fixture(scope="module")
def lib():
    return _lib.lib()


def test_every_declared_symbol_is_exported(lib):
    names = declared_functions()
    assert len(names) >= 39
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing
    # the ctypes table covers exactly the header
    assert set(_lib.SIGNATURES) == set(names)


def test_library_has_no_cpu_fallback_symbols():
    """The product library never links the oracle."""
    out = open(_lib.LIB_PATH, "rb").read()
    assert b"oracle_" not in out


class Env:
    """Host stand-ins for device buffers: validation reads only the addresses."""

    def __init__(self, lib, rows=2, cols=3, nnz=3):
        self.lib = lib
        self.h = ctypes.c_void_p(0)
        assert lib.aclsparseCreate(ctypes.byref(self.h)) == Status.SUCCESS
        assert lib.aclsparseSetStream(self.h, ctypes.c_void_p(_lib.HIP_NULL_STREAM)) == Status.SUCCESS
        self.bufs = [np.zeros(max(n, 1) * 8 + 64, np.uint8) for n in (rows + 1, nnz, nnz, cols, rows, cols, rows)]
        self.rp, self.ci, self.va, self.xv, self.yv, self.xt, self.yt = [self._al(b) for b in self.bufs]
        self.rows, self.cols, self.nnz = rows, cols, nnz
        self.alpha, self.beta = ctypes.c_float(1.0), ctypes.c_float(0.0)

    @staticmethod
    def _al(b):
        return (b.ctypes.data + 63) & ~63

    def csr(self, rows=None, cols=None, nnz=None, ptrs=True, vtype=DataType.FLOAT, ptr_type=IndexType.I32,
            idx_type=IndexType.I32, base=IndexBase.ZERO):
        d = ctypes.c_void_p(0)
        r = self.rows if rows is None else rows
        c = self.cols if cols is None else cols
        n = self.nnz if nnz is None else nnz
        p = (lambda a: ctypes.c_void_p(a)) if ptrs else (lambda a: ctypes.c_void_p(0))
        st = self.lib.aclsparseCreateCsr(ctypes.byref(d), r, c, n, p(self.rp), p(self.ci), p(self.va), int(ptr_type),
                                         int(idx_type), int(base), int(vtype))
        assert st == Status.SUCCESS
        return d

    def vec(self, n, addr, vtype=DataType.FLOAT):
        d = ctypes.c_void_p(0)
        assert self.lib.aclsparseCreateDnVec(ctypes.byref(d), n, ctypes.c_void_p(addr), int(vtype)) == Status.SUCCESS
        return d

    def size(self, op, A, x, y, c=F32, alg=0, alpha=None, beta=None, h=None):
        s = ctypes.c_size_t(0)
        st = self.lib.aclsparseSpMVGetBufferSize(self.h if h is None else h, op,
                                                 ctypes.byref(self.alpha) if alpha is None else alpha, A, x,
                                                 ctypes.byref(self.beta) if beta is None else beta, y, c, alg,
                                                 ctypes.byref(s))
        return st, s.value

    def run(self, fn, op, A, x, y, ws, c=F32, alg=0):
        return getattr(self.lib, fn)(self.h, op, ctypes.byref(self.alpha), A, x, ctypes.byref(self.beta), y, c, alg,
                                     ws)


@pytest.fixture
def env(lib):
    e = Env(lib)
    yield e
    lib.aclsparseDestroy(e.h)


# ------------------------------- handle --------------------------------------

def test_handle_lifecycle(lib):
    h = ctypes.c_void_p(0)
    assert lib.aclsparseCreate(None) == Status.HANDLE_IS_NULLPTR
    assert lib.aclsparseCreate(ctypes.byref(h)) == Status.SUCCESS
    assert lib.aclsparseCreate(ctypes.byref(h)) == Status.INVALID_VALUE  # would overwrite a live handle
    v = ctypes.c_int(0)
    assert lib.aclsparseGetVersion(h, ctypes.byref(v)) == Status.SUCCESS and v.value > 0
    # the reference answers the version without a handle (aclsparse_auxiliary.cpp:239-247)
    assert lib.aclsparseGetVersion(None, ctypes.byref(v)) == Status.SUCCESS
    assert lib.aclsparseGetVersion(h, None) == Status.INVALID_VALUE
    mode = ctypes.c_int32(-1)
    assert lib.aclsparseGetPointerMode(h, ctypes.byref(mode)) == Status.SUCCESS and mode.value == PointerMode.HOST
    assert lib.aclsparseSetPointerMode(h, int(PointerMode.DEVICE)) == Status.SUCCESS
    assert lib.aclsparseGetPointerMode(h, ctypes.byref(mode)) == Status.SUCCESS and mode.value == PointerMode.DEVICE
    assert lib.aclsparseSetPointerMode(h, 7) == Status.INVALID_VALUE
    s = ctypes.c_void_p(0)
    assert lib.aclsparseSetStream(h, ctypes.c_void_p(0x1234)) == Status.SUCCESS
    assert lib.aclsparseGetStream(h, ctypes.byref(s)) == Status.SUCCESS and s.value == 0x1234
    assert lib.aclsparseGetStream(h, None) == Status.INVALID_VALUE
    buf = np.zeros(4096, np.uint8)
    assert lib.aclsparseSetWorkspace(h, ctypes.c_void_p(buf.ctypes.data), 0) == Status.INVALID_VALUE
    assert lib.aclsparseSetWorkspace(h, ctypes.c_void_p(buf.ctypes.data), 4096) == Status.SUCCESS
    w, n = ctypes.c_void_p(0), ctypes.c_size_t(0)
    assert lib.aclsparseGetWorkspace(h, ctypes.byref(w), ctypes.byref(n)) == Status.SUCCESS
    assert w.value == buf.ctypes.data and n.value == 4096
    assert lib.aclsparseSetWorkspace(h, None, 0) == Status.SUCCESS  # unbinds
    assert lib.aclsparseSetStream(h, None) == Status.SUCCESS
    assert lib.aclsparseDestroy(h) == Status.SUCCESS
    assert lib.aclsparseDestroy(None) == Status.HANDLE_IS_NULLPTR  # aclsparse_auxiliary.cpp:133-139


# ------------------------------ descriptors -----------------------------------

def test_dnvec_descriptor(lib):
    data = np.zeros(16, np.float32)
    d = ctypes.c_void_p(0)
    assert lib.aclsparseCreateDnVec(ctypes.byref(d), -1, None, F32) == Status.INVALID_VALUE
    assert lib.aclsparseCreateDnVec(ctypes.byref(d), 16, ctypes.c_void_p(data.ctypes.data), F32) == Status.SUCCESS
    n, p, t = ctypes.c_int64(0), ctypes.c_void_p(0), ctypes.c_int32(0)
    assert lib.aclsparseDnVecGet(d, ctypes.byref(n), ctypes.byref(p), ctypes.byref(t)) == Status.SUCCESS
    assert (n.value, p.value, t.value) == (16, data.ctypes.data, F32)
    s = ctypes.c_int64(0)
    assert lib.aclsparseDnVecGetStride(d, ctypes.byref(s)) == Status.SUCCESS and s.value == 1
    assert lib.aclsparseDnVecSetStride(d, 0) == Status.INVALID_VALUE
    assert lib.aclsparseDnVecSetStride(d, 3) == Status.SUCCESS
    assert lib.aclsparseDnVecGetStride(d, ctypes.byref(s)) == Status.SUCCESS and s.value == 3
    assert lib.aclsparseDnVecSetValues(d, None) == Status.SUCCESS  # delayed binding
    assert lib.aclsparseDnVecGetValues(d, ctypes.byref(p)) == Status.SUCCESS and p.value is None
    assert lib.aclsparseDestroyDnVec(d) == Status.SUCCESS
    assert lib.aclsparseDestroyDnVec(None) == Status.SUCCESS


def test_csr_descriptor(lib):
    e = Env(lib)
    A = e.csr(base=IndexBase.ONE)
    f = ctypes.c_int32(-1)
    assert lib.aclsparseSpMatGetFormat(A, ctypes.byref(f)) == Status.SUCCESS and f.value == Format.CSR
    assert lib.aclsparseSpMatGetIndexBase(A, ctypes.byref(f)) == Status.SUCCESS and f.value == IndexBase.ONE
    r, c, n = ctypes.c_int64(0), ctypes.c_int64(0), ctypes.c_int64(0)
    assert lib.aclsparseSpMatGetSize(A, ctypes.byref(r), ctypes.byref(c), ctypes.byref(n)) == Status.SUCCESS
    assert (r.value, c.value, n.value) == (2, 3, 3)
    ptrs = [ctypes.c_void_p(0) for _ in range(3)]
    ts = [ctypes.c_int32(0) for _ in range(4)]
    assert lib.aclsparseCsrGet(A, ctypes.byref(r), ctypes.byref(c), ctypes.byref(n), *[ctypes.byref(p) for p in ptrs],
                               *[ctypes.byref(t) for t in ts]) == Status.SUCCESS
    assert [p.value for p in ptrs] == [e.rp, e.ci, e.va]
    assert [t.value for t in ts] == [IndexType.I32, IndexType.I32, IndexBase.ONE, F32]
    s = [ctypes.c_int64(0) for _ in range(3)]
    assert lib.aclsparseCsrGetStrides(A, *[ctypes.byref(v) for v in s]) == Status.SUCCESS
    assert [v.value for v in s] == [1, 1, 1]
    assert lib.aclsparseCsrSetStrides(A, 2, 3, 4) == Status.SUCCESS
    assert lib.aclsparseCsrGetStrides(A, *[ctypes.byref(v) for v in s]) == Status.SUCCESS
    assert [v.value for v in s] == [2, 3, 4]
    assert lib.aclsparseCsrSetStrides(A, 0, 1, 1) == Status.INVALID_VALUE
    # row offsets are required when rows > 0, indices and values when nnz > 0
    assert lib.aclsparseCsrSetPointers(A, None, None, None) == Status.INVALID_VALUE
    assert lib.aclsparseCsrSetPointers(A, ctypes.c_void_p(e.rp), ctypes.c_void_p(e.ci), None) == Status.INVALID_VALUE
    assert lib.aclsparseCsrSetPointers(A, ctypes.c_void_p(e.rp), ctypes.c_void_p(e.ci),
                                       ctypes.c_void_p(e.va)) == Status.SUCCESS
    assert lib.aclsparseSpMatSetValues(A, ctypes.c_void_p(e.va)) == Status.SUCCESS
    v = ctypes.c_void_p(0)
    assert lib.aclsparseSpMatGetValues(A, ctypes.byref(v)) == Status.SUCCESS and v.value == e.va
    assert lib.aclsparseDestroySpMat(A) == Status.SUCCESS
    assert lib.aclsparseDestroySpMat(None) == Status.SUCCESS
    d = ctypes.c_void_p(0)
    assert lib.aclsparseCreateCsr(ctypes.byref(d), -1, 3, 0, None, None, None, 0, 0, 0, F32) == Status.INVALID_VALUE
    lib.aclsparseDestroy(e.h)


# --------------------------- SpMV validation ----------------------------------

def test_spmv_buffer_size_positive_and_aligned(env):
    A = env.csr()
    x, y = env.vec(3, env.xv), env.vec(2, env.yv)
    st, n = env.size(N, A, x, y)
    assert st == Status.SUCCESS and n >= 64 and n % 64 == 0
    xt, yt = env.vec(2, env.xt), env.vec(3, env.yt)
    st, nt = env.size(T, A, xt, yt)
    assert st == Status.SUCCESS and nt >= 64 and nt % 64 == 0


# (name, rows, cols, nnz, row offset type, value type, op) of the five benchmark configurations
BENCH_SHAPES = [
    ("c1", 4096, 4096, 167936, IndexType.I32, DataType.FLOAT, N),
    ("c2", 4194304, 4194304, 20963328, IndexType.I32, DataType.FLOAT, N),
    ("c3", 8388608, 8388608, 134217728, IndexType.I32, DataType.FLOAT, N),
    ("c4", 16777216, 16777216, 536870912, IndexType.I64, DataType.FLOAT16, N),
    ("c5", 2097152, 2097152, 22649242, IndexType.I32, DataType.FLOAT, T),
]


def _align64(n):
    return (n + 63) // 64 * 64


@pytest.mark.parametrize("shape", BENCH_SHAPES, ids=[s[0] for s in BENCH_SHAPES])
def test_spmv_alg1_workspace_is_reference_sized(shape, env):
    """CSR_ALG1 sizes the reference's workspace (sparse/spmv/arch35/spmv_tiling_data.h:104-141):
    align64(align64(192 + (rows+1)*rowBytes) + cols*accBytes for a transpose), within 2x plus a
    fixed 128 KiB (the row-block partition, the long-row tasks and their scan storage come on top);
    DEFAULT keeps the larger layout of the staged / narrow / CSC tables, never smaller than ALG1's."""
    name, rows, cols, nnz, ptype, vtype, op = shape
    A = env.csr(rows=rows, cols=cols, nnz=nnz, ptrs=False, vtype=vtype, ptr_type=ptype)
    xr, yr = (rows, cols) if op == T else (cols, rows)
    x, y = env.vec(xr, 0, vtype), env.vec(yr, 0, vtype)
    st, lean = env.size(op, A, x, y, alg=int(SpMVAlg.CSR_ALG1))
    assert st == Status.SUCCESS and lean % 64 == 0
    rb = 8 if ptype == IndexType.I64 else 4
    ref = _align64(_align64(192 + (rows + 1) * rb) + (cols * 4 if op == T else 0))
    assert ref <= lean <= 2 * ref + (128 << 10), (name, lean, ref)
    st, full = env.size(op, A, x, y, alg=int(SpMVAlg.DEFAULT))
    assert st == Status.SUCCESS and full >= lean


def test_spmv_handle_checks(env, lib):
    A = env.csr()
    x, y = env.vec(3, env.xv), env.vec(2, env.yv)
    s = ctypes.c_size_t(0)
    assert lib.aclsparseSpMVGetBufferSize(None, N, ctypes.byref(env.alpha), A, x, ctypes.byref(env.beta), y, F32, 0,
                                          ctypes.byref(s)) == Status.HANDLE_IS_NULLPTR
    h = ctypes.c_void_p(0)
    assert lib.aclsparseCreate(ctypes.byref(h)) == Status.SUCCESS
    # the stream must be set before any SpMV call
    assert env.size(N, A, x, y, h=h)[0] == Status.INVALID_VALUE
    lib.aclsparseDestroy(h)


def test_spmv_rejects_unsupported_op_compute_alg(env):
    A = env.csr()
    x, y = env.vec(3, env.xv), env.vec(2, env.yv)
    assert env.size(9, A, x, y)[0] == Status.NOT_SUPPORTED
    assert env.size(N, A, x, y, c=int(DataType.FLOAT16))[0] == Status.NOT_SUPPORTED
    assert env.size(N, A, x, y, alg=17)[0] == Status.NOT_SUPPORTED
    assert env.size(N, None, x, y)[0] == Status.INVALID_VALUE


def test_spmv_rejects_null_and_misaligned_scalars(env):
    A = env.csr()
    x, y = env.vec(3, env.xv), env.vec(2, env.yv)
    raw = (ctypes.c_uint8 * 16)()
    mis = ctypes.c_void_p(ctypes.addressof(raw) + 1)
    assert env.size(N, A, x, y, alpha=ctypes.c_void_p(0))[0] == Status.INVALID_VALUE
    assert env.size(N, A, x, y, alpha=mis)[0] == Status.INVALID_VALUE


def test_spmv_rejects_type_combinations(env):
    x, y = env.vec(3, env.xv), env.vec(2, env.yv)
    A16 = env.csr(vtype=DataType.FLOAT16)
    assert env.size(N, A16, x, y)[0] == Status.NOT_SUPPORTED  # fp16 A with fp32 x
    x16, y16 = env.vec(3, env.xv, DataType.FLOAT16), env.vec(2, env.yv, DataType.FLOAT16)
    assert env.size(N, A16, x16, y16)[0] == Status.SUCCESS
    yb = env.vec(2, env.yv, DataType.BF16)
    assert env.size(N, A16, x16, yb)[0] == Status.NOT_SUPPORTED
    A8 = env.csr(vtype=DataType.INT8)
    x8, y32 = env.vec(3, env.xv, DataType.INT8), env.vec(2, env.yv, DataType.INT32)
    ai = ctypes.c_int32(1)
    assert env.size(N, A8, x8, y32, c=int(DataType.INT32), alpha=ctypes.byref(ai), beta=ctypes.byref(ai))[0] == \
        Status.SUCCESS
    assert env.size(N, A8, x8, env.vec(2, env.yv, DataType.FLOAT))[0] == Status.SUCCESS
    assert env.size(N, env.csr(idx_type=IndexType.I64), x, y)[0] == Status.NOT_SUPPORTED


def test_spmv_accepts_i64_row_offsets(env):
    x, y = env.vec(3, env.xv), env.vec(2, env.yv)
    assert env.size(N, env.csr(ptr_type=IndexType.I64), x, y)[0] == Status.SUCCESS


def test_spmv_transpose_beyond_int32_nnz_not_supported(env):
    """Transposes sum each column in CSR order through a CSC pattern limited to
    INT32_MAX entries (the reference's own nnz bound, sparse/spmv/README.md
    arch35 constraints); with 64-bit row offsets a larger matrix is still
    accepted for op = N but rejected, for every algorithm, for T and H."""
    big = (1 << 31) + 5
    A = env.csr(rows=1 << 20, cols=1 << 20, nnz=big, ptr_type=IndexType.I64, ptrs=False)
    xn, yn = env.vec(1 << 20, 0), env.vec(1 << 20, 0)
    assert env.size(N, A, xn, yn)[0] == Status.SUCCESS
    for op in (T, H):
        for alg in (SpMVAlg.DEFAULT, SpMVAlg.CSR_ALG1, SpMVAlg.CSR_ALG2):
            assert env.size(op, A, xn, yn, alg=int(alg))[0] == Status.NOT_SUPPORTED
    edge = env.csr(rows=1 << 20, cols=1 << 20, nnz=(1 << 31) - 1, ptr_type=IndexType.I64, ptrs=False)
    assert env.size(T, edge, xn, yn, alg=int(SpMVAlg.CSR_ALG2))[0] == Status.SUCCESS


def test_spmv_rejects_wrong_vector_sizes(env):
    A = env.csr()
    assert env.size(N, A, env.vec(2, env.xv), env.vec(2, env.yv))[0] == Status.INVALID_VALUE
    assert env.size(T, A, env.vec(3, env.xv), env.vec(2, env.yv))[0] == Status.INVALID_VALUE


def test_spmv_rejects_nonzero_nnz_with_zero_dimensions(env):
    """spmv_test.cpp:543-568: nnz > 0 with rows == 0 or cols == 0."""
    ws = np.zeros(512, np.uint8)
    wsp = ctypes.c_void_p(Env._al(ws))
    for zero_rows in (False, True):
        A = env.csr(rows=0 if zero_rows else 2, cols=2 if zero_rows else 0, nnz=1, ptrs=False)
        for op in (N, T):
            tr = op == T
            x = env.vec(0 if zero_rows == tr else 2, 0)
            y = env.vec(2 if zero_rows == tr else 0, 0)
            assert env.size(op, A, x, y)[0] == Status.INVALID_VALUE
            assert env.run("aclsparseSpMVPreprocess", op, A, x, y, wsp) == Status.INVALID_VALUE
            assert env.run("aclsparseSpMV", op, A, x, y, wsp) == Status.INVALID_VALUE


def test_spmv_workspace_query_before_binding_storage(env):
    """spmv_test.cpp:570-593: sizes are known before storage is bound; running unbound fails."""
    A = env.csr(ptrs=False)
    x, y = env.vec(3, 0), env.vec(2, 0)
    st, n = env.size(N, A, x, y)
    assert st == Status.SUCCESS and n > 0
    ws = np.zeros(n + 64, np.uint8)
    assert env.run("aclsparseSpMVPreprocess", N, A, x, y, ctypes.c_void_p(Env._al(ws))) == Status.INVALID_VALUE
    assert env.run("aclsparseSpMV", N, A, x, y, ctypes.c_void_p(Env._al(ws))) == Status.INVALID_VALUE


def test_spmv_workspace_checks(env):
    A = env.csr()
    x, y = env.vec(3, env.xv), env.vec(2, env.yv)
    assert env.run("aclsparseSpMV", N, A, x, y, None) == Status.INSUFFICIENT_RESOURCES
    ws = np.zeros(4096, np.uint8)
    assert env.run("aclsparseSpMV", N, A, x, y, ctypes.c_void_p(Env._al(ws) + 4)) == Status.INVALID_VALUE


def test_spmv_rejects_aliased_storage(env):
    A = env.csr()
    x = env.vec(3, env.xv)
    y = env.vec(2, env.xv)  # y aliases x
    ws = np.zeros(8192, np.uint8)
    assert env.run("aclsparseSpMV", N, A, x, y, ctypes.c_void_p(Env._al(ws))) == Status.INVALID_VALUE


# --------------------------- SpMVOp validation --------------------------------

def test_spmvop_validation(env, lib):
    A = env.csr()
    x, y, z = env.vec(3, env.xv), env.vec(2, env.yv), env.vec(2, env.yt)
    s = ctypes.c_size_t(7)
    bs = lib.aclsparseSpMVOp_bufferSize
    assert bs(None, N, A, x, y, z, F32, 0, ctypes.byref(s)) == Status.HANDLE_IS_NULLPTR
    assert bs(env.h, T, A, x, y, z, F32, 0, ctypes.byref(s)) == Status.NOT_SUPPORTED
    assert bs(env.h, N, A, x, y, z, int(DataType.INT32), 0, ctypes.byref(s)) == Status.NOT_SUPPORTED
    assert bs(env.h, N, env.csr(vtype=DataType.FLOAT16), x, y, z, F32, 0, ctypes.byref(s)) == Status.NOT_SUPPORTED
    assert bs(env.h, N, A, x, y, z, F32, 9, ctypes.byref(s)) != Status.SUCCESS
    assert bs(env.h, N, A, x, y, z, F32, int(SpMVOpAlg.ALG1), ctypes.byref(s)) == Status.SUCCESS and s.value == 0
    d = ctypes.c_void_p(0)
    cd = lib.aclsparseSpMVOp_createDescr
    assert cd(env.h, ctypes.byref(d), N, A, x, y, z, F32, int(SpMVOpAlg.ALG2), None) == Status.INVALID_VALUE
    assert cd(env.h, None, N, A, x, y, z, F32, 1, None) == Status.INVALID_VALUE
    assert cd(env.h, ctypes.byref(d), N, A, x, y, z, F32, int(SpMVOpAlg.DEFAULT), None) == Status.SUCCESS
    plan = ctypes.c_void_p(0)
    assert lib.aclsparseSpMVOp_createPlan(env.h, d, ctypes.byref(plan), None, 0) == Status.SUCCESS
    assert lib.aclsparseSpMVOp_createPlan(env.h, d, None, None, 0) == Status.INVALID_VALUE
    a, b = ctypes.c_float(1), ctypes.c_float(0)
    ex = lib.aclsparseSpMVOp
    assert ex(env.h, plan, None, ctypes.byref(b), x, y, z) == Status.INVALID_VALUE
    assert ex(env.h, plan, ctypes.byref(a), ctypes.byref(b), x, y, env.vec(3, env.yt)) == Status.INVALID_VALUE
    assert lib.aclsparseSpMVOp_destroyPlan(plan) == Status.SUCCESS
    assert lib.aclsparseSpMVOp_destroyDescr(d) == Status.SUCCESS


def test_package_import_registers_aten_mv_for_csr_on_rocm():
    # the reference's package implements aten::mv for its device's CSR key on import
    import torch
    import ops_sparse  # noqa: F401
    dump = torch._C._dispatch_dump("aten::mv")
    line = next(l for l in dump.splitlines() if l.startswith("SparseCsrCUDA:"))
    assert "ops_sparse" in line and "aten.py" in line


# ------------------------- dense matrix / SpMMOp --------------------------------

def test_dnmat_descriptor(lib):
    """aclsparseCreateDnMat rules (sparse/common/aclsparse_descr.cpp:1102-1152) and the getters."""
    data = np.zeros(64, np.float32)
    p = ctypes.c_void_p(data.ctypes.data)
    d = ctypes.c_void_p(0)
    cr = lib.aclsparseCreateDnMat
    R, C = int(Order.ROW), int(Order.COL)
    assert cr(None, 2, 3, 3, p, F32, R) == Status.INVALID_VALUE
    assert cr(ctypes.byref(d), -1, 3, 3, p, F32, R) == Status.INVALID_VALUE
    assert cr(ctypes.byref(d), 2, 1 << 31, 1 << 31, p, F32, R) == Status.INVALID_VALUE
    assert cr(ctypes.byref(d), 2, 3, -1, p, F32, R) == Status.INVALID_VALUE
    assert cr(ctypes.byref(d), 2, 3, 3, None, F32, R) == Status.INVALID_VALUE
    assert cr(ctypes.byref(d), 0, 3, 3, None, F32, R) == Status.SUCCESS  # empty: storage may be null
    assert lib.aclsparseDestroyDnMat(d) == Status.SUCCESS
    assert cr(ctypes.byref(d), 2, 3, 3, p, 99, R) == Status.INVALID_VALUE
    assert cr(ctypes.byref(d), 2, 3, 3, p, F32, 2) == Status.INVALID_VALUE
    assert cr(ctypes.byref(d), 2, 3, 2, p, F32, R) == Status.INVALID_VALUE  # ld < cols
    assert cr(ctypes.byref(d), 2, 3, 1, p, F32, C) == Status.INVALID_VALUE  # ld < rows
    assert cr(ctypes.byref(d), 2, 3, 5, p, F32, R) == Status.SUCCESS
    r, c, ld, v = ctypes.c_int64(0), ctypes.c_int64(0), ctypes.c_int64(0), ctypes.c_void_p(0)
    t, o = ctypes.c_int32(-1), ctypes.c_int32(-1)
    assert lib.aclsparseDnMatGet(d, ctypes.byref(r), ctypes.byref(c), ctypes.byref(ld), ctypes.byref(v),
                                 ctypes.byref(t), ctypes.byref(o)) == Status.SUCCESS
    assert (r.value, c.value, ld.value, v.value, t.value, o.value) == (2, 3, 5, data.ctypes.data, F32, R)
    assert lib.aclsparseConstDnMatGet(d, None, None, None, None, None, None) == Status.SUCCESS  # outputs optional
    assert lib.aclsparseDnMatSetValues(d, None) == Status.SUCCESS
    assert lib.aclsparseDnMatGetValues(d, ctypes.byref(v)) == Status.SUCCESS and not v.value
    assert lib.aclsparseDestroyDnMat(d) == Status.SUCCESS
    assert lib.aclsparseDestroyDnMat(None) == Status.SUCCESS
    assert lib.aclsparseDnMatGetValues(None, ctypes.byref(v)) == Status.INVALID_VALUE


def _dnmat(lib, rows, cols, addr, vtype=DataType.FLOAT, order=Order.ROW, ld=None):
    d = ctypes.c_void_p(0)
    if ld is None:
        ld = cols if order == Order.ROW else rows
    assert lib.aclsparseCreateDnMat(ctypes.byref(d), rows, cols, max(ld, 1), ctypes.c_void_p(addr), int(vtype),
                                    int(order)) == Status.SUCCESS
    return d


def test_spmmop_validation(env, lib):
    """Status codes of the SpMMOp exception tests (test/spmm_op/arch35/spmm_op_test.cpp:523-731) and
    the host checks of sparse/spmm_op/arch35/spmm_op_host.cpp; nothing here reaches a launch."""
    A = env.csr()  # 2 x 3, fp32
    B = _dnmat(lib, 3, 4, env.xv)
    Cm = _dnmat(lib, 2, 4, env.yt)
    s = ctypes.c_size_t(7)
    bs = lib.aclsparseSpMMOp_bufferSize
    assert bs(None, N, N, A, B, Cm, F32, 0, ctypes.byref(s)) == Status.HANDLE_IS_NULLPTR
    assert bs(env.h, N, N, None, B, Cm, F32, 0, ctypes.byref(s)) == Status.INVALID_VALUE
    assert bs(env.h, N, N, A, None, Cm, F32, 0, ctypes.byref(s)) == Status.INVALID_VALUE
    assert bs(env.h, N, N, A, B, None, F32, 0, ctypes.byref(s)) == Status.INVALID_VALUE
    assert bs(env.h, N, N, A, B, Cm, F32, 0, None) == Status.INVALID_VALUE
    assert bs(env.h, N, N, A, B, Cm, int(DataType.DOUBLE), 0, ctypes.byref(s)) == Status.NOT_SUPPORTED
    assert bs(env.h, T, N, A, B, Cm, F32, 0, ctypes.byref(s)) == Status.NOT_SUPPORTED
    assert bs(env.h, N, H, A, B, Cm, F32, 0, ctypes.byref(s)) == Status.NOT_SUPPORTED
    assert bs(env.h, N, N, A, B, Cm, F32, 9, ctypes.byref(s)) == Status.NOT_SUPPORTED
    assert bs(env.h, N, N, env.csr(vtype=DataType.BF16), B, Cm, F32, 0, ctypes.byref(s)) == Status.NOT_SUPPORTED
    assert bs(env.h, N, N, env.csr(idx_type=IndexType.I64), B, Cm, F32, 0, ctypes.byref(s)) == Status.NOT_SUPPORTED
    # null row offsets (nnz = 0, so indices and values may be null)
    assert bs(env.h, N, N, env.csr(nnz=0, ptrs=False), B, Cm, F32, 0, ctypes.byref(s)) == Status.INVALID_VALUE
    for alg in (SpMMOpAlg.DEFAULT, SpMMOpAlg.ALG1, SpMMOpAlg.ALG1_HIGH_PRECISION):
        assert bs(env.h, N, N, A, B, Cm, F32, int(alg), ctypes.byref(s)) == Status.SUCCESS and s.value == 0
    assert bs(env.h, N, N, A, B, Cm, F32, int(SpMMOpAlg.ALG2), ctypes.byref(s)) == Status.SUCCESS
    assert s.value >= 256 + 2 * 4 and s.value % 64 == 0
    d = ctypes.c_void_p(0)
    cd = lib.aclsparseSpMMOp_createDescr
    assert cd(None, ctypes.byref(d), N, N, A, B, Cm, F32, 0, None) == Status.HANDLE_IS_NULLPTR
    assert cd(env.h, None, N, N, A, B, Cm, F32, 0, None) == Status.INVALID_VALUE
    assert cd(env.h, ctypes.byref(d), N, N, A, B, Cm, F32, int(SpMMOpAlg.ALG2), None) == Status.INVALID_VALUE
    assert cd(env.h, ctypes.byref(d), N, N, A, B, Cm, F32, int(SpMMOpAlg.ALG1), None) == Status.SUCCESS
    plan = ctypes.c_void_p(0)
    cp = lib.aclsparseSpMMOp_createPlan
    assert cp(None, d, ctypes.byref(plan), None, 0) == Status.HANDLE_IS_NULLPTR
    assert cp(env.h, None, ctypes.byref(plan), None, 0) == Status.INVALID_VALUE
    assert cp(env.h, d, None, None, 0) == Status.INVALID_VALUE
    lto = np.zeros(16, np.uint8)
    assert cp(env.h, d, ctypes.byref(plan), ctypes.c_void_p(lto.ctypes.data), 16) == Status.NOT_SUPPORTED
    assert cp(env.h, d, ctypes.byref(plan), None, 0) == Status.SUCCESS
    sg = lib.aclsparseSpMMOp_setGlobalUserData
    assert sg(None, plan, b"x", None, 0) == Status.HANDLE_IS_NULLPTR
    assert sg(env.h, None, b"x", None, 0) == Status.INVALID_VALUE
    assert sg(env.h, plan, b"x", None, 4) == Status.INVALID_VALUE
    assert sg(env.h, plan, b"x", None, 0) == Status.SUCCESS
    a, b = ctypes.c_float(1), ctypes.c_float(0)
    ex = lib.aclsparseSpMMOp
    pa, pb = ctypes.byref(a), ctypes.byref(b)
    assert ex(None, plan, pa, pb, B, Cm) == Status.HANDLE_IS_NULLPTR
    assert ex(env.h, None, pa, pb, B, Cm) == Status.INVALID_VALUE
    assert ex(env.h, plan, None, pb, B, Cm) == Status.INVALID_VALUE
    assert ex(env.h, plan, pa, None, B, Cm) == Status.INVALID_VALUE
    assert ex(env.h, plan, pa, pb, None, Cm) == Status.INVALID_VALUE
    # B with k = 2 rows against A's k = 3 (DimMismatch), C with the wrong row count
    assert ex(env.h, plan, pa, pb, _dnmat(lib, 2, 4, env.xv), Cm) == Status.INVALID_VALUE
    assert ex(env.h, plan, pa, pb, B, _dnmat(lib, 3, 4, env.yt)) == Status.INVALID_VALUE
    # B of another dtype (UnsupportedDtypeCombo)
    assert ex(env.h, plan, pa, pb, _dnmat(lib, 3, 4, env.xv, DataType.FLOAT16), Cm) == Status.NOT_SUPPORTED
    # ld above the int32 range
    Bw = _dnmat(lib, 3, 4, env.xv, ld=1 << 31)
    assert ex(env.h, plan, pa, pb, Bw, Cm) == Status.NOT_SUPPORTED
    assert lib.aclsparseSpMMOp_destroyPlan(plan) == Status.SUCCESS
    assert lib.aclsparseSpMMOp_destroyPlan(None) == Status.SUCCESS
    assert lib.aclsparseSpMMOp_destroyDescr(d) == Status.SUCCESS
    assert lib.aclsparseSpMMOp_destroyDescr(None) == Status.SUCCESS
    # opB = T: B is n x k
    assert cd(env.h, ctypes.byref(d), N, T, A, B, Cm, F32, 0, None) == Status.SUCCESS
    assert cp(env.h, d, ctypes.byref(plan), None, 0) == Status.SUCCESS
    assert ex(env.h, plan, pa, pb, B, Cm) == Status.INVALID_VALUE  # 3 x 4 is not n x k = 4 x 3
    lib.aclsparseSpMMOp_destroyPlan(plan)
    lib.aclsparseSpMMOp_destroyDescr(d)


def test_bridge_operators_defined_without_cpu_fallback():
    # torch_npu/spmv_npu.cpp:410-437: ops_sparse::spmv and the ops_sparse_test::spmv_npu hook,
    # with device kernels only (test_spmv_npu.py:104-113: CPU tensors raise, no fallback)
    import torch
    import ops_sparse  # noqa: F401

    assert "spmv(Tensor mat, Tensor vec) -> Tensor" in str(torch.ops.ops_sparse.spmv.default._schema)
    schema = str(torch.ops.ops_sparse_test.spmv_npu.default._schema)
    assert "Tensor(a!) y" in schema and schema.endswith("-> Tensor(a!)")
    for key in ("CUDA", "SparseCsrCUDA"):
        assert torch._C._dispatch_has_kernel_for_dispatch_key("ops_sparse::spmv", key)
    assert torch._C._dispatch_has_kernel_for_dispatch_key("ops_sparse_test::spmv_npu", "CUDA")
    assert not torch._C._dispatch_has_kernel_for_dispatch_key("ops_sparse_test::spmv_npu", "CPU")
    row_ptr = torch.tensor([0, 0], dtype=torch.int32)
    empty_i, empty_f = torch.empty(0, dtype=torch.int32), torch.empty(0, dtype=torch.float32)
    with pytest.raises(RuntimeError):
        torch.ops.ops_sparse_test.spmv_npu(row_ptr, empty_i, empty_f, empty_f, empty_f, 1.0, 0.0, "N", 0)


def test_library_build_id_matches_the_sources(lib):
    """The loaded library was compiled from this tree's sources and flags."""
    from ops_sparse.build import file_build_id, source_hash

    assert _lib.library_build_id(lib) == source_hash() == file_build_id(_lib.LIB_PATH)


def test_stale_library_is_refused(tmp_path):
    """A library whose build id differs from the tree's is refused by the loader
    (checked in a fresh process on a copy with one byte of its id changed)."""
    import shutil
    import subprocess
    import sys

    from ops_sparse.build import BUILD_ID_PREFIX

    data = bytearray(open(_lib.LIB_PATH, "rb").read())
    i = data.find(BUILD_ID_PREFIX) + len(BUILD_ID_PREFIX)
    data[i] = ord("0") if data[i] != ord("0") else ord("1")
    stale = tmp_path / "lib" / "libaclsparse_hip.so"
    stale.parent.mkdir()
    stale.write_bytes(bytes(data))
    code = ("import sys; sys.path.insert(0, sys.argv[1]); from ops_sparse import _lib; "
            "_lib.LIB_PATH = sys.argv[2]\n"
            "try:\n    _lib.lib()\nexcept RuntimeError as e:\n    print('refused' if 'stale' in str(e) else e)\n"
            "else:\n    print('loaded')")
    pkg = os.path.dirname(os.path.dirname(_lib.__file__))
    out = subprocess.run([sys.executable, "-c", code, pkg, str(stale)], capture_output=True, text=True, timeout=120)
    assert out.stdout.strip().splitlines()[-1] == "refused", out.stdout + out.stderr


def test_host_scalars_follow_the_extension_conversions():
    """HostScalar mirrors the torch extension's (sparse/spmv/torch_extension/csrc/spmv.cpp:162-190)."""
    from ops_sparse.spmv import HostScalar

    def i32(v):
        return ctypes.cast(HostScalar(v, DataType.INT32).ptr, ctypes.POINTER(ctypes.c_int32)).contents.value

    assert i32(-7) == -7 and i32(2**31 - 1) == 2**31 - 1 and i32(-2**31) == -2**31
    assert i32(2.9) == 2 and i32(-2.9) == -2  # static_cast<int32_t> truncates
    for bad, msg in ((2**31, "out of the int32 range"), (-2**31 - 1, "out of the int32 range"),
                     (complex(1, 1), "imaginary part")):
        with pytest.raises(ValueError, match=msg):
            HostScalar(bad, DataType.INT32)
    assert ctypes.cast(HostScalar(1.5, DataType.FLOAT).ptr, ctypes.POINTER(ctypes.c_float)).contents.value == 1.5
    assert ctypes.cast(HostScalar(complex(1.5, 0), DataType.FLOAT).ptr,
                       ctypes.POINTER(ctypes.c_float)).contents.value == 1.5
    with pytest.raises(ValueError, match="real SpMV compute type cannot use a complex scalar"):
        HostScalar(complex(1, 2), DataType.FLOAT)
    c = ctypes.cast(HostScalar(complex(1, 2), DataType.COMPLEX64).ptr, ctypes.POINTER(_lib.Complex)).contents
    assert (c.x, c.y) == (1.0, 2.0)


def test_bridge_int32_scalar_checks():
    """The bridge's MakeScalars (torch_npu/spmv_npu.cpp:113-124) wants integral int32 scalars."""
    from ops_sparse.bridge import _check_int32_scalars

    _check_int32_scalars(2, -3)
    _check_int32_scalars(np.int64(5), 2**31 - 1)
    for a, b, msg in ((2.5, 1, "integral"), (2, 1.0, "integral"), (True, 0, "integral"), (2**31, 0, "fit int32"),
                      (0, -2**31 - 1, "fit int32")):
        with pytest.raises(RuntimeError, match=msg):
            _check_int32_scalars(a, b)


@pytest.mark.parametrize("rows,cols,nnz", [(1 << 19, 1 << 22, 1 << 22), (1 << 20, 1 << 19, 1 << 24)])
def test_staged_tables_follow_the_size_rule(rows, cols, nnz, env):
    """The DEFAULT workspace holds the staged-gather tables (slots, columns and gathered x: several
    bytes per entry) from 2^22 entries with an x of 8 MB or more, and from 2^24 entries with an x
    of 1 to 8 MB; one entry below the threshold it does not."""
    sizes = []
    for n in (nnz - 1, nnz):
        A = env.csr(rows=rows, cols=cols, nnz=n, ptrs=False)
        x, y = env.vec(cols, 0), env.vec(rows, 0)
        st, full = env.size(N, A, x, y, alg=int(SpMVAlg.DEFAULT))
        assert st == Status.SUCCESS
        sizes.append(full)
    assert sizes[1] - sizes[0] > 4 * nnz, sizes  # the staged tables appear at the threshold
