"""ctypes view of the CPU oracle (oracle/lib/liboracle.so).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and the
cpu_baseline leg of bench.py, as the checker or the timed CPU baseline.  The
product never imports this module.  Inputs are numpy arrays; CSR data must be
base 0 and contiguous (row offsets are converted to int64 here).
"""
import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "lib", "liboracle.so")
_LIB = None

K_F32, K_F16, K_BF16 = 0, 1, 2


def build():
    subprocess.run(["make", "-s", "-C", _HERE], check=True)


def lib():
    global _LIB
    if _LIB is None:
        if not os.path.exists(LIB_PATH):
            build()
        _LIB = ctypes.CDLL(LIB_PATH)
        _LIB.oracle_half_from_float.restype = ctypes.c_uint16
        _LIB.oracle_half_from_float.argtypes = [ctypes.c_float]
        _LIB.oracle_float_from_half.restype = ctypes.c_float
        _LIB.oracle_float_from_half.argtypes = [ctypes.c_uint16]
        _LIB.oracle_bf16_from_float.restype = ctypes.c_uint16
        _LIB.oracle_bf16_from_float.argtypes = [ctypes.c_float]
        _LIB.oracle_float_from_bf16.restype = ctypes.c_float
        _LIB.oracle_float_from_bf16.argtypes = [ctypes.c_uint16]
        _LIB.oracle_items_per_block.restype = ctypes.c_int64
        _LIB.oracle_items_per_block.argtypes = [ctypes.c_int64, ctypes.c_int64]
        _LIB.oracle_num_blocks.restype = ctypes.c_int64
        _LIB.oracle_num_blocks.argtypes = [ctypes.c_int64, ctypes.c_int64]
        _LIB.oracle_verify_mixed.restype = ctypes.c_int
    return _LIB


def _p(a):
    return a.ctypes.data_as(ctypes.c_void_p)


def _i64(a):
    return np.ascontiguousarray(a, dtype=np.int64)


def _c(a, dt):
    return np.ascontiguousarray(a, dtype=dt)


_D = ctypes.c_double
_I = ctypes.c_int64


def _map(fn, v, out_dtype):
    """Applies a scalar conversion elementwise (scalars in, scalar out)."""
    if np.ndim(v) == 0:
        return fn(v)
    a = np.asarray(v).ravel()
    return np.fromiter((fn(e) for e in a.tolist()), dtype=out_dtype, count=a.size).reshape(np.shape(v))


def half_from_float(v):
    return _map(lambda e: lib().oracle_half_from_float(float(e)), v, np.uint16)


def float_from_half(b):
    return _map(lambda e: lib().oracle_float_from_half(int(e)), b, np.float32)


def bf16_from_float(v):
    return _map(lambda e: lib().oracle_bf16_from_float(float(e)), v, np.uint16)


def float_from_bf16(b):
    return _map(lambda e: lib().oracle_float_from_bf16(int(e)), b, np.float32)


def spmv_f64(row_ptr, col, val, x, y, alpha, beta):
    """SpmvCpu in double for fp32 inputs: returns float64 z (non-transpose)."""
    rp = _i64(row_ptr)
    rows = rp.size - 1
    z = np.empty(rows, dtype=np.float64)
    lib().oracle_spmv_f64(_I(rows), _p(rp), _p(_c(col, np.int32)), _p(_c(val, np.float32)), _p(_c(x, np.float32)),
                          _p(_c(y, np.float32)), _D(alpha), _D(beta), _p(z))
    return z


def spmv_f64_threads(row_ptr, col, val, x, y, alpha, beta, threads):
    """spmv_f64 split over `threads` POSIX threads by row ranges (same per-row arithmetic)."""
    rp = _i64(row_ptr)
    rows = rp.size - 1
    z = np.empty(rows, dtype=np.float64)
    st = lib().oracle_spmv_f64_threads(_I(rows), _p(rp), _p(_c(col, np.int32)), _p(_c(val, np.float32)),
                                       _p(_c(x, np.float32)), _p(_c(y, np.float32)), _D(alpha), _D(beta), _p(z),
                                       ctypes.c_int(int(threads)))
    if st != 0:
        raise RuntimeError("oracle_spmv_f64_threads failed")
    return z


def spmv_trans_f64(row_ptr, col, val, x, y, cols, alpha, beta):
    rp = _i64(row_ptr)
    rows = rp.size - 1
    z = np.empty(cols, dtype=np.float64)
    lib().oracle_spmv_trans_f64(_I(rows), _I(cols), _p(rp), _p(_c(col, np.int32)), _p(_c(val, np.float32)),
                                _p(_c(x, np.float32)), _p(_c(y, np.float32)), _D(alpha), _D(beta), _p(z))
    return z


def _kind(bits_dtype_name):
    return {"float16": K_F16, "bfloat16": K_BF16, "float32": K_F32}[bits_dtype_name]


def spmv_lowp(row_ptr, col, val_bits, x_bits, y_bits, kind, y_kind, alpha, beta, transpose=False, cols=None):
    """fp16/bf16 values and x (as uint16 bit arrays, or float32 when kind is K_F32), fp32 compute.

    Returns z as uint16 bits (y_kind f16/bf16) or float32 (y_kind f32).
    """
    rp = _i64(row_ptr)
    rows = rp.size - 1
    n = cols if transpose else rows
    vdt = np.float32 if kind == K_F32 else np.uint16
    ydt = np.float32 if y_kind == K_F32 else np.uint16
    z = np.empty(n, dtype=ydt)
    args = (_p(rp), _p(_c(col, np.int32)), _p(_c(val_bits, vdt)), _p(_c(x_bits, vdt)), _p(_c(y_bits, ydt)),
            ctypes.c_int(kind), ctypes.c_int(y_kind), ctypes.c_float(alpha), ctypes.c_float(beta))
    if transpose:
        acc = np.empty(n, dtype=np.float32)
        lib().oracle_spmv_trans_lowp(_I(rows), _I(cols), *args, _p(acc), _p(z))
    else:
        lib().oracle_spmv_lowp(_I(rows), *args, _p(z))
    return z


def row_scale(row_ptr, col, val, x, y, kind, y_kind, alpha, beta, transpose=False, cols=None):
    """|alpha|*sum|a_ij x_j| + |beta y_i| for every output element (float64)."""
    rp = _i64(row_ptr)
    rows = rp.size - 1
    cols = cols if cols is not None else rows
    n = cols if transpose else rows
    vdt = np.float32 if kind == K_F32 else np.uint16
    ydt = np.float32 if y_kind == K_F32 else np.uint16
    s = np.empty(n, dtype=np.float64)
    lib().oracle_row_scale(_I(rows), _I(cols), _p(rp), _p(_c(col, np.int32)), _p(_c(val, vdt)), _p(_c(x, vdt)),
                           _p(_c(y, ydt)), ctypes.c_int(kind), ctypes.c_int(y_kind), ctypes.c_int(int(transpose)),
                           _D(alpha), _D(beta), _p(s))
    return s


def spmv_i8(row_ptr, col, val, x, y, alpha, beta, transpose=False, cols=None):
    rp = _i64(row_ptr)
    rows = rp.size - 1
    cols = cols if cols is not None else rows
    n = cols if transpose else rows
    z = np.empty(n, dtype=np.int32)
    acc = np.empty(n, dtype=np.int64)
    lib().oracle_spmv_i8(_I(rows), _I(cols), _p(rp), _p(_c(col, np.int32)), _p(_c(val, np.int8)),
                         _p(_c(x, np.int8)), _p(_c(y, np.int32)), ctypes.c_int(int(transpose)),
                         ctypes.c_int32(alpha), ctypes.c_int32(beta), _p(z), _p(acc))
    return z


def spmv_c64(row_ptr, col, val, x, y, cols, op, alpha, beta, val_is_real=False):
    """complex64 SpMV in double; val/x (complex64 or float32) and y (complex64) numpy arrays."""
    rp = _i64(row_ptr)
    rows = rp.size - 1
    n = rows if op == 0 else cols
    vdt = np.float32 if val_is_real else np.complex64
    z = np.empty(2 * n, dtype=np.float64)
    a, b = complex(alpha), complex(beta)
    lib().oracle_spmv_c64(_I(rows), _I(cols), _p(rp), _p(_c(col, np.int32)), _p(_c(val, vdt)), _p(_c(x, vdt)),
                          _p(_c(y, np.complex64)), ctypes.c_int(int(val_is_real)), ctypes.c_int(op),
                          _D(a.real), _D(a.imag), _D(b.real), _D(b.imag), _p(z))
    return z[0::2] + 1j * z[1::2]


def items_per_block(rows, nnz):
    return lib().oracle_items_per_block(rows, nnz)


def num_blocks(rows, nnz):
    return lib().oracle_num_blocks(rows, nnz)


def partition(row_ptr, nnz, rows=None, stride=1, base=0):
    """(normalised row offsets, block start rows, block start offsets) of the row-block partition.

    ``row_ptr`` is the physical array (``rows+1`` logical entries ``stride`` apart).
    """
    rp = _i64(row_ptr)
    if rows is None:
        rows = (rp.size - 1) // stride
    norm = np.empty(rows + 1, dtype=np.int64)
    nb = num_blocks(rows, nnz)
    blocks = np.empty(nb + 1, dtype=np.int32)
    bnnz = np.empty(nb + 1, dtype=np.int64)
    lib().oracle_spmv_partition(_I(rows), _I(nnz), _p(rp), _I(stride), _I(base), _p(norm), _p(blocks), _p(bnnz))
    return norm, blocks, bnnz


def task_table(block_nnz, long_chunks, chunk=512):
    """(task_start[B+1], task_block[total]) of the long-block task table.

    This build's own design (no reference counterpart): block b, whose
    non-zeros are [block_nnz[b], block_nnz[b+1]), is read in chunks of
    ``chunk`` slots starting at its first non-zero rounded down to a multiple
    of 4; a block of more than ``long_chunks`` chunks becomes one task per
    chunk.  task_start is the exclusive scan of the per-block task counts and
    task_block names the block of every task.
    """
    bn = _i64(block_nnz)
    k0, k1 = bn[:-1], bn[1:]
    chunks = (k1 - k0 + (k0 & 3) + chunk - 1) // chunk
    counts = np.where(chunks > long_chunks, chunks, 0)
    start = np.zeros(bn.size, dtype=np.int64)
    np.cumsum(counts, out=start[1:])
    return start.astype(np.int32), np.repeat(np.arange(k0.size, dtype=np.int32), counts)


def verify_mixed(golden, actual, rtol, atol, max_abs, ratio, exact=False):
    """Reference Verification(): returns (passed, matched_ratio, max_abs_error)."""
    g = np.ascontiguousarray(golden, dtype=np.float64)
    a = np.ascontiguousarray(actual, dtype=np.float64)
    if g.size != a.size:
        return False, 0.0, float("inf")
    r = ctypes.c_double(0)
    m = ctypes.c_double(0)
    st = lib().oracle_verify_mixed(_I(g.size), _p(g), _p(a), _D(rtol), _D(atol), _D(max_abs), _D(ratio),
                                   ctypes.c_int(int(exact)), ctypes.byref(r), ctypes.byref(m))
    return st == 0, r.value, m.value


# Per-dtype mixed tolerance of the reference (test/spmv/arch22/spmv_test.cpp:365-384)
MIXED_TOL = {
    "float32": (2.0 ** -10, 2.0 ** -16, 1e-2, 0.99),
    "float16": (2.0 ** -9, 2.0 ** -9, 1e-1, 0.99),
    "bfloat16": (2.0 ** -6, 2.0 ** -6, 1.0, 0.99),
    "int32": (0.0, 0.0, 0.0, 1.0),
}


def spmvop_tables(row_ptr, num_blocks):
    """(reorder, scratch, bin_edge) of the reference's SpMVOp ALG2 preprocess."""
    rp = _i64(row_ptr)
    m = rp.size - 1
    reorder = np.empty(max(m, 1), dtype=np.int32)
    scratch = np.empty(max(m, 1), dtype=np.int32)
    t1 = np.empty(max(m, 1), dtype=np.int32)
    t2 = np.empty(max(m, 1), dtype=np.int32)
    edge = np.empty(num_blocks + 1, dtype=np.int32)
    lib().oracle_spmvop_tables(ctypes.c_int32(m), _p(rp), ctypes.c_uint32(num_blocks), _p(reorder), _p(scratch),
                               _p(t1), _p(t2), _p(edge))
    return reorder[:m], scratch[:m], edge


def verify_mere_mare(golden, actual, threshold, multiplier):
    """(passed, mere, mare) of the reference's MERE/MARE strategy."""
    g = np.ascontiguousarray(golden, dtype=np.float32)
    a = np.ascontiguousarray(actual, dtype=np.float32)
    mere, mare = ctypes.c_double(0), ctypes.c_double(0)
    ok = lib().oracle_verify_mere_mare(_I(g.size), _p(g), _p(a), _D(threshold), _D(multiplier), ctypes.byref(mere),
                                       ctypes.byref(mare))
    return bool(ok), mere.value, mare.value
