"""ctypes view of the CPU oracle (oracle/lib/liboracle.so).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and the
cpu_baseline leg of bench.py, as the checker or the timed CPU baseline.  The
product never imports this module.  Inputs are numpy arrays; CSR data must be
contiguous (row offsets are converted to int64 here) and base 0, except for the
SpMMOp functions, which take the index base.  The SpMV restatement is
spmv_oracle.c, the SpMMOp one spmm_oracle.c; spmvop_inputs.cpp rebuilds the
SpMVOp tests' inputs.
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


def spmv_lowp_threads(row_ptr, col, val_bits, x_bits, y_bits, kind, y_kind, alpha, beta, threads):
    """spmv_lowp (non-transpose) over ``threads`` POSIX threads by row ranges: bit-identical results."""
    rp = _i64(row_ptr)
    rows = rp.size - 1
    vdt = np.float32 if kind == K_F32 else np.uint16
    ydt = np.float32 if y_kind == K_F32 else np.uint16
    z = np.empty(rows, dtype=ydt)
    rc = lib().oracle_spmv_lowp_threads(_I(rows), _p(rp), _p(_c(col, np.int32)), _p(_c(val_bits, vdt)),
                                        _p(_c(x_bits, vdt)), _p(_c(y_bits, ydt)), ctypes.c_int(kind),
                                        ctypes.c_int(y_kind), ctypes.c_float(alpha), ctypes.c_float(beta), _p(z),
                                        ctypes.c_int(threads))
    if rc != 0:
        raise RuntimeError("pthread_create failed")
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


def merge_path_tiles(norm_row_ptr, items):
    """Corners of the merge-path tiles of a CSR matrix (Merrill & Garland, SC'16, "Merge-based
    parallel sparse matrix-vector multiplication"): the path walks the row ends
    a[i] = rp[i+1] and the entry indices 0..nnz-1, taking a row end first when
    a[i] <= the next entry index; tile t starts at diagonal min(t*items, rows+nnz).
    Returns (rows_done[T+1], entries_done[T+1]) for the normalised row offsets
    ``norm_row_ptr`` (rp[0] = 0).  The staged-gather tiles of this build; no
    reference counterpart (the reference has no merge-path partition)."""
    rp = np.asarray(norm_row_ptr, np.int64)
    rows = rp.size - 1
    nnz = int(rp[-1])
    total = rows + nnz
    tiles = -(-total // items)
    d = np.minimum(np.arange(tiles + 1, dtype=np.int64) * items, total)
    lo = np.maximum(d - nnz, 0)
    hi = np.minimum(d, rows)
    while np.any(lo < hi):
        act = lo < hi
        mid = (lo + hi) >> 1
        go_right = act & (rp[np.minimum(mid + 1, rows)] <= d - 1 - mid)
        lo = np.where(go_right, mid + 1, lo)
        hi = np.where(act & ~go_right, mid, hi)
    return lo.astype(np.int32), d - lo


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


# ------------------------------- SpMMOp -------------------------------------

def mt19937(seed, count):
    """The first ``count`` words of std::mt19937(seed)."""
    out = np.empty(count, dtype=np.uint32)
    lib().oracle_mt19937_fill(ctypes.c_uint32(seed & 0xFFFFFFFF), _I(count), _p(out))
    return out


def uniform_real(seed, lo, hi, count):
    """``count`` draws of libstdc++'s uniform_real_distribution<double>(lo, hi) over std::mt19937(seed)."""
    out = np.empty(count, dtype=np.float64)
    lib().oracle_uniform_real(ctypes.c_uint32(seed & 0xFFFFFFFF), _D(lo), _D(hi), _I(count), _p(out))
    return out


def half_from_float_away(v):
    """fp32 -> fp16 bits, round to nearest with ties away from zero."""
    f = lib().oracle_half_from_float_away
    f.restype = ctypes.c_uint16
    f.argtypes = [ctypes.c_float]
    v = np.asarray(v, dtype=np.float32)
    return np.array([f(float(x)) for x in v.ravel()], dtype=np.uint16).reshape(v.shape)


def spmm_sparsity(m, k, ratio, lo, hi, seed, unsorted=False, base=0):
    """MakeSpmmSparsity (test/spmm_op/spmm_op_golden.h:82-137): (row_ptr int64, col int32, values fp64),
    row_ptr / col carrying ``base``."""
    rp = np.zeros(m + 1, dtype=np.int64)
    if m <= 0 or k <= 0:
        return rp + base, np.zeros(0, np.int32), np.zeros(0, np.float64)
    thr = int(ratio * 100)
    ii = (np.arange(m) % 100)[:, None] * 7
    jj = (np.arange(k) % 100)[None, :] * 13
    mask = (ii + jj) % 100 < thr
    rows, cols = np.nonzero(mask)  # row-major order, the generator's loop order
    nnz = rows.size
    rp[1:] = np.cumsum(mask.sum(axis=1))
    col = cols.astype(np.int32)
    val = uniform_real(seed, lo, hi, nnz)
    if unsorted:  # ShuffleCsrRowPairs (:40-65): per-row Fisher-Yates with std::mt19937(seed + i)
        for i in range(m):
            s, e = int(rp[i]), int(rp[i + 1])
            if e - s <= 1:
                continue
            words = mt19937((seed + i) & 0xFFFFFFFF, e - s - 1)
            for t, j in enumerate(range(e - 1, s, -1)):
                kk = s + int(words[t]) % (j - s + 1)
                col[j], col[kk] = col[kk], col[j]
                val[j], val[kk] = val[kk], val[j]
    return rp + base, col + base, val


def spmm_f32(m, k, n, row_ptr, col, val, base, b, ldb, b_contig, c, ldc, c_row, alpha, beta, kahan=False,
             half_out=False):
    """The SpMMOp kernel's fp32 steps; returns the new C storage (float32, same layout as ``c``)."""
    rp = _i64(row_ptr)
    out = np.array(c, dtype=np.float32, copy=True).ravel()
    lib().oracle_spmm_f32(_I(m), _I(k), _I(n), _p(rp), _p(_c(col, np.int32)), _p(_c(val, np.float32)),
                          _I(len(col)), ctypes.c_int32(base), _p(_c(b, np.float32)), _I(ldb), ctypes.c_int32(b_contig),
                          _p(out), _I(ldc), ctypes.c_int32(c_row), ctypes.c_float(alpha), ctypes.c_float(beta),
                          ctypes.c_int32(int(kahan)), ctypes.c_int32(int(half_out)))
    return out


def spmm_golden_f64(m, k, n, row_ptr, col, val, base, b, b_trans, c_init, alpha, beta):
    """SpmmGolden (fp64): b and c_init in canonical row-major order; returns (m*n,) float64."""
    out = np.empty(max(m * n, 1), dtype=np.float64)
    lib().oracle_spmm_golden_f64(_I(m), _I(k), _I(n), _p(_i64(row_ptr)), _p(_c(col, np.int32)),
                                 _p(_c(val, np.float64)), ctypes.c_int32(base), _p(_c(b, np.float64)),
                                 ctypes.c_int32(int(b_trans)), _p(_c(c_init, np.float64)), _D(alpha), _D(beta),
                                 _p(out))
    return out[:m * n]


# MIXED_TOLERANCE rows of test/frame/verify.h:230-236: (rtol, atol, fixed limit, mantissa bits, emin)
FRAME_MIXED = {"float32": (2.0 ** -13, 2.0 ** -13, 1e-2, 23, -126), "float16": (2.0 ** -10, 2.0 ** -10, 1e-1, 10, -14)}


def verify_frame_mixed(golden, actual, dtype):
    """MixedToleranceStrategy (test/frame/verify.h:207-320): returns (passed, matched_ratio, max_abs_error).
    An element fails when |a-g| > atol + rtol*|g|; the check fails when fewer than 99% match, or when
    any |a-g| exceeds max(fixed, 32 ulp(|g|)), or any value is NaN/Inf."""
    rtol, atol, fixed, mbits, emin = FRAME_MIXED[dtype]
    g = np.asarray(golden, dtype=np.float32).astype(np.float64).ravel()
    a = np.asarray(actual, dtype=np.float32).astype(np.float64).ravel()
    if g.size == 0:
        return True, 1.0, 0.0
    bad = ~np.isfinite(g) | ~np.isfinite(a)
    diff = np.abs(a - g)
    ga = np.abs(g)
    _, ex = np.frexp(ga)
    ulp = np.where(ga == 0, 2.0 ** (emin - mbits), np.ldexp(1.0, np.maximum(ex - 1, emin) - mbits))
    fails = (diff > atol + rtol * ga) | bad
    hard = bad | (diff > np.maximum(fixed, 32.0 * ulp))
    ratio = 1.0 - fails.sum() / g.size
    return bool(ratio >= 0.99 and not hard.any()), float(ratio), float(np.nanmax(np.where(bad, 0, diff)))


# ---------------------------- SpMVOp test inputs ------------------------------

_INPUTS = None
_PATTERNS = {"random": 0, "diag": 1, "empty": 2}


def _inputs_lib():
    global _INPUTS
    if _INPUTS is None:
        path = os.path.join(_HERE, "lib", "liboracle_inputs.so")
        if not os.path.exists(path):
            build()
        _INPUTS = ctypes.CDLL(path)
        f = _INPUTS.oracle_spmvop_inputs
        f.restype = ctypes.c_int64
        f.argtypes = [ctypes.c_int64, ctypes.c_int64, ctypes.c_double, ctypes.c_double, ctypes.c_uint32,
                      ctypes.c_int, ctypes.c_int, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p,
                      ctypes.c_int64, ctypes.c_void_p, ctypes.c_void_p]
    return _INPUTS


def spmvop_inputs(m, k, sparsity, empty_prob, seed, pattern="random", unsorted=False):
    """The reference SpMVOp test's A (int64 row offsets, int32 columns, fp32 values), x and y
    (test/spmv_op/arch35/spmv_op_test.cpp:50-101, test/frame/fill.h:71-141) as this toolchain's
    C++ standard library draws them (oracle/spmvop_inputs.cpp)."""
    f = _inputs_lib().oracle_spmvop_inputs
    pat = _PATTERNS[pattern]
    mm = max(m, 0)
    rp = np.zeros(mm + 1, np.int32)
    nnz = f(m, k, sparsity, empty_prob, seed & 0xFFFFFFFF, pat, int(unsorted), _p(rp), None, None, 0, None, None)
    col = np.zeros(max(nnz, 1), np.int32)
    val = np.zeros(max(nnz, 1), np.float32)
    x = np.zeros(max(k, 1), np.float32)
    y = np.zeros(max(mm, 1), np.float32)
    f(m, k, sparsity, empty_prob, seed & 0xFFFFFFFF, pat, int(unsorted), _p(rp), _p(col), _p(val), nnz, _p(x),
      _p(y))
    return rp.astype(np.int64), col[:nnz], val[:nnz], x[:max(k, 0)], y[:mm]
