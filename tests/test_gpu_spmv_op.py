"""GPU parity of the aclsparseSpMVOp family (through the C ABI).

Cases come from the reference's own parameter table
(test/spmv_op/arch35/spmv_op_test.csv, kept as tests/golden/spmv_op_cases.csv):
shape, sparsity, empty-row probability, seed, alpha, beta, pointer mode, row
offset type, Z/Y aliasing, unsorted columns, algorithm and the MERE/MARE
thresholds.  The matrices and vectors are the reference's own: the oracle's
input generator (oracle/spmvop_inputs.cpp) makes the same C++ standard-library
draws as the reference's SparseFillGenerator and test body (binomial row
lengths, distinct uniform columns, uniform values in [-5, 5], x and y in
[-3, 3] from seeds + 1 and + 2, row-wise shuffles for unsorted cases), as this
toolchain's libstdc++ computes them.  The golden is the fp64 oracle rounded to
fp32 (the reference's SpMVOpGolden, test/spmv_op/spmv_op_golden.h), checked
with the reference's MERE/MARE verifier (test/frame/verify.h:126-175) as
restated in the oracle.

The ALG2 preprocess tables (row reorder by descending length, sorted lengths,
bin edges) are compared bit-exactly with the oracle's restatement of the
reference's host-side construction (sparse/spmv_op/arch35/spmv_op_host.cpp).
"""
import csv
import ctypes
import os

import numpy as np
import pytest
import torch

import oracle
from ops_sparse import _lib
from ops_sparse._lib import DataType, Operation, SpMVOpAlg, Status
from ops_sparse.spmv import CsrDescr, DnVecDescr, Handle, SpMVOp

pytestmark = pytest.mark.gpu

_CSV = os.path.join(os.path.dirname(__file__), "golden", "spmv_op_cases.csv")
CASES = list(csv.DictReader(open(_CSV)))
ALG = {"DEFAULT": SpMVOpAlg.DEFAULT, "ALG1": SpMVOpAlg.ALG1, "ALG2": SpMVOpAlg.ALG2}

# layout of the ALG2 buffer (ops-sparse_amd/csrc/spmv_op_kernels.hip, SpmvOpComputeLayout)
_HDR, _ALIGN = 256, 64


def _align(v):
    return (v + _ALIGN - 1) & ~(_ALIGN - 1)


def alg2_offsets(m, bins):
    rb = 4 * m
    reorder = _HDR
    tmp_reorder = _align(reorder + rb)
    scratch = _align(tmp_reorder + rb)
    tmp_scratch = _align(scratch + rb)
    bin_edge = _align(tmp_scratch + rb)
    return reorder, tmp_scratch, bin_edge


def num_bins(m, dev):
    cus = torch.cuda.get_device_properties(dev).multi_processor_count
    return max(1, min(cus, -(-m // 128))) if m > 0 else 0


def make_inputs(m, k, sparsity, empty_prob, seed, pattern, unsorted):
    """The reference test's A (int64 offsets), x and y for one CSV row."""
    return oracle.spmvop_inputs(m, k, sparsity, empty_prob, seed, pattern, unsorted)


def run_case(c, dev, alg=None):
    m, k = int(c["m"]), int(c["k"])
    seed = int(c["seed"])
    rp, col, val, x, y = make_inputs(m, k, float(c["sparsity"]), float(c["empty_row_prob"]), seed, c["pattern"],
                                     c["unsorted"] == "1")
    alpha, beta = float(c["alpha"]), float(c["beta"])
    ptr_dtype = torch.int64 if c["row_offset_type"] == "i64" else torch.int32
    d_rp = torch.from_numpy(rp).to(ptr_dtype).to(dev)
    d_col = torch.from_numpy(col).to(dev)
    d_val = torch.from_numpy(val).to(dev)
    d_x = torch.from_numpy(x).to(dev)
    d_y = torch.from_numpy(y).to(dev)
    alias = c["alias_z_y"] == "1"
    d_z = d_y if alias else torch.full((max(m, 0),), float("nan"), device=dev)
    op = SpMVOp(m, k, d_rp, d_col, d_val, d_x, d_y, d_z, alg=ALG[alg or c["alg"]])
    if c["pointer_mode"] == "DEVICE":
        op.run(torch.tensor([alpha], device=dev), torch.tensor([beta], device=dev))
    else:
        op.run(alpha, beta)
    torch.cuda.synchronize()
    golden = oracle.spmv_f64(rp, col, val, x, y, alpha, beta).astype(np.float32) if m > 0 else np.zeros(0)
    return op, golden, d_z.cpu().numpy(), rp


@pytest.mark.parametrize("case", CASES, ids=lambda c: c["case_name"])
def test_reference_spmv_op_case(case, dev):
    op, golden, z, _ = run_case(case, dev)
    op.close()
    if golden.size == 0:
        return
    ok, mere, mare = oracle.verify_mere_mare(golden, z, float(case["mere_threshold"]),
                                             float(case["mare_multiplier"]))
    assert ok, f"MERE {mere:.3g} MARE {mare:.3g}"


@pytest.mark.parametrize("name", ["L1_2048x2048_medium", "L1_i64_scaled", "L1_empty_rows_most", "L1_10000x10000",
                                  "L1_1048576x1_extreme", "L1_2048x2048_dense50pct", "L0_unsorted_large"])
def test_alg2_on_alg1_cases(name, dev):
    """Every ALG1 shape also runs under ALG2 (binned, reordered rows)."""
    case = next(c for c in CASES if c["case_name"] == name)
    op, golden, z, _ = run_case(case, dev, alg="ALG2")
    op.close()
    ok, mere, mare = oracle.verify_mere_mare(golden, z, float(case["mere_threshold"]),
                                             float(case["mare_multiplier"]))
    assert ok, f"MERE {mere:.3g} MARE {mare:.3g}"


@pytest.mark.parametrize("name", ["L1_ALG2_2048", "L1_ALG2_4096", "L1_ALG2_i64", "L1_empty_rows_most",
                                  "L1_1048576x1_extreme", "L0_diag_8x8", "L1_2048x2048_full"])
def test_alg2_tables_bit_exact(name, dev):
    """reorder / sorted lengths / bin_edge equal the oracle's restatement bit for bit."""
    case = next(c for c in CASES if c["case_name"] == name)
    op, _, _, rp = run_case(case, dev, alg="ALG2")
    m = rp.size - 1
    bins = num_bins(m, dev)
    off_reorder, off_sorted, off_edge = alg2_offsets(m, bins)
    buf = op.buffer.cpu().numpy()
    got_reorder = buf[off_reorder:off_reorder + 4 * m].view(np.int32)
    got_sorted = buf[off_sorted:off_sorted + 4 * m].view(np.int32)
    got_edge = buf[off_edge:off_edge + 4 * (bins + 1)].view(np.int32)
    reorder, scratch, edge = oracle.spmvop_tables(rp, bins)
    np.testing.assert_array_equal(got_reorder, reorder)
    np.testing.assert_array_equal(got_sorted, scratch)
    np.testing.assert_array_equal(got_edge, edge)
    op.close()


def test_alg2_tables_known_answer(dev):
    """Hand-checked ALG2 tables: lengths [1,3,0,3,2] sort (stable, descending) to rows [1,3,4,0,2]."""
    rp = np.array([0, 1, 4, 4, 7, 9], np.int64)
    reorder, scratch, edge = oracle.spmvop_tables(rp, 1)
    np.testing.assert_array_equal(reorder, [1, 3, 4, 0, 2])
    np.testing.assert_array_equal(scratch, [3, 3, 2, 1, 0])
    assert edge[0] == 0 and edge[-1] == 5
    col = np.array([0, 0, 1, 2, 0, 1, 2, 1, 2], np.int32)
    val = np.arange(1, 10, dtype=np.float32)
    x = np.array([1.0, 2.0, 3.0], np.float32)
    d = [torch.from_numpy(a).to(dev) for a in (rp.astype(np.int32), col, val, x)]
    y = torch.zeros(5, device=dev)
    z = torch.zeros(5, device=dev)
    op = SpMVOp(5, 3, *d, y, z, alg=SpMVOpAlg.ALG2)
    op.run(1.0, 0.0)
    torch.cuda.synchronize()
    m, bins = 5, num_bins(5, dev)
    o_r, o_s, o_e = alg2_offsets(m, bins)
    buf = op.buffer.cpu().numpy()
    np.testing.assert_array_equal(buf[o_r:o_r + 20].view(np.int32), [1, 3, 4, 0, 2])
    np.testing.assert_array_equal(buf[o_s:o_s + 20].view(np.int32), [3, 3, 2, 1, 0])
    np.testing.assert_allclose(z.cpu().numpy(), [1.0, 2 + 6 + 12.0, 0.0, 5 + 12 + 21.0, 16 + 27.0])
    op.close()


def test_nnz_zero_beta_y_and_reexecute(dev):
    """nnz == 0: Z = beta*Y (the reference's beta_y kernel); executing twice is idempotent."""
    m, k = 300, 17
    rp = torch.zeros(m + 1, dtype=torch.int32, device=dev)
    e_i = torch.empty(0, dtype=torch.int32, device=dev)
    e_f = torch.empty(0, dtype=torch.float32, device=dev)
    x = torch.randn(k, device=dev)
    y = torch.randn(m, device=dev)
    for alg in (SpMVOpAlg.ALG1, SpMVOpAlg.ALG2):
        z = torch.full((m,), 7.0, device=dev)
        op = SpMVOp(m, k, rp, e_i, e_f, x, y, z, alg=alg)
        for _ in range(2):
            op.run(2.0, 1.5)
            torch.cuda.synchronize()
            np.testing.assert_array_equal(z.cpu().numpy(), (np.float32(1.5) * y.cpu().numpy()))
        op.run(2.0, 0.0)
        torch.cuda.synchronize()
        np.testing.assert_array_equal(z.cpu().numpy(), np.zeros(m, np.float32))
        op.close()


def test_beta_zero_ignores_nan_y(dev):
    """beta == 0 does not read Y: NaN in Y does not reach Z."""
    rp, col, val, _, _ = make_inputs(500, 400, 0.9, 0.0, 7, "random", False)
    rng = np.random.default_rng(8)
    x = rng.uniform(-3, 3, 400).astype(np.float32)
    for alg in (SpMVOpAlg.ALG1, SpMVOpAlg.ALG2):
        y = torch.full((500,), float("nan"), device=dev)
        z = torch.zeros(500, device=dev)
        d = [torch.from_numpy(a).to(dev) for a in (rp.astype(np.int32), col, val, x)]
        op = SpMVOp(500, 400, *d, y, z, alg=alg)
        op.run(1.0, 0.0)
        torch.cuda.synchronize()
        golden = oracle.spmv_f64(rp, col, val, x, np.zeros(500, np.float32), 1.0, 0.0).astype(np.float32)
        ok, mere, mare = oracle.verify_mere_mare(golden, z.cpu().numpy(), 1e-6, 5.0)
        assert ok, (alg, mere, mare)
        op.close()


def test_plan_reuse_with_new_vectors(dev):
    """One plan, executed against different X/Y/Z descriptors of the same sizes."""
    rp, col, val, _, _ = make_inputs(3000, 2000, 0.98, 0.1, 11, "random", False)
    d = [torch.from_numpy(a).to(dev) for a in (rp.astype(np.int32), col, val)]
    rng = np.random.default_rng(12)
    x1 = rng.uniform(-3, 3, 2000).astype(np.float32)
    y1 = rng.uniform(-3, 3, 3000).astype(np.float32)
    tx, ty, tz = torch.from_numpy(x1).to(dev), torch.from_numpy(y1).to(dev), torch.zeros(3000, device=dev)
    op = SpMVOp(3000, 2000, *d, tx, ty, tz, alg=SpMVOpAlg.ALG2)
    for trial in range(3):
        x = rng.uniform(-3, 3, 2000).astype(np.float32)
        y = rng.uniform(-3, 3, 3000).astype(np.float32)
        tx.copy_(torch.from_numpy(x))
        ty.copy_(torch.from_numpy(y))
        op.run(0.5, -2.0)
        torch.cuda.synchronize()
        golden = oracle.spmv_f64(rp, col, val, x, y, 0.5, -2.0).astype(np.float32)
        ok, mere, mare = oracle.verify_mere_mare(golden, tz.cpu().numpy(), 1e-6, 5.0)
        assert ok, (trial, mere, mare)
    op.close()


def test_long_rows_compensated_sum(dev):
    """Rows of up to 200k terms with heavy cancellation: the compensated dot keeps MERE below 1e-6."""
    m, k = 64, 200000
    rng = np.random.default_rng(21)
    lengths = rng.integers(0, k, m)
    lengths[0], lengths[1] = k, 0
    rp = np.zeros(m + 1, np.int64)
    np.cumsum(lengths, out=rp[1:])
    col = np.concatenate([np.sort(rng.choice(k, n, replace=False)) for n in lengths]).astype(np.int32)
    val = rng.uniform(-3, 3, col.size).astype(np.float32)
    x = rng.uniform(-3, 3, k).astype(np.float32)
    y = rng.uniform(-3, 3, m).astype(np.float32)
    for alg in (SpMVOpAlg.ALG1, SpMVOpAlg.ALG2):
        d = [torch.from_numpy(a).to(dev) for a in (rp.astype(np.int32), col, val, x, y)]
        z = torch.zeros(m, device=dev)
        op = SpMVOp(m, k, *d, z, alg=alg)
        op.run(1.0, 1.0)
        torch.cuda.synchronize()
        golden = oracle.spmv_f64(rp, col, val, x, y, 1.0, 1.0).astype(np.float32)
        ok, mere, mare = oracle.verify_mere_mare(golden, z.cpu().numpy(), 1e-6, 5.0)
        assert ok, (alg, mere, mare)
        op.close()


def test_status_codes(dev):
    """Validation order and error codes of the reference (spmv_op_host.cpp)."""
    lib = _lib.lib()
    m, k = 8, 8
    rp = torch.arange(m + 1, dtype=torch.int32, device=dev)
    col = torch.arange(m, dtype=torch.int32, device=dev)
    val = torch.ones(m, device=dev)
    x, y, z = torch.ones(k, device=dev), torch.ones(m, device=dev), torch.zeros(m, device=dev)
    h = Handle(torch.cuda.current_stream(dev).cuda_stream)
    A = CsrDescr(m, k, rp, col, val)
    vx, vy, vz = DnVecDescr(k, x), DnVecDescr(m, y), DnVecDescr(m, z)
    size = ctypes.c_size_t(0)
    N, T = int(Operation.NON_TRANSPOSE), int(Operation.TRANSPOSE)
    F, H16 = int(DataType.FLOAT), int(DataType.FLOAT16)
    assert lib.aclsparseSpMVOp_bufferSize(None, N, A.d, vx.d, vy.d, vz.d, F, 0, ctypes.byref(size)) == \
        Status.HANDLE_IS_NULLPTR
    assert lib.aclsparseSpMVOp_bufferSize(h.h, T, A.d, vx.d, vy.d, vz.d, F, 0, ctypes.byref(size)) == \
        Status.NOT_SUPPORTED
    assert lib.aclsparseSpMVOp_bufferSize(h.h, N, A.d, vx.d, vy.d, vz.d, H16, 0, ctypes.byref(size)) == \
        Status.NOT_SUPPORTED
    assert lib.aclsparseSpMVOp_bufferSize(h.h, N, A.d, vx.d, vy.d, vz.d, F, 0, None) == Status.INVALID_VALUE
    assert lib.aclsparseSpMVOp_bufferSize(h.h, N, A.d, vx.d, vy.d, vz.d, F, int(SpMVOpAlg.ALG1),
                                          ctypes.byref(size)) == Status.SUCCESS
    descr = ctypes.c_void_p(0)
    # ALG2 needs a buffer
    assert lib.aclsparseSpMVOp_createDescr(h.h, ctypes.byref(descr), N, A.d, vx.d, vy.d, vz.d, F,
                                           int(SpMVOpAlg.ALG2), None) == Status.INVALID_VALUE
    buf = torch.empty(1 << 16, dtype=torch.uint8, device=dev)
    # misaligned buffer
    assert lib.aclsparseSpMVOp_createDescr(h.h, ctypes.byref(descr), N, A.d, vx.d, vy.d, vz.d, F,
                                           int(SpMVOpAlg.ALG2), ctypes.c_void_p(buf.data_ptr() + 4)) == \
        Status.INVALID_VALUE
    assert lib.aclsparseSpMVOp_createDescr(h.h, ctypes.byref(descr), N, A.d, vx.d, vy.d, vz.d, F,
                                           int(SpMVOpAlg.ALG1), None) == Status.SUCCESS
    plan = ctypes.c_void_p(0)
    dummy = ctypes.c_int(0)
    assert lib.aclsparseSpMVOp_createPlan(h.h, descr, ctypes.byref(plan), ctypes.byref(dummy), 4) == \
        Status.NOT_SUPPORTED
    assert lib.aclsparseSpMVOp_createPlan(h.h, descr, ctypes.byref(plan), None, 0) == Status.SUCCESS
    a, b = ctypes.c_float(1.0), ctypes.c_float(0.0)
    assert lib.aclsparseSpMVOp(None, plan, ctypes.byref(a), ctypes.byref(b), vx.d, vy.d, vz.d) == \
        Status.HANDLE_IS_NULLPTR
    assert lib.aclsparseSpMVOp(h.h, None, ctypes.byref(a), ctypes.byref(b), vx.d, vy.d, vz.d) == \
        Status.INVALID_VALUE
    assert lib.aclsparseSpMVOp(h.h, plan, None, ctypes.byref(b), vx.d, vy.d, vz.d) == Status.INVALID_VALUE
    wrong = DnVecDescr(m + 1, torch.zeros(m + 1, device=dev))
    assert lib.aclsparseSpMVOp(h.h, plan, ctypes.byref(a), ctypes.byref(b), vx.d, vy.d, wrong.d) == \
        Status.INVALID_VALUE
    assert lib.aclsparseSpMVOp(h.h, plan, ctypes.byref(a), ctypes.byref(b), vx.d, vy.d, vz.d) == Status.SUCCESS
    torch.cuda.synchronize()
    np.testing.assert_array_equal(z.cpu().numpy(), np.ones(m, np.float32))
    assert lib.aclsparseSpMVOp_destroyPlan(plan) == Status.SUCCESS
    assert lib.aclsparseSpMVOp_destroyDescr(descr) == Status.SUCCESS
    assert lib.aclsparseSpMVOp_destroyPlan(None) == Status.SUCCESS
    assert lib.aclsparseSpMVOp_destroyDescr(None) == Status.SUCCESS


@pytest.mark.parametrize("i64", [False, True])
def test_alg2_row_blocks_reproducible_and_correctly_rounded(i64, dev):
    """ALG2 runs on the SpMV row blocks (short rows per lane, lane groups, whole-wave rows carried
    across chunks): repeated runs and rebuilt descriptors are bit-identical, and every z is within
    2 ulp of the fp64 golden (plus 1e-12 of the row scale for cancelling rows)."""
    rng = np.random.default_rng(77)
    lengths = np.concatenate([rng.integers(0, 6, 20000), rng.integers(20, 60, 500), [3000, 0, 9000, 1],
                              rng.integers(0, 3, 4000)])
    m, k = lengths.size, 50000
    rp = np.zeros(m + 1, np.int64)
    np.cumsum(lengths, out=rp[1:])
    col = rng.integers(0, k, int(rp[-1])).astype(np.int32)
    val = rng.uniform(-3, 3, col.size).astype(np.float32)
    x = rng.uniform(-3, 3, k).astype(np.float32)
    y = rng.uniform(-3, 3, m).astype(np.float32)
    d = [torch.from_numpy(a).to(dev) for a in (rp.astype(np.int64 if i64 else np.int32), col, val, x, y)]
    outs = []
    for _ in range(2):
        z = torch.full((m,), float("nan"), device=dev)
        op = SpMVOp(m, k, *d, z, alg=SpMVOpAlg.ALG2)
        op.run(1.25, -0.5)
        op.run(1.25, -0.5)
        torch.cuda.synchronize()
        outs.append(z.cpu().numpy())
        op.close()
    assert np.array_equal(outs[0].view(np.uint32), outs[1].view(np.uint32))
    golden = oracle.spmv_f64(rp, col, val, x, y, 1.25, -0.5)
    scale = oracle.row_scale(rp, col, val, x, y, oracle.K_F32, oracle.K_F32, 1.25, -0.5, cols=k)
    g32 = golden.astype(np.float32)
    ulp = np.spacing(np.abs(g32)).astype(np.float64)
    err = np.abs(outs[0].astype(np.float64) - golden)
    assert np.all(err <= 2 * ulp + 1e-12 * scale), float(np.max(err / (ulp + 1e-30)))


@pytest.mark.parametrize("alg", [SpMVOpAlg.ALG1, SpMVOpAlg.ALG2])
@pytest.mark.parametrize("i64", [False, True])
def test_one_based_indices_and_long_rows(alg, i64, dev):
    """Index base 1 (row offsets and columns), rows from empty to several chunks long."""
    rng = np.random.default_rng(5)
    lengths = np.concatenate([rng.integers(0, 7, 3000), [1500, 0, 40, 700], rng.integers(0, 20, 500)])
    m, k = lengths.size, 4000
    rp = np.zeros(m + 1, np.int64)
    np.cumsum(lengths, out=rp[1:])
    col = rng.integers(0, k, int(rp[-1])).astype(np.int32)
    val = rng.uniform(-3, 3, col.size).astype(np.float32)
    x = rng.uniform(-3, 3, k).astype(np.float32)
    y = rng.uniform(-3, 3, m).astype(np.float32)
    d_rp = torch.from_numpy(rp + 1).to(torch.int64 if i64 else torch.int32).to(dev)
    d = [torch.from_numpy(a).to(dev) for a in (col + 1, val, x, y)]
    z = torch.full((m,), float("nan"), device=dev)
    op = SpMVOp(m, k, d_rp, *d, z, alg=alg, base=1)
    op.run(0.75, 1.5)
    torch.cuda.synchronize()
    golden = oracle.spmv_f64(rp, col, val, x, y, 0.75, 1.5).astype(np.float32)
    ok, mere, mare = oracle.verify_mere_mare(golden, z.cpu().numpy(), 1e-6, 5.0)
    assert ok, (mere, mare)
    op.close()


def _spmv_flag(op):
    """The path flag in the header of the SpMV workspace inside an ALG2 buffer (found by its magic word,
    after the reference's tables): 0 col_ind, 3 narrow columns, 5 narrow columns on entry-aligned blocks."""
    buf = op.buffer.cpu().numpy()
    words = buf[: buf.size // 4 * 4].view(np.uint32)
    hits = np.nonzero(words[::16] == 0x4D505348)[0]  # 64-byte aligned header starts
    assert hits.size >= 1
    return int(words[hits[-1] * 16 + 32])


@pytest.mark.parametrize("case", ["laplacian", "long_rows"])
def test_alg2_narrow_columns(case, dev):
    """ALG2 on matrices of at least 2^20 entries: createDescr builds the 16-bit column copy (flag 5 for the
    Laplacian, whose 480-entry chunks fit; flag 3 for rows of 2000 entries). Bit-identical across runs and
    rebuilt descriptors, within 2 ulp of the fp64 golden like every ALG2 result, and equal in value to ALG1
    within the same bound."""
    if case == "laplacian":
        w = __import__("ops_sparse.workloads", fromlist=["laplacian_2d"]).laplacian_2d(n=1024)
        rp, col, val = w.row_ptr.numpy().astype(np.int64), w.col_ind.numpy(), w.values.numpy()
        m = k = w.rows
        want = 5
    else:
        m = k = 1024
        band = 2001
        off = np.arange(band) - band // 2
        col = np.clip(np.arange(m)[:, None] + off[None, :], 0, m - 1).reshape(-1).astype(np.int32)
        rp = np.arange(0, m * band + 1, band, dtype=np.int64)
        val = np.random.default_rng(3).uniform(-2, 2, col.size).astype(np.float32)
        want = 3
    rng = np.random.default_rng(9)
    x = rng.uniform(-3, 3, k).astype(np.float32)
    y = rng.uniform(-3, 3, m).astype(np.float32)
    d = [torch.from_numpy(a).to(dev) for a in (rp.astype(np.int32), col, val, x, y)]
    outs = []
    for alg in (SpMVOpAlg.ALG2, SpMVOpAlg.ALG2, SpMVOpAlg.ALG1):
        z = torch.full((m,), float("nan"), device=dev)
        op = SpMVOp(m, k, *d, z, alg=alg)
        op.run(1.25, -0.5)  # issued right after createDescr: every kernel variant, gated on the device flag
        torch.cuda.synchronize()
        first = z.clone()
        op.run(1.25, -0.5)  # the choice on the host: one kernel
        torch.cuda.synchronize()
        assert torch.equal(first.view(torch.int32), z.view(torch.int32))
        if alg == SpMVOpAlg.ALG2:
            assert _spmv_flag(op) == want
        outs.append(z.cpu().numpy())
        op.close()
    assert np.array_equal(outs[0].view(np.uint32), outs[1].view(np.uint32))
    golden = oracle.spmv_f64(rp, col, val, x, y, 1.25, -0.5)
    scale = oracle.row_scale(rp, col, val, x, y, oracle.K_F32, oracle.K_F32, 1.25, -0.5, cols=k)
    ulp = np.spacing(np.abs(golden.astype(np.float32))).astype(np.float64)
    for o in (outs[0], outs[2]):
        err = np.abs(o.astype(np.float64) - golden)
        assert np.all(err <= 2 * ulp + 1e-12 * scale), float(np.max(err / (ulp + 1e-30)))
