"""CPU checks that pin the oracle: the reference's known-answer vectors, and
independent mathematics (scipy, numpy's IEEE conversions, brute force,
closed forms) chosen so that a dropped term, a wrong index or a swapped
operand in the oracle fails one of them."""
import json
import math
import os

import numpy as np
import pytest
import scipy.sparse as sp
import torch

import oracle

KATS = json.load(open(os.path.join(os.path.dirname(__file__), "golden", "reference_kats.json")))


def rand_csr(rows, cols, density, seed, empty_prob=0.0):
    rng = np.random.default_rng(seed)
    m = sp.random(rows, cols, density=density, format="csr", random_state=rng, dtype=np.float64)
    if empty_prob:
        keep = rng.random(rows) >= empty_prob
        m = sp.diags(keep.astype(np.float64)) @ m
        m = m.tocsr()
        m.eliminate_zeros()
    m.data = rng.uniform(-3, 3, m.nnz)
    rp = m.indptr.astype(np.int64)
    col = m.indices.astype(np.int32)
    val = m.data.astype(np.float32)
    return rp, col, val


# ------------------------------ reference KATs -------------------------------

@pytest.mark.parametrize("case", KATS["csv_cases"], ids=lambda c: c["name"])
def test_oracle_reference_csv_cases(case):
    """Both applications of the reference's three-stage cases (spmv_test.cpp:69-212)."""
    b = case["base"]
    rp = np.array(case["row_ptr"], np.int64) - b
    col = np.array(case["col_ind"], np.int32) - b
    val = np.array(case["values"], np.float32)
    x = np.array(case["x"], np.float32)
    y = np.array(case["y"], np.float32)
    a, bt = case["alpha"], case["beta"]
    if case["op"] == "N":
        f = lambda yy: oracle.spmv_f64(rp, col, val, x, yy, a, bt)
    else:
        f = lambda yy: oracle.spmv_trans_f64(rp, col, val, x, yy, case["cols"], a, bt)
    z1 = f(y)
    np.testing.assert_allclose(z1, case["expected_first"], atol=case["tolerance"], rtol=0)
    z2 = f(z1.astype(np.float32))
    np.testing.assert_allclose(z2, case["expected_second"], atol=case["tolerance"], rtol=0)


def test_oracle_zero_nnz_beta():
    k = KATS["zero_nnz_beta"]
    rp = np.array(k["row_ptr"], np.int64)
    z = oracle.spmv_f64(rp, np.zeros(0, np.int32), np.zeros(0, np.float32), np.array(k["x"], np.float32),
                        np.array(k["y"], np.float32), k["alpha"], k["beta"])
    np.testing.assert_array_equal(z, k["expected"])


def test_oracle_repeated_coordinates():
    k = KATS["repeated_coordinates"]
    z = oracle.spmv_f64(np.array(k["row_ptr"]), np.array(k["col_ind"]), np.array(k["values"], np.float32),
                        np.array(k["x"], np.float32), np.array(k["y"], np.float32), k["alpha"], k["beta"])
    assert z[0] == k["expected"][0]


def test_oracle_golden_precision():
    """2^24 + 1 - 2^24 = 1 needs a wider-than-fp32 accumulator (spmv_test.cpp:350-361)."""
    k = KATS["golden_precision"]
    z = oracle.spmv_f64(np.array(k["row_ptr"]), np.array(k["col_ind"]), np.array(k["values"], np.float32),
                        np.array(k["x"], np.float32), np.zeros(1, np.float32), 1.0, 0.0)
    assert z[0] == k["expected"]


def test_oracle_fp16_round_half_even():
    k = KATS["fp16_halfway"]
    z = oracle.spmv_lowp(np.array(k["row_ptr"]), np.array(k["col_ind"]), np.array(k["values_bits"], np.uint16),
                         np.array(k["x_bits"], np.uint16), np.array(k["y_bits"], np.uint16), oracle.K_F16,
                         oracle.K_F16, k["alpha"], k["beta"])
    assert list(z) == k["expected_bits"]


@pytest.mark.parametrize("op", ["N", "T", "H"])
@pytest.mark.parametrize("rows", [2, 4096])
def test_oracle_int8_saturation(op, rows):
    k = KATS["int8_saturation"]
    rp = np.array([0, 1] + [2] * (rows - 1), np.int64)
    tr = op != "N"
    x = np.full(rows if tr else 2, 127, np.int8)
    y = np.zeros(2 if tr else rows, np.int32)
    z = oracle.spmv_i8(rp, np.array(k["col_ind"]), np.array(k["values"], np.int8), x, y, k["alpha"], k["beta"],
                       transpose=tr, cols=2)
    assert list(z[:2]) == k["expected_head"]
    assert np.all(z[2:] == 0)


def test_oracle_complex_conjugate_transpose():
    k = KATS["complex_conj_transpose"]
    c = lambda v: np.array([complex(a, b) for a, b in v], np.complex64)
    z = oracle.spmv_c64(np.array(k["row_ptr"]), np.array(k["col_ind"]), c(k["values"]), c(k["x"]), c(k["y"]),
                        k["cols"], 2, complex(*k["alpha"]), complex(*k["beta"]))
    np.testing.assert_allclose(z, [complex(a, b) for a, b in k["expected"]], atol=1e-12)


@pytest.mark.parametrize("rows", [2, 65, 4096])
def test_oracle_strided_partition_and_values(rows):
    """The strided fixture of spmv_test.cpp:255-374, through the partition's stride/base handling."""
    k = KATS["strided"]
    s = k["strides"]["row"]
    rp, ci, va = [1], [], []
    for r in range(rows):
        if r % 2 == 0:
            ci += [1, 3]
            va += [2.0, 3.0]
        else:
            ci.append(2)
            va.append(4.0)
        rp.append(len(va) + 1)
    phys = np.full(len(rp) * s, k["index_sentinel"], np.int64)
    phys[::s] = rp
    norm, _, _ = oracle.partition(phys, len(va), rows=rows, stride=s, base=1)
    np.testing.assert_array_equal(norm, np.array(rp) - 1)
    z = oracle.spmv_f64(norm, np.array(ci) - 1, np.array(va, np.float32), np.array([1, 2, 3], np.float32),
                        np.full(rows, k["y_init"], np.float32), k["alpha"], k["beta"])
    exp = [k["expected_n"]["even_row"] if r % 2 == 0 else k["expected_n"]["odd_row"] for r in range(rows)]
    np.testing.assert_array_equal(z, exp)
    even, odd = (rows + 1) // 2, rows // 2
    zt = oracle.spmv_trans_f64(norm, np.array(ci) - 1, np.array(va, np.float32), np.ones(rows, np.float32),
                               np.full(3, k["y_init"], np.float32), 3, k["alpha"], k["beta"])
    np.testing.assert_array_equal(zt, [4.0 * even + 15, 8.0 * odd + 15, 6.0 * even + 15])


_TOLMAP = {"float32": "float32", "exact_float": "float32", "int32": "int32"}


@pytest.mark.parametrize("i", range(len(KATS["verifier"]["cases"])))
def test_oracle_mixed_verifier_known_answers(i):
    """The reference verifier's own self-test cases (spmv_test_verification.h:111-165)."""
    c = KATS["verifier"]["cases"][i]
    g = np.array([float(v) for v in c["golden"]])
    a = np.array([float(v) for v in c["actual"]])
    tol = oracle.MIXED_TOL[_TOLMAP[c["tol"]]]
    ok, _, _ = oracle.verify_mixed(g, a, *tol, exact=c["tol"] == "exact_float")
    assert ok == c["passed"]


def test_oracle_mixed_verifier_diagnostics():
    d = KATS["verifier"]["diagnostics"]
    g = np.array(d["golden_head"] + [1.0] * (d["n"] - 2))
    a = np.array(d["actual_head"] + [1.0] * (d["n"] - 2))
    ok, ratio, max_abs = oracle.verify_mixed(g, a, *oracle.MIXED_TOL["float32"])
    assert ok == d["passed"]
    assert max_abs == pytest.approx(0.02, rel=1e-6)


# ------------------------------- mathematics ---------------------------------

@pytest.mark.parametrize("seed", [1, 2, 3])
def test_oracle_matches_scipy(seed):
    rows, cols = 700, 900
    rp, col, val = rand_csr(rows, cols, 0.02, seed, empty_prob=0.2)
    rng = np.random.default_rng(seed + 10)
    x = rng.uniform(-1, 1, cols).astype(np.float32)
    y = rng.uniform(-1, 1, rows).astype(np.float32)
    yt = rng.uniform(-1, 1, cols).astype(np.float32)
    A = sp.csr_matrix((val.astype(np.float64), col, rp), shape=(rows, cols))
    z = oracle.spmv_f64(rp, col, val, x, y, 1.5, -0.25)
    np.testing.assert_allclose(z, 1.5 * (A @ x.astype(np.float64)) - 0.25 * y, rtol=1e-12, atol=1e-12)
    zt = oracle.spmv_trans_f64(rp, col, val, y, yt, cols, -0.5, 2.0)
    np.testing.assert_allclose(zt, -0.5 * (A.T @ y.astype(np.float64)) + 2.0 * yt, rtol=1e-12, atol=1e-12)
    # complex, N/T/H against scipy with conjugation applied by hand
    cv = (val + 1j * rng.uniform(-1, 1, val.size)).astype(np.complex64)
    C = sp.csr_matrix((cv.astype(np.complex128), col, rp), shape=(rows, cols))
    xc = (rng.uniform(-1, 1, cols) + 1j * rng.uniform(-1, 1, cols)).astype(np.complex64)
    xr = (rng.uniform(-1, 1, rows) + 1j * rng.uniform(-1, 1, rows)).astype(np.complex64)
    yc = (rng.uniform(-1, 1, rows) + 1j * rng.uniform(-1, 1, rows)).astype(np.complex64)
    yk = (rng.uniform(-1, 1, cols) + 1j * rng.uniform(-1, 1, cols)).astype(np.complex64)
    al, be = 0.5 - 1j, 1j
    np.testing.assert_allclose(oracle.spmv_c64(rp, col, cv, xc, yc, cols, 0, al, be),
                               al * (C @ xc.astype(np.complex128)) + be * yc, rtol=1e-10, atol=1e-10)
    np.testing.assert_allclose(oracle.spmv_c64(rp, col, cv, xr, yk, cols, 1, al, be),
                               al * (C.T @ xr.astype(np.complex128)) + be * yk, rtol=1e-10, atol=1e-10)
    np.testing.assert_allclose(oracle.spmv_c64(rp, col, cv, xr, yk, cols, 2, al, be),
                               al * (C.conj().T @ xr.astype(np.complex128)) + be * yk, rtol=1e-10, atol=1e-10)


def test_half_and_bf16_conversions_match_ieee():
    """Every fp16 and bf16 bit pattern round-trips; fp32->fp16 RNE equals numpy's IEEE cast and
    fp32->bf16 equals torch's RNE cast on a sweep including halfway and overflow values."""
    bits = np.arange(1 << 16, dtype=np.uint16)
    f16 = bits.view(np.float16)
    got = oracle.float_from_half(bits)
    ok = ~np.isnan(f16)
    np.testing.assert_array_equal(got[ok], f16[ok].astype(np.float32))
    assert np.all(np.isnan(got[~ok]))
    fb = oracle.float_from_bf16(bits)
    # (NaN payloads are compared as NaN: returning through a C float quiets signalling NaNs)
    nb = np.isnan(fb)
    np.testing.assert_array_equal(fb.view(np.uint32)[~nb], (bits.astype(np.uint32) << 16)[~nb])
    assert np.array_equal(nb, ((bits & 0x7F80) == 0x7F80) & ((bits & 0x7F) != 0))
    rng = np.random.default_rng(5)
    v = np.concatenate([
        rng.uniform(-70000, 70000, 200000), rng.uniform(-1e-4, 1e-4, 100000), rng.standard_normal(100000),
        (np.arange(-2048, 2048) + 0.5) * 2.0 ** -10,  # halfway points of the fp16 grid near 1
        [65504.0, 65519.99, 65520.0, 1e30, -1e30, 2.0 ** -24, 2.0 ** -25, 3 * 2.0 ** -26, 0.0, -0.0],
    ]).astype(np.float32)
    np.testing.assert_array_equal(oracle.half_from_float(v), v.astype(np.float16).view(np.uint16))
    exp_bf = torch.from_numpy(v).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    np.testing.assert_array_equal(oracle.bf16_from_float(v), exp_bf)


def test_lowp_oracle_against_fp32_compute():
    """fp16 inputs, fp32 accumulation in row order, fp16 RNE store; y in fp32 variant unrounded."""
    rows, cols = 300, 200
    rp, col, val = rand_csr(rows, cols, 0.05, 9)
    rng = np.random.default_rng(9)
    vh = val.astype(np.float16)
    xh = rng.uniform(-2, 2, cols).astype(np.float16)
    yh = rng.uniform(-2, 2, rows).astype(np.float16)
    z = oracle.spmv_lowp(rp, col, vh.view(np.uint16), xh.view(np.uint16), yh.view(np.uint16), oracle.K_F16,
                         oracle.K_F16, 1.25, 0.5).view(np.float16)
    exp = np.empty(rows, np.float32)
    for r in range(rows):
        acc = np.float32(0)
        for q in range(rp[r], rp[r + 1]):
            acc = np.float32(acc + np.float32(vh[q]) * np.float32(xh[col[q]]))
        exp[r] = np.float32(np.float32(1.25) * acc) + np.float32(np.float32(0.5) * np.float32(yh[r]))
    np.testing.assert_allclose(z.astype(np.float32), exp.astype(np.float16).astype(np.float32), rtol=2e-3,
                               atol=2e-3)


def test_int8_against_int64_closed_form():
    rows, cols = 200, 150
    rp, col, _ = rand_csr(rows, cols, 0.1, 4)
    rng = np.random.default_rng(4)
    v = rng.integers(-128, 128, col.size).astype(np.int8)
    x = rng.integers(-128, 128, cols).astype(np.int8)
    y = rng.integers(-2 ** 31, 2 ** 31, rows).astype(np.int32)
    A = sp.csr_matrix((v.astype(np.int64), col, rp), shape=(rows, cols))
    for alpha, beta in [(3, 0), (1, 1), (-7, 2), (2 ** 31 - 1, -1)]:
        z = oracle.spmv_i8(rp, col, v, x, y, alpha, beta)
        exact = alpha * (A @ x.astype(np.int64)) + beta * y.astype(np.int64)
        np.testing.assert_array_equal(z, np.clip(exact, -2 ** 31, 2 ** 31 - 1))


# -------------------------------- partition ----------------------------------

@pytest.mark.parametrize("rows,nnz", [(0, 0), (1, 0), (5, 0), (1, 1), (3, 10 ** 6), (1000, 41000), (10 ** 5, 10 ** 5),
                                      (777, 123456), (2 ** 20, 2 ** 24)])
def test_items_per_block_closed_form(rows, nnz):
    t = 2032 if nnz == 0 else min(2032, 496 + (16 * 496 * rows) // nnz)
    assert oracle.items_per_block(rows, nnz) == t
    assert oracle.num_blocks(rows, nnz) == -(-(16 * rows + nnz) // t)


@pytest.mark.parametrize("seed", range(6))
def test_partition_brute_force(seed):
    rng = np.random.default_rng(seed)
    rows = int(rng.integers(1, 3000))
    lengths = rng.choice([0, 1, 3, 40, 700, 5000], size=rows, p=[0.2, 0.3, 0.2, 0.2, 0.09, 0.01])
    rp = np.zeros(rows + 1, np.int64)
    np.cumsum(lengths, out=rp[1:])
    nnz = int(rp[-1])
    norm, blocks, bnnz = oracle.partition(rp, nnz)
    t = oracle.items_per_block(rows, nnz)
    nb = oracle.num_blocks(rows, nnz)
    w = 16 * np.arange(rows + 1) + rp
    for b in range(nb):
        exp = next((r for r in range(rows) if w[r] >= b * t), rows)
        assert blocks[b] == exp
        assert bnnz[b] == rp[blocks[b]]
    assert blocks[nb] == rows and blocks[0] == 0
    assert np.all(np.diff(blocks) >= 0)
    # a block never starts more than (T / 16) rows after the previous one
    assert np.all(np.diff(blocks[:-1]) <= t // 16 + 1)


@pytest.mark.parametrize("seed", range(4))
@pytest.mark.parametrize("long_chunks", [1, 4])
def test_task_table_covers_long_blocks_exactly(seed, long_chunks):
    # brute force on the slots: walking each block's 512-slot chunks from its 16-byte-aligned
    # first non-zero must cover [k0, k1) exactly; blocks of more than long_chunks chunks get one
    # task per chunk, in block order, and no other block gets any
    rng = np.random.default_rng(100 + seed)
    rows = int(rng.integers(1, 2000))
    lengths = rng.choice([0, 2, 9, 300, 4000, 40000], size=rows, p=[0.2, 0.3, 0.3, 0.15, 0.04, 0.01])
    rp = np.zeros(rows + 1, np.int64)
    np.cumsum(lengths, out=rp[1:])
    nnz = int(rp[-1])
    _, _, bnnz = oracle.partition(rp, nnz)
    start, tblock = oracle.task_table(bnnz, long_chunks)
    nb = bnnz.size - 1
    assert start[0] == 0 and start[nb] == tblock.size
    covered = np.zeros(nnz, np.int32)
    for b in range(nb):
        k0, k1 = int(bnnz[b]), int(bnnz[b + 1])
        s0 = k0 - k0 % 4
        chunks = []
        while s0 + 512 * len(chunks) < k1:
            lo = max(k0, s0 + 512 * len(chunks))
            hi = min(k1, s0 + 512 * (len(chunks) + 1))
            covered[lo:hi] += 1
            chunks.append((lo, hi))
        n = int(start[b + 1] - start[b])
        assert n == (len(chunks) if len(chunks) > long_chunks else 0)
        assert np.all(tblock[start[b]:start[b + 1]] == b)
    assert np.all(covered == 1)


def test_partition_clamps_out_of_range_offsets():
    rp = np.array([5, 3, 100, 7], np.int64)  # base 1: logical [4, 2, 99, 6], nnz 6
    norm, _, _ = oracle.partition(rp, 6, base=1)
    np.testing.assert_array_equal(norm, [4, 2, 6, 6])


# ------------------------------ SpMVOp ALG2 tables ----------------------------

def _bin_edges_vectorised(sorted_lengths, bins):
    """Bin edges from the inclusive scan: lb(b) = 1 + first i with run[i] >= per*b,
    then the one-edge-per-row rule edge[b] = max(lb(b), edge[b-1] + 1)."""
    m = sorted_lengths.size
    run = np.cumsum(sorted_lengths.astype(np.int64))
    total = int(run[-1]) if m else 0
    per = -(-total // bins) if total > 0 else 0
    edge = [0]
    for b in range(1, bins):
        lb = int(np.searchsorted(run, per * b, side="left")) + 1
        e = max(lb, edge[-1] + 1)
        edge.append(min(e, m) if e <= m else m)
    edge.append(m)
    # once an edge reached m the remaining bins are empty
    for b in range(1, bins + 1):
        if edge[b - 1] >= m:
            edge[b] = m
    return np.array(edge, np.int32)


@pytest.mark.parametrize("seed,m,bins", [(0, 1, 1), (1, 5, 3), (2, 128, 1), (3, 1000, 8), (4, 5000, 40),
                                         (5, 20000, 157), (6, 300, 256), (7, 70000, 256)])
def test_spmvop_tables(seed, m, bins):
    rng = np.random.default_rng(seed)
    lengths = rng.choice([0, 1, 2, 7, 50, 900], size=m, p=[0.3, 0.2, 0.2, 0.2, 0.08, 0.02])
    rp = np.zeros(m + 1, np.int64)
    np.cumsum(lengths, out=rp[1:])
    reorder, scratch, edge = oracle.spmvop_tables(rp, bins)
    exp_order = np.argsort(-lengths, kind="stable")
    np.testing.assert_array_equal(reorder, exp_order)
    np.testing.assert_array_equal(scratch, lengths[exp_order])
    np.testing.assert_array_equal(edge, _bin_edges_vectorised(lengths[exp_order], bins))
    assert edge[0] == 0 and edge[-1] == m and np.all(np.diff(edge) >= 0)


def test_spmvop_tables_hand_checked():
    # lengths [4, 4, 4, 4]: total 16, 2 bins of 8 -> the edge after row 2
    rp = np.array([0, 4, 8, 12, 16])
    _, _, edge = oracle.spmvop_tables(rp, 2)
    np.testing.assert_array_equal(edge, [0, 2, 4])
    # one long row and many empty rows: the long row closes every bin it reaches, one edge per row
    rp = np.array([0, 100, 100, 100, 100])
    reorder, scratch, edge = oracle.spmvop_tables(rp, 3)
    np.testing.assert_array_equal(reorder, [0, 1, 2, 3])
    np.testing.assert_array_equal(edge, [0, 1, 2, 4])


# ----------------------------- MERE / MARE verifier ---------------------------

def test_mere_mare_closed_form():
    eps = 2.0 ** -14
    g = np.array([1.0, 2.0, -4.0, 0.0], np.float32)
    a = np.array([1.0 + 2 ** -20, 2.0, -4.0 - 2 ** -18, 0.0], np.float32)
    ok, mere, mare = oracle.verify_mere_mare(g, a, 1e-6, 5.0)
    rel = np.array([2 ** -20 / (1 + eps), 0.0, 2 ** -18 / (4 + eps), 0.0])
    assert mere == pytest.approx(rel.mean(), rel=1e-12)
    assert mare == pytest.approx(rel.max(), rel=1e-12)
    assert ok == (rel.mean() < 1e-6 and rel.max() < 5e-6)
    # a one-sided NaN fails; NaN on both sides is skipped
    assert not oracle.verify_mere_mare(np.ones(3), np.array([1, np.nan, 1]), 1e-6, 5.0)[0]
    assert oracle.verify_mere_mare(np.array([1, np.nan, 1]), np.array([1, np.nan, 1]), 1e-6, 5.0)[0]
    # an outlier above multiplier*threshold fails even when the mean passes
    g = np.ones(1000, np.float32)
    a = g.copy()
    a[0] = 1.0 + 2 ** -15
    ok, mere, mare = oracle.verify_mere_mare(g, a, 1e-6, 5.0)
    assert mere < 1e-6 and mare > 5e-6 and not ok


def test_trans_lowp_and_row_scale_closed_forms():
    """Transposed fp16/bf16 oracle against an fp32 brute force; the tolerance scale against numpy."""
    rows, cols = 120, 90
    rp, col, val = rand_csr(rows, cols, 0.08, 13)
    rng = np.random.default_rng(14)
    x = rng.uniform(-2, 2, rows).astype(np.float32)
    y = rng.uniform(-2, 2, cols).astype(np.float32)
    vb = torch.from_numpy(val).to(torch.bfloat16)
    xb = torch.from_numpy(x).to(torch.bfloat16)
    vbits = vb.view(torch.int16).numpy().view(np.uint16)
    xbits = xb.view(torch.int16).numpy().view(np.uint16)
    z = oracle.spmv_lowp(rp, col, vbits, xbits, y, oracle.K_BF16, oracle.K_F32, 0.75, -1.5, transpose=True,
                         cols=cols)
    acc = np.zeros(cols, np.float32)
    vf, xf = vb.float().numpy(), xb.float().numpy()
    for r in range(rows):
        for q in range(rp[r], rp[r + 1]):
            acc[col[q]] = np.float32(acc[col[q]] + np.float32(vf[q] * xf[r]))
    exp = np.float32(0.75) * acc + np.float32(-1.5) * y
    np.testing.assert_allclose(z, exp, rtol=1e-6, atol=1e-6)
    A = sp.csr_matrix((val.astype(np.float64), col, rp), shape=(rows, cols))
    xn = rng.uniform(-2, 2, cols).astype(np.float32)
    yn = rng.uniform(-2, 2, rows).astype(np.float32)
    s = oracle.row_scale(rp, col, val, xn, yn, oracle.K_F32, oracle.K_F32, -2.0, 0.5, cols=cols)
    np.testing.assert_allclose(s, 2.0 * (abs(A) @ np.abs(xn.astype(np.float64))) + 0.5 * np.abs(yn), rtol=1e-12)
    st = oracle.row_scale(rp, col, val, x, y, oracle.K_F32, oracle.K_F32, -2.0, 0.5, transpose=True, cols=cols)
    np.testing.assert_allclose(st, 2.0 * (abs(A).T @ np.abs(x.astype(np.float64))) + 0.5 * np.abs(y), rtol=1e-12)


def test_threaded_spmv_matches_serial_bit_for_bit():
    # the parallel CPU baseline splits rows only: every row keeps the serial summation order
    rng = np.random.default_rng(3)
    lengths = rng.integers(0, 40, 5000)
    rp = np.zeros(lengths.size + 1, np.int64)
    np.cumsum(lengths, out=rp[1:])
    col = rng.integers(0, 700, int(rp[-1])).astype(np.int32)
    val = rng.standard_normal(col.size).astype(np.float32)
    x = rng.standard_normal(700).astype(np.float32)
    y = rng.standard_normal(lengths.size).astype(np.float32)
    a = oracle.spmv_f64(rp, col, val, x, y, 1.5, -0.5)
    for t in (1, 3, 8):
        assert np.array_equal(oracle.spmv_f64_threads(rp, col, val, x, y, 1.5, -0.5, t), a)
    # fp16 / bf16 values and x, fp32 compute, 16-bit outputs
    for kind in (oracle.K_F16, oracle.K_BF16):
        vb = (oracle.half_from_float(val) if kind == oracle.K_F16 else oracle.bf16_from_float(val))
        xb = (oracle.half_from_float(x) if kind == oracle.K_F16 else oracle.bf16_from_float(x))
        yb = (oracle.half_from_float(y) if kind == oracle.K_F16 else oracle.bf16_from_float(y))
        s = oracle.spmv_lowp(rp, col, vb, xb, yb, kind, kind, 1.5, -0.5)
        for t in (1, 3, 8):
            assert np.array_equal(oracle.spmv_lowp_threads(rp, col, vb, xb, yb, kind, kind, 1.5, -0.5, t), s)


def _walk_merge_path(rp, items):
    """Brute force: walk the merge path one item at a time (row end first when its
    entries are all consumed) and record the corner at every multiple of ``items``."""
    rows, nnz = rp.size - 1, int(rp[-1])
    i = j = 0
    corners = [(0, 0)]
    for step in range(1, rows + nnz + 1):
        if i < rows and rp[i + 1] <= j:
            i += 1
        else:
            j += 1
        if step % items == 0 or step == rows + nnz:
            corners.append((i, j))
    return np.array([c[0] for c in corners]), np.array([c[1] for c in corners])


@pytest.mark.parametrize("seed", range(12))
def test_merge_path_tiles_match_a_walk_of_the_path(seed):
    rng = np.random.default_rng(seed)
    rows = int(rng.integers(1, 300))
    kind = seed % 3
    if kind == 0:
        lengths = rng.integers(0, 12, rows)
    elif kind == 1:  # many empty rows, a few long ones
        lengths = np.where(rng.random(rows) < 0.1, rng.integers(20, 400, rows), 0)
    else:
        lengths = np.zeros(rows, np.int64)
        lengths[rng.integers(0, rows)] = int(rng.integers(1, 900))
    rp = np.zeros(rows + 1, np.int64)
    np.cumsum(lengths, out=rp[1:])
    for items in (1, 2, 7, 64, 1000):
        r, e = oracle.merge_path_tiles(rp, items)
        rw, ew = _walk_merge_path(rp, items)
        np.testing.assert_array_equal(r, rw)
        np.testing.assert_array_equal(e, ew)
        # every tile holds exactly `items` items but the last; rows done and entries done never decrease
        assert np.all(np.diff(r + e)[:-1] == items) and np.all(np.diff(r) >= 0) and np.all(np.diff(e) >= 0)
        # a corner's completed rows have all their entries consumed
        assert np.all(rp[r] <= e)
