"""Pins the SpMMOp oracle (oracle/spmm_oracle.c) before the GPU tests trust it.

* std::mt19937 and libstdc++'s uniform_real_distribution<double>: against
  draws printed by a g++-built program (tests/golden/libstdcxx_uniform.json),
  the C++ standard's 10000th-word check, and numpy's MT19937 (genrand_res53
  built from the same two words);
* the fp16 ties-away cast: every fp16 midpoint rounds away from zero, every
  other value as numpy's round-to-nearest;
* the fp64 golden: against scipy's dense product for every opB / index base;
* the fp32 restatement: within fp32 error of the golden, layout-independent
  (row- and column-major B and C give the same bits), Kahan closer to fp64
  than plain summation on cancelling rows, the fp16 store = clamp then cast;
* the sparsity generator: a hand-derived 4x4 pattern, row shuffles that only
  permute each row, and the golden unchanged by them;
* the MIXED_TOLERANCE verifier on constructed pass / fail cases.
"""
import json
import os

import numpy as np
import pytest
import scipy.sparse as sp

import oracle

H = os.path.join(os.path.dirname(__file__), "golden")
VEC = json.load(open(os.path.join(H, "libstdcxx_uniform.json")))


def test_mt19937_matches_libstdcxx_and_the_standard():
    for case in VEC["raw"]:
        got = oracle.mt19937(case["seed"], len(case["words"]))
        np.testing.assert_array_equal(got, np.array(case["words"], dtype=np.uint32))
    assert int(oracle.mt19937(5489, 10000)[-1]) == 4123659995 == VEC["default_10000th"]


@pytest.mark.parametrize("seed", [0, 7, 101, 20260909])
def test_mt19937_matches_numpy_res53(seed):
    w = oracle.mt19937(seed, 2000).astype(np.float64)
    a, b = np.floor(w[0::2] / 32), np.floor(w[1::2] / 64)
    res53 = (a * 67108864.0 + b) / 9007199254740992.0
    np.testing.assert_array_equal(res53, np.random.RandomState(seed).random_sample(1000))


def test_uniform_real_matches_libstdcxx():
    for case in VEC["uniform"]:
        got = oracle.uniform_real(case["seed"], case["lo"], case["hi"], len(case["values"]))
        np.testing.assert_array_equal(got, np.array(case["values"], dtype=np.float64))


def _halves():
    h = np.arange(0x7C00, dtype=np.uint16)  # every finite positive fp16
    return h, h.view(np.float16).astype(np.float32)


def test_half_ties_away_on_every_midpoint():
    h, f = _halves()
    lo, hi = f[:-1].astype(np.float64), f[1:].astype(np.float64)
    mid = ((lo + hi) / 2).astype(np.float32)  # exact: fp16 midpoints fit fp32
    assert np.all(mid.astype(np.float64) == (lo + hi) / 2)
    got = oracle.half_from_float_away(mid)
    np.testing.assert_array_equal(got, h[1:])
    np.testing.assert_array_equal(oracle.half_from_float_away(-mid), h[1:] | 0x8000)
    # the midpoint below the smallest subnormal rounds up to it, half of that to zero
    assert oracle.half_from_float_away(np.float32(2.0 ** -25)) == 1
    assert oracle.half_from_float_away(np.float32(2.0 ** -26)) == 0


def test_half_away_equals_nearest_off_midpoints():
    rng = np.random.default_rng(3)
    v = np.concatenate([rng.uniform(-65504, 65504, 20000), rng.uniform(-1, 1, 20000) * 2.0 ** -14,
                        rng.standard_normal(20000)]).astype(np.float32)
    ref = v.astype(np.float16)
    lo = ref.astype(np.float64)
    # exclude exact midpoints (where the two rules differ)
    with np.errstate(over="ignore"):
        nxt = np.nextafter(ref, np.float16(np.inf) * np.sign(v).astype(np.float16)).astype(np.float64)
    keep = np.abs(v.astype(np.float64) - lo) != np.abs(nxt - lo) / 2
    np.testing.assert_array_equal(oracle.half_from_float_away(v[keep]), ref[keep].view(np.uint16))


def _case(m, k, n, ratio, seed, base=0, unsorted=False):
    rp, col, val = oracle.spmm_sparsity(m, k, ratio, -1.0, 1.0, seed, unsorted, base)
    b = oracle.uniform_real(seed + 100, -1.0, 1.0, k * n)
    c = oracle.uniform_real(seed + 200, -1.0, 1.0, m * n)
    return rp, col, val, b, c


@pytest.mark.parametrize("b_trans", [False, True])
@pytest.mark.parametrize("base", [0, 1])
def test_golden_matches_dense_product(b_trans, base):
    m, k, n = 37, 23, 19
    rp, col, val, b, c = _case(m, k, n, 0.4, 11, base)
    A = sp.csr_matrix((val, col - base, rp - base), shape=(m, k)).toarray()
    B = b.reshape(n, k).T if b_trans else b.reshape(k, n)
    want = 1.5 * A @ B - 0.25 * c.reshape(m, n)
    got = oracle.spmm_golden_f64(m, k, n, rp, col, val, base, b, b_trans, c, 1.5, -0.25)
    np.testing.assert_allclose(got.reshape(m, n), want, rtol=1e-13, atol=1e-13)


def _f32(m, k, n, rp, col, val, base, b, c, alpha, beta, b_trans, b_row, c_row, kahan=False):
    """Runs the fp32 restatement with B / C stored in the requested orders; returns C (m, n)."""
    Bl = b.reshape(n, k) if b_trans else b.reshape(k, n)  # logical storage shape of B
    store_b = Bl if b_row else Bl.T
    ldb = Bl.shape[1] if b_row else Bl.shape[0]
    contig = b_row != b_trans
    C = c.reshape(m, n)
    store_c = C if c_row else C.T
    out = oracle.spmm_f32(m, k, n, rp, col, val.astype(np.float32), base, np.ascontiguousarray(store_b, np.float32),
                          ldb, contig, np.ascontiguousarray(store_c, np.float32), n if c_row else m, c_row, alpha, beta,
                          kahan)
    return out.reshape(m, n) if c_row else out.reshape(n, m).T


@pytest.mark.parametrize("b_trans", [False, True])
def test_f32_restatement_within_fp32_of_golden_in_every_layout(b_trans):
    m, k, n = 45, 31, 27
    rp, col, val, b, c = _case(m, k, n, 0.5, 5)
    gold = oracle.spmm_golden_f64(m, k, n, rp, col, val.astype(np.float32).astype(np.float64), 0,
                                  b.astype(np.float32).astype(np.float64), b_trans,
                                  c.astype(np.float32).astype(np.float64), 0.75, 0.5).reshape(m, n)
    outs = [_f32(m, k, n, rp, col, val, 0, b, c, 0.75, 0.5, b_trans, br, cr) for br in (1, 0) for cr in (1, 0)]
    for o in outs[1:]:
        np.testing.assert_array_equal(o, outs[0])
    lens = np.diff(rp)[:, None]
    np.testing.assert_allclose(outs[0], gold, rtol=0, atol=float(4 * lens.max() * 2.0 ** -24 * np.abs(gold).max()))


def test_kahan_beats_plain_sum_on_cancelling_rows():
    m, k, n = 8, 4000, 4
    rng = np.random.default_rng(1)
    rp = np.arange(m + 1, dtype=np.int64) * k
    col = np.tile(np.arange(k, dtype=np.int32), m)
    val = np.where(np.arange(m * k) % 2 == 0, 1.0, -1.0) * (1.0 + rng.uniform(0, 1e-3, m * k))
    val = val.astype(np.float32).astype(np.float64)
    b = rng.uniform(0.5, 1.5, k * n).astype(np.float32).astype(np.float64)
    c = np.zeros(m * n)
    gold = oracle.spmm_golden_f64(m, k, n, rp, col, val, 0, b, False, c, 1.0, 0.0).reshape(m, n)
    plain = _f32(m, k, n, rp, col, val, 0, b, c, 1.0, 0.0, False, 1, 1)
    kahan = _f32(m, k, n, rp, col, val, 0, b, c, 1.0, 0.0, False, 1, 1, kahan=True)
    assert np.abs(kahan - gold).max() < 0.25 * np.abs(plain - gold).max()


def test_fp16_store_is_clamp_then_ties_away():
    m, k, n = 4, 3, 5
    rp = np.array([0, 1, 2, 3, 3], np.int64)
    col = np.array([0, 1, 2], np.int32)
    val = np.array([1.0, 1.0, 1.0])
    b = np.array([70000.0, -70000.0, 2.0 ** -25, 1.0, 1.5,
                  1.0 + 2.0 ** -11, -(1.0 + 3 * 2.0 ** -11), 3.0, -5.0, 0.0,
                  2048.0 + 1.0, 1.0e-8, -0.0, 7.0, 8.0])
    out = oracle.spmm_f32(m, k, n, rp, col, val, 0, b, n, 1, np.zeros(m * n, np.float32), n, 1, 1.0, 0.0,
                          half_out=True).reshape(m, n)
    row = lambda i: b[5 * i:5 * i + 5].astype(np.float32)
    for i in range(3):
        v = np.clip(row(i), -65504, 65504)
        np.testing.assert_array_equal(out[i], oracle.half_from_float_away(v).view(np.float16).astype(np.float32))
    np.testing.assert_array_equal(out[3], 0.0)  # empty row: alpha * 0
    assert out[0, 0] == 65504.0 and out[0, 1] == -65504.0 and out[1, 0] == 1.0 + 2.0 ** -10
    assert out[2, 0] == 2050.0  # 2049 is a midpoint of fp16 spacing 2: away from zero


def test_sparsity_pattern_and_row_shuffle():
    rp, col, val = oracle.spmm_sparsity(4, 4, 0.5, -1, 1, 9)
    # key(i, j) = (7i + 13j) % 100 < 50: rows 0 and 1 full, rows 2 and 3 drop j = 3 (53, 60)
    np.testing.assert_array_equal(rp, [0, 4, 8, 11, 14])
    np.testing.assert_array_equal(col, [0, 1, 2, 3, 0, 1, 2, 3, 0, 1, 2, 0, 1, 2])
    np.testing.assert_array_equal(val, oracle.uniform_real(9, -1, 1, 14))
    m, k, n = 50, 40, 6
    rp0, col0, val0 = oracle.spmm_sparsity(m, k, 0.6, -1, 1, 3)
    rp1, col1, val1 = oracle.spmm_sparsity(m, k, 0.6, -1, 1, 3, unsorted=True)
    np.testing.assert_array_equal(rp0, rp1)
    assert not np.array_equal(col0, col1)
    for i in range(m):
        s, e = rp0[i], rp0[i + 1]
        o0, o1 = np.argsort(col0[s:e]), np.argsort(col1[s:e])
        np.testing.assert_array_equal(col0[s:e][o0], col1[s:e][o1])
        np.testing.assert_array_equal(val0[s:e][o0], val1[s:e][o1])
    b = oracle.uniform_real(7, -1, 1, k * n)
    c = np.zeros(m * n)
    g0 = oracle.spmm_golden_f64(m, k, n, rp0, col0, val0, 0, b, False, c, 1.0, 0.0)
    g1 = oracle.spmm_golden_f64(m, k, n, rp1, col1, val1, 0, b, False, c, 1.0, 0.0)
    np.testing.assert_allclose(g0, g1, rtol=1e-12, atol=1e-12)
    rpb, colb, _ = oracle.spmm_sparsity(4, 4, 0.5, -1, 1, 9, base=1)
    np.testing.assert_array_equal(rpb, rp + 1)
    np.testing.assert_array_equal(colb, col + 1)


def test_frame_mixed_verifier():
    g = np.linspace(-2, 2, 1000).astype(np.float32)
    assert oracle.verify_frame_mixed(g, g, "float32")[0]
    a = g.copy()
    a[:5] += 1e-3  # 0.5% beyond atol + rtol*|g|, inside the 1e-2 hard limit
    ok, ratio, _ = oracle.verify_frame_mixed(g, a, "float32")
    assert ok and ratio == pytest.approx(0.995)
    a[:20] += 1e-3  # 2% fail
    assert not oracle.verify_frame_mixed(g, a, "float32")[0]
    a = g.copy()
    a[0] += 0.02  # one element beyond max(1e-2, 32 ulp)
    assert not oracle.verify_frame_mixed(g, a, "float32")[0]
    a = g.copy()
    a[0] = np.nan
    assert not oracle.verify_frame_mixed(g, a, "float32")[0]
    h = np.linspace(-2, 2, 1000).astype(np.float16).astype(np.float32)
    assert oracle.verify_frame_mixed(h, h + np.float32(5e-4), "float16")[0]


def _uniform_float(seed, lo, hi, count):
    """libstdc++ uniform_real_distribution<float>: generate_canonical<float, 24> takes one
    32-bit word, float(w) / 2^32 (in float), then u * (hi - lo) + lo in float."""
    w = oracle.mt19937(seed, count).astype(np.float32)
    u = w / np.float32(4294967296.0)
    u = np.where(u >= 1, np.nextafter(np.float32(1), np.float32(0)), u).astype(np.float32)
    return (u * np.float32(hi - lo) + np.float32(lo)).astype(np.float32)


def test_spmvop_inputs_follow_the_reference_generator():
    """SpMVOp test inputs (oracle/spmvop_inputs.cpp): x and y are the float draws of
    mt19937(seed+1) / mt19937(seed+2) in [-3, 3]; rows hold distinct sorted columns (shuffled
    row-wise for unsorted cases, same multiset), values in [-5, 5], lengths near the binomial
    mean; diag and empty patterns; the same call gives the same bits."""
    m, k, seed = 300, 200, 77
    rp, col, val, x, y = oracle.spmvop_inputs(m, k, 0.9, 0.0, seed)
    np.testing.assert_array_equal(x, _uniform_float(seed + 1, -3.0, 3.0, k))
    np.testing.assert_array_equal(y, _uniform_float(seed + 2, -3.0, 3.0, m))
    lens = np.diff(rp)
    assert abs(lens.mean() - 0.1 * k) < 3 and np.all(lens >= 0)
    for i in range(m):
        c = col[rp[i]:rp[i + 1]]
        assert np.all(np.diff(c) > 0) and (c.size == 0 or (c[0] >= 0 and c[-1] < k))
    assert np.all(np.abs(val) <= 5.0) and np.all(np.isfinite(val))
    rp2, col2, val2, _, _ = oracle.spmvop_inputs(m, k, 0.9, 0.0, seed)
    np.testing.assert_array_equal(col, col2)
    np.testing.assert_array_equal(val, val2)
    rpu, colu, valu, _, _ = oracle.spmvop_inputs(m, k, 0.9, 0.0, seed, unsorted=True)
    np.testing.assert_array_equal(rpu, rp)
    assert not np.array_equal(colu, col)
    for i in range(m):
        s, e = rp[i], rp[i + 1]
        o = np.argsort(colu[s:e])
        np.testing.assert_array_equal(colu[s:e][o], col[s:e])
        np.testing.assert_array_equal(valu[s:e][o], val[s:e])
    rpe, cole, _, _, _ = oracle.spmvop_inputs(m, k, 0.5, 0.9, seed)  # 90% empty rows
    assert (np.diff(rpe) == 0).mean() > 0.8
    rpd, cold, vald, _, _ = oracle.spmvop_inputs(5, 5, 0.0, 0.0, 1, "diag")
    np.testing.assert_array_equal(rpd, np.arange(6))
    np.testing.assert_array_equal(cold, np.arange(5))
    np.testing.assert_array_equal(vald, np.ones(5, np.float32))
    rpz, colz, _, _, _ = oracle.spmvop_inputs(4, 3, 0.5, 0.0, 1, "empty")
    assert colz.size == 0 and np.all(rpz == 0)
    # dense rows (sparsity 0): the attempt budget runs out and the row completes from the unused columns
    rpf, colf, _, _, _ = oracle.spmvop_inputs(20, 50, 0.0, 0.0, 3)
    np.testing.assert_array_equal(np.diff(rpf), np.full(20, 50))
