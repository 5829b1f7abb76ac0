"""GPU parity of the column-bucketed transpose (fp32 values, opA = T or H) through the C ABI.

Preprocess takes this path for fp32 transposes of at least 2^20 entries when
every bucket of columns fits pass 2's LDS; each test reads the choice from the
workspace header (staged_flag) so that a case meant for the bucketed kernels
cannot pass on the CSC kernels, and the other way round.
"""
import ctypes

import numpy as np
import pytest
import torch

from helpers import assert_close
from ops_sparse._lib import Operation, PointerMode
from ops_sparse.spmv import CsrSpMV
from ops_sparse import workloads as wl

pytestmark = pytest.mark.gpu

REGION_TARGET = 24576
REGION_CAP = 32768


def header(plan):
    h = np.frombuffer(plan.workspace[:192].cpu().numpy().tobytes(), dtype=np.uint64)
    return int(h[16] & 0xFFFFFFFF), int(h[16] >> 32), int(h[17])


def bucket_width(cols, nnz):
    target = REGION_TARGET * cols // nnz
    shift = 6
    while shift < 16 and (2 << shift) <= target:
        shift += 1
    return 1 << shift


def run(w, op=Operation.TRANSPOSE, preprocess=True, y0=None):
    y = (w.y0 if y0 is None else y0).clone()
    plan = CsrSpMV(w.rows, w.cols, w.row_ptr, w.col_ind, w.values, w.x, y, w.alpha, w.beta, op=op,
                   base=w.meta.get("base", 0))
    if preprocess:
        plan.preprocess()
    plan.run()
    torch.cuda.synchronize()
    return y, plan


def host(w):
    h = w.to("cpu")
    b = w.meta.get("base", 0)
    if b:
        h.col_ind = h.col_ind - b
        h.row_ptr = h.row_ptr - b
    return h


def transpose_workload(dev, rows, cols, mean, seed, base=0, rdtype=torch.int32, alpha=1.0, beta=2.0):
    g = torch.Generator(device="cpu")
    g.manual_seed(seed)
    lengths = torch.poisson(torch.full((rows,), mean), generator=g).to(torch.int64)
    row_ptr, col = wl.csr_from_lengths(lengths, cols, g, "cpu", distinct=False)
    n = col.numel()
    vals = torch.rand(n, generator=g) * 2 - 1
    x = torch.rand(rows, generator=g) * 2 - 1
    y0 = torch.rand(cols, generator=g) * 2 - 1
    w = wl.Workload(f"bt_{rows}x{cols}", rows, cols, (row_ptr + base).to(rdtype), (col + base).to(torch.int32),
                    vals, x, y0, alpha, beta, trans="T", meta={"base": base})
    return w.to(dev)


def test_c5_takes_the_bucketed_path_and_matches_oracle(dev):
    w = wl.poisson_transpose().to(dev)
    y, plan = run(w)
    flag, buckets, tiles = header(plan)
    assert flag == 1, "c5's buckets fit the column pass's LDS: the bucketed kernels run"
    assert buckets == -(-w.cols // bucket_width(w.cols, w.nnz))
    assert_close(w.to("cpu"), y)
    # again from the same y: bit-identical (every column is summed in row order), on a new plan
    # (its first SpMV launches both kernel sets, which read the device flag) and on this plan
    # once Preprocess's choice has reached the host (only the bucketed kernels are launched)
    y3, _ = run(w)
    assert torch.equal(y.view(torch.int32), y3.view(torch.int32))
    first = y.clone()
    y.copy_(w.y0)
    plan.run()
    torch.cuda.synchronize()
    assert torch.equal(first.view(torch.int32), y.view(torch.int32))


def test_conjugate_transpose_int64_base1_beta0_ignores_nan_y(dev):
    w = transpose_workload(dev, rows=1 << 20, cols=3 << 18, mean=9.0, seed=5, base=1, rdtype=torch.int64,
                           alpha=-1.5, beta=0.0)
    y0 = torch.full((w.cols,), float("nan"), device=dev)
    y, plan = run(w, op=Operation.CONJUGATE_TRANSPOSE, y0=y0)
    assert header(plan)[0] == 1
    assert bool(torch.isfinite(y).all())
    assert_close(host(w), y)


def test_rectangular_device_scalars(dev):
    w = transpose_workload(dev, rows=3 << 20, cols=1 << 20, mean=2.0, seed=8, alpha=0.75, beta=-0.5)
    y = w.y0.clone()
    plan = CsrSpMV(w.rows, w.cols, w.row_ptr, w.col_ind, w.values, w.x, y, 1.0, 0.0, op=Operation.TRANSPOSE)
    plan.handle.set_pointer_mode(PointerMode.DEVICE)
    da = torch.tensor([0.75], device=dev)
    db = torch.tensor([-0.5], device=dev)
    plan.alpha = type("P", (), {"ptr": ctypes.c_void_p(da.data_ptr())})()
    plan.beta = type("P", (), {"ptr": ctypes.c_void_p(db.data_ptr())})()
    plan.preprocess()
    plan.run()
    torch.cuda.synchronize()
    assert header(plan)[0] == 1
    assert_close(w.to("cpu"), y)


def test_a_giant_column_keeps_the_csc_kernels(dev):
    """One column holding more entries than pass 2's LDS: Preprocess keeps the CSC kernels."""
    w = transpose_workload(dev, rows=1 << 20, cols=1 << 20, mean=3.0, seed=9)
    col = w.col_ind.clone()
    g = torch.Generator(device=dev)
    g.manual_seed(3)
    hot = torch.rand(col.numel(), generator=g, device=dev) < (2 * REGION_CAP) / col.numel()
    col[hot] = 12345
    w.col_ind = col
    y, plan = run(w)
    assert header(plan)[0] == 0
    assert_close(w.to("cpu"), y)


def test_entries_outside_the_rows_are_ignored(dev):
    """row_ptr[0] > 0: the leading entries belong to no row and must not reach y."""
    w = transpose_workload(dev, rows=1 << 20, cols=1 << 19, mean=4.0, seed=10)
    lead = 7
    w.row_ptr = w.row_ptr + lead
    w.col_ind = torch.cat([torch.arange(lead, dtype=torch.int32, device=dev), w.col_ind])
    w.values = torch.cat([torch.full((lead,), 1e6, device=dev), w.values])
    y, plan = run(w)
    assert header(plan)[0] == 1
    assert_close(w.to("cpu"), y)


def test_without_preprocess_runs_the_csc_kernels(dev):
    w = transpose_workload(dev, rows=1 << 20, cols=1 << 20, mean=6.0, seed=11)
    y, plan = run(w, preprocess=False)
    assert header(plan)[0] == 0
    assert_close(w.to("cpu"), y)


def banded_workload(dev, n=1536, beta=0.5, base=0):
    """A 5-point Laplacian (banded, long runs per tile) as a transpose workload."""
    w = wl.laplacian_2d(n=n)
    w = wl.Workload(w.name + "_T", w.rows, w.cols, (w.row_ptr + base).to(torch.int32),
                    (w.col_ind + base).to(torch.int32), w.values * (1.0 + 0.25 * torch.rand(w.nnz)),
                    w.x, w.y0, 1.5, beta, trans="T", meta={"base": base})
    return w.to(dev)


def test_banded_transpose_takes_the_one_pass_kernel(dev):
    """Long runs: Preprocess picks the one-pass banded column kernel, on its 16-bit copies (flag 4: every
    entry's row within 16 bits of its CSC block's first column, its CSR position within 16 bits of its CSC
    index); repeated runs are
    bit-identical on a new plan (every kernel set launched, gated on the device flag) and on this plan
    once the choice has reached the host (only the banded kernel launched)."""
    w = banded_workload(dev)
    assert w.nnz >= 1 << 20
    y, plan = run(w)
    assert header(plan)[0] == 4
    assert_close(w.to("cpu"), y)
    y3, _ = run(w)
    assert torch.equal(y.view(torch.int32), y3.view(torch.int32))
    first = y.clone()
    y.copy_(w.y0)
    plan.run()
    torch.cuda.synchronize()
    assert torch.equal(first.view(torch.int32), y.view(torch.int32))


def test_banded_conjugate_transpose_base1_beta0_ignores_nan_y(dev):
    w = banded_workload(dev, n=1100, beta=0.0, base=1)
    y0 = torch.full((w.cols,), float("nan"), device=dev)
    y, plan = run(w, op=Operation.CONJUGATE_TRANSPOSE, y0=y0)
    assert header(plan)[0] == 4
    assert bool(torch.isfinite(y).all())
    assert_close(host(w), y)


def test_banded_transpose_int64_offsets_keeps_the_csc_kernels(dev):
    """The one-pass banded kernel takes 32-bit row offsets: with int64 offsets Preprocess keeps the
    CSC kernels (flag 0) and the result is still right, on the first SpMV (every kernel set launched)
    and once the choice is on the host."""
    w = banded_workload(dev, n=1100)
    w.row_ptr = w.row_ptr.to(torch.int64)
    y, plan = run(w)
    assert header(plan)[0] == 0
    assert_close(w.to("cpu"), y)
    first = y.clone()
    y.copy_(w.y0)
    plan.run()
    torch.cuda.synchronize()
    assert torch.equal(first.view(torch.int32), y.view(torch.int32))


def test_banded_transpose_far_band_keeps_32_bit_streams(dev):
    """A Laplacian plus a band 40 000 columns off the diagonal: still banded (long runs, flag 2), but those
    entries' rows and positions are out of 16-bit reach, so the kernel streams the 32-bit arrays; the result
    is checked against the oracle and is bit-identical on a second run."""
    n = 1100
    m = n * n
    i = torch.arange(m, dtype=torch.int64)
    cols = [i - n, i - 1, i, i + 1, i + n, i + 40000]
    r = torch.cat([i] * len(cols))
    c = torch.cat(cols)
    ok = (c >= 0) & (c < m)
    r, c = r[ok], c[ok]
    order = torch.argsort(r * m + c)
    r, c = r[order], c[order]
    row_ptr = torch.zeros(m + 1, dtype=torch.int64)
    row_ptr[1:] = torch.cumsum(torch.bincount(r, minlength=m), 0)
    g = torch.Generator(device="cpu")
    g.manual_seed(12)
    vals = torch.rand(c.numel(), generator=g) * 2 - 1
    x = torch.rand(m, generator=g) * 2 - 1
    y0 = torch.rand(m, generator=g) * 2 - 1
    w = wl.Workload("laplace_far_T", m, m, row_ptr.to(torch.int32), c.to(torch.int32), vals, x, y0, 1.25, -0.5,
                    trans="T").to(dev)
    y, plan = run(w)
    flag, _, _ = header(plan)
    assert flag == 2
    assert_close(w.to("cpu"), y)
    first = y.clone()
    y.copy_(w.y0)
    plan.run()
    torch.cuda.synchronize()
    assert torch.equal(first.view(torch.int32), y.view(torch.int32))


@pytest.mark.parametrize("extra", [5000, 9000])
def test_banded_transpose_long_column_tasks(dev, extra):
    """A Laplacian plus one column holding `extra` more entries (rows within extra/2 of it): still the
    one-pass banded kernel on 16-bit copies (flag 4), with that column's block several chunks long, so
    it is summed by tasks whose partial sums are combined; checked against the oracle and bit-identical
    on a second run."""
    n = 1100
    m = n * n
    i = torch.arange(m, dtype=torch.int64)
    r = torch.cat([i] * 5)
    c = torch.cat([i - n, i - 1, i, i + 1, i + n])
    c0 = m // 2 + 17
    rr = torch.arange(c0 - extra // 2, c0 + extra // 2 + 1, dtype=torch.int64)
    r = torch.cat([r, rr])
    c = torch.cat([c, torch.full_like(rr, c0)])
    ok = (c >= 0) & (c < m)
    key = torch.unique(r[ok] * m + c[ok])
    r, c = key // m, key % m
    row_ptr = torch.zeros(m + 1, dtype=torch.int64)
    row_ptr[1:] = torch.cumsum(torch.bincount(r, minlength=m), 0)
    g = torch.Generator(device="cpu")
    g.manual_seed(extra)
    vals = torch.rand(c.numel(), generator=g) * 2 - 1
    x = torch.rand(m, generator=g) * 2 - 1
    y0 = torch.rand(m, generator=g) * 2 - 1
    w = wl.Workload("laplace_longcol_T", m, m, row_ptr.to(torch.int32), c.to(torch.int32), vals, x, y0, 0.75, 1.5,
                    trans="T").to(dev)
    y, plan = run(w)
    assert header(plan)[0] == 4
    assert_close(w.to("cpu"), y)
    first = y.clone()
    y.copy_(w.y0)
    plan.run()
    torch.cuda.synchronize()
    assert torch.equal(first.view(torch.int32), y.view(torch.int32))


@pytest.mark.parametrize("tail", [1, 2, 3, 5, 7, 8])
def test_entry_counts_of_every_remainder_mod_8(dev, tail):
    """nnz = 8q + tail (tail = 8: a multiple of 8): pass 2 reads each bucket's products and places
    by 16-byte loads from an 8-entry boundary, so the last bucket's final loads cross the end of the
    arrays at every offset; every column, the last (partial) bucket's included, must match the
    oracle."""
    w = transpose_workload(dev, rows=1 << 20, cols=(1 << 20) + 1237 * tail, mean=5.0, seed=20 + tail)
    keep = (w.nnz // 8 - 1) * 8 + tail
    drop = w.nnz - keep
    rp = w.row_ptr.clone()
    rp[-1] -= drop  # the last rows lose their final entries
    rp = torch.minimum(rp, rp[-1])
    w.row_ptr = rp
    w.col_ind = w.col_ind[:keep].contiguous()
    w.values = w.values[:keep].contiguous()
    assert w.nnz == keep and keep % 8 == tail % 8
    y, plan = run(w)
    assert header(plan)[0] == 1
    assert_close(w.to("cpu"), y)


def test_random_pattern_with_few_wide_buckets_takes_the_bucketed_kernels(dev):
    """2 M random entries over 1 M columns: the buckets are few and wide, so the tiles' runs are long
    (about 110 entries), but every tile has a run in every bucket: the pattern is scattered and the
    bucketed kernels take it (the one-pass banded kernel would gather every value from afar)."""
    w = transpose_workload(dev, rows=1 << 18, cols=1 << 20, mean=8.5, seed=31)
    assert w.nnz >= 1 << 21
    y, plan = run(w)
    flag, buckets, tiles = header(plan)
    assert flag == 1
    assert w.nnz / (buckets * tiles) > 64  # long runs, yet scattered
    assert_close(w.to("cpu"), y)


@pytest.mark.parametrize("seed", [41, 42])
def test_mixed_row_lengths_meet_the_middle_of_every_tile(dev, seed):
    """Rows of 0-120 entries (10% empty) with random columns: pass 1 spreads x and places the
    products half a tile at a time, so short rows, rows longer than 32 entries (spread by a wave)
    and empty rows meet the middle of the tile's entries, and runs cross the middle of its slots,
    at every offset.  Bit-identical on a second run."""
    rows, cols = 300_001, (1 << 20) + 77
    rng = np.random.default_rng(seed)
    lengths = torch.from_numpy(np.where(rng.random(rows) < 0.1, 0, rng.integers(1, 121, rows)).astype(np.int64))
    g = torch.Generator(device="cpu")
    g.manual_seed(seed)
    row_ptr, col = wl.csr_from_lengths(lengths, cols, g, "cpu", distinct=False)
    n = col.numel()
    w = wl.Workload(f"bt_mixed_{seed}", rows, cols, row_ptr.to(torch.int32), col.to(torch.int32),
                    torch.rand(n, generator=g) * 2 - 1, torch.rand(rows, generator=g) * 2 - 1,
                    torch.rand(cols, generator=g) * 2 - 1, 0.75, -1.0, trans="T").to(dev)
    y, plan = run(w)
    assert header(plan)[0] == 1
    assert_close(w.to("cpu"), y)
    y2, _ = run(w)
    assert torch.equal(y.view(torch.int32), y2.view(torch.int32))
