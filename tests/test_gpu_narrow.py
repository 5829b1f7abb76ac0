"""GPU parity of the narrow-column row kernel through the C ABI.

For non-transpose matrices of at least 2^20 entries with fp32 / fp16 / bf16
values and fp32 compute (or int8 values with int32 compute), Preprocess writes
every entry's column as a signed 16-bit offset from the first row of its row
block when all of them fit, and the row kernel streams that copy (2 bytes per
entry) instead of col_ind (4 bytes).  The header's path flag reads 5 when the
entry-aligned row blocks fit (every 480-entry chunk's rows end within 512
entries and number at most 127: a wave loads its window before its block's
metadata arrives), else 3 (the merge-path blocks).  On the merge-path blocks
the sums are the col_ind kernel's, in the same order, so those cases are also
checked bit for bit against the SpMV without Preprocess (flag 0); every case
is checked against the oracle.
"""
import numpy as np
import pytest
import torch

import oracle
from helpers import assert_close
from ops_sparse import workloads as wl
from ops_sparse.spmv import CsrSpMV

pytestmark = pytest.mark.gpu

NARROW_MIN_NNZ = 1 << 20
NARROW = 3         # path flag: row kernel on the 16-bit copies, merge-path row blocks
ENTRY = 5          # path flag: the same on entry-aligned row blocks (loads issued before the block's metadata)
ENTRY_CHUNK = 480  # entries per entry-aligned block


def flag(plan):
    h = np.frombuffer(plan.workspace[:192].cpu().numpy().tobytes(), dtype=np.uint32)
    return int(h[32]), int(h[40])  # staged_flag, narrow_bad


def bits(t):
    return t.view(torch.int16) if t.element_size() == 2 else t.view(torch.int32)


def run(w, preprocess=True, y0=None, settle=True):
    y = (w.y0 if y0 is None else y0).to(w.out_dtype).clone()
    plan = CsrSpMV(w.rows, w.cols, w.row_ptr, w.col_ind, w.values, w.x, y, w.alpha, w.beta,
                   base=w.meta.get("base", 0))
    if preprocess:
        plan.preprocess()
        if settle:
            torch.cuda.synchronize()  # the path choice reaches the host: one kernel set launched
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


def check(w, expect_flag, y0=None):
    """Oracle parity, the expected path, bit equality with the first SpMV after Preprocess (issued
    before the choice reached the host: every kernel set launched, each gated on the device flag) and,
    on the merge-path blocks, with the col_ind kernel (no Preprocess)."""
    y, plan = run(w, y0=y0)
    assert flag(plan)[0] == expect_flag
    assert_close(host(w), y)
    y_plain, plan0 = run(w, preprocess=False, y0=y0)
    assert flag(plan0)[0] == 0
    if expect_flag == NARROW:  # the same row blocks: the same sums in the same order
        assert torch.equal(bits(y), bits(y_plain))
    else:  # other row blocks: a row that crossed a chunk edge is summed in another order
        assert_close(host(w), y_plain)
    y_first, _ = run(w, y0=y0, settle=False)
    assert torch.equal(bits(y), bits(y_first))
    return y, plan


def banded(dev, rows, band, vdtype=torch.float32, rdtype=torch.int32, base=0, alpha=1.25, beta=0.5, seed=4,
           spread=1):
    """Rows of `band` entries at columns row + spread*(j - band//2), clipped to the matrix."""
    g = torch.Generator(device="cpu")
    g.manual_seed(seed)
    off = (torch.arange(band) - band // 2) * spread
    col = (torch.arange(rows)[:, None] + off[None, :]).clamp(0, rows - 1).reshape(-1)
    rp = torch.arange(0, rows * band + 1, band, dtype=torch.int64)
    vals = (torch.rand(col.numel(), generator=g) * 2 - 1).to(vdtype)
    x = (torch.rand(rows, generator=g) * 2 - 1).to(vdtype)
    out = torch.float32 if vdtype == torch.float32 else vdtype
    y0 = (torch.rand(rows, generator=g) * 2 - 1).to(out)
    w = wl.Workload(f"banded{band}_{rows}", rows, rows, (rp + base).to(rdtype), (col + base).to(torch.int32),
                    vals, x, y0, alpha, beta, out_dtype=out, meta={"base": base})
    return w.to(dev)


def test_laplacian_c2_takes_the_narrow_kernel(dev):
    w = wl.laplacian_2d().to(dev)
    check(w, ENTRY)


@pytest.mark.parametrize("vdtype", [torch.float16, torch.bfloat16], ids=["f16", "bf16"])
def test_half_values_int64_offsets_base1(vdtype, dev):
    w = banded(dev, rows=1 << 18, band=9, vdtype=vdtype, rdtype=torch.int64, base=1, spread=3000)
    check(w, ENTRY)


def entry_block_first_rows(row_ptr):
    """First row of each row's entry-aligned block: block t holds the rows starting in [480 t, 480 (t+1))."""
    rp = row_ptr.cpu().numpy().astype(np.int64)
    rp = rp - rp[0]
    t = rp[:-1] // ENTRY_CHUNK
    return torch.from_numpy(np.searchsorted(rp, t * ENTRY_CHUNK, side="left").astype(np.int64))


def test_offsets_at_the_16_bit_limits(dev):
    """Columns at offsets -32768 and +32767 from the first row of their block fit; one more does not."""
    rows, band = 1 << 17, 9
    w = banded(dev, rows=rows, band=band, spread=1)
    r0 = entry_block_first_rows(w.row_ptr).to(dev)
    col = w.col_ind.view(rows, band).clone()
    lo, hi = r0 - 32768, r0 + 32767
    col[:, 0] = torch.where(lo >= 0, lo, col[:, 0].to(torch.int64)).to(torch.int32)
    col[:, -1] = torch.where(hi < rows, hi, col[:, -1].to(torch.int64)).to(torch.int32)
    w.col_ind = col.reshape(-1).contiguous()
    assert int((w.col_ind.view(rows, band)[:, 0].to(torch.int64) - r0).min()) == -32768
    assert int((w.col_ind.view(rows, band)[:, -1].to(torch.int64) - r0).max()) == 32767
    check(w, ENTRY)
    for delta in (-32769, 32768):
        far = w.col_ind.clone()
        i = rows // 2
        c = int(r0[i]) + delta
        assert 0 <= c < rows
        far[i * band + (0 if delta < 0 else band - 1)] = c
        w2 = wl.Workload(w.name, w.rows, w.cols, w.row_ptr, far, w.values, w.x, w.y0, w.alpha, w.beta,
                         out_dtype=w.out_dtype, meta=w.meta)
        y, plan = run(w2)
        assert flag(plan) == (0, 1)
        assert_close(host(w2), y)


def test_long_rows_run_as_tasks(dev):
    """Rows of 3000 entries within +-1500 columns: blocks of one row, split into chunk tasks (too long for
    the entry-aligned blocks' 512-entry windows: flag 3)."""
    rows = 1 << 10
    w = banded(dev, rows=rows, band=3001, spread=1, beta=0.0)
    assert w.nnz >= NARROW_MIN_NNZ
    y, _ = check(w, NARROW, y0=torch.full_like(w.y0, float("nan")))  # beta = 0: y is never read
    assert bool(torch.isfinite(y).all())


def test_entries_outside_the_rows_are_ignored(dev):
    w = banded(dev, rows=1 << 18, band=5, spread=700)
    lead = 5
    w.row_ptr = w.row_ptr + lead
    w.col_ind = torch.cat([torch.full((lead,), 1 << 30, dtype=torch.int32, device=dev), w.col_ind])
    w.values = torch.cat([torch.full((lead,), 1e6, device=dev), w.values])
    check(w, ENTRY)


def test_small_matrices_keep_col_ind(dev):
    w = banded(dev, rows=1 << 16, band=5)
    assert w.nnz < NARROW_MIN_NNZ
    y, plan = run(w)
    assert flag(plan)[0] == 0
    assert_close(host(w), y)


def test_values_updated_after_preprocess(dev):
    """Preprocess reads the pattern only: new values and x are used by the next SpMV."""
    w = banded(dev, rows=1 << 18, band=7, spread=100)
    y, plan = run(w)
    assert flag(plan)[0] == ENTRY
    w.values.mul_(-0.5).add_(0.25)
    w.x.copy_(torch.flip(w.x, [0]))
    y.copy_(w.y0)
    plan.run()
    torch.cuda.synchronize()
    assert_close(host(w), y)


def test_narrow_spmv_in_a_hip_graph(dev):
    from test_gpu_staged import _graph_matches_eager
    w = banded(dev, rows=1 << 18, band=11, vdtype=torch.float16, spread=50)
    plan = _graph_matches_eager(w, dev)
    assert flag(plan)[0] == ENTRY


def int8_case(dev, rows, band, spread, alpha, beta, seed=7, extreme=False, i64=False):
    g = torch.Generator(device="cpu")
    g.manual_seed(seed)
    off = (torch.arange(band) - band // 2) * spread
    col = (torch.arange(rows)[:, None] + off[None, :]).clamp(0, rows - 1).reshape(-1).to(torch.int32)
    rp = torch.arange(0, rows * band + 1, band, dtype=torch.int64)
    if extreme:  # every product 16384 (or -16384 for negative x): row sums far beyond 2^24
        val = torch.full((col.numel(),), -128, dtype=torch.int8)
        x = torch.where(torch.rand(rows, generator=g) < 0.5, -128, 127).to(torch.int8)
    else:
        val = torch.randint(-128, 128, (col.numel(),), generator=g, dtype=torch.int8)
        x = torch.randint(-128, 128, (rows,), generator=g, dtype=torch.int8)
    y0 = torch.randint(-(1 << 30), 1 << 30, (rows,), generator=g, dtype=torch.int32)
    ref = oracle.spmv_i8(rp.numpy(), col.numpy(), val.numpy(), x.numpy(), y0.numpy(), alpha, beta)
    rpd = rp.to(torch.int64 if i64 else torch.int32).to(dev)
    return (rows, rpd, col.to(dev), val.to(dev), x.to(dev), y0.to(dev)), ref


def run_int8(args, alpha, beta, preprocess=True, settle=True):
    from ops_sparse._lib import DataType
    rows, rp, col, val, x, y0 = args
    y = y0.clone()
    plan = CsrSpMV(rows, rows, rp, col, val, x, y, alpha, beta, compute_type=DataType.INT32)
    if preprocess:
        plan.preprocess()
        if settle:
            torch.cuda.synchronize()
    plan.run()
    torch.cuda.synchronize()
    return y, plan


@pytest.mark.parametrize("i64", [False, True], ids=["i32", "i64"])
def test_int8_narrow_exact(i64, dev):
    """int8 values and x, int32 y: the fp32 row kernel on the narrow copy, bit-exact against the int64
    oracle (saturating epilogue), and equal to the col_ind kernel and to the first SpMV after Preprocess."""
    args, ref = int8_case(dev, rows=1 << 18, band=9, spread=1000, alpha=3, beta=-2, i64=i64)
    y, plan = run_int8(args, 3, -2)
    assert flag(plan)[0] == ENTRY
    np.testing.assert_array_equal(y.cpu().numpy(), ref)
    y0, plan0 = run_int8(args, 3, -2, preprocess=False)
    assert flag(plan0)[0] == 0
    np.testing.assert_array_equal(y0.cpu().numpy(), ref)
    y1, _ = run_int8(args, 3, -2, settle=False)
    np.testing.assert_array_equal(y1.cpu().numpy(), ref)


def test_int8_long_rows_beyond_fp32_exactness(dev):
    """Rows of 3001 products of magnitude 16384 (sums near 2^25.6, past fp32's exact integers) split over
    several chunks, and an alpha that saturates some rows: exact, on the narrow copy and on col_ind."""
    args, ref = int8_case(dev, rows=1 << 10, band=3001, spread=1, alpha=50, beta=1, extreme=True)
    sat = (ref == 2147483647) | (ref == -2147483648)
    assert np.any(sat) and not np.all(sat)
    y, plan = run_int8(args, 50, 1)
    assert flag(plan)[0] == NARROW
    np.testing.assert_array_equal(y.cpu().numpy(), ref)
    y0, _ = run_int8(args, 50, 1, preprocess=False)
    np.testing.assert_array_equal(y0.cpu().numpy(), ref)


def test_many_empty_rows_keep_the_merge_path_blocks(dev):
    """Every other row empty and rows of 2 entries: 480 entries span 480 rows, more than a wave's 127, so the
    entry-aligned blocks do not fit and the narrow copy follows the merge-path blocks (flag 3)."""
    rows = 1 << 20
    g = torch.Generator(device="cpu")
    g.manual_seed(21)
    lengths = torch.where(torch.arange(rows) % 2 == 0, 2, 0).to(torch.int64)
    rp = torch.zeros(rows + 1, dtype=torch.int64)
    rp[1:] = torch.cumsum(lengths, 0)
    r = torch.repeat_interleave(torch.arange(rows), lengths)
    col = (r + torch.randint(-500, 500, (r.numel(),), generator=g)).clamp(0, rows - 1).to(torch.int32)
    vals = torch.rand(col.numel(), generator=g) * 2 - 1
    x = torch.rand(rows, generator=g) * 2 - 1
    y0 = torch.rand(rows, generator=g) * 2 - 1
    w = wl.Workload("alternate_empty", rows, rows, rp.to(torch.int32), col, vals, x, y0, 1.0, 0.5).to(dev)
    assert w.nnz >= NARROW_MIN_NNZ
    check(w, NARROW)
