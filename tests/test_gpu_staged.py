"""GPU parity of the staged-gather path (x segments staged in LDS, merge-path tiles) through the C ABI.

The path is considered for non-transpose fp32-compute matrices of at least
2^22 entries whose x is at least 8 MiB (2^24 entries for an x of 1 to 8 MiB),
and taken when Preprocess finds the columns scattered; most cases here hold
33.5M+ entries (the oracle runs well under a second each), and the size rule
itself is checked at its edges.  Each test also reads the path
Preprocess chose from the workspace header, so a case meant for the staged
kernels cannot pass on the row kernels, and the other way round.
"""
import numpy as np
import pytest
import torch

import oracle
from helpers import assert_close
from ops_sparse import workloads as wl
from ops_sparse.spmv import CsrSpMV

pytestmark = pytest.mark.gpu

STAGE_MIN_NNZ = 1 << 25


def tile_items(values):
    """Rows + entries per merge-path tile: 8184 for fp32 values, 16376 for fp16 / bf16."""
    return 8184 if values.dtype == torch.float32 else 16376


def header(plan):
    """(staged_flag, buckets, tiles, tile_row_offset, tile_nnz_offset) from the workspace header."""
    h = np.frombuffer(plan.workspace[:192].cpu().numpy().tobytes(), dtype=np.uint64)
    return int(h[16] & 0xFFFFFFFF), int(h[16] >> 32), int(h[17]), int(h[18]), int(h[19])


def run(w, dev, preprocess=True):
    y = w.y0.to(w.out_dtype).clone()
    plan = CsrSpMV(w.rows, w.cols, w.row_ptr, w.col_ind, w.values, w.x, y, w.alpha, w.beta,
                   base=w.meta.get("base", 0))
    if preprocess:
        plan.preprocess()
    plan.run()
    torch.cuda.synchronize()
    return y, plan


def random_rows(dev, rows, cols, lengths, vdtype, rdtype, alpha=1.0, beta=0.0, seed=1, base=0):
    g = torch.Generator(device=dev)
    g.manual_seed(seed)
    row_ptr, col = wl.csr_from_lengths(lengths, cols, g, dev, distinct=False)
    n = col.numel()
    vals = (torch.rand(n, generator=g, device=dev) * 2 - 1).to(vdtype)
    x = (torch.rand(cols, generator=g, device=dev) * 2 - 1).to(vdtype)
    out = torch.float32 if vdtype == torch.float32 else vdtype
    y0 = (torch.rand(rows, generator=g, device=dev) * 2 - 1).to(out)
    w = wl.Workload(f"staged_{rows}x{cols}_{vdtype}", rows, cols, (row_ptr + base).to(rdtype),
                    (col + base).to(torch.int32), vals, x, y0, alpha, beta, out_dtype=out, meta={"base": base})
    return w


def host_workload(w):
    """The workload on the host with base-0 column indices (the oracle's convention)."""
    h = w.to("cpu")
    b = w.meta.get("base", 0)
    if b:
        h.col_ind = h.col_ind - b
        h.row_ptr = h.row_ptr - b
    return h


def check_tiles(w, plan):
    flag, buckets, tiles, tr_off, tn_off = header(plan)
    rp = w.row_ptr.cpu().numpy().astype(np.int64)
    rp = rp - rp[0]
    r_ref, e_ref = oracle.merge_path_tiles(rp, tile_items(w.values))
    assert tiles + 1 == r_ref.size
    ws = plan.workspace
    tr = np.frombuffer(ws[tr_off:tr_off + 4 * (tiles + 1)].cpu().numpy().tobytes(), dtype=np.int32)
    tn = np.frombuffer(ws[tn_off:tn_off + 8 * (tiles + 1)].cpu().numpy().tobytes(), dtype=np.int64)
    np.testing.assert_array_equal(tr, r_ref)
    np.testing.assert_array_equal(tn, e_ref)


CASES = [
    # (name, rows, cols, row lengths kind, value dtype, row offsets dtype, alpha, beta, base);
    # "giant" rows hold their columns in random order (the reference does not ask for sorted
    # columns), "giant_sorted" sorted: then a tile of the row touches few x lines and the
    # row kernels keep it
    ("uniform32_fp16_i64", 1 << 20, 1 << 22, "uniform32", torch.float16, torch.int64, 1.0, 0.0, 0),
    ("uniform32_bf16_i32_beta", 1 << 20, 1 << 22, "uniform32", torch.bfloat16, torch.int32, 1.5, -0.5, 0),
    ("uniform32_fp32_i32_base1", 1 << 20, 1 << 21, "uniform32", torch.float32, torch.int32, 1.5, 0.5, 1),
    ("zipf_fp32_i64_long_rows", 1 << 21, 1 << 21, "zipf", torch.float32, torch.int64, 1.0, 2.0, 0),
    ("one_giant_row_fp32", 1024, 1 << 22, "giant", torch.float32, torch.int32, -2.0, 1.0, 0),
    ("one_giant_sorted_row_fp32", 1024, 1 << 22, "giant_sorted", torch.float32, torch.int32, -2.0, 1.0, 0),
    ("sparse_rows_fp16", 3 << 23, 1 << 23, "sparse", torch.float16, torch.int64, 1.0, 0.0, 0),
    # odd sizes: rows and columns not multiples of anything, an odd entry count (the value,
    # slot and row-offset loads of the last tile end inside a dword), a partial last segment
    ("ragged_fp16_i32_odd", (1 << 20) + 7, 3 * (1 << 21) + 12345, "ragged", torch.float16, torch.int32, 0.75, 0.25,
     0),
    ("ragged_fp32_i64_odd_base1", (1 << 20) + 3, (1 << 22) + 1, "ragged", torch.float32, torch.int64, 1.0, 0.0, 1),
    # rows of 0-120 entries: the wide (fp16 / bf16) tiles sum their products in two halves, and
    # short rows, rows longer than 32 entries (summed by a wave) and empty rows all meet the
    # middle of some tile, on either side of it or across it
    # x of just under 128 MiB: 1024 buckets, the most the staged tables allow, so pass B's run map
    # and staging area (sized at launch for the bucket count) are at their largest
    ("max_buckets_fp16", 1 << 20, (1 << 26) - 3, "uniform32", torch.float16, torch.int32, 1.0, 0.0, 0),
    ("max_buckets_fp32_beta", 1 << 20, (1 << 25) - 1, "uniform32", torch.float32, torch.int64, 0.5, 1.5, 0),
    ("mixed_lengths_fp16_i64", 650_000, 1 << 22, "mixed", torch.float16, torch.int64, 1.0, 0.0, 0),
    ("mixed_lengths_bf16_i32_beta", 650_001, (1 << 22) + 5, "mixed", torch.bfloat16, torch.int32, -1.25, 0.5, 0),
]


def lengths_for(kind, rows, seed=3):
    rng = np.random.default_rng(seed)
    if kind == "uniform32":
        return torch.full((rows,), 32, dtype=torch.int64)
    if kind == "zipf":  # Zipf(2) rescaled to a mean of 17, capped at 200k, permuted; many rows cross tiles
        z = np.minimum(rng.zipf(2.0, size=rows), 200000).astype(np.float64)
        ln = np.floor(z * (17.0 * rows / z.sum()) + rng.random(rows)).astype(np.int64)
        return torch.from_numpy(np.clip(ln, 0, 200000)[rng.permutation(rows)])
    if kind in ("giant", "giant_sorted"):  # one row spans thousands of tiles, the others are empty or short
        ln = rng.integers(0, 3, rows)
        ln[rows // 3] = STAGE_MIN_NNZ + 12345
        return torch.from_numpy(ln.astype(np.int64))
    if kind == "ragged":  # 25..40 entries per row, an odd total
        ln = rng.integers(25, 41, rows)
        if ln.sum() % 2 == 0:
            ln[-1] += 1
        return torch.from_numpy(ln.astype(np.int64))
    if kind == "mixed":  # 0..120 entries per row, 10% empty rows
        ln = np.where(rng.random(rows) < 0.1, 0, rng.integers(1, 121, rows))
        return torch.from_numpy(ln.astype(np.int64))
    if kind == "sparse":  # 2 entries per row on average, 40% empty rows: tiles hold many rows
        ln = np.where(rng.random(rows) < 0.4, 0, rng.integers(1, 6, rows))
        return torch.from_numpy(ln.astype(np.int64))
    raise ValueError(kind)


@pytest.mark.parametrize("case", CASES, ids=[c[0] for c in CASES])
def test_staged_path_matches_oracle(case, dev):
    name, rows, cols, kind, vdt, rdt, alpha, beta, base = case
    w = random_rows(dev, rows, cols, lengths_for(kind, rows), vdt, rdt, alpha, beta, base=base)
    if kind == "giant":
        g = torch.Generator(device=dev)
        g.manual_seed(11)
        w.col_ind = w.col_ind[torch.randperm(w.nnz, generator=g, device=dev)]
    assert w.nnz >= STAGE_MIN_NNZ
    y, plan = run(w, dev)
    flag, buckets, tiles, _, _ = header(plan)
    if kind == "giant_sorted":
        assert flag == 0, "a sorted row touches few x lines per tile: the row kernels keep it"
        assert_close(host_workload(w), y)
        return
    assert flag == 1, "scattered columns must take the staged path"
    seg = (128 * 1024) // w.x.element_size()
    assert buckets == -(-cols // seg)
    check_tiles(w, plan)
    h = host_workload(w)
    err = assert_close(h, y)
    # the same plan again: bit-identical (the summation order is fixed by the pattern)
    y1 = y.clone()
    plan.run()
    torch.cuda.synchronize()
    if beta == 0.0:
        assert torch.equal(y.view(torch.int16) if y.element_size() == 2 else y.view(torch.int32),
                           y1.view(torch.int16) if y.element_size() == 2 else y1.view(torch.int32))
    print(f"{name}: nnz={w.nnz} tiles={tiles} buckets={buckets} max scaled error {err:.3e}")


@pytest.mark.parametrize("rows,per,cols,staged", [
    (1 << 19, 8, 1 << 22, True),     # 4 M entries, x 16 MiB: staged
    ((1 << 19) - 64, 8, 1 << 22, False),  # just under 2^22 entries: the row kernels
    (1 << 20, 8, 1 << 19, False),    # 8 M entries, x 2 MiB: the row kernels (L2-sized x)
    (1 << 20, 16, 1 << 19, True),    # 16 M entries, x 2 MiB: staged
])
def test_staged_size_rule(rows, per, cols, staged, dev):
    w = random_rows(dev, rows, cols, torch.full((rows,), per, dtype=torch.int64), torch.float32, torch.int32, 1.25,
                    -0.5)
    y, plan = run(w, dev)
    assert header(plan)[0] == (1 if staged else 0)
    assert_close(host_workload(w), y)


def test_banded_matrix_keeps_the_row_kernels(dev):
    """Eligible by size, but each tile touches few x lines: Preprocess keeps the row kernels, on the
    narrow column copy over entry-aligned row blocks (flag 5: every column lies within 16 bits of its row
    block's first row; the copy overlays the staged tables)."""
    rows = 1 << 21
    band = 17
    rp = torch.arange(0, rows * band + 1, band, dtype=torch.int64, device=dev)
    off = torch.arange(band, device=dev) - band // 2
    col = (torch.arange(rows, device=dev)[:, None] + off[None, :]).clamp(0, rows - 1).reshape(-1).to(torch.int32)
    g = torch.Generator(device=dev)
    g.manual_seed(9)
    vals = torch.rand(col.numel(), generator=g, device=dev) * 2 - 1
    x = torch.rand(rows, generator=g, device=dev) * 2 - 1
    y0 = torch.rand(rows, generator=g, device=dev) * 2 - 1
    w = wl.Workload("banded17", rows, rows, rp.to(torch.int32), col, vals, x, y0, 1.0, 0.5)
    assert w.nnz >= STAGE_MIN_NNZ
    y, plan = run(w, dev)
    assert header(plan)[0] == 5
    assert_close(w.to("cpu"), y)


def test_staged_values_updated_in_place_and_no_preprocess(dev):
    """Preprocess reads only the pattern: values and x updated in place after it are used by the next
    SpMV; without Preprocess the same matrix runs on the row kernels with the same result (tolerance)."""
    rows, cols = 1 << 20, 1 << 22
    w = random_rows(dev, rows, cols, lengths_for("uniform32", rows), torch.float32, torch.int32, 1.0, 0.0)
    y, plan = run(w, dev)
    assert header(plan)[0] == 1
    w.values.mul_(-0.75).add_(0.125)
    w.x.copy_(torch.flip(w.x, [0]))
    plan.run()
    torch.cuda.synchronize()
    assert_close(w.to("cpu"), y)
    y2, plan2 = run(w, dev, preprocess=False)
    assert header(plan2)[0] == 0  # no Preprocess: no staged tables
    assert_close(w.to("cpu"), y2)


def test_staged_plan_with_an_unaligned_x_runs_the_row_kernels(dev):
    """Pass A reads x by 16-byte vectors: after a staged Preprocess, an SpMV whose x is bound at a
    4-byte offset (the plan still matches: x is not part of it) takes the row kernels instead, on
    the whole matrix, and then an aligned x takes the staged kernels again."""
    from ops_sparse.spmv import DnVecDescr

    rows, cols = 1 << 20, 1 << 22
    w = random_rows(dev, rows, cols, lengths_for("uniform32", rows), torch.float32, torch.int32, 1.0, 0.5)
    y, plan = run(w, dev)
    assert header(plan)[0] == 1
    want = host_workload(w)
    big = torch.zeros(cols + 4, dtype=torch.float32, device=dev)
    xm = big[1:cols + 1]
    xm.copy_(w.x)
    assert xm.data_ptr() % 16 != 0
    aligned = plan.x
    plan.x = DnVecDescr(cols, xm)
    y.copy_(w.y0)
    plan.run()
    torch.cuda.synchronize()
    assert_close(want, y)
    plan.x = aligned
    y.copy_(w.y0)
    plan.run()
    torch.cuda.synchronize()
    assert_close(want, y)


def test_re_preprocess_switches_between_staged_and_row_kernels(dev):
    """The same descriptor and workspace: random columns (staged gather), then the columns rewritten
    in place to a band and Preprocess called again (the row kernels on the 16-bit column copy), then
    random again: every SpMV matches the oracle for the columns it was given."""
    rows, cols, per = 1 << 20, 1 << 22, 8
    w = random_rows(dev, rows, cols, torch.full((rows,), per, dtype=torch.int64), torch.float32, torch.int32, 1.0,
                    0.5)
    y = w.y0.clone()
    plan = CsrSpMV(w.rows, w.cols, w.row_ptr, w.col_ind, w.values, w.x, y, w.alpha, w.beta)
    scattered = w.col_ind.clone()
    band = (torch.arange(rows, device=dev, dtype=torch.int32)[:, None] +
            torch.arange(per, device=dev, dtype=torch.int32)[None, :]).reshape(-1)  # columns row .. row+7
    for cols_now, want_flag in ((scattered, (1,)), (band, (3, 5)), (scattered, (1,))):
        w.col_ind.copy_(cols_now)
        torch.cuda.synchronize()
        plan.preprocess()
        y.copy_(w.y0)
        plan.run()
        torch.cuda.synchronize()
        assert header(plan)[0] in want_flag
        assert_close(host_workload(w), y)


def test_staged_device_scalars_and_beta_zero_ignores_nan_y(dev):
    from ops_sparse._lib import PointerMode

    rows, cols = 1 << 20, 1 << 22
    w = random_rows(dev, rows, cols, lengths_for("uniform32", rows), torch.float16, torch.int64, 1.0, 0.0)
    y = torch.full((rows,), float("nan"), dtype=torch.float16, device=dev)
    plan = CsrSpMV(w.rows, w.cols, w.row_ptr, w.col_ind, w.values, w.x, y, 1.0, 0.0)
    plan.handle.set_pointer_mode(PointerMode.DEVICE)
    import ctypes
    da = torch.tensor([1.0], device=dev)
    db = torch.tensor([0.0], device=dev)
    plan.alpha = type("P", (), {"ptr": ctypes.c_void_p(da.data_ptr())})()
    plan.beta = type("P", (), {"ptr": ctypes.c_void_p(db.data_ptr())})()
    plan.preprocess()
    plan.run()
    torch.cuda.synchronize()
    assert header(plan)[0] == 1
    assert bool(torch.isfinite(y).all())
    assert_close(w.to("cpu"), y)


def _graph_matches_eager(w, dev, op=None):
    """Preprocess, an eager SpMV, then the SpMV captured in a HIP graph and replayed three times with
    eager SpMVs between the replays: every replay equals the eager result bit for bit.  Under capture
    the library makes no host calls on the stream (no event query): the captured SpMV launches every
    kernel set, each reading the path flag Preprocess left on the device."""
    from ops_sparse._lib import Operation
    op = Operation.NON_TRANSPOSE if op is None else op
    s = torch.cuda.Stream()
    y = w.y0.to(w.out_dtype).clone()
    torch.cuda.synchronize()  # the inputs were written on the default stream
    with torch.cuda.stream(s):
        plan = CsrSpMV(w.rows, w.cols, w.row_ptr, w.col_ind, w.values, w.x, y, w.alpha, w.beta, op=op,
                       base=w.meta.get("base", 0))
        plan.preprocess()
        plan.run()
    torch.cuda.synchronize()
    eager = y.clone()
    g = torch.cuda.CUDAGraph()
    y.copy_(w.y0.to(w.out_dtype))
    torch.cuda.synchronize()
    with torch.cuda.graph(g, stream=s):
        plan.run()
    bits = (lambda t: t.view(torch.int16)) if eager.element_size() == 2 else (lambda t: t.view(torch.int32))
    for _ in range(3):
        y.copy_(w.y0.to(w.out_dtype))
        torch.cuda.synchronize()
        with torch.cuda.stream(s):
            g.replay()
        torch.cuda.synchronize()
        assert torch.equal(bits(y), bits(eager))
        y.copy_(w.y0.to(w.out_dtype))
        torch.cuda.synchronize()
        with torch.cuda.stream(s):  # eager work between replays
            plan.run()
        torch.cuda.synchronize()
        assert torch.equal(bits(y), bits(eager))
    return plan


def test_staged_spmv_in_a_hip_graph(dev):
    rows, cols = 1 << 20, 1 << 22
    w = random_rows(dev, rows, cols, lengths_for("uniform32", rows), torch.float16, torch.int64, 1.0, 0.5)
    plan = _graph_matches_eager(w, dev)
    assert header(plan)[0] == 1


@pytest.mark.parametrize("kind", ["bucketed", "banded"])
def test_transposes_in_a_hip_graph(kind, dev):
    from ops_sparse._lib import Operation
    if kind == "bucketed":
        w = wl.poisson_transpose(rows=1 << 20).to(dev)
    else:
        w = wl.laplacian_2d(n=1536).to(dev)
        w.trans = "T"
    plan = _graph_matches_eager(w, dev, Operation.TRANSPOSE)
    assert header(plan)[0] == (1 if kind == "bucketed" else 4)
