"""Seeded synthetic CSR workloads of the five benchmark configurations.

Generators run on any torch device (the GPU for full-size inputs, the CPU for
small test cases) and return a :class:`Workload`.  The byte model
(:func:`algorithmic_bytes`) counts every array once: row offsets, col_ind and
values once, x once (compulsory), y written once and read once more when
beta != 0.

Configurations (BASELINE.json "configs"):
  c1  4096 x 4096, exactly 41 distinct sorted columns per row, fp32, alpha=1 beta=0
  c2  5-point 2-D Laplacian on a 2048^2 grid, fp32, alpha=1.5 beta=0.5
  c3  8,388,608^2, Zipf(2.0) row lengths rescaled to mean 16, capped at 200,000,
      rows permuted, fp32, alpha=1 beta=0
  c4  16,777,216^2, 32 uniform sorted columns per row, fp16 or bf16 values and x,
      fp32 compute, int64 row offsets, alpha=1 beta=0
  c5  2,097,152^2, Poisson(12) row lengths with 10% of rows empty, fp32,
      op=TRANSPOSE, alpha=1 beta=2
Every generator takes a ``scale`` divisor so tests can run the same
distribution at a size the CPU oracle finishes in seconds.
"""
from dataclasses import dataclass, field

import numpy as np
import torch


@dataclass
class Workload:
    name: str
    rows: int
    cols: int
    row_ptr: torch.Tensor
    col_ind: torch.Tensor
    values: torch.Tensor
    x: torch.Tensor
    y0: torch.Tensor
    alpha: float
    beta: float
    trans: str = "N"
    out_dtype: torch.dtype = torch.float32
    meta: dict = field(default_factory=dict)

    @property
    def nnz(self):
        return int(self.col_ind.numel())

    def to(self, device):
        t = lambda v: v.to(device)
        return Workload(self.name, self.rows, self.cols, t(self.row_ptr), t(self.col_ind), t(self.values),
                        t(self.x), t(self.y0), self.alpha, self.beta, self.trans, self.out_dtype, dict(self.meta))


def _elem_bytes(dtype):
    return torch.empty((), dtype=dtype).element_size()


def algorithmic_bytes(w):
    """Bytes one SpMV must move at minimum (each array once; y read only if beta != 0)."""
    vb = _elem_bytes(w.values.dtype)
    ob = _elem_bytes(w.out_dtype)
    rb = _elem_bytes(w.row_ptr.dtype)
    x_len = w.rows if w.trans != "N" else w.cols
    y_len = w.cols if w.trans != "N" else w.rows
    y_bytes = ob * y_len * (2 if w.beta != 0 else 1)
    return rb * (w.rows + 1) + (4 + vb) * w.nnz + vb * x_len + y_bytes


STAGE_SEGMENT_BYTES = 128 * 1024  # x per bucket of the staged path
STAGE_CHUNK_BYTES = 8  # staged x moves in chunks of this many bytes (runs padded to whole chunks)


def staged_bytes(w):
    """Bytes one SpMV moves on the staged-gather path (its design traffic).

    Pass A reads every staged slot's column within its bucket (2 B) and
    writes the gathered x value (vb), reading x once; pass B reads the values,
    every entry's slot (2 B) and the staged x values again, the low 16 bits of
    the normalised row offsets (2 B per row), the run table (4 B per tile and
    bucket) and y; col_ind is not
    read at all after Preprocess.  Staged slots are the entries plus the
    padding of every (tile, bucket) run to whole chunks of STAGE_CHUNK_BYTES (half a chunk
    less one slot per run on average).  Tiles hold 8184 rows + entries for
    fp32 values and 16376 for fp16 / bf16.
    """
    vb = _elem_bytes(w.values.dtype)
    ob = _elem_bytes(w.out_dtype)
    rb = 2  # pass B reads the low halves of the row offsets
    items = 8184 if vb == 4 else 16376
    tiles = -(-(w.rows + w.nnz) // items)
    buckets = -(-(w.cols * vb) // STAGE_SEGMENT_BYTES) + 1
    chunk = STAGE_CHUNK_BYTES // vb
    slots = w.nnz + (chunk - 1) / 2 * buckets * tiles
    y_bytes = ob * w.rows * (2 if w.beta != 0 else 1)
    return int(rb * (w.rows + 2) + (2 + vb) * slots + (vb + 2) * w.nnz + vb * slots + vb * w.cols + y_bytes
               + 4 * (tiles + 1) * buckets)


def flops(w):
    return 2 * w.nnz


def _gen(device, seed):
    g = torch.Generator(device=device)
    g.manual_seed(seed)
    return g


def _uniform(n, gen, device, lo=-1.0, hi=1.0, dtype=torch.float32):
    return (torch.rand(n, generator=gen, device=device, dtype=torch.float32) * (hi - lo) + lo).to(dtype)


def csr_from_lengths(lengths, n_cols, gen, device, distinct=True):
    """Row offsets + sorted uniform columns for the given row lengths.

    Columns are drawn uniformly; with ``distinct`` duplicates inside a row are
    dropped (so a row may end up slightly shorter than requested: the exact
    count is what the returned offsets say).
    """
    lengths = lengths.to(device=device, dtype=torch.int64)
    m = lengths.numel()
    nnz = int(lengths.sum().item())
    rows = torch.repeat_interleave(torch.arange(m, device=device, dtype=torch.int64), lengths)
    cols = torch.randint(0, n_cols, (nnz,), generator=gen, device=device, dtype=torch.int64)
    keys = rows * n_cols + cols
    del rows, cols
    keys = torch.sort(keys).values
    if distinct:
        keys = torch.unique_consecutive(keys)
    row_of = torch.div(keys, n_cols, rounding_mode="floor")
    col = (keys - row_of * n_cols).to(torch.int32)
    del keys
    counts = torch.bincount(row_of, minlength=m)
    del row_of
    row_ptr = torch.zeros(m + 1, dtype=torch.int64, device=device)
    torch.cumsum(counts, 0, out=row_ptr[1:])
    return row_ptr, col


def c1_uniform41(device="cpu", seed=20260502, rows=4096, cols=4096, per_row=41):
    """Exactly ``per_row`` distinct sorted columns per row (sampling without replacement)."""
    g = _gen("cpu", seed)
    col = torch.empty(rows * per_row, dtype=torch.int32)
    for i in range(rows):
        col[i * per_row:(i + 1) * per_row] = torch.sort(torch.randperm(cols, generator=g)[:per_row]).values
    row_ptr = torch.arange(0, rows * per_row + 1, per_row, dtype=torch.int32)
    values = _uniform(rows * per_row, g, "cpu")
    x = _uniform(cols, g, "cpu")
    y0 = _uniform(rows, g, "cpu")
    w = Workload("c1_uniform41_fp32", rows, cols, row_ptr, col, values, x, y0, 1.0, 0.0)
    return w.to(device)


def laplacian_2d(n=2048, device="cpu", seed=20260503, alpha=1.5, beta=0.5):
    """5-point Laplacian on an n x n grid: 4 on the diagonal, -1 for each neighbour."""
    m = n * n
    idx = torch.arange(m, device=device, dtype=torch.int64)
    gi, gj = idx // n, idx % n
    cand = torch.stack([idx - n, idx - 1, idx, idx + 1, idx + n], dim=1)
    ok = torch.stack([gi > 0, gj > 0, torch.ones_like(gi, dtype=torch.bool), gj < n - 1, gi < n - 1], dim=1)
    counts = ok.sum(dim=1)
    row_ptr = torch.zeros(m + 1, dtype=torch.int64, device=device)
    torch.cumsum(counts, 0, out=row_ptr[1:])
    col = cand[ok].to(torch.int32)
    vals = torch.where(cand == idx[:, None], 4.0, -1.0)[ok].to(torch.float32)
    g = _gen(device, seed)
    x = _uniform(m, g, device)
    y0 = _uniform(m, g, device)
    return Workload(f"c2_laplacian_{n}x{n}_fp32", m, m, row_ptr.to(torch.int32), col, vals, x, y0, alpha, beta,
                    meta={"grid": n})


def zipf_rows(rows=8388608, device="cpu", seed=20260504, mean=16.0, cap=200000, exponent=2.0):
    """Zipf(exponent) row lengths (capped, rescaled to ``mean``), rows permuted, uniform sorted columns."""
    rng = np.random.default_rng(seed)
    cap = min(cap, rows)
    z = np.minimum(rng.zipf(exponent, size=rows), cap).astype(np.float64)
    u = rng.random(rows)  # unbiased rounding of the scaled lengths
    target = int(round(mean * rows))

    def total(f):
        # expected entries once duplicate columns are dropped: a row of L
        # uniform draws over `rows` columns keeps rows*(1-(1-1/rows)^L)
        lengths = np.minimum(np.floor(z * f + u), cap)
        return float(-rows * np.expm1(lengths * np.log1p(-1.0 / rows)).sum())

    # The cap takes mass from the longest rows (and dropping duplicate columns
    # a little more), so a plain rescale to the mean falls short of it: bisect
    # the scale factor until the expected entry count reaches the target.
    lo = mean * rows / z.sum()
    hi = lo
    while total(hi) < target and hi < 1e12:
        hi *= 2.0
    for _ in range(64):
        mid = 0.5 * (lo + hi)
        if total(mid) >= target:
            hi = mid
        else:
            lo = mid
    lengths = np.minimum(np.floor(z * hi + u), cap).astype(np.int64)
    lengths = lengths[rng.permutation(rows)]
    g = _gen(device, seed)
    row_ptr, col = csr_from_lengths(torch.from_numpy(lengths), rows, g, device)
    nnz = col.numel()
    values = _uniform(nnz, g, device)
    x = _uniform(rows, g, device)
    y0 = _uniform(rows, g, device)
    return Workload(f"c3_zipf{exponent:g}_mean{mean:g}_{rows}_fp32", rows, rows, row_ptr.to(torch.int32), col,
                    values, x, y0, 1.0, 0.0, meta={"max_row": int(lengths.max())})


def uniform_rows_lowp(rows=16777216, device="cpu", seed=20260505, per_row=32, dtype=torch.float16):
    """``per_row`` uniform sorted columns per row (repeats allowed), int64 row offsets, 16-bit values and x."""
    g = _gen(device, seed)
    col = torch.randint(0, rows, (rows, per_row), generator=g, device=device, dtype=torch.int32)
    col = torch.sort(col, dim=1).values.reshape(-1)
    row_ptr = torch.arange(0, rows * per_row + 1, per_row, dtype=torch.int64, device=device)
    values = torch.randn(rows * per_row, generator=g, device=device, dtype=torch.float32).to(dtype)
    x = _uniform(rows, g, device, dtype=dtype)
    y0 = torch.zeros(rows, dtype=dtype, device=device)
    tag = "fp16" if dtype == torch.float16 else "bf16"
    return Workload(f"c4_uniform{per_row}_{rows}_{tag}_i64", rows, rows, row_ptr, col, values, x, y0, 1.0, 0.0,
                    out_dtype=dtype)


def poisson_transpose(rows=2097152, device="cpu", seed=20260506, mean=12.0, empty_frac=0.1):
    """Poisson(mean) row lengths, ``empty_frac`` of rows forced empty, op=TRANSPOSE, alpha=1 beta=2."""
    g = _gen(device, seed)
    lengths = torch.poisson(torch.full((rows,), mean, device=device), generator=g).to(torch.int64)
    empty = torch.rand(rows, generator=g, device=device) < empty_frac
    lengths = torch.where(empty, torch.zeros_like(lengths), lengths)
    lengths = torch.clamp(lengths, max=rows)
    row_ptr, col = csr_from_lengths(lengths, rows, g, device)
    nnz = col.numel()
    values = _uniform(nnz, g, device)
    x = _uniform(rows, g, device)
    y0 = _uniform(rows, g, device)
    return Workload(f"c5_poisson{mean:g}_T_{rows}_fp32", rows, rows, row_ptr.to(torch.int32), col, values, x, y0,
                    1.0, 2.0, trans="T")


def config(name, device="cpu", scale=1, dtype=torch.float16):
    """Workload for config c1..c5; ``scale`` divides the row count (tests use scale > 1)."""
    if name == "c1":
        return c1_uniform41(device)
    if name == "c2":
        n = max(8, 2048 // int(round(scale ** 0.5)))
        return laplacian_2d(n, device)
    if name == "c3":
        return zipf_rows(max(1024, 8388608 // scale), device, cap=max(64, 200000 // scale))
    if name == "c4":
        return uniform_rows_lowp(max(1024, 16777216 // scale), device, dtype=dtype)
    if name == "c5":
        return poisson_transpose(max(1024, 2097152 // scale), device)
    raise ValueError(name)
