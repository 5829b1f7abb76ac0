"""Seeded random matrices at the sizes where the staged gather (opA = N) and the column-bucketed
transpose (opA = T, H) take over, against the oracle through the C ABI.

Every case draws its shape, row-length law, value type, row-offset type, index base, scalars and
operation from its seed, checks that Preprocess chose the path the case is meant for (the
workspace header's path flag), compares with the oracle, and runs again for bit-identical output.
"""
import numpy as np
import pytest
import torch

from helpers import assert_close
from ops_sparse import workloads as wl
from ops_sparse._lib import Operation
from ops_sparse.spmv import CsrSpMV

pytestmark = pytest.mark.gpu


def _lengths(rng, rows, mean, law):
    if law == "uniform":
        return rng.integers(max(1, int(mean) - 4), int(mean) + 5, rows)
    if law == "poisson":
        ln = rng.poisson(mean, rows)
        ln[rng.random(rows) < 0.1] = 0  # empty rows
        return ln
    z = np.minimum(rng.zipf(2.2, rows), 50000).astype(np.float64)  # heavy tail: rows across tiles
    return np.floor(z * (mean * rows / z.sum()) + rng.random(rows)).astype(np.int64)


def _case(seed, dev):
    rng = np.random.default_rng(1000 + seed)
    transpose = seed % 4 == 3
    vdt = torch.float32 if transpose else [torch.float32, torch.float16, torch.bfloat16][seed % 3]
    rows = int(rng.integers(1 << 18, 1 << 21))
    mean = float(rng.uniform(6, 24))
    law = ["uniform", "poisson", "zipf"][(seed // 3) % 3]
    ln = _lengths(rng, rows, mean, law)
    nnz = int(ln.sum())
    floor = 1 << 22 if not transpose else 1 << 21
    if nnz < floor:  # scale the rows' lengths up to the path's size
        ln = ln * (floor // max(nnz, 1) + 1)
        nnz = int(ln.sum())
    vb = 4 if vdt == torch.float32 else 2
    cols = int(rng.integers((8 << 20) // vb, (64 << 20) // vb)) if not transpose else int(rng.integers(1 << 20, 1 << 22))
    base = int(rng.integers(0, 2))
    rdt = [torch.int32, torch.int64][int(rng.integers(0, 2))]
    alpha = float(rng.choice([1.0, -0.75, 2.5]))
    beta = float(rng.choice([0.0, 0.5, -1.25]))
    g = torch.Generator(device=dev)
    g.manual_seed(seed)
    row_ptr, col = wl.csr_from_lengths(torch.from_numpy(ln.astype(np.int64)), cols, g, dev, distinct=False)
    vals = (torch.rand(col.numel(), generator=g, device=dev) * 2 - 1).to(vdt)
    xn = rows if transpose else cols
    yn = cols if transpose else rows
    x = (torch.rand(xn, generator=g, device=dev) * 2 - 1).to(vdt)
    out = torch.float32 if vdt == torch.float32 else vdt
    y0 = (torch.rand(yn, generator=g, device=dev) * 2 - 1).to(out)
    trans = "T" if transpose else "N"
    w = wl.Workload(f"fuzz{seed}_{law}_{rows}x{cols}_{trans}", rows, cols, (row_ptr + base).to(rdt),
                    (col + base).to(torch.int32), vals, x, y0, alpha, beta, trans=trans, out_dtype=out,
                    meta={"base": base})
    return w


def _host(w):
    h = w.to("cpu")
    b = w.meta.get("base", 0)
    if b:
        h.col_ind = h.col_ind - b
        h.row_ptr = h.row_ptr - b
    return h


@pytest.mark.parametrize("seed", range(16))
def test_large_random_matrix(seed, dev):
    w = _case(seed, dev)
    op = Operation.TRANSPOSE if w.trans == "T" else Operation.NON_TRANSPOSE
    y = w.y0.clone()
    plan = CsrSpMV(w.rows, w.cols, w.row_ptr, w.col_ind, w.values, w.x, y, w.alpha, w.beta, op=op,
                   base=w.meta["base"])
    plan.preprocess()
    plan.run()
    torch.cuda.synchronize()
    flag = int(np.frombuffer(plan.workspace[:192].cpu().numpy().tobytes(), dtype=np.uint32)[32])
    if w.trans == "N" or w.row_ptr.dtype == torch.int32:
        # random columns: the staged gather, or for a transpose with 32-bit offsets the bucketed kernels
        assert flag == 1, f"{w.name}: path flag {flag}"
    print(f"{w.name}: nnz={w.nnz} dtype={w.values.dtype} base={w.meta['base']} flag={flag}")
    assert_close(_host(w), y)
    first = y.clone()
    y.copy_(w.y0)
    plan.run()
    torch.cuda.synchronize()
    bits = (lambda t: t.view(torch.int16)) if y.element_size() == 2 else (lambda t: t.view(torch.int32))
    assert torch.equal(bits(first), bits(y))
