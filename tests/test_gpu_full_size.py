"""Full-size parity of the largest configuration (c4: 16,777,216 rows, 536,870,912
non-zeros, fp16 / bf16 values and x, fp32 compute, int64 row offsets) through the C ABI.

The whole output is computed on the GPU; the oracle then recomputes a sampled
subset of rows (the first and last 4096 rows and 2^20 seeded random rows)
from the same host arrays, and every row is checked for the properties the
domain fixes (finite output; rows without entries are exactly zero).
"""
import numpy as np
import pytest
import torch

from helpers import TOL, oracle_result, scaled_error, to_f64
from ops_sparse import workloads as wl
from ops_sparse.spmv import CsrSpMV

pytestmark = pytest.mark.gpu


def sub_csr(rp, rows):
    """Row offsets and entry positions of the sub-matrix made of ``rows`` (int64 numpy)."""
    starts, ends = rp[rows], rp[rows + 1]
    lens = ends - starts
    sub_rp = np.zeros(rows.size + 1, np.int64)
    np.cumsum(lens, out=sub_rp[1:])
    pos = np.repeat(starts - sub_rp[:-1], lens) + np.arange(sub_rp[-1], dtype=np.int64)
    return sub_rp, pos


def sampled_rows(n, edge=4096, random=1 << 20, seed=7):
    rng = np.random.default_rng(seed)
    pick = np.concatenate([np.arange(min(edge, n)), np.arange(max(0, n - edge), n),
                           rng.integers(0, n, size=min(random, n))])
    return np.unique(pick)


def check_sampled(w, y, rows=None):
    """Oracle on a row sample of workload ``w`` (device tensors) against the device result ``y``."""
    rp = w.row_ptr.cpu().numpy().astype(np.int64)
    rows = sampled_rows(w.rows) if rows is None else rows
    sub_rp, pos = sub_csr(rp, rows)
    pos_t = torch.from_numpy(pos).to(w.col_ind.device)
    sub = wl.Workload(w.name + "_sample", rows.size, w.cols, torch.from_numpy(sub_rp), w.col_ind[pos_t].cpu(),
                      w.values[pos_t].cpu(), w.x.cpu(), w.y0.cpu()[torch.from_numpy(rows)], w.alpha, w.beta,
                      out_dtype=w.out_dtype)
    golden, scale = oracle_result(sub)
    got = to_f64(y.cpu()[torch.from_numpy(rows)])
    err = scaled_error(got, golden, scale)
    tol = TOL[w.out_dtype]
    worst = int(np.argmax(err))
    assert err.max() <= tol, (f"{w.name}: row {rows[worst]}: scaled error {err[worst]:.3e} > {tol}: got "
                              f"{got[worst]!r} golden {golden[worst]!r} scale {scale[worst]!r}")
    return float(err.max())


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16], ids=["fp16", "bf16"])
def test_config4_full_size_sampled_oracle(dtype, dev):
    w = wl.uniform_rows_lowp(device=dev, dtype=dtype)
    assert w.rows == 16777216 and w.nnz == 536870912 and w.row_ptr.dtype == torch.int64
    y = torch.full((w.rows,), float("nan"), dtype=dtype, device=dev)  # beta = 0: y must not be read
    plan = CsrSpMV(w.rows, w.cols, w.row_ptr, w.col_ind, w.values, w.x, y, w.alpha, w.beta)
    plan.preprocess()
    plan.run()
    torch.cuda.synchronize()
    # every row: finite; c4 has no empty rows, so no row is exactly the beta*y of an empty row
    assert bool(torch.isfinite(y).all())
    err = check_sampled(w, y)
    print(f"{w.name}: sampled max scaled error {err:.3e}")
    # a second SpMV on the same plan gives the same bits (fixed summation order)
    y2 = torch.empty_like(y)
    plan2 = CsrSpMV(w.rows, w.cols, w.row_ptr, w.col_ind, w.values, w.x, y2, w.alpha, w.beta)
    plan2.preprocess()
    plan2.run()
    torch.cuda.synchronize()
    assert torch.equal(y2.view(torch.int16), y.view(torch.int16))


def test_config4_full_size_reference_sized_workspace(dev):
    """c4 fp16 under CSR_ALG1: the reference-sized workspace (normalised row offsets and the row-block
    partition, no staged tables) and the row kernel, on the sampled oracle."""
    from ops_sparse._lib import SpMVAlg

    w = wl.uniform_rows_lowp(device=dev, dtype=torch.float16)
    y = torch.full((w.rows,), float("nan"), dtype=torch.float16, device=dev)
    plan = CsrSpMV(w.rows, w.cols, w.row_ptr, w.col_ind, w.values, w.x, y, w.alpha, w.beta,
                   alg=SpMVAlg.CSR_ALG1)
    ref = (192 + (w.rows + 1) * 8 + 63) // 64 * 64  # the reference's formula with 8-byte row offsets
    assert plan.buffer_size <= 2 * ref
    plan.preprocess()
    plan.run()
    torch.cuda.synchronize()
    assert bool(torch.isfinite(y).all())
    err = check_sampled(w, y)
    print(f"{w.name} ALG1: workspace {plan.buffer_size} B, sampled max scaled error {err:.3e}")


@pytest.mark.parametrize("op", ["T", "H"])
def test_complex_laplacian_transpose_full_size(op, dev):
    """The headline Laplacian (4,194,304 rows, 20,963,328 entries: more entries than one capped grid
    covers) with complex64 values, x and y, opA = T and H after Preprocess: the one-pass banded
    transpose (path flag 6, packed 16-bit rows and positions) against the fp64 oracle on every column,
    and bit-identical to the product and column passes (the same SpMV without Preprocess)."""
    import bench
    from ops_sparse._lib import Operation
    import oracle

    w = bench.make("c2_c64_H", dev)
    o = Operation.TRANSPOSE if op == "T" else Operation.CONJUGATE_TRANSPOSE
    outs = []
    for pre in (True, False):
        y = w.y0.clone()
        plan = CsrSpMV(w.rows, w.cols, w.row_ptr, w.col_ind, w.values, w.x, y, w.alpha, w.beta, op=o)
        if pre:
            plan.preprocess()
            torch.cuda.synchronize()
            h = np.frombuffer(plan.workspace[:192].cpu().numpy().tobytes(), dtype=np.uint32)
            assert int(h[32]) == 6
        plan.run()
        torch.cuda.synchronize()
        outs.append(y.cpu())
        del plan
    assert torch.equal(outs[0], outs[1])
    z = oracle.spmv_c64(w.row_ptr.cpu().numpy(), w.col_ind.cpu().numpy(), w.values.cpu().numpy(),
                        w.x.cpu().numpy(), w.y0.cpu().numpy(), w.cols, 1 if op == "T" else 2, w.alpha, w.beta)
    np.testing.assert_allclose(outs[0].numpy(), z, rtol=1e-4, atol=1e-4)


def test_laplacian_transpose_full_size(dev):
    """The headline Laplacian with opA = T after Preprocess at full size: the banded one-pass kernel on
    its 16-bit copies (path flag 4) against the oracle on every column, and bit-identical on a second run."""
    import bench
    from helpers import assert_close
    from ops_sparse._lib import Operation

    w = bench.make("c2_T", dev)
    y = w.y0.clone()
    plan = CsrSpMV(w.rows, w.cols, w.row_ptr, w.col_ind, w.values, w.x, y, w.alpha, w.beta,
                   op=Operation.TRANSPOSE)
    plan.preprocess()
    torch.cuda.synchronize()
    h = np.frombuffer(plan.workspace[:192].cpu().numpy().tobytes(), dtype=np.uint32)
    assert int(h[32]) == 4
    plan.run()
    torch.cuda.synchronize()
    first = y.clone()
    assert_close(w, y)
    y.copy_(w.y0)
    plan.run()
    torch.cuda.synchronize()
    assert torch.equal(first.view(torch.int32), y.view(torch.int32))
