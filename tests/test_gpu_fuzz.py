"""Seeded random cases over the whole dtype/op matrix of aclsparseSpMV, against the CPU oracle.

Each case draws a row-length mix (empty, short, 9-16, long), index base, row-offset width,
operation, scalars (zeros included) and whether Preprocess runs, so every kernel path (stream,
int8/complex stream, CSC column pass, general kernel) is exercised with the others' edge cases.
"""
import numpy as np
import pytest
import torch

import oracle
from helpers import assert_close
from ops_sparse import workloads as wl
from ops_sparse._lib import Operation, SpMVAlg
from ops_sparse.spmv import CsrSpMV

pytestmark = pytest.mark.gpu

KINDS = ["f32", "f16", "bf16", "f16->f32", "i8->i32", "i8->f32", "c64", "f32->c64"]
OPS = {"N": Operation.NON_TRANSPOSE, "T": Operation.TRANSPOSE, "H": Operation.CONJUGATE_TRANSPOSE}


def _case(seed):
    rng = np.random.default_rng(1000 + seed)
    kind = KINDS[seed % len(KINDS)]
    ops = ["N", "T", "H"] if kind == "c64" else ["N", "T"]
    op = ops[rng.integers(len(ops))]
    rows = int(rng.integers(1, 3000))
    cols = int(rng.integers(1, 3000))
    mix = rng.choice([0, 1, 3, 5, 12, 16, 40, 700, 2500], size=rows,
                     p=[0.15, 0.2, 0.2, 0.15, 0.1, 0.08, 0.07, 0.04, 0.01])
    base = int(rng.integers(2))
    i64 = bool(rng.integers(2))
    alpha = [0.0, 1.0, -1.5, 2.25][rng.integers(4)]
    beta = [0.0, 1.0, 0.5, -2.0][rng.integers(4)]
    pre = bool(rng.integers(2))
    alg = [SpMVAlg.DEFAULT, SpMVAlg.CSR_ALG1, SpMVAlg.CSR_ALG2][rng.integers(3)]
    return rng, kind, op, rows, cols, mix, base, i64, alpha, beta, pre, alg


@pytest.mark.parametrize("seed", range(96))
def test_random_case(seed, dev):
    rng, kind, op, rows, cols, mix, base, i64, alpha, beta, pre, alg = _case(seed)
    g = torch.Generator().manual_seed(seed)
    rp, col = wl.csr_from_lengths(torch.from_numpy(mix.astype(np.int64)), cols, g, "cpu")
    n = col.numel()
    trans = op != "N"
    xlen, ylen = (rows, cols) if trans else (cols, rows)
    u = lambda k: torch.rand(k, generator=g) * 2 - 1
    if kind.startswith("i8"):
        val = torch.randint(-128, 128, (n,), generator=g, dtype=torch.int8)
        x = torch.randint(-128, 128, (xlen,), generator=g, dtype=torch.int8)
        alpha, beta = int(alpha * 2), int(beta * 2)
        y0 = torch.randint(-5000, 5000, (ylen,), generator=g, dtype=torch.int32) if kind == "i8->i32" else u(ylen)
    elif kind == "c64":
        val, x, y0 = torch.complex(u(n), u(n)), torch.complex(u(xlen), u(xlen)), torch.complex(u(ylen), u(ylen))
        alpha, beta = complex(alpha, 0.5), complex(beta, -0.25)
    elif kind == "f32->c64":
        val, x, y0 = u(n), u(xlen), torch.complex(u(ylen), u(ylen))
        alpha, beta = complex(alpha, 0.75), complex(beta, 0.5)
    else:
        vdt = {"f32": torch.float32, "f16": torch.float16, "bf16": torch.bfloat16, "f16->f32": torch.float16}[kind]
        odt = torch.float32 if kind in ("f32", "f16->f32") else vdt
        val, x, y0 = u(n).to(vdt), u(xlen).to(vdt), u(ylen).to(odt)
    y = y0.to(dev).clone()
    d_rp = (rp + base).to(torch.int64 if i64 else torch.int32).to(dev)
    plan = CsrSpMV(rows, cols, d_rp, (col + base).to(dev), val.to(dev), x.to(dev), y, alpha, beta, op=OPS[op],
                   base=base, alg=alg)
    if pre:
        plan.preprocess()
    plan.run()
    torch.cuda.synchronize()
    got = y.cpu()
    rpn, coln = rp.numpy(), col.numpy()
    if kind == "i8->i32":
        ref = oracle.spmv_i8(rpn, coln, val.numpy(), x.numpy(), y0.numpy(), alpha, beta, transpose=trans, cols=cols)
        np.testing.assert_array_equal(got.numpy(), ref)
        return
    if kind in ("c64", "f32->c64"):
        real = kind == "f32->c64"
        ref = oracle.spmv_c64(rpn, coln, val.numpy(), x.numpy(), y0.numpy(), cols, {"N": 0, "T": 1, "H": 2}[op],
                              alpha, beta, val_is_real=real)
        w = wl.Workload("fuzz", rows, cols, rp.to(torch.int32), col, val.abs().float(), x.abs().float(),
                        y0.abs().float(), abs(alpha), abs(beta), trans="T" if trans else "N")
        scale = oracle.row_scale(rpn, coln, w.values.numpy(), w.x.numpy(), w.y0.numpy(), oracle.K_F32, oracle.K_F32,
                                 abs(alpha), abs(beta), trans, cols)
        err = np.abs(got.numpy().astype(np.complex128) - ref) / np.maximum(scale, 1e-30)
        err[np.abs(got.numpy().astype(np.complex128) - ref) == 0] = 0.0
        assert err.max(initial=0.0) <= 1e-5, (kind, op, float(err.max()))
        return
    if kind == "i8->f32":
        valf, xf = val.float(), x.float()  # int8 values are exact in fp32
        w = wl.Workload("fuzz", rows, cols, rp.to(torch.int32), col, valf, xf, y0, float(alpha), float(beta),
                        trans="T" if trans else "N")
    else:
        w = wl.Workload("fuzz", rows, cols, rp.to(torch.int32), col, val, x, y0, alpha, beta,
                        trans="T" if trans else "N", out_dtype=y0.dtype)
    assert_close(w, got)
