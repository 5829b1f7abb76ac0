"""Shared checks: run the HIP path and compare with the CPU oracle."""
import numpy as np
import torch

import oracle

# fp32 1e-5 and fp16/bf16 (fp32 compute) 1e-2, relative
# to the row scale |alpha|*sum|a_ij x_j| + |beta y_i|
TOL = {torch.float32: 1e-5, torch.float16: 1e-2, torch.bfloat16: 1e-2}

_KIND = {torch.float32: oracle.K_F32, torch.float16: oracle.K_F16, torch.bfloat16: oracle.K_BF16}


def host_bits(t):
    """numpy view of a tensor: 16-bit floats as uint16 bit patterns."""
    t = t.detach().cpu().contiguous()
    if t.dtype in (torch.float16, torch.bfloat16):
        return t.view(torch.int16).numpy().view(np.uint16)
    return t.numpy()


def to_f64(t):
    return t.detach().cpu().to(torch.float64).numpy()


def oracle_result(w):
    """(golden float64, row scale) for a Workload on the host."""
    rp = w.row_ptr.cpu().numpy().astype(np.int64)
    col = w.col_ind.cpu().numpy()
    vk = _KIND[w.values.dtype]
    yk = _KIND[w.out_dtype]
    val, x, y = host_bits(w.values), host_bits(w.x), host_bits(w.y0.to(w.out_dtype))
    transpose = w.trans != "N"
    scale = oracle.row_scale(rp, col, val, x, y, vk, yk, w.alpha, w.beta, transpose, w.cols)
    if vk == oracle.K_F32 and yk == oracle.K_F32:
        if transpose:
            g = oracle.spmv_trans_f64(rp, col, val, x, y, w.cols, w.alpha, w.beta)
        else:
            g = oracle.spmv_f64(rp, col, val, x, y, w.alpha, w.beta)
    else:
        z = oracle.spmv_lowp(rp, col, val, x, y, vk, yk, w.alpha, w.beta, transpose, w.cols)
        g = (torch.from_numpy(z.view(np.int16)).view(w.out_dtype).to(torch.float64).numpy()
             if yk != oracle.K_F32 else z.astype(np.float64))
    return g, scale


def scaled_error(got, golden, scale):
    denom = np.maximum(scale, np.finfo(np.float64).tiny)
    err = np.abs(got - golden) / denom
    # outputs that are exactly zero in both get error 0 even when scale == 0
    err[(got == golden)] = 0.0
    return err


def assert_close(w, y, golden=None, scale=None):
    if golden is None:
        golden, scale = oracle_result(w)
    got = to_f64(y)
    assert np.all(np.isfinite(got)), "non-finite output"
    err = scaled_error(got, golden, scale)
    tol = TOL[w.out_dtype]
    worst = int(np.argmax(err)) if err.size else 0
    assert err.size == 0 or err.max() <= tol, (
        f"{w.name}: max scaled error {err.max():.3e} > {tol} at {worst}: got {got[worst]!r} "
        f"golden {golden[worst]!r} scale {scale[worst]!r}")
    return float(err.max()) if err.size else 0.0
