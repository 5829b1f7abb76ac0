"""The ``ops_sparse`` / ``ops_sparse_test`` operator libraries on a ROCm device.

Mirrors the reference's optional PyTorch bridge (torch_npu/spmv_npu.cpp:410-444):

* ``torch.ops.ops_sparse.spmv(Tensor mat, Tensor vec) -> Tensor``: ``mat @ vec``
  for a 2-D CSR ``mat`` (SpmvMv, :384-407: alpha 1, beta 0, int8 -> int32 out),
  registered for the dense and the CSR dispatch keys of the device (``CUDA`` and
  ``SparseCsrCUDA`` on ROCm, ``PrivateUse1`` / ``SparseCsrPrivateUse1`` there);
* ``torch.ops.ops_sparse_test.spmv_npu(row_ptr, col_ind, values, x, y, alpha,
  beta, trans, base) -> Tensor``: ``y = alpha * op(A) * x + beta * y`` in place,
  returning ``y`` itself (SpmvNpu / RunSpmv, :354-382), int32 indices only
  (CheckIndex, :62-67).

Neither library has a CPU kernel, so a call with CPU tensors raises (the
dispatcher's NotImplementedError, a RuntimeError) instead of falling back.
Argument errors raise RuntimeError, as TORCH_CHECK does there.  The schema of
``spmv_npu`` marks ``y`` as written and aliased by the result.
"""
import torch

from ._lib import Operation
from .spmv import CsrSpMV, _validate_npu_args, mv as _mv

_LIBS = None


def _spmv(mat, vec):
    """SpmvMv: device, layout and shape checks with the bridge's messages, then ``mv``."""
    if not mat.is_cuda:
        raise RuntimeError("mat must be on a ROCm device")
    if not vec.is_cuda or vec.dim() != 1 or not vec.is_contiguous():
        raise RuntimeError("vec must be a contiguous one-dimensional tensor on a ROCm device")
    if mat.layout != torch.sparse_csr or mat.dim() != 2:
        raise RuntimeError("ops_sparse::spmv requires a two-dimensional CSR matrix")
    if mat.device != vec.device:
        raise RuntimeError("mat and vec must be on the same ROCm device")
    if mat.size(1) != vec.numel():
        raise RuntimeError(f"SpMV matrix columns must equal vector length, got {mat.size(1)} columns and "
                           f"{vec.numel()} elements")
    try:
        return _mv(mat, vec)
    except ValueError as e:
        raise RuntimeError(str(e)) from None


def _spmv_npu(row_ptr, col_ind, values, x, y, alpha, beta, trans, base):
    """RunSpmv: y = alpha*op(A)*x + beta*y into ``y`` itself; returns ``y``."""
    for name, t in (("row_ptr", row_ptr), ("col_ind", col_ind)):
        if t.dtype != torch.int32:
            raise RuntimeError(f"{name} must use int32 indices for SpMV")
    for name, t in (("row_ptr", row_ptr), ("col_ind", col_ind), ("values", values), ("x", x), ("y", y)):
        if t.dim() != 1 or not t.is_contiguous():
            raise RuntimeError(f"{name} must be a contiguous one-dimensional tensor")
    try:
        rows, cols, _ = _validate_npu_args(row_ptr, col_ind, values, x, y, trans, base)
    except ValueError as e:
        raise RuntimeError(str(e)) from None
    op = {"N": Operation.NON_TRANSPOSE, "T": Operation.TRANSPOSE, "H": Operation.CONJUGATE_TRANSPOSE}[trans]
    plan = CsrSpMV(rows, cols, row_ptr, col_ind, values, x, y, alpha, beta, op=op, base=base)
    plan.preprocess()
    plan.run()
    return y


def register():
    """Define both libraries and their ROCm kernels (idempotent)."""
    global _LIBS
    if _LIBS is not None:
        return _LIBS
    main = torch.library.Library("ops_sparse", "DEF")
    main.define("spmv(Tensor mat, Tensor vec) -> Tensor")
    main.impl("spmv", _spmv, "CUDA")
    main.impl("spmv", _spmv, "SparseCsrCUDA")
    test = torch.library.Library("ops_sparse_test", "DEF")
    test.define("spmv_npu(Tensor row_ptr, Tensor col_ind, Tensor values, Tensor x, Tensor(a!) y, Scalar alpha, "
                "Scalar beta, str trans, int base) -> Tensor(a!)")
    test.impl("spmv_npu", _spmv_npu, "CUDA")
    _LIBS = (main, test)
    return _LIBS


register()
