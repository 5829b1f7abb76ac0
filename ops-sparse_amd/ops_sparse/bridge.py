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

# value dtypes SpmvMv accepts for mat and vec (int8 gives an int32 result)
_MV_DTYPES = (torch.int8, torch.float16, torch.bfloat16, torch.float32, torch.complex64)


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
    if mat.dtype not in _MV_DTYPES or vec.dtype not in _MV_DTYPES:
        # ToAclDataType (torch_npu/spmv_npu.cpp:286-297): anything else is rejected
        raise RuntimeError(f"unsupported A5 SpMV tensor dtype: mat {mat.dtype}, vec {vec.dtype} (supported: "
                           "int8, float16, bfloat16, float32, complex64)")
    try:
        return _mv(mat, vec)
    except (ValueError, TypeError) as e:
        raise RuntimeError(str(e)) from None


def _check_int32_scalars(alpha, beta):
    """MakeScalars for INT32 compute (torch_npu/spmv_npu.cpp:113-124): integral scalars
    (a Python int; a float such as 2.0 is not integral) that fit int32."""
    import numbers

    for v in (alpha, beta):
        if isinstance(v, bool) or not isinstance(v, numbers.Integral):
            raise RuntimeError("INT32 SpMV alpha/beta must be integral scalars")
    for v in (alpha, beta):
        if not -2**31 <= int(v) <= 2**31 - 1:
            raise RuntimeError("INT32 SpMV alpha/beta must fit int32")


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
    if y.dtype == torch.int32:
        _check_int32_scalars(alpha, beta)
    op = {"N": Operation.NON_TRANSPOSE, "T": Operation.TRANSPOSE, "H": Operation.CONJUGATE_TRANSPOSE}[trans]
    try:
        plan = CsrSpMV(rows, cols, row_ptr, col_ind, values, x, y, alpha, beta, op=op, base=base)
    except ValueError as e:  # real compute with a complex scalar
        raise RuntimeError(str(e)) from None
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
