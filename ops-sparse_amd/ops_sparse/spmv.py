"""Host-side mirror of the reference's SpMV torch binding, over the C ABI.

Reference interface mirrored here (sparse/spmv/torch_extension/csrc/spmv.cpp):
  * ``mv(mat, vec)``                 -- SpMvCsr (:290-322): A @ vec for a sparse
                                       CSR tensor, alpha=1, beta=0, base 0,
                                       int64 indices narrowed to int32, int8
                                       values produce int32.
  * ``spmv_npu(row_ptr, col_ind, values, x, y, alpha, beta, trans, base)``
                                     -- SpMvNpu (:381-411): explicit CSR arrays,
                                       y is not modified, the result is returned.
  * ``spmv_npu_workspace(...)``      -- SpMvNpuWorkspace (:416-460).
The names keep the reference's ``_npu`` suffix so callers switch by import
only; ``spmv_device`` / ``spmv_device_workspace`` are the same functions.

Everything runs through libaclsparse_hip.so on the current torch stream; torch
provides device memory and the stream, nothing else.  There is no CPU path.
"""
import ctypes

import torch

from . import _lib
from ._lib import DataType, IndexBase, IndexType, Operation, PointerMode, SpMVAlg, check

_INT32_MAX = 2**31 - 1

_ACL_DTYPE = {
    torch.int8: DataType.INT8,
    torch.float16: DataType.FLOAT16,
    torch.bfloat16: DataType.BF16,
    torch.float32: DataType.FLOAT,
    torch.int32: DataType.INT32,
    torch.complex64: DataType.COMPLEX64,
}

# values dtype -> allowed output dtypes (csrc/spmv.cpp:129-147)
_VALID_COMBOS = {
    torch.int8: (torch.int32, torch.float32),
    torch.float16: (torch.float16, torch.float32),
    torch.bfloat16: (torch.bfloat16, torch.float32),
    torch.float32: (torch.float32, torch.complex64),
    torch.complex64: (torch.complex64,),
}


def acl_dtype(dtype):
    try:
        return _ACL_DTYPE[dtype]
    except KeyError:
        raise TypeError(f"SpMV supports int8, float16, bfloat16, float32, int32 and complex64, got {dtype}")


def compute_type_for(out_dtype):
    """INT32 output -> exact integer path, complex64 -> complex, else FP32 (csrc/spmv.cpp:150-159)."""
    if out_dtype == torch.int32:
        return DataType.INT32
    if out_dtype == torch.complex64:
        return DataType.COMPLEX64
    return DataType.FLOAT


def _stream_ptr(device):
    s = torch.cuda.current_stream(device).cuda_stream
    return s if s != 0 else _lib.HIP_NULL_STREAM


def _ptr(t):
    return ctypes.c_void_p(t.data_ptr()) if t is not None and t.numel() > 0 else ctypes.c_void_p(0)


class HostScalar:
    """alpha/beta in the compute type, kept alive for the duration of a call.

    Conversions follow the torch extension's HostScalar
    (sparse/spmv/torch_extension/csrc/spmv.cpp:162-190): INT32 compute rejects
    a non-zero imaginary part and values outside the int32 range and truncates
    the real part; real compute rejects a non-zero imaginary part; complex
    compute keeps both parts.  Violations raise ValueError.
    """

    def __init__(self, value, compute_type):
        value = complex(value)
        if compute_type == DataType.COMPLEX64:
            self._obj = _lib.Complex(value.real, value.imag)
            return
        if value.imag != 0.0:
            kind = "int32 SpMV" if compute_type == DataType.INT32 else "real SpMV compute type"
            raise ValueError(f"{kind} cannot use a complex scalar, but got imaginary part {value.imag}")
        if compute_type == DataType.INT32:
            if not -2.0**31 <= value.real <= float(_INT32_MAX):
                raise ValueError(f"int32 SpMV scalar {value.real} is out of the int32 range")
            self._obj = ctypes.c_int32(int(value.real))
        else:
            self._obj = ctypes.c_float(value.real)

    @property
    def ptr(self):
        return ctypes.cast(ctypes.pointer(self._obj), ctypes.c_void_p)


class Handle:
    """aclsparseHandle_t bound to a torch stream."""

    def __init__(self, stream=None):
        self._lib = _lib.lib()
        self.h = ctypes.c_void_p(0)
        check("aclsparseCreate", self._lib.aclsparseCreate(ctypes.byref(self.h)))
        if stream is not None:
            self.set_stream(stream)

    def set_stream(self, stream_ptr):
        check("aclsparseSetStream", self._lib.aclsparseSetStream(self.h, ctypes.c_void_p(stream_ptr)))

    def set_pointer_mode(self, mode):
        check("aclsparseSetPointerMode", self._lib.aclsparseSetPointerMode(self.h, int(mode)))

    def close(self):
        if self.h:
            self._lib.aclsparseDestroy(self.h)
            self.h = ctypes.c_void_p(0)

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class CsrDescr:
    """aclsparseSpMatDescr_t for a CSR matrix held in torch tensors (weak references, like the C API)."""

    def __init__(self, rows, cols, row_ptr, col_ind, values, base=0, value_dtype=None):
        self._lib = _lib.lib()
        self.d = ctypes.c_void_p(0)
        ptr_type = IndexType.I64 if row_ptr is not None and row_ptr.dtype == torch.int64 else IndexType.I32
        vdt = value_dtype if value_dtype is not None else values.dtype
        nnz = col_ind.numel() if col_ind is not None else 0
        check("aclsparseCreateCsr", self._lib.aclsparseCreateCsr(
            ctypes.byref(self.d), int(rows), int(cols), int(nnz), _ptr(row_ptr), _ptr(col_ind), _ptr(values),
            int(ptr_type), int(IndexType.I32), int(base), int(acl_dtype(vdt))))

    def set_strides(self, row_stride, col_stride, val_stride):
        check("aclsparseCsrSetStrides", self._lib.aclsparseCsrSetStrides(self.d, row_stride, col_stride, val_stride))

    def close(self):
        if self.d:
            self._lib.aclsparseDestroySpMat(self.d)
            self.d = ctypes.c_void_p(0)

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class DnVecDescr:
    def __init__(self, size, tensor, dtype=None):
        self._lib = _lib.lib()
        self.d = ctypes.c_void_p(0)
        dt = dtype if dtype is not None else tensor.dtype
        check("aclsparseCreateDnVec", self._lib.aclsparseCreateDnVec(
            ctypes.byref(self.d), int(size), _ptr(tensor), int(acl_dtype(dt))))

    def set_stride(self, stride):
        check("aclsparseDnVecSetStride", self._lib.aclsparseDnVecSetStride(self.d, stride))

    def close(self):
        if self.d:
            self._lib.aclsparseDestroyDnVec(self.d)
            self.d = ctypes.c_void_p(0)

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class CsrSpMV:
    """Three-stage SpMV (GetBufferSize -> Preprocess -> SpMV) on fixed tensors.

    Mirrors RunSpMv (csrc/spmv.cpp:219-259) but keeps the descriptors and the
    workspace alive so the product can be executed repeatedly (the benchmark
    times only :meth:`run`).
    """

    def __init__(self, rows, cols, row_ptr, col_ind, values, x, y, alpha=1.0, beta=0.0,
                 op=Operation.NON_TRANSPOSE, base=0, alg=SpMVAlg.DEFAULT, compute_type=None):
        self._lib = _lib.lib()
        device = values.device if values is not None else y.device
        self.device = device
        self.op = Operation(op)
        self.alg = SpMVAlg(alg)
        self.compute_type = compute_type if compute_type is not None else compute_type_for(y.dtype)
        self.handle = Handle(_stream_ptr(device))
        self.mat = CsrDescr(rows, cols, row_ptr, col_ind, values, base, value_dtype=x.dtype)
        transpose = self.op != Operation.NON_TRANSPOSE
        self.x = DnVecDescr(rows if transpose else cols, x)
        self.y = DnVecDescr(cols if transpose else rows, y)
        self.tensors = (row_ptr, col_ind, values, x, y)
        self.alpha = HostScalar(alpha, self.compute_type)
        self.beta = HostScalar(beta, self.compute_type)
        size = ctypes.c_size_t(0)
        check("aclsparseSpMVGetBufferSize", self._lib.aclsparseSpMVGetBufferSize(
            self.handle.h, int(self.op), self.alpha.ptr, self.mat.d, self.x.d, self.beta.ptr, self.y.d,
            int(self.compute_type), int(self.alg), ctypes.byref(size)))
        self.buffer_size = size.value
        self.workspace = torch.empty(max(self.buffer_size, 64), dtype=torch.uint8, device=device)

    def preprocess(self):
        check("aclsparseSpMVPreprocess", self._lib.aclsparseSpMVPreprocess(
            self.handle.h, int(self.op), self.alpha.ptr, self.mat.d, self.x.d, self.beta.ptr, self.y.d,
            int(self.compute_type), int(self.alg), ctypes.c_void_p(self.workspace.data_ptr())))

    def run(self):
        check("aclsparseSpMV", self._lib.aclsparseSpMV(
            self.handle.h, int(self.op), self.alpha.ptr, self.mat.d, self.x.d, self.beta.ptr, self.y.d,
            int(self.compute_type), int(self.alg), ctypes.c_void_p(self.workspace.data_ptr())))


def _validate_npu_args(row_ptr, col_ind, values, x, y, trans, base):
    """Argument checks and shape inference of ValidateSpMvNpuArgs (csrc/spmv.cpp:334-379)."""
    tensors = (row_ptr, col_ind, values, x, y)
    if not all(t.is_cuda for t in tensors):
        raise ValueError("all tensors must be on a ROCm device")
    if len({t.device for t in tensors}) != 1:
        raise ValueError("all tensors must be on the same device")
    if row_ptr.dtype not in (torch.int32, torch.int64) or col_ind.dtype != torch.int32:
        raise ValueError("row_ptr must be int32 or int64 and col_ind int32")
    if col_ind.numel() != values.numel():
        raise ValueError(f"col_ind and values length mismatch: {col_ind.numel()} vs {values.numel()}")
    if x.dtype != values.dtype:
        raise ValueError(f"x and values must have the same dtype, got {x.dtype} and {values.dtype}")
    if base not in (0, 1):
        raise ValueError(f"base must be 0 or 1, got {base}")
    if trans not in ("N", "T", "H"):
        raise ValueError(f"trans must be N, T or H, got {trans}")
    if x.dim() != 1 or y.dim() != 1:
        raise ValueError("x and y must be one-dimensional")
    if row_ptr.numel() < 1:
        raise ValueError("row_ptr must not be empty")
    if (row_ptr.numel() - 1 > _INT32_MAX or x.numel() > _INT32_MAX or y.numel() > _INT32_MAX):
        raise ValueError(f"SpMV dims must stay within the int32 limit {_INT32_MAX}")
    if y.dtype not in _VALID_COMBOS.get(values.dtype, ()):
        raise ValueError(f"unsupported SpMV dtype combination: values {values.dtype} -> y {y.dtype}")
    rows = row_ptr.numel() - 1
    is_trans = trans != "N"
    cols = y.size(0) if is_trans else x.size(0)
    need_x = rows if is_trans else cols
    need_y = cols if is_trans else rows
    if x.size(0) < need_x or y.size(0) < need_y:
        raise ValueError("x or y is too small for the requested op")
    return rows, cols, is_trans


def spmv_npu(row_ptr, col_ind, values, x, y, alpha=1.0, beta=0.0, trans="N", base=0):
    """y_out = alpha*op(A)*x + beta*y from explicit CSR arrays; ``y`` is left unchanged."""
    rows, cols, is_trans = _validate_npu_args(row_ptr, col_ind, values, x, y, trans, base)
    beta_zero = complex(beta) == 0
    y_out = torch.empty_like(y) if (beta_zero and not is_trans) else y.clone(memory_format=torch.contiguous_format)
    op = Operation.NON_TRANSPOSE if trans == "N" else (
        Operation.CONJUGATE_TRANSPOSE if trans == "H" else Operation.TRANSPOSE)
    plan = CsrSpMV(rows, cols, row_ptr.contiguous(), col_ind.contiguous(), values.contiguous(), x.contiguous(),
                   y_out, alpha, beta, op=op, base=base)
    plan.preprocess()
    plan.run()
    return y_out


def spmv_npu_workspace(row_ptr, col_ind, values, x, y, alpha=1.0, beta=0.0, trans="N", base=0):
    """Workspace bytes aclsparseSpMVGetBufferSize reports for the same call."""
    rows, cols, is_trans = _validate_npu_args(row_ptr, col_ind, values, x, y, trans, base)
    op = Operation.TRANSPOSE if is_trans else Operation.NON_TRANSPOSE
    plan = CsrSpMV(rows, cols, row_ptr, col_ind, values, x, y, alpha, beta, op=op, base=base)
    return plan.buffer_size


spmv_device = spmv_npu
spmv_device_workspace = spmv_npu_workspace


def mv(mat, vec):
    """A @ vec for a torch sparse CSR tensor on a ROCm device (SpMvCsr semantics)."""
    if mat.layout != torch.sparse_csr:
        raise ValueError(f"mat must use the sparse CSR layout, got {mat.layout}")
    if not (mat.is_cuda and vec.is_cuda) or mat.device != vec.device:
        raise ValueError("mat and vec must be on the same ROCm device")
    if mat.dim() != 2 or vec.dim() != 1 or vec.layout != torch.strided:
        raise ValueError("mat must be 2-D sparse CSR and vec a 1-D dense vector")
    if mat.dtype != vec.dtype:
        raise ValueError(f"mat and vec must have the same dtype, got {mat.dtype} and {vec.dtype}")
    if mat.size(1) != vec.size(0):
        raise ValueError(f"mat and vec shapes cannot be multiplied ({tuple(mat.shape)} and {tuple(vec.shape)})")
    if mat.size(0) > _INT32_MAX or mat.size(1) > _INT32_MAX or mat._nnz() > _INT32_MAX:
        raise ValueError("mat exceeds the int32 CSR limit")
    out_dtype = torch.int32 if mat.dtype == torch.int8 else mat.dtype
    y = torch.empty(mat.size(0), dtype=out_dtype, device=mat.device)
    if mat.size(0) == 0:
        return y
    if mat.size(1) == 0 or mat._nnz() == 0:
        return y.zero_()
    row_ptr = mat.crow_indices().to(torch.int32).contiguous()
    col_ind = mat.col_indices().to(torch.int32).contiguous()
    values = mat.values().contiguous()
    plan = CsrSpMV(mat.size(0), mat.size(1), row_ptr, col_ind, values, vec.contiguous(), y, 1.0, 0.0)
    plan.preprocess()
    plan.run()
    return y


class SpMVOp:
    """aclsparseSpMVOp on torch tensors: Z = alpha*A*X + beta*Y (fp32, NON_TRANSPOSE).

    Mirrors the reference's seven-call sequence (sparse/spmv_op/arch35/spmv_op_host.cpp):
    bufferSize -> createDescr (ALG2 builds the reorder / bin_edge tables) ->
    createPlan -> execute (:meth:`run`) -> destroyPlan / destroyDescr.
    """

    def __init__(self, rows, cols, row_ptr, col_ind, values, x, y, z, alg=_lib.SpMVOpAlg.DEFAULT, base=0):
        self._lib = _lib.lib()
        self.handle = Handle(_stream_ptr(values.device))
        self.mat = CsrDescr(rows, cols, row_ptr, col_ind, values, base)
        self.x = DnVecDescr(cols, x)
        self.y = DnVecDescr(rows, y)
        self.z = DnVecDescr(rows, z)
        self.tensors = (row_ptr, col_ind, values, x, y, z)
        size = ctypes.c_size_t(0)
        check("aclsparseSpMVOp_bufferSize", self._lib.aclsparseSpMVOp_bufferSize(
            self.handle.h, int(Operation.NON_TRANSPOSE), self.mat.d, self.x.d, self.y.d, self.z.d,
            int(DataType.FLOAT), int(alg), ctypes.byref(size)))
        self.buffer_size = size.value
        self.buffer = torch.empty(max(size.value, 64), dtype=torch.uint8, device=values.device)
        self.descr = ctypes.c_void_p(0)
        check("aclsparseSpMVOp_createDescr", self._lib.aclsparseSpMVOp_createDescr(
            self.handle.h, ctypes.byref(self.descr), int(Operation.NON_TRANSPOSE), self.mat.d, self.x.d, self.y.d,
            self.z.d, int(DataType.FLOAT), int(alg), ctypes.c_void_p(self.buffer.data_ptr())))
        self.plan = ctypes.c_void_p(0)
        check("aclsparseSpMVOp_createPlan", self._lib.aclsparseSpMVOp_createPlan(
            self.handle.h, self.descr, ctypes.byref(self.plan), None, 0))

    def run(self, alpha=1.0, beta=0.0):
        """Execute; alpha/beta are Python floats (HOST pointer mode) or one-element
        device tensors (the handle is switched to DEVICE pointer mode)."""
        if isinstance(alpha, torch.Tensor):
            self.handle.set_pointer_mode(PointerMode.DEVICE)
            a, b = ctypes.c_void_p(alpha.data_ptr()), ctypes.c_void_p(beta.data_ptr())
            check("aclsparseSpMVOp", self._lib.aclsparseSpMVOp(
                self.handle.h, self.plan, a, b, self.x.d, self.y.d, self.z.d))
            return
        self.handle.set_pointer_mode(PointerMode.HOST)
        a, b = ctypes.c_float(alpha), ctypes.c_float(beta)
        check("aclsparseSpMVOp", self._lib.aclsparseSpMVOp(
            self.handle.h, self.plan, ctypes.byref(a), ctypes.byref(b), self.x.d, self.y.d, self.z.d))

    def close(self):
        if self.plan:
            self._lib.aclsparseSpMVOp_destroyPlan(self.plan)
            self.plan = ctypes.c_void_p(0)
        if self.descr:
            self._lib.aclsparseSpMVOp_destroyDescr(self.descr)
            self.descr = ctypes.c_void_p(0)

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
