"""aclsparseSpMMOp on torch tensors: C = alpha * A * op(B) + beta * C.

Mirrors the reference's seven-call sequence (sparse/spmm_op/arch35/spmm_op_host.cpp):
bufferSize -> createDescr (ALG2 builds the reorder / bin_edge tables) ->
createPlan -> execute (:meth:`SpMMOp.run`, B and C may change between runs)
-> destroyPlan / destroyDescr.  A is CSR (fp32 or fp16 values, int32 or int64
row offsets, index base 0 or 1); B and C are dense tensors of A's dtype in
row or column order.
"""
import ctypes

import torch

from . import _lib
from ._lib import DataType, Operation, Order, PointerMode, SpMMOpAlg, check
from .spmv import CsrDescr, Handle, _ptr, _stream_ptr, acl_dtype


class DnMatDescr:
    """aclsparseDnMatDescr_t over a torch tensor's storage (weak reference, like the C API)."""

    def __init__(self, rows, cols, ld, tensor, order=Order.ROW, dtype=None):
        self._lib = _lib.lib()
        self.d = ctypes.c_void_p(0)
        dt = dtype if dtype is not None else tensor.dtype
        check("aclsparseCreateDnMat", self._lib.aclsparseCreateDnMat(
            ctypes.byref(self.d), int(rows), int(cols), int(ld), _ptr(tensor), int(acl_dtype(dt)), int(order)))

    @classmethod
    def of(cls, t):
        """Descriptor of a 2-D tensor: row order when its last dimension is contiguous,
        column order when its first is (a transposed view)."""
        r, c = t.shape
        if t.stride(1) == 1 and (r <= 1 or t.stride(0) >= max(c, 1)):
            return cls(r, c, max(t.stride(0), c, 1), t, Order.ROW)
        if t.stride(0) == 1 and (c <= 1 or t.stride(1) >= max(r, 1)):
            return cls(r, c, max(t.stride(1), r, 1), t, Order.COL)
        raise ValueError("dense operands must be row- or column-major views")

    def close(self):
        if self.d:
            self._lib.aclsparseDestroyDnMat(self.d)
            self.d = ctypes.c_void_p(0)

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class SpMMOp:
    """Plan for C = alpha * A * op(B) + beta * C with a fixed CSR A and opB."""

    def __init__(self, rows, cols, row_ptr, col_ind, values, b, c, op_b=Operation.NON_TRANSPOSE,
                 alg=SpMMOpAlg.DEFAULT, base=0):
        self._lib = _lib.lib()
        self.handle = Handle(_stream_ptr(values.device))
        self.mat = CsrDescr(rows, cols, row_ptr, col_ind, values, base)
        self.tensors = (row_ptr, col_ind, values)
        self.op_b = op_b
        bd, cd = DnMatDescr.of(b), DnMatDescr.of(c)
        size = ctypes.c_size_t(0)
        check("aclsparseSpMMOp_bufferSize", self._lib.aclsparseSpMMOp_bufferSize(
            self.handle.h, int(Operation.NON_TRANSPOSE), int(op_b), self.mat.d, bd.d, cd.d, int(DataType.FLOAT),
            int(alg), ctypes.byref(size)))
        self.buffer_size = size.value
        self.buffer = torch.empty(max(size.value, 64), dtype=torch.uint8, device=values.device)
        self.descr = ctypes.c_void_p(0)
        check("aclsparseSpMMOp_createDescr", self._lib.aclsparseSpMMOp_createDescr(
            self.handle.h, ctypes.byref(self.descr), int(Operation.NON_TRANSPOSE), int(op_b), self.mat.d, bd.d,
            cd.d, int(DataType.FLOAT), int(alg), ctypes.c_void_p(self.buffer.data_ptr())))
        self.plan = ctypes.c_void_p(0)
        check("aclsparseSpMMOp_createPlan", self._lib.aclsparseSpMMOp_createPlan(
            self.handle.h, self.descr, ctypes.byref(self.plan), None, 0))

    def run(self, b, c, alpha=1.0, beta=0.0):
        """C = alpha * A * op(B) + beta * C on the handle's stream; alpha/beta are Python
        floats (HOST pointer mode) or one-element fp32 device tensors (DEVICE mode)."""
        bd, cd = DnMatDescr.of(b), DnMatDescr.of(c)
        if isinstance(alpha, torch.Tensor):
            self.handle.set_pointer_mode(PointerMode.DEVICE)
            a, bt = ctypes.c_void_p(alpha.data_ptr()), ctypes.c_void_p(beta.data_ptr())
        else:
            self.handle.set_pointer_mode(PointerMode.HOST)
            af, bf = ctypes.c_float(alpha), ctypes.c_float(beta)
            a, bt = ctypes.byref(af), ctypes.byref(bf)
        check("aclsparseSpMMOp", self._lib.aclsparseSpMMOp(self.handle.h, self.plan, a, bt, bd.d, cd.d))

    def close(self):
        if self.plan:
            self._lib.aclsparseSpMMOp_destroyPlan(self.plan)
            self.plan = ctypes.c_void_p(0)
        if self.descr:
            self._lib.aclsparseSpMMOp_destroyDescr(self.descr)
            self.descr = ctypes.c_void_p(0)

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
