"""MI355X (gfx950) CSR SpMV behind the ops-sparse C API.

``ops_sparse.spmv`` mirrors the reference's torch binding (mv / spmv_npu /
spmv_npu_workspace); ``ops_sparse._lib`` is the ctypes view of
libaclsparse_hip.so.  Importing the package does not load the library; the
first call does, and raises if the library has not been built.
"""
from . import _lib  # noqa: F401
from .spmv import CsrSpMV, SpMVOp, mv, spmv_device, spmv_device_workspace, spmv_npu, spmv_npu_workspace  # noqa: F401
