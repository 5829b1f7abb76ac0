"""MI355X (gfx950) CSR SpMV behind the ops-sparse C API.

``ops_sparse.spmv`` mirrors the reference's torch binding (mv / spmv_npu /
spmv_npu_workspace) and the SpMVOp plan sequence, ``ops_sparse.spmm`` the
SpMMOp plan sequence; ``ops_sparse._lib`` is the ctypes view of
libaclsparse_hip.so.  Importing the package implements ``aten::mv`` for CSR
tensors on ROCm devices (``torch.mv(csr, vec)``) with this library, as the
reference package does for the NPU, and defines the reference bridge's
``torch.ops.ops_sparse.spmv`` and ``torch.ops.ops_sparse_test.spmv_npu``.  It does not load the library; the first
call does, and raises if the library has not been built.
"""
from . import _lib  # noqa: F401
from .spmv import CsrSpMV, SpMVOp, mv, spmv_device, spmv_device_workspace, spmv_npu, spmv_npu_workspace  # noqa: F401
from .spmm import DnMatDescr, SpMMOp  # noqa: F401
from . import bridge  # noqa: F401,E402  (defines ops_sparse::spmv and ops_sparse_test::spmv_npu)
from . import aten  # noqa: F401,E402  (registers aten::mv for SparseCsrCUDA)
