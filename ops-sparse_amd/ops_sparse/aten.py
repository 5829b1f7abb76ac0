"""``torch.mv(csr, vec)`` on a ROCm device routed to this library.

Mirrors the reference's ATen registration
(sparse/spmv/torch_extension/spmv.py:43-46), which implements ``aten::mv``
for the ``SparseCsrPrivateUse1`` key.  On ROCm a CSR tensor on the GPU
dispatches through ``SparseCsrCUDA``, so that is the key implemented here.
No schema is defined: ``aten::mv`` already has one, and its Meta kernel
stays PyTorch's.  Semantics are ``SpMvCsr``'s: ``alpha = 1, beta = 0``; the
checks and messages are the bridge's (torch_npu/spmv_npu.cpp:384-407, 442-445).

The registration replaces PyTorch's own CSR ``mv`` kernel for the process,
as importing the reference package does for the NPU.
"""
import warnings

import torch

from .bridge import _spmv

_LIB = None


def register():
    """Implement aten::mv for SparseCsrCUDA with the bridge's ``spmv`` (SpmvMv) kernel (idempotent)."""
    global _LIB
    if _LIB is not None:
        return _LIB
    lib = torch.library.Library("aten", "IMPL")
    with warnings.catch_warnings():
        # PyTorch warns that a built-in kernel is being overridden: that is the point.
        warnings.simplefilter("ignore", UserWarning)
        lib.impl("mv", _spmv, "SparseCsrCUDA")
    _LIB = lib
    return lib


register()
