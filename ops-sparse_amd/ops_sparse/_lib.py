"""ctypes binding of libaclsparse_hip.so (the C ABI declared in include/cann_ops_sparse.h).

The library is loaded from ``ops-sparse_amd/lib`` in the source tree.  There is
no CPU fallback: if the shared library is missing, :func:`lib` raises.
"""
import ctypes
import enum
import os

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_DIR = os.path.join(os.path.dirname(_HERE), "lib")
LIB_PATH = os.environ.get("ACLSPARSE_HIP_LIB", os.path.join(LIB_DIR, "libaclsparse_hip.so"))


class Status(enum.IntEnum):
    """aclsparseStatus_t (include/cann_ops_sparse.h:124-174 of the reference)."""
    SUCCESS = 0
    NOT_INITIALIZED = 1
    ALLOC_FAILED = 2
    INVALID_VALUE = 3
    ARCH_MISMATCH = 4
    EXECUTION_FAILED = 5
    INTERNAL_ERROR = 6
    MATRIX_TYPE_NOT_SUPPORTED = 7
    NOT_SUPPORTED = 8
    INSUFFICIENT_RESOURCES = 9
    HANDLE_IS_NULLPTR = 10


class DataType(enum.IntEnum):
    """aclDataType values (CANN acl_base_rt.h)."""
    FLOAT = 0
    FLOAT16 = 1
    INT8 = 2
    INT32 = 3
    UINT8 = 4
    INT16 = 6
    UINT16 = 7
    UINT32 = 8
    INT64 = 9
    UINT64 = 10
    DOUBLE = 11
    BOOL = 12
    COMPLEX64 = 16
    BF16 = 27


class Operation(enum.IntEnum):
    NON_TRANSPOSE = 0
    TRANSPOSE = 1
    CONJUGATE_TRANSPOSE = 2


class SpMVAlg(enum.IntEnum):
    DEFAULT = 0
    COO_ALG1 = 1
    COO_ALG2 = 2
    CSR_ALG1 = 3
    CSR_ALG2 = 4
    SELL_ALG1 = 5
    CSR_ALG_CUBE = 6


class SpMVOpAlg(enum.IntEnum):
    DEFAULT = 0
    ALG1 = 1
    ALG2 = 2


class SpMMOpAlg(enum.IntEnum):
    DEFAULT = 0
    ALG1 = 1
    ALG2 = 2
    ALG1_HIGH_PRECISION = 3


class Order(enum.IntEnum):
    ROW = 0
    COL = 1


class IndexType(enum.IntEnum):
    I32 = 0
    I64 = 1


class IndexBase(enum.IntEnum):
    ZERO = 0
    ONE = 1


class PointerMode(enum.IntEnum):
    HOST = 0
    DEVICE = 1


class Format(enum.IntEnum):
    COO = 0
    CSR = 1
    CSC = 2
    BLOCKED_ELL = 3
    SLICED_ELL = 4
    BSR = 5


class Complex(ctypes.Structure):
    _fields_ = [("x", ctypes.c_float), ("y", ctypes.c_float)]


HIP_NULL_STREAM = 1  # ACL_SPARSE_HIP_NULL_STREAM

_vp = ctypes.c_void_p
_pvp = ctypes.POINTER(ctypes.c_void_p)
_i64 = ctypes.c_int64
_pi64 = ctypes.POINTER(ctypes.c_int64)
_i32 = ctypes.c_int32
_sz = ctypes.c_size_t

# name -> argtypes; every function returns aclsparseStatus_t (int) unless RESTYPES says otherwise
RESTYPES = {"aclsparseHipBuildId": ctypes.c_char_p}
SIGNATURES = {
    "aclsparseHipBuildId": [],
    "aclsparseCreate": [_pvp],
    "aclsparseDestroy": [_vp],
    "aclsparseSetStream": [_vp, _vp],
    "aclsparseGetStream": [_vp, _pvp],
    "aclsparseSetWorkspace": [_vp, _vp, _sz],
    "aclsparseGetWorkspace": [_vp, _pvp, ctypes.POINTER(_sz)],
    "aclsparseGetVersion": [_vp, ctypes.POINTER(ctypes.c_int)],
    "aclsparseSetPointerMode": [_vp, _i32],
    "aclsparseGetPointerMode": [_vp, ctypes.POINTER(_i32)],
    "aclsparseCreateDnVec": [_pvp, _i64, _vp, _i32],
    "aclsparseCreateConstDnVec": [_pvp, _i64, _vp, _i32],
    "aclsparseDestroyDnVec": [_vp],
    "aclsparseDnVecGet": [_vp, _pi64, _pvp, ctypes.POINTER(_i32)],
    "aclsparseDnVecGetValues": [_vp, _pvp],
    "aclsparseDnVecSetValues": [_vp, _vp],
    "aclsparseDnVecSetStride": [_vp, _i64],
    "aclsparseDnVecGetStride": [_vp, _pi64],
    "aclsparseCreateCsr": [_pvp, _i64, _i64, _i64, _vp, _vp, _vp, _i32, _i32, _i32, _i32],
    "aclsparseCreateConstCsr": [_pvp, _i64, _i64, _i64, _vp, _vp, _vp, _i32, _i32, _i32, _i32],
    "aclsparseCsrSetPointers": [_vp, _vp, _vp, _vp],
    "aclsparseCsrSetStrides": [_vp, _i64, _i64, _i64],
    "aclsparseCsrGetStrides": [_vp, _pi64, _pi64, _pi64],
    "aclsparseDestroySpMat": [_vp],
    "aclsparseSpMatGetFormat": [_vp, ctypes.POINTER(_i32)],
    "aclsparseSpMatGetIndexBase": [_vp, ctypes.POINTER(_i32)],
    "aclsparseSpMatGetValues": [_vp, _pvp],
    "aclsparseSpMatSetValues": [_vp, _vp],
    "aclsparseSpMatGetSize": [_vp, _pi64, _pi64, _pi64],
    "aclsparseCsrGet": [_vp, _pi64, _pi64, _pi64, _pvp, _pvp, _pvp, ctypes.POINTER(_i32),
                        ctypes.POINTER(_i32), ctypes.POINTER(_i32), ctypes.POINTER(_i32)],
    "aclsparseSpMVGetBufferSize": [_vp, _i32, _vp, _vp, _vp, _vp, _vp, _i32, _i32, ctypes.POINTER(_sz)],
    "aclsparseSpMVPreprocess": [_vp, _i32, _vp, _vp, _vp, _vp, _vp, _i32, _i32, _vp],
    "aclsparseSpMV": [_vp, _i32, _vp, _vp, _vp, _vp, _vp, _i32, _i32, _vp],
    "aclsparseSpMVNoAlloc": [_vp, _i32, _vp, _vp, _vp, _vp, _vp, _i32, _i32],
    "aclsparseSpMVOp_bufferSize": [_vp, _i32, _vp, _vp, _vp, _vp, _i32, _i32, ctypes.POINTER(_sz)],
    "aclsparseSpMVOp_createDescr": [_vp, _pvp, _i32, _vp, _vp, _vp, _vp, _i32, _i32, _vp],
    "aclsparseSpMVOp_destroyDescr": [_vp],
    "aclsparseSpMVOp_createPlan": [_vp, _vp, _pvp, _vp, _sz],
    "aclsparseSpMVOp_destroyPlan": [_vp],
    "aclsparseSpMVOp_setGlobalUserData": [_vp, _vp, ctypes.c_char_p, _vp, _sz],
    "aclsparseSpMVOp": [_vp, _vp, _vp, _vp, _vp, _vp, _vp],
    "aclsparseCreateDnMat": [_pvp, _i64, _i64, _i64, _vp, _i32, _i32],
    "aclsparseCreateConstDnMat": [_pvp, _i64, _i64, _i64, _vp, _i32, _i32],
    "aclsparseDestroyDnMat": [_vp],
    "aclsparseDnMatGet": [_vp, _pi64, _pi64, _pi64, _pvp, ctypes.POINTER(_i32), ctypes.POINTER(_i32)],
    "aclsparseConstDnMatGet": [_vp, _pi64, _pi64, _pi64, _pvp, ctypes.POINTER(_i32), ctypes.POINTER(_i32)],
    "aclsparseDnMatGetValues": [_vp, _pvp],
    "aclsparseConstDnMatGetValues": [_vp, _pvp],
    "aclsparseDnMatSetValues": [_vp, _vp],
    "aclsparseSpMMOp_bufferSize": [_vp, _i32, _i32, _vp, _vp, _vp, _i32, _i32, ctypes.POINTER(_sz)],
    "aclsparseSpMMOp_createDescr": [_vp, _pvp, _i32, _i32, _vp, _vp, _vp, _i32, _i32, _vp],
    "aclsparseSpMMOp_destroyDescr": [_vp],
    "aclsparseSpMMOp_createPlan": [_vp, _vp, _pvp, _vp, _sz],
    "aclsparseSpMMOp_destroyPlan": [_vp],
    "aclsparseSpMMOp_setGlobalUserData": [_vp, _vp, ctypes.c_char_p, _vp, _sz],
    "aclsparseSpMMOp": [_vp, _vp, _vp, _vp, _vp, _vp],
}

_LIB = None


def library_build_id(handle):
    """The build id compiled into a loaded library (aclsparseHipBuildId)."""
    fn = handle.aclsparseHipBuildId
    fn.argtypes = []
    fn.restype = ctypes.c_char_p
    return fn().decode()


def lib():
    """Loads the HIP library once; raises if it has not been built or was built
    from sources other than the ones in this tree."""
    global _LIB
    if _LIB is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(
                f"{LIB_PATH} is missing: build it with `python -c 'import __graft_entry__ as g; g.build()'` "
                "(there is no CPU fallback for the SpMV path)")
        handle = ctypes.CDLL(LIB_PATH)
        from .build import CSRC, source_hash

        if os.path.isdir(CSRC) and "ACLSPARSE_HIP_LIB" not in os.environ:
            want, got = source_hash(), library_build_id(handle)
            if want != got:
                raise RuntimeError(f"{LIB_PATH} is stale: built from sources {got}, the tree holds {want}; "
                                   "rebuild it with `python -c 'import __graft_entry__ as g; g.build()'`")
        for name, args in SIGNATURES.items():
            fn = getattr(handle, name)
            fn.argtypes = args
            fn.restype = RESTYPES.get(name, ctypes.c_int)
        _LIB = handle
    return _LIB


class AclSparseError(RuntimeError):
    def __init__(self, fn, status):
        super().__init__(f"{fn} failed with {Status(status).name} ({status})")
        self.status = Status(status)


def check(fn_name, status):
    if status != Status.SUCCESS:
        raise AclSparseError(fn_name, status)
