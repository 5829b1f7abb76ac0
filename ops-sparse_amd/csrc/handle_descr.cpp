// Handle and descriptor entry points of libaclsparse_hip.
//
// Semantics follow sparse/common/aclsparse_auxiliary.cpp:103-180 (handle) and
// sparse/common/aclsparse_descr.cpp:346-416,620-720,942-1100 (CSR / DnVec
// descriptors) and :1102-1302 (dense matrix descriptors): status codes, null tolerance of the destroy calls, delayed
// binding of null storage and the plan reset rules.
#include <hip/hip_runtime.h>

#include <cstdint>
#include <limits>
#include <new>

#include "aclsparse_internal.h"

namespace {

bool IsValidValueType(aclDataType t)
{
    switch (t) {
        case ACL_FLOAT: case ACL_FLOAT16: case ACL_DOUBLE: case ACL_INT8: case ACL_INT16:
        case ACL_INT32: case ACL_INT64: case ACL_UINT8: case ACL_UINT16: case ACL_UINT32:
        case ACL_UINT64: case ACL_BF16: case ACL_COMPLEX64:
            return true;
        default:
            return false;
    }
}

// Element stride must be positive and keep (size-1)*stride addressable
// (sparse/common/aclsparse_descr.cpp:167-177).
bool IsValidElementStride(uint64_t logicalSize, int64_t stride)
{
    if (stride <= 0) return false;
    if (logicalSize <= 1U) return true;
    return static_cast<uint64_t>(stride) <=
           static_cast<uint64_t>(std::numeric_limits<int64_t>::max()) / (logicalSize - 1U);
}

bool IsIndexType(aclsparseIndexType_t t) { return t == ACL_SPARSE_INDEX_32I || t == ACL_SPARSE_INDEX_64I; }

aclsparseStatus_t CheckHandle(aclsparseHandle_t handle)
{
    if (handle == nullptr) return ACL_SPARSE_STATUS_HANDLE_IS_NULLPTR;
    if (handle->signature != aclsp::kHandleSignature) return ACL_SPARSE_STATUS_INVALID_VALUE;
    return ACL_SPARSE_STATUS_SUCCESS;
}

bool IsMat(aclsparseConstSpMatDescr_t d) { return d != nullptr && d->signature == aclsp::kSpMatSignature; }
bool IsVec(aclsparseConstDnVecDescr_t d) { return d != nullptr && d->signature == aclsp::kDnVecSignature; }
bool IsDnMat(aclsparseConstDnMatDescr_t d) { return d != nullptr && d->signature == aclsp::kDnMatSignature; }

void ResetPlan(aclsparseSpMatDescr* d) { d->plan = SpmvPlan{}; }

}  // namespace

extern "C" {

// ------------------------------- handle -------------------------------------

aclsparseStatus_t aclsparseCreate(aclsparseHandle_t* handle)
{
    if (handle == nullptr) return ACL_SPARSE_STATUS_HANDLE_IS_NULLPTR;
    if (*handle != nullptr) return ACL_SPARSE_STATUS_INVALID_VALUE;  // would leak an existing handle
    auto* h = new (std::nothrow) aclsparseContext();
    if (h == nullptr) return ACL_SPARSE_STATUS_ALLOC_FAILED;
    *handle = h;
    return ACL_SPARSE_STATUS_SUCCESS;
}

aclsparseStatus_t aclsparseDestroy(aclsparseHandle_t handle)
{
    aclsparseStatus_t st = CheckHandle(handle);
    if (st != ACL_SPARSE_STATUS_SUCCESS) return st;
    if (handle->default_workspace != nullptr) {
        hipStream_t s = handle->stream == ACL_SPARSE_HIP_NULL_STREAM ? nullptr
                                                                    : static_cast<hipStream_t>(handle->stream);
        if (handle->stream != nullptr) (void)hipStreamSynchronize(s);
        (void)hipFree(handle->default_workspace);
    }
    handle->signature = 0;
    delete handle;
    return ACL_SPARSE_STATUS_SUCCESS;
}

aclsparseStatus_t aclsparseSetStream(aclsparseHandle_t handle, aclrtStream stream)
{
    aclsparseStatus_t st = CheckHandle(handle);
    if (st != ACL_SPARSE_STATUS_SUCCESS) return st;
    if (handle->stream != stream) {
        ++handle->stream_epoch;
        if (handle->stream_epoch == 0) handle->stream_epoch = 1;
    }
    handle->stream = stream;
    return ACL_SPARSE_STATUS_SUCCESS;
}

aclsparseStatus_t aclsparseGetStream(aclsparseHandle_t handle, aclrtStream* stream)
{
    aclsparseStatus_t st = CheckHandle(handle);
    if (st != ACL_SPARSE_STATUS_SUCCESS) return st;
    if (stream == nullptr) return ACL_SPARSE_STATUS_INVALID_VALUE;
    *stream = handle->stream;
    return ACL_SPARSE_STATUS_SUCCESS;
}

aclsparseStatus_t aclsparseSetWorkspace(aclsparseHandle_t handle, void* workspace, size_t workspaceSize)
{
    aclsparseStatus_t st = CheckHandle(handle);
    if (st != ACL_SPARSE_STATUS_SUCCESS) return st;
    if (workspace == nullptr) {  // back to the library default workspace
        handle->user_workspace = nullptr;
        handle->user_workspace_size = 0;
        return ACL_SPARSE_STATUS_SUCCESS;
    }
    if (workspaceSize == 0) return ACL_SPARSE_STATUS_INVALID_VALUE;
    // Grow-only: a smaller user workspace keeps the current one
    // (include/cann_ops_sparse.h:1578-1590).
    if (handle->user_workspace != nullptr && workspaceSize <= handle->user_workspace_size) {
        return ACL_SPARSE_STATUS_SUCCESS;
    }
    handle->user_workspace = workspace;
    handle->user_workspace_size = workspaceSize;
    return ACL_SPARSE_STATUS_SUCCESS;
}

aclsparseStatus_t aclsparseGetWorkspace(aclsparseHandle_t handle, void** workspace, size_t* workspaceSize)
{
    aclsparseStatus_t st = CheckHandle(handle);
    if (st != ACL_SPARSE_STATUS_SUCCESS) return st;
    if (workspace == nullptr || workspaceSize == nullptr) return ACL_SPARSE_STATUS_INVALID_VALUE;
    if (handle->user_workspace != nullptr) {
        *workspace = handle->user_workspace;
        *workspaceSize = handle->user_workspace_size;
        return ACL_SPARSE_STATUS_SUCCESS;
    }
    if (handle->default_workspace == nullptr) {
        // The 4 MiB default workspace is allocated on first use rather than at
        // aclsparseCreate, so a handle can be created and validated without a
        // device.  The SpMV path itself never uses it (caller-owned buffers).
        if (hipMalloc(&handle->default_workspace, aclsp::kDefaultWorkspaceBytes) != hipSuccess) {
            handle->default_workspace = nullptr;
            return ACL_SPARSE_STATUS_ALLOC_FAILED;
        }
        handle->default_workspace_size = aclsp::kDefaultWorkspaceBytes;
    }
    *workspace = handle->default_workspace;
    *workspaceSize = handle->default_workspace_size;
    return ACL_SPARSE_STATUS_SUCCESS;
}

// Build id: SHA-256 (first 32 hex digits) of the native sources, the public
// header and the compiler flags, set by the build script.  The prefix lets the
// id be read from the library file without loading it.
#ifndef ACLSPARSE_HIP_BUILD_ID
#define ACLSPARSE_HIP_BUILD_ID "unknown"
#endif
static const char kBuildIdRecord[] = "aclsparse-hip-build-id:" ACLSPARSE_HIP_BUILD_ID;

const char* aclsparseHipBuildId(void) { return kBuildIdRecord + sizeof("aclsparse-hip-build-id:") - 1; }

aclsparseStatus_t aclsparseGetVersion(aclsparseHandle_t handle, int* version)
{
    (void)handle;  // may be null
    if (version == nullptr) return ACL_SPARSE_STATUS_INVALID_VALUE;
    *version = aclsp::kVersion;
    return ACL_SPARSE_STATUS_SUCCESS;
}

aclsparseStatus_t aclsparseSetPointerMode(aclsparseHandle_t handle, aclsparsePointerMode_t mode)
{
    aclsparseStatus_t st = CheckHandle(handle);
    if (st != ACL_SPARSE_STATUS_SUCCESS) return st;
    if (mode != ACL_SPARSE_POINTER_MODE_HOST && mode != ACL_SPARSE_POINTER_MODE_DEVICE) {
        return ACL_SPARSE_STATUS_INVALID_VALUE;
    }
    handle->pointer_mode = mode;
    return ACL_SPARSE_STATUS_SUCCESS;
}

aclsparseStatus_t aclsparseGetPointerMode(aclsparseHandle_t handle, aclsparsePointerMode_t* mode)
{
    aclsparseStatus_t st = CheckHandle(handle);
    if (st != ACL_SPARSE_STATUS_SUCCESS) return st;
    if (mode == nullptr) return ACL_SPARSE_STATUS_INVALID_VALUE;
    *mode = handle->pointer_mode;
    return ACL_SPARSE_STATUS_SUCCESS;
}

// ------------------------------- dense vector -------------------------------

aclsparseStatus_t aclsparseCreateDnVec(aclsparseDnVecDescr_t* dnVecDescr, int64_t size, void* values,
                                       aclDataType valueType)
{
    if (dnVecDescr == nullptr || size < 0 || !IsValidValueType(valueType)) return ACL_SPARSE_STATUS_INVALID_VALUE;
    auto* d = new (std::nothrow) aclsparseDnVecDescr();
    if (d == nullptr) return ACL_SPARSE_STATUS_ALLOC_FAILED;
    d->nums = static_cast<uint64_t>(size);
    d->values = values;  // null allowed: workspace can be queried before binding
    d->value_type = valueType;
    *dnVecDescr = d;
    return ACL_SPARSE_STATUS_SUCCESS;
}

aclsparseStatus_t aclsparseCreateConstDnVec(aclsparseConstDnVecDescr_t* dnVecDescr, int64_t size,
                                            const void* values, aclDataType valueType)
{
    if (dnVecDescr == nullptr) return ACL_SPARSE_STATUS_INVALID_VALUE;
    aclsparseDnVecDescr_t tmp = nullptr;
    aclsparseStatus_t st = aclsparseCreateDnVec(&tmp, size, const_cast<void*>(values), valueType);
    if (st == ACL_SPARSE_STATUS_SUCCESS) *dnVecDescr = tmp;
    return st;
}

aclsparseStatus_t aclsparseDestroyDnVec(aclsparseConstDnVecDescr_t dnVecDescr)
{
    if (dnVecDescr == nullptr) return ACL_SPARSE_STATUS_SUCCESS;
    if (!IsVec(dnVecDescr)) return ACL_SPARSE_STATUS_INVALID_VALUE;
    auto* d = const_cast<aclsparseDnVecDescr*>(dnVecDescr);
    d->signature = 0;
    delete d;
    return ACL_SPARSE_STATUS_SUCCESS;
}

aclsparseStatus_t aclsparseDnVecGet(aclsparseDnVecDescr_t dnVecDescr, int64_t* size, void** values,
                                    aclDataType* valueType)
{
    if (!IsVec(dnVecDescr) || size == nullptr || values == nullptr || valueType == nullptr) {
        return ACL_SPARSE_STATUS_INVALID_VALUE;
    }
    *size = static_cast<int64_t>(dnVecDescr->nums);
    *values = dnVecDescr->values;
    *valueType = dnVecDescr->value_type;
    return ACL_SPARSE_STATUS_SUCCESS;
}

aclsparseStatus_t aclsparseDnVecGetValues(aclsparseDnVecDescr_t dnVecDescr, void** values)
{
    if (!IsVec(dnVecDescr) || values == nullptr) return ACL_SPARSE_STATUS_INVALID_VALUE;
    *values = dnVecDescr->values;
    return ACL_SPARSE_STATUS_SUCCESS;
}

aclsparseStatus_t aclsparseDnVecSetValues(aclsparseDnVecDescr_t dnVecDescr, void* values)
{
    if (!IsVec(dnVecDescr)) return ACL_SPARSE_STATUS_INVALID_VALUE;
    dnVecDescr->values = values;
    return ACL_SPARSE_STATUS_SUCCESS;
}

aclsparseStatus_t aclsparseDnVecSetStride(aclsparseDnVecDescr_t dnVecDescr, int64_t stride)
{
    if (!IsVec(dnVecDescr) || !IsValidElementStride(dnVecDescr->nums, stride)) {
        return ACL_SPARSE_STATUS_INVALID_VALUE;
    }
    dnVecDescr->stride = stride;
    return ACL_SPARSE_STATUS_SUCCESS;
}

aclsparseStatus_t aclsparseDnVecGetStride(aclsparseConstDnVecDescr_t dnVecDescr, int64_t* stride)
{
    if (!IsVec(dnVecDescr) || stride == nullptr) return ACL_SPARSE_STATUS_INVALID_VALUE;
    *stride = dnVecDescr->stride;
    return ACL_SPARSE_STATUS_SUCCESS;
}

// ------------------------------- CSR matrix ---------------------------------

aclsparseStatus_t aclsparseCreateCsr(aclsparseSpMatDescr_t* spMatDescr, int64_t rows, int64_t cols, int64_t nnz,
                                     void* csrRowOffsets, void* csrColInd, void* csrValues,
                                     aclsparseIndexType_t csrRowOffsetsType, aclsparseIndexType_t csrColIndType,
                                     aclsparseIndexBase_t idxBase, aclDataType valueType)
{
    if (spMatDescr == nullptr || rows < 0 || cols < 0 || nnz < 0) return ACL_SPARSE_STATUS_INVALID_VALUE;
    if (!IsIndexType(csrRowOffsetsType) || !IsIndexType(csrColIndType)) return ACL_SPARSE_STATUS_INVALID_VALUE;
    if (idxBase != ACL_SPARSE_INDEX_BASE_ZERO && idxBase != ACL_SPARSE_INDEX_BASE_ONE) {
        return ACL_SPARSE_STATUS_INVALID_VALUE;
    }
    if (!IsValidValueType(valueType)) return ACL_SPARSE_STATUS_INVALID_VALUE;
    auto* d = new (std::nothrow) aclsparseSpMatDescr();
    if (d == nullptr) return ACL_SPARSE_STATUS_ALLOC_FAILED;
    d->rows = static_cast<uint64_t>(rows);
    d->cols = static_cast<uint64_t>(cols);
    d->nnz = static_cast<uint64_t>(nnz);
    d->ptrs = csrRowOffsets;  // null pointers allowed for delayed binding
    d->idxs = csrColInd;
    d->values = csrValues;
    d->ptr_type = csrRowOffsetsType;
    d->idx_type = csrColIndType;
    d->base = idxBase;
    d->value_type = valueType;
    *spMatDescr = d;
    return ACL_SPARSE_STATUS_SUCCESS;
}

aclsparseStatus_t aclsparseCreateConstCsr(aclsparseConstSpMatDescr_t* spMatDescr, int64_t rows, int64_t cols,
                                          int64_t nnz, const void* csrRowOffsets, const void* csrColInd,
                                          const void* csrValues, aclsparseIndexType_t csrRowOffsetsType,
                                          aclsparseIndexType_t csrColIndType, aclsparseIndexBase_t idxBase,
                                          aclDataType valueType)
{
    if (spMatDescr == nullptr) return ACL_SPARSE_STATUS_INVALID_VALUE;
    aclsparseSpMatDescr_t tmp = nullptr;
    aclsparseStatus_t st = aclsparseCreateCsr(&tmp, rows, cols, nnz, const_cast<void*>(csrRowOffsets),
                                              const_cast<void*>(csrColInd), const_cast<void*>(csrValues),
                                              csrRowOffsetsType, csrColIndType, idxBase, valueType);
    if (st == ACL_SPARSE_STATUS_SUCCESS) *spMatDescr = tmp;
    return st;
}

aclsparseStatus_t aclsparseCsrSetPointers(aclsparseSpMatDescr_t descr, void* rowOffsets, void* colIndices,
                                          void* values)
{
    if (!IsMat(descr) || descr->format != ACL_SPARSE_FORMAT_CSR) return ACL_SPARSE_STATUS_INVALID_VALUE;
    // Row offsets are required whenever the matrix has rows; colInd/values
    // whenever it has non-zeros.
    if ((descr->rows > 0 && rowOffsets == nullptr) ||
        (descr->nnz > 0 && (colIndices == nullptr || values == nullptr))) {
        return ACL_SPARSE_STATUS_INVALID_VALUE;
    }
    if (descr->ptrs != rowOffsets || descr->idxs != colIndices || descr->values != values) ResetPlan(descr);
    descr->ptrs = rowOffsets;
    descr->idxs = colIndices;
    descr->values = values;
    return ACL_SPARSE_STATUS_SUCCESS;
}

aclsparseStatus_t aclsparseCsrSetStrides(aclsparseSpMatDescr_t descr, int64_t rowOffsetsStride,
                                         int64_t colIndStride, int64_t valuesStride)
{
    if (!IsMat(descr) || descr->format != ACL_SPARSE_FORMAT_CSR ||
        !IsValidElementStride(descr->rows + 1U, rowOffsetsStride) ||
        !IsValidElementStride(descr->nnz, colIndStride) || !IsValidElementStride(descr->nnz, valuesStride)) {
        return ACL_SPARSE_STATUS_INVALID_VALUE;
    }
    descr->ptr_stride = rowOffsetsStride;
    descr->idx_stride = colIndStride;
    descr->value_stride = valuesStride;
    ResetPlan(descr);  // sparse/common/aclsparse_descr.cpp:966-971
    return ACL_SPARSE_STATUS_SUCCESS;
}

aclsparseStatus_t aclsparseCsrGetStrides(aclsparseConstSpMatDescr_t descr, int64_t* rowOffsetsStride,
                                         int64_t* colIndStride, int64_t* valuesStride)
{
    if (!IsMat(descr) || descr->format != ACL_SPARSE_FORMAT_CSR || rowOffsetsStride == nullptr ||
        colIndStride == nullptr || valuesStride == nullptr) {
        return ACL_SPARSE_STATUS_INVALID_VALUE;
    }
    *rowOffsetsStride = descr->ptr_stride;
    *colIndStride = descr->idx_stride;
    *valuesStride = descr->value_stride;
    return ACL_SPARSE_STATUS_SUCCESS;
}

aclsparseStatus_t aclsparseDestroySpMat(aclsparseConstSpMatDescr_t spMatDescr)
{
    if (spMatDescr == nullptr) return ACL_SPARSE_STATUS_SUCCESS;
    if (!IsMat(spMatDescr)) return ACL_SPARSE_STATUS_INVALID_VALUE;
    auto* d = const_cast<aclsparseSpMatDescr*>(spMatDescr);
    aclsp::ReleasePathChoice(d->staged_choice);  // back to the pool, without waiting for its copy
    d->signature = 0;
    delete d;
    return ACL_SPARSE_STATUS_SUCCESS;
}

aclsparseStatus_t aclsparseSpMatGetFormat(aclsparseConstSpMatDescr_t spMatDescr, aclsparseFormat_t* format)
{
    if (!IsMat(spMatDescr)) return ACL_SPARSE_STATUS_INVALID_VALUE;
    if (format != nullptr) *format = spMatDescr->format;
    return ACL_SPARSE_STATUS_SUCCESS;
}

aclsparseStatus_t aclsparseSpMatGetIndexBase(aclsparseConstSpMatDescr_t spMatDescr, aclsparseIndexBase_t* idxBase)
{
    if (!IsMat(spMatDescr)) return ACL_SPARSE_STATUS_INVALID_VALUE;
    if (idxBase != nullptr) *idxBase = spMatDescr->base;
    return ACL_SPARSE_STATUS_SUCCESS;
}

aclsparseStatus_t aclsparseSpMatGetValues(aclsparseSpMatDescr_t spMatDescr, void** values)
{
    if (!IsMat(spMatDescr)) return ACL_SPARSE_STATUS_INVALID_VALUE;
    if (values != nullptr) *values = spMatDescr->values;
    return ACL_SPARSE_STATUS_SUCCESS;
}

aclsparseStatus_t aclsparseSpMatSetValues(aclsparseSpMatDescr_t spMatDescr, void* values)
{
    if (!IsMat(spMatDescr)) return ACL_SPARSE_STATUS_INVALID_VALUE;
    if (spMatDescr->values != values) ResetPlan(spMatDescr);  // sparse/common/aclsparse_descr.cpp:1071-1082
    spMatDescr->values = values;
    return ACL_SPARSE_STATUS_SUCCESS;
}

aclsparseStatus_t aclsparseSpMatGetSize(aclsparseConstSpMatDescr_t spMatDescr, int64_t* rows, int64_t* cols,
                                        int64_t* nnz)
{
    if (!IsMat(spMatDescr)) return ACL_SPARSE_STATUS_INVALID_VALUE;
    if (rows != nullptr) *rows = static_cast<int64_t>(spMatDescr->rows);
    if (cols != nullptr) *cols = static_cast<int64_t>(spMatDescr->cols);
    if (nnz != nullptr) *nnz = static_cast<int64_t>(spMatDescr->nnz);
    return ACL_SPARSE_STATUS_SUCCESS;
}

aclsparseStatus_t aclsparseCsrGet(aclsparseSpMatDescr_t spMatDescr, int64_t* rows, int64_t* cols, int64_t* nnz,
                                  void** csrRowOffsets, void** csrColInd, void** csrValues,
                                  aclsparseIndexType_t* csrRowOffsetsType, aclsparseIndexType_t* csrColIndType,
                                  aclsparseIndexBase_t* idxBase, aclDataType* valueType)
{
    if (!IsMat(spMatDescr) || spMatDescr->format != ACL_SPARSE_FORMAT_CSR || rows == nullptr || cols == nullptr ||
        nnz == nullptr || csrRowOffsets == nullptr || csrColInd == nullptr || csrValues == nullptr ||
        csrRowOffsetsType == nullptr || csrColIndType == nullptr || idxBase == nullptr || valueType == nullptr) {
        return ACL_SPARSE_STATUS_INVALID_VALUE;
    }
    *rows = static_cast<int64_t>(spMatDescr->rows);
    *cols = static_cast<int64_t>(spMatDescr->cols);
    *nnz = static_cast<int64_t>(spMatDescr->nnz);
    *csrRowOffsets = spMatDescr->ptrs;
    *csrColInd = spMatDescr->idxs;
    *csrValues = spMatDescr->values;
    *csrRowOffsetsType = spMatDescr->ptr_type;
    *csrColIndType = spMatDescr->idx_type;
    *idxBase = spMatDescr->base;
    *valueType = spMatDescr->value_type;
    return ACL_SPARSE_STATUS_SUCCESS;
}

// ------------------------------- dense matrix -------------------------------
// Validation order and status codes of sparse/common/aclsparse_descr.cpp:1102-1302.

aclsparseStatus_t aclsparseCreateDnMat(aclsparseDnMatDescr_t* dnMatDescr, int64_t rows, int64_t cols, int64_t ld,
                                       void* values, aclDataType valueType, aclsparseOrder_t order)
{
    if (dnMatDescr == nullptr) return ACL_SPARSE_STATUS_INVALID_VALUE;
    if (rows < 0 || cols < 0) return ACL_SPARSE_STATUS_INVALID_VALUE;
    if (rows > INT32_MAX || cols > INT32_MAX) return ACL_SPARSE_STATUS_INVALID_VALUE;
    if (ld < 0) return ACL_SPARSE_STATUS_INVALID_VALUE;
    if (rows != 0 && cols != 0 && values == nullptr) return ACL_SPARSE_STATUS_INVALID_VALUE;
    if (!IsValidValueType(valueType)) return ACL_SPARSE_STATUS_INVALID_VALUE;
    if (order != ACL_SPARSE_ORDER_ROW && order != ACL_SPARSE_ORDER_COL) return ACL_SPARSE_STATUS_INVALID_VALUE;
    if (order == ACL_SPARSE_ORDER_ROW && ld < cols) return ACL_SPARSE_STATUS_INVALID_VALUE;
    if (order == ACL_SPARSE_ORDER_COL && ld < rows) return ACL_SPARSE_STATUS_INVALID_VALUE;
    auto* d = new (std::nothrow) aclsparseDnMatDescr();
    if (d == nullptr) return ACL_SPARSE_STATUS_ALLOC_FAILED;
    d->rows = rows;
    d->cols = cols;
    d->ld = ld;
    d->values = values;
    d->value_type = valueType;
    d->order = order;
    *dnMatDescr = d;
    return ACL_SPARSE_STATUS_SUCCESS;
}

aclsparseStatus_t aclsparseCreateConstDnMat(aclsparseConstDnMatDescr_t* dnMatDescr, int64_t rows, int64_t cols,
                                            int64_t ld, const void* values, aclDataType valueType,
                                            aclsparseOrder_t order)
{
    if (dnMatDescr == nullptr) return ACL_SPARSE_STATUS_INVALID_VALUE;
    aclsparseDnMatDescr_t tmp = nullptr;
    aclsparseStatus_t st = aclsparseCreateDnMat(&tmp, rows, cols, ld, const_cast<void*>(values), valueType, order);
    if (st == ACL_SPARSE_STATUS_SUCCESS) *dnMatDescr = tmp;
    return st;
}

aclsparseStatus_t aclsparseDestroyDnMat(aclsparseConstDnMatDescr_t dnMatDescr)
{
    if (dnMatDescr == nullptr) return ACL_SPARSE_STATUS_SUCCESS;
    if (!IsDnMat(dnMatDescr)) return ACL_SPARSE_STATUS_INVALID_VALUE;
    auto* d = const_cast<aclsparseDnMatDescr*>(dnMatDescr);
    d->signature = 0;
    delete d;
    return ACL_SPARSE_STATUS_SUCCESS;
}

aclsparseStatus_t aclsparseConstDnMatGet(aclsparseConstDnMatDescr_t dnMatDescr, int64_t* rows, int64_t* cols,
                                         int64_t* ld, const void** values, aclDataType* valueType,
                                         aclsparseOrder_t* order)
{
    // every output is optional
    if (!IsDnMat(dnMatDescr)) return ACL_SPARSE_STATUS_INVALID_VALUE;
    if (rows != nullptr) *rows = dnMatDescr->rows;
    if (cols != nullptr) *cols = dnMatDescr->cols;
    if (ld != nullptr) *ld = dnMatDescr->ld;
    if (values != nullptr) *values = dnMatDescr->values;
    if (valueType != nullptr) *valueType = dnMatDescr->value_type;
    if (order != nullptr) *order = dnMatDescr->order;
    return ACL_SPARSE_STATUS_SUCCESS;
}

aclsparseStatus_t aclsparseDnMatGet(aclsparseDnMatDescr_t dnMatDescr, int64_t* rows, int64_t* cols, int64_t* ld,
                                    void** values, aclDataType* valueType, aclsparseOrder_t* order)
{
    return aclsparseConstDnMatGet(dnMatDescr, rows, cols, ld, const_cast<const void**>(values), valueType, order);
}

aclsparseStatus_t aclsparseConstDnMatGetValues(aclsparseConstDnMatDescr_t dnMatDescr, const void** values)
{
    if (!IsDnMat(dnMatDescr)) return ACL_SPARSE_STATUS_INVALID_VALUE;
    if (values != nullptr) *values = dnMatDescr->values;
    return ACL_SPARSE_STATUS_SUCCESS;
}

aclsparseStatus_t aclsparseDnMatGetValues(aclsparseDnMatDescr_t dnMatDescr, void** values)
{
    return aclsparseConstDnMatGetValues(dnMatDescr, const_cast<const void**>(values));
}

aclsparseStatus_t aclsparseDnMatSetValues(aclsparseDnMatDescr_t dnMatDescr, void* values)
{
    if (!IsDnMat(dnMatDescr)) return ACL_SPARSE_STATUS_INVALID_VALUE;
    dnMatDescr->values = values;
    return ACL_SPARSE_STATUS_SUCCESS;
}

}  // extern "C"
