// aclsparseSpMVOp_* entry points: Z = alpha*A*X + beta*Y, fp32, CSR with
// I32/I64 row offsets, deterministic compensated accumulation.
//
// Validation and status semantics restate sparse/spmv_op/arch35/spmv_op_host.cpp:
// common checks (:88-102), matrix checks (:57-86), alg (:104-113),
// bufferSize (:515-560), createDescr (:631-674), destroyDescr (:677-684),
// createPlan (:687-713, an epilogue LTO buffer is NOT_SUPPORTED),
// destroyPlan (:716-723), setGlobalUserData (:726-750), execute (:753-773,
// vector checks :199-250, nnz == 0 -> Z = beta*Y :362-417).
#include <hip/hip_runtime.h>

#include <cstring>
#include <new>

#include "aclsparse_internal.h"

namespace {

bool HandleOk(aclsparseHandle_t h) { return h != nullptr && h->signature == aclsp::kHandleSignature; }

void* StreamOf(aclsparseHandle_t h)
{
    // SpMVOp launches on the handle's stream; an unset stream is the HIP
    // null stream (the reference launches on whatever stream the handle has).
    return (h->stream == nullptr || h->stream == ACL_SPARSE_HIP_NULL_STREAM) ? nullptr : h->stream;
}

aclsparseStatus_t ValidateCommon(aclsparseOperation_t opA, aclDataType computeType)
{
    if (opA != ACL_SPARSE_OP_NON_TRANSPOSE) return ACL_SPARSE_STATUS_NOT_SUPPORTED;
    if (computeType != ACL_FLOAT) return ACL_SPARSE_STATUS_NOT_SUPPORTED;
    return ACL_SPARSE_STATUS_SUCCESS;
}

aclsparseStatus_t ValidateMat(aclsparseConstSpMatDescr_t A)
{
    if (A == nullptr || A->signature != aclsp::kSpMatSignature) return ACL_SPARSE_STATUS_INVALID_VALUE;
    if (A->format != ACL_SPARSE_FORMAT_CSR) return ACL_SPARSE_STATUS_NOT_SUPPORTED;
    if (A->value_type != ACL_FLOAT) return ACL_SPARSE_STATUS_NOT_SUPPORTED;
    if (A->idx_type != ACL_SPARSE_INDEX_32I) return ACL_SPARSE_STATUS_NOT_SUPPORTED;
    if (A->ptr_type != ACL_SPARSE_INDEX_32I && A->ptr_type != ACL_SPARSE_INDEX_64I) {
        return ACL_SPARSE_STATUS_NOT_SUPPORTED;
    }
    return ACL_SPARSE_STATUS_SUCCESS;
}

aclsparseStatus_t ValidateAlg(aclsparseSpMVOpAlg_t alg)
{
    return (alg == ACL_SPARSE_SPMVOP_ALG_DEFAULT || alg == ACL_SPARSE_SPMVOP_ALG1 || alg == ACL_SPARSE_SPMVOP_ALG2)
               ? ACL_SPARSE_STATUS_SUCCESS
               : ACL_SPARSE_STATUS_NOT_SUPPORTED;
}

bool IsVec(aclsparseConstDnVecDescr_t v) { return v != nullptr && v->signature == aclsp::kDnVecSignature; }

}  // namespace

extern "C" {

aclsparseStatus_t aclsparseSpMVOp_bufferSize(aclsparseHandle_t handle, aclsparseOperation_t opA,
                                             aclsparseConstSpMatDescr_t matA, aclsparseConstDnVecDescr_t vecX,
                                             aclsparseConstDnVecDescr_t vecY, aclsparseDnVecDescr_t vecZ,
                                             aclDataType computeType, aclsparseSpMVOpAlg_t alg, size_t* bufferSize)
{
    (void)vecX;
    (void)vecY;
    (void)vecZ;
    if (handle == nullptr) return ACL_SPARSE_STATUS_HANDLE_IS_NULLPTR;
    if (!HandleOk(handle)) return ACL_SPARSE_STATUS_INVALID_VALUE;
    aclsparseStatus_t st = ValidateCommon(opA, computeType);
    if (st != ACL_SPARSE_STATUS_SUCCESS) return st;
    st = ValidateMat(matA);
    if (st != ACL_SPARSE_STATUS_SUCCESS) return st;
    st = ValidateAlg(alg);
    if (st != ACL_SPARSE_STATUS_SUCCESS) return st;
    if (bufferSize == nullptr) return ACL_SPARSE_STATUS_INVALID_VALUE;
    if (matA->rows > 0x7FFFFFFFULL) return ACL_SPARSE_STATUS_NOT_SUPPORTED;
    if (alg == ACL_SPARSE_SPMVOP_ALG2) {
        const int64_t m = static_cast<int64_t>(matA->rows);
        *bufferSize = aclsp::SpmvOpComputeLayout(m, static_cast<int64_t>(matA->cols), static_cast<int64_t>(matA->nnz),
                                                 matA->ptr_type, aclsp::SpmvOpNumBins(m))
                          .total;
    } else {
        *bufferSize = 0;
    }
    return ACL_SPARSE_STATUS_SUCCESS;
}

aclsparseStatus_t aclsparseSpMVOp_createDescr(aclsparseHandle_t handle, aclsparseSpMVOpDescr_t* descr,
                                              aclsparseOperation_t opA, aclsparseConstSpMatDescr_t matA,
                                              aclsparseConstDnVecDescr_t vecX, aclsparseConstDnVecDescr_t vecY,
                                              aclsparseDnVecDescr_t vecZ, aclDataType computeType,
                                              aclsparseSpMVOpAlg_t alg, void* buffer)
{
    (void)vecX;
    (void)vecY;
    (void)vecZ;
    if (handle == nullptr) return ACL_SPARSE_STATUS_HANDLE_IS_NULLPTR;
    if (!HandleOk(handle)) return ACL_SPARSE_STATUS_INVALID_VALUE;
    if (descr == nullptr) return ACL_SPARSE_STATUS_INVALID_VALUE;
    aclsparseStatus_t st = ValidateMat(matA);
    if (st != ACL_SPARSE_STATUS_SUCCESS) return st;
    st = ValidateAlg(alg);
    if (st != ACL_SPARSE_STATUS_SUCCESS) return st;
    if (alg == ACL_SPARSE_SPMVOP_ALG2 && buffer == nullptr) return ACL_SPARSE_STATUS_INVALID_VALUE;
    st = ValidateCommon(opA, computeType);
    if (st != ACL_SPARSE_STATUS_SUCCESS) return st;
    if (matA->rows > 0x7FFFFFFFULL) return ACL_SPARSE_STATUS_NOT_SUPPORTED;
    if (matA->base != ACL_SPARSE_INDEX_BASE_ZERO && matA->base != ACL_SPARSE_INDEX_BASE_ONE) {
        return ACL_SPARSE_STATUS_INVALID_VALUE;
    }
    if (alg == ACL_SPARSE_SPMVOP_ALG2 && reinterpret_cast<uintptr_t>(buffer) % aclsp::kWsAlign != 0U) {
        return ACL_SPARSE_STATUS_INVALID_VALUE;
    }
    auto* d = new (std::nothrow) aclsparseSpMVOpDescr();
    if (d == nullptr) return ACL_SPARSE_STATUS_ALLOC_FAILED;
    d->m = matA->rows;
    d->n = matA->cols;
    d->nnz = matA->nnz;
    d->base = matA->base;
    d->row_type = matA->ptr_type;
    d->row_offsets = matA->ptrs;
    d->col_ind = static_cast<const int32_t*>(matA->idxs);
    d->values = static_cast<const float*>(matA->values);
    d->alg = alg == ACL_SPARSE_SPMVOP_ALG_DEFAULT ? ACL_SPARSE_SPMVOP_ALG1 : alg;
    if (d->alg == ACL_SPARSE_SPMVOP_ALG2) {
        d->buffer = buffer;
        d->num_bins = aclsp::SpmvOpNumBins(static_cast<int64_t>(d->m));
        if (d->m > 0) {
            if (d->row_offsets == nullptr) {
                delete d;
                return ACL_SPARSE_STATUS_INVALID_VALUE;
            }
            (void)hipGetLastError();
            d->narrow = aclsp::SpmvOpNarrowUsable(*d);
            if (aclsp::LaunchSpmvOpPreprocess(*d, StreamOf(handle)) != 0 || hipGetLastError() != hipSuccess) {
                aclsp::ReleasePathChoice(d->choice);
                delete d;
                return ACL_SPARSE_STATUS_EXECUTION_FAILED;
            }
            if (d->narrow) {
                aclsp::PublishPathChoice(d->choice, aclsp::SpmvOpSpmvWorkspace(*d), StreamOf(handle));
            }
        }
    }
    *descr = d;
    return ACL_SPARSE_STATUS_SUCCESS;
}

aclsparseStatus_t aclsparseSpMVOp_destroyDescr(aclsparseSpMVOpDescr_t descr)
{
    if (descr == nullptr) return ACL_SPARSE_STATUS_SUCCESS;
    if (descr->signature != aclsp::kSpMVOpDescrSignature) return ACL_SPARSE_STATUS_INVALID_VALUE;
    descr->signature = 0;
    aclsp::ReleasePathChoice(descr->choice);
    delete descr;
    return ACL_SPARSE_STATUS_SUCCESS;
}

aclsparseStatus_t aclsparseSpMVOp_createPlan(aclsparseHandle_t handle, aclsparseSpMVOpDescr_t descr,
                                             aclsparseSpMVOpPlan_t* plan, const void* epilogueLTOBuffer,
                                             size_t epilogueLTOBufferSize)
{
    if (handle == nullptr) return ACL_SPARSE_STATUS_HANDLE_IS_NULLPTR;
    if (!HandleOk(handle)) return ACL_SPARSE_STATUS_INVALID_VALUE;
    if (descr == nullptr || descr->signature != aclsp::kSpMVOpDescrSignature) return ACL_SPARSE_STATUS_INVALID_VALUE;
    if (plan == nullptr) return ACL_SPARSE_STATUS_INVALID_VALUE;
    // Only the identity epilogue exists: a JIT epilogue module is not supported.
    if (epilogueLTOBuffer != nullptr || epilogueLTOBufferSize > 0) return ACL_SPARSE_STATUS_NOT_SUPPORTED;
    auto* p = new (std::nothrow) aclsparseSpMVOpPlan();
    if (p == nullptr) return ACL_SPARSE_STATUS_ALLOC_FAILED;
    p->descr = descr;
    p->alg = descr->alg;
    *plan = p;
    return ACL_SPARSE_STATUS_SUCCESS;
}

aclsparseStatus_t aclsparseSpMVOp_destroyPlan(aclsparseSpMVOpPlan_t plan)
{
    if (plan == nullptr) return ACL_SPARSE_STATUS_SUCCESS;
    if (plan->signature != aclsp::kSpMVOpPlanSignature) return ACL_SPARSE_STATUS_INVALID_VALUE;
    plan->signature = 0;
    delete plan;
    return ACL_SPARSE_STATUS_SUCCESS;
}

aclsparseStatus_t aclsparseSpMVOp_setGlobalUserData(aclsparseHandle_t handle, aclsparseSpMVOpPlan_t plan,
                                                    const char* epilogueDataName, void* epilogueData,
                                                    size_t epilogueDataSize)
{
    (void)epilogueDataName;
    if (handle == nullptr) return ACL_SPARSE_STATUS_HANDLE_IS_NULLPTR;
    if (plan == nullptr) return ACL_SPARSE_STATUS_INVALID_VALUE;
    if ((epilogueData == nullptr) != (epilogueDataSize == 0)) return ACL_SPARSE_STATUS_INVALID_VALUE;
    return ACL_SPARSE_STATUS_SUCCESS;  // identity epilogue: nothing to bind
}

aclsparseStatus_t aclsparseSpMVOp(aclsparseHandle_t handle, aclsparseSpMVOpPlan_t plan, const void* alpha,
                                  const void* beta, aclsparseConstDnVecDescr_t vecX, aclsparseConstDnVecDescr_t vecY,
                                  aclsparseDnVecDescr_t vecZ)
{
    if (handle == nullptr) return ACL_SPARSE_STATUS_HANDLE_IS_NULLPTR;
    if (!HandleOk(handle)) return ACL_SPARSE_STATUS_INVALID_VALUE;
    if (plan == nullptr || plan->signature != aclsp::kSpMVOpPlanSignature) return ACL_SPARSE_STATUS_INVALID_VALUE;
    const aclsparseSpMVOpDescr* d = plan->descr;
    if (d == nullptr || d->signature != aclsp::kSpMVOpDescrSignature) return ACL_SPARSE_STATUS_INVALID_VALUE;
    if (alpha == nullptr || beta == nullptr) return ACL_SPARSE_STATUS_INVALID_VALUE;
    if (!IsVec(vecX) || !IsVec(vecY) || !IsVec(vecZ)) return ACL_SPARSE_STATUS_INVALID_VALUE;
    if (vecX->value_type != ACL_FLOAT || vecY->value_type != ACL_FLOAT || vecZ->value_type != ACL_FLOAT) {
        return ACL_SPARSE_STATUS_NOT_SUPPORTED;
    }
    const bool deviceScalars = handle->pointer_mode == ACL_SPARSE_POINTER_MODE_DEVICE;
    float a = 0.0f, b = 0.0f;
    if (!deviceScalars) {
        std::memcpy(&a, alpha, sizeof(float));
        std::memcpy(&b, beta, sizeof(float));
    }
    const uint64_t m = d->m, n = d->n;
    if (n > 0 && vecX->values == nullptr) return ACL_SPARSE_STATUS_INVALID_VALUE;
    // Y may stay unbound when beta is a host zero (or lives in device memory).
    const bool skipY = deviceScalars || b == 0.0f;
    if (!skipY && m > 0 && vecY->values == nullptr) return ACL_SPARSE_STATUS_INVALID_VALUE;
    if (m > 0 && vecZ->values == nullptr) return ACL_SPARSE_STATUS_INVALID_VALUE;
    if (vecX->nums != n || vecY->nums != m || vecZ->nums != m) return ACL_SPARSE_STATUS_INVALID_VALUE;
    if (m > 0x7FFFFFFFULL) return ACL_SPARSE_STATUS_NOT_SUPPORTED;
    if (m == 0) return ACL_SPARSE_STATUS_SUCCESS;
    if (d->nnz > 0 && (d->row_offsets == nullptr || d->col_ind == nullptr || d->values == nullptr)) {
        return ACL_SPARSE_STATUS_INVALID_VALUE;
    }
    if (d->alg == ACL_SPARSE_SPMVOP_ALG2 && d->num_bins == 0) return ACL_SPARSE_STATUS_INVALID_VALUE;
    (void)hipGetLastError();
    if (aclsp::LaunchSpmvOpExecute(*d, vecX->values, vecY->values, vecZ->values, a, b, alpha, beta, deviceScalars,
                                   StreamOf(handle)) != 0 ||
        hipGetLastError() != hipSuccess) {
        return ACL_SPARSE_STATUS_EXECUTION_FAILED;
    }
    return ACL_SPARSE_STATUS_SUCCESS;
}

}  // extern "C"
