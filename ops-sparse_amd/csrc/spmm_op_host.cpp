// aclsparseSpMMOp_* entry points: C = alpha*A*op(B) + beta*C, A CSR (fp32 or
// fp16 values, I32/I64 row offsets), B and C dense (row or column order),
// fp32 accumulation, deterministic.
//
// Validation order and status codes restate
// sparse/spmm_op/arch35/spmm_op_host.cpp: matrix enums and pointers
// (:69-147), opA/opB/computeType (:150-170), alg (:173-183), bufferSize
// (:189-233, :695-740), createDescr (:239-258, :961-1002; ALG2 builds the
// length-sorted tables once, here on the device), createPlan (:264-283,
// :1015-1043), setGlobalUserData (:1056-1080) and execute (:289-480,
// :659-690: m == 0 or n == 0 launch nothing, nnz == 0 -> C = beta*C).
#include <hip/hip_runtime.h>

#include <cstdint>
#include <cstring>
#include <new>

#include "aclsparse_internal.h"

namespace {

bool HandleOk(aclsparseHandle_t h) { return h != nullptr && h->signature == aclsp::kHandleSignature; }

void* StreamOf(aclsparseHandle_t h)
{
    return (h->stream == nullptr || h->stream == ACL_SPARSE_HIP_NULL_STREAM) ? nullptr : h->stream;
}

bool IsDnMat(aclsparseConstDnMatDescr_t d) { return d != nullptr && d->signature == aclsp::kDnMatSignature; }

aclsparseStatus_t ValidateMat(aclsparseConstSpMatDescr_t A)
{
    if (A == nullptr || A->signature != aclsp::kSpMatSignature) return ACL_SPARSE_STATUS_INVALID_VALUE;
    if (A->format != ACL_SPARSE_FORMAT_CSR) return ACL_SPARSE_STATUS_NOT_SUPPORTED;
    if (A->value_type != ACL_FLOAT && A->value_type != ACL_FLOAT16) return ACL_SPARSE_STATUS_NOT_SUPPORTED;
    if (A->idx_type != ACL_SPARSE_INDEX_32I) return ACL_SPARSE_STATUS_NOT_SUPPORTED;
    if (A->ptr_type != ACL_SPARSE_INDEX_32I && A->ptr_type != ACL_SPARSE_INDEX_64I) {
        return ACL_SPARSE_STATUS_NOT_SUPPORTED;
    }
    if (A->base != ACL_SPARSE_INDEX_BASE_ZERO && A->base != ACL_SPARSE_INDEX_BASE_ONE) {
        return ACL_SPARSE_STATUS_NOT_SUPPORTED;
    }
    // row offsets are always needed; indices and values once there are entries
    if (A->ptrs == nullptr) return ACL_SPARSE_STATUS_INVALID_VALUE;
    if (A->nnz > 0 && (A->idxs == nullptr || A->values == nullptr)) return ACL_SPARSE_STATUS_INVALID_VALUE;
    if (A->nnz > static_cast<uint64_t>(INT32_MAX)) return ACL_SPARSE_STATUS_NOT_SUPPORTED;
    return ACL_SPARSE_STATUS_SUCCESS;
}

aclsparseStatus_t ValidateCommon(aclsparseOperation_t opA, aclsparseOperation_t opB, aclDataType computeType)
{
    if (opA != ACL_SPARSE_OP_NON_TRANSPOSE) return ACL_SPARSE_STATUS_NOT_SUPPORTED;
    if (opB != ACL_SPARSE_OP_NON_TRANSPOSE && opB != ACL_SPARSE_OP_TRANSPOSE) return ACL_SPARSE_STATUS_NOT_SUPPORTED;
    if (computeType != ACL_FLOAT) return ACL_SPARSE_STATUS_NOT_SUPPORTED;
    return ACL_SPARSE_STATUS_SUCCESS;
}

aclsparseStatus_t ValidateAlg(aclsparseSpMMOpAlg_t alg)
{
    return (alg == ACL_SPARSE_SPMMOP_ALG_DEFAULT || alg == ACL_SPARSE_SPMMOP_ALG1 || alg == ACL_SPARSE_SPMMOP_ALG2 ||
            alg == ACL_SPARSE_SPMMOP_ALG1_HIGH_PRECISION)
               ? ACL_SPARSE_STATUS_SUCCESS
               : ACL_SPARSE_STATUS_NOT_SUPPORTED;
}

// Execute-time checks of B and C against the descriptor (dtype, shapes,
// order, leading dimensions, strides the kernels address, storage).
aclsparseStatus_t ValidateDnMats(const aclsparseSpMMOpDescr* d, aclsparseConstDnMatDescr_t B,
                                 aclsparseConstDnMatDescr_t C)
{
    if (!IsDnMat(B) || !IsDnMat(C)) return ACL_SPARSE_STATUS_INVALID_VALUE;
    if (B->value_type != d->value_type || C->value_type != d->value_type) return ACL_SPARSE_STATUS_NOT_SUPPORTED;
    const int64_t m = static_cast<int64_t>(d->m), k = static_cast<int64_t>(d->k), n = C->cols;
    if (C->rows != m) return ACL_SPARSE_STATUS_INVALID_VALUE;
    if (n < 0) return ACL_SPARSE_STATUS_INVALID_VALUE;
    if (n > INT32_MAX) return ACL_SPARSE_STATUS_NOT_SUPPORTED;
    if (d->op_b == ACL_SPARSE_OP_NON_TRANSPOSE) {
        if (B->rows != k || B->cols != n) return ACL_SPARSE_STATUS_INVALID_VALUE;
    } else {
        if (B->cols != k || B->rows != n) return ACL_SPARSE_STATUS_INVALID_VALUE;
    }
    if (B->order != ACL_SPARSE_ORDER_ROW && B->order != ACL_SPARSE_ORDER_COL) return ACL_SPARSE_STATUS_INVALID_VALUE;
    if (C->order != ACL_SPARSE_ORDER_ROW && C->order != ACL_SPARSE_ORDER_COL) return ACL_SPARSE_STATUS_INVALID_VALUE;
    const int64_t bMin = B->order == ACL_SPARSE_ORDER_ROW ? B->cols : B->rows;
    const int64_t cMin = C->order == ACL_SPARSE_ORDER_ROW ? C->cols : C->rows;
    if (B->ld < bMin || C->ld < cMin) return ACL_SPARSE_STATUS_INVALID_VALUE;
    if (B->ld > INT32_MAX || C->ld > INT32_MAX) return ACL_SPARSE_STATUS_NOT_SUPPORTED;
    const int64_t strideLimit = static_cast<int64_t>(UINT32_MAX) / (B->value_type == ACL_FLOAT ? 4 : 2);
    if (B->ld > strideLimit || C->ld > strideLimit) return ACL_SPARSE_STATUS_NOT_SUPPORTED;
    if (B->values == nullptr || C->values == nullptr) return ACL_SPARSE_STATUS_INVALID_VALUE;
    return ACL_SPARSE_STATUS_SUCCESS;
}

aclsp::SpmmOpLayout LayoutOf(int64_t m, uint32_t bins) { return aclsp::SpmmOpComputeLayout(m, bins); }

}  // namespace

extern "C" {

aclsparseStatus_t aclsparseSpMMOp_bufferSize(aclsparseHandle_t handle, aclsparseOperation_t opA,
                                             aclsparseOperation_t opB, aclsparseConstSpMatDescr_t matA,
                                             aclsparseConstDnMatDescr_t matB, aclsparseDnMatDescr_t matC,
                                             aclDataType computeType, aclsparseSpMMOpAlg_t alg, size_t* bufferSize)
{
    if (handle == nullptr) return ACL_SPARSE_STATUS_HANDLE_IS_NULLPTR;
    if (!HandleOk(handle)) return ACL_SPARSE_STATUS_INVALID_VALUE;
    aclsparseStatus_t st = ValidateCommon(opA, opB, computeType);
    if (st != ACL_SPARSE_STATUS_SUCCESS) return st;
    st = ValidateMat(matA);
    if (st != ACL_SPARSE_STATUS_SUCCESS) return st;
    st = ValidateAlg(alg);
    if (st != ACL_SPARSE_STATUS_SUCCESS) return st;
    if (matB == nullptr || matC == nullptr || bufferSize == nullptr) return ACL_SPARSE_STATUS_INVALID_VALUE;
    if (!IsDnMat(matB) || !IsDnMat(matC)) return ACL_SPARSE_STATUS_INVALID_VALUE;
    if (matA->cols > static_cast<uint64_t>(INT32_MAX)) return ACL_SPARSE_STATUS_NOT_SUPPORTED;
    if (matB->ld > INT32_MAX || matC->ld > INT32_MAX) return ACL_SPARSE_STATUS_NOT_SUPPORTED;
    if (matA->rows > static_cast<uint64_t>(INT32_MAX)) return ACL_SPARSE_STATUS_NOT_SUPPORTED;
    if (alg == ACL_SPARSE_SPMMOP_ALG2) {
        const int64_t m = static_cast<int64_t>(matA->rows);
        *bufferSize = LayoutOf(m, aclsp::SpmvOpNumBins(m)).total;
    } else {
        *bufferSize = 0;
    }
    return ACL_SPARSE_STATUS_SUCCESS;
}

aclsparseStatus_t aclsparseSpMMOp_createDescr(aclsparseHandle_t handle, aclsparseSpMMOpDescr_t* descr,
                                              aclsparseOperation_t opA, aclsparseOperation_t opB,
                                              aclsparseConstSpMatDescr_t matA, aclsparseConstDnMatDescr_t matB,
                                              aclsparseDnMatDescr_t matC, aclDataType computeType,
                                              aclsparseSpMMOpAlg_t alg, void* buffer)
{
    (void)matB;
    (void)matC;
    if (handle == nullptr) return ACL_SPARSE_STATUS_HANDLE_IS_NULLPTR;
    if (!HandleOk(handle)) return ACL_SPARSE_STATUS_INVALID_VALUE;
    if (descr == nullptr) return ACL_SPARSE_STATUS_INVALID_VALUE;
    aclsparseStatus_t st = ValidateMat(matA);
    if (st != ACL_SPARSE_STATUS_SUCCESS) return st;
    st = ValidateAlg(alg);
    if (st != ACL_SPARSE_STATUS_SUCCESS) return st;
    if (alg == ACL_SPARSE_SPMMOP_ALG2 && buffer == nullptr) return ACL_SPARSE_STATUS_INVALID_VALUE;
    st = ValidateCommon(opA, opB, computeType);
    if (st != ACL_SPARSE_STATUS_SUCCESS) return st;
    if (matA->rows > static_cast<uint64_t>(INT32_MAX)) return ACL_SPARSE_STATUS_NOT_SUPPORTED;
    auto* d = new (std::nothrow) aclsparseSpMMOpDescr();
    if (d == nullptr) return ACL_SPARSE_STATUS_ALLOC_FAILED;
    d->m = matA->rows;
    d->k = matA->cols;
    d->nnz = matA->nnz;
    d->base = matA->base;
    d->row_type = matA->ptr_type;
    d->value_type = matA->value_type;
    d->op_b = opB;
    d->row_offsets = matA->ptrs;
    d->col_ind = static_cast<const int32_t*>(matA->idxs);
    d->values = matA->values;
    d->alg = alg == ACL_SPARSE_SPMMOP_ALG_DEFAULT ? ACL_SPARSE_SPMMOP_ALG1 : alg;
    if (d->alg == ACL_SPARSE_SPMMOP_ALG2) {
        const int64_t m = static_cast<int64_t>(d->m);
        d->buffer = buffer;
        d->num_bins = aclsp::SpmvOpNumBins(m);
        if (m > 0) {
            const aclsp::SpmmOpLayout l = LayoutOf(m, d->num_bins);
            uint8_t* ws = static_cast<uint8_t*>(buffer);
            aclsp::LengthTables t{};
            t.row_offsets = d->row_offsets;
            t.rowptr64 = d->row_type == ACL_SPARSE_INDEX_64I;
            t.m = m;
            t.bins = d->num_bins;
            t.reorder = reinterpret_cast<int32_t*>(ws + l.reorder);
            t.tmp_reorder = reinterpret_cast<int32_t*>(ws + l.tmp_reorder);
            t.scratch = reinterpret_cast<int32_t*>(ws + l.scratch);
            t.tmp_scratch = reinterpret_cast<int32_t*>(ws + l.tmp_scratch);
            t.bin_edge = reinterpret_cast<int32_t*>(ws + l.bin_edge);
            t.running = reinterpret_cast<int64_t*>(ws + l.running);
            t.temp = ws + l.temp;
            t.temp_bytes = l.temp_bytes;
            (void)hipGetLastError();
            if (aclsp::LaunchLengthTables(t, StreamOf(handle)) != 0 || hipGetLastError() != hipSuccess) {
                delete d;
                return ACL_SPARSE_STATUS_EXECUTION_FAILED;
            }
        }
    }
    *descr = d;
    return ACL_SPARSE_STATUS_SUCCESS;
}

aclsparseStatus_t aclsparseSpMMOp_destroyDescr(aclsparseSpMMOpDescr_t descr)
{
    if (descr == nullptr) return ACL_SPARSE_STATUS_SUCCESS;
    if (descr->signature != aclsp::kSpMMOpDescrSignature) return ACL_SPARSE_STATUS_INVALID_VALUE;
    descr->signature = 0;
    delete descr;
    return ACL_SPARSE_STATUS_SUCCESS;
}

aclsparseStatus_t aclsparseSpMMOp_createPlan(aclsparseHandle_t handle, aclsparseSpMMOpDescr_t descr,
                                             aclsparseSpMMOpPlan_t* plan, const void* epilogueLTOBuffer,
                                             size_t epilogueLTOBufferSize)
{
    if (handle == nullptr) return ACL_SPARSE_STATUS_HANDLE_IS_NULLPTR;
    if (!HandleOk(handle)) return ACL_SPARSE_STATUS_INVALID_VALUE;
    if (descr == nullptr || descr->signature != aclsp::kSpMMOpDescrSignature) return ACL_SPARSE_STATUS_INVALID_VALUE;
    if (plan == nullptr) return ACL_SPARSE_STATUS_INVALID_VALUE;
    // Only the identity epilogue exists: a JIT epilogue module is not supported.
    if (epilogueLTOBuffer != nullptr || epilogueLTOBufferSize > 0) return ACL_SPARSE_STATUS_NOT_SUPPORTED;
    auto* p = new (std::nothrow) aclsparseSpMMOpPlan();
    if (p == nullptr) return ACL_SPARSE_STATUS_ALLOC_FAILED;
    p->descr = descr;
    p->alg = descr->alg;
    *plan = p;
    return ACL_SPARSE_STATUS_SUCCESS;
}

aclsparseStatus_t aclsparseSpMMOp_destroyPlan(aclsparseSpMMOpPlan_t plan)
{
    if (plan == nullptr) return ACL_SPARSE_STATUS_SUCCESS;
    if (plan->signature != aclsp::kSpMMOpPlanSignature) return ACL_SPARSE_STATUS_INVALID_VALUE;
    plan->signature = 0;
    delete plan;
    return ACL_SPARSE_STATUS_SUCCESS;
}

aclsparseStatus_t aclsparseSpMMOp_setGlobalUserData(aclsparseHandle_t handle, aclsparseSpMMOpPlan_t plan,
                                                    const char* epilogueDataName, void* epilogueData,
                                                    size_t epilogueDataSize)
{
    (void)epilogueDataName;
    if (handle == nullptr) return ACL_SPARSE_STATUS_HANDLE_IS_NULLPTR;
    if (plan == nullptr) return ACL_SPARSE_STATUS_INVALID_VALUE;
    if ((epilogueData == nullptr) != (epilogueDataSize == 0)) return ACL_SPARSE_STATUS_INVALID_VALUE;
    return ACL_SPARSE_STATUS_SUCCESS;  // identity epilogue: nothing to bind
}

aclsparseStatus_t aclsparseSpMMOp(aclsparseHandle_t handle, aclsparseSpMMOpPlan_t plan, const void* alpha,
                                  const void* beta, aclsparseConstDnMatDescr_t matB, aclsparseDnMatDescr_t matC)
{
    if (handle == nullptr) return ACL_SPARSE_STATUS_HANDLE_IS_NULLPTR;
    if (!HandleOk(handle)) return ACL_SPARSE_STATUS_INVALID_VALUE;
    if (plan == nullptr || plan->signature != aclsp::kSpMMOpPlanSignature) return ACL_SPARSE_STATUS_INVALID_VALUE;
    const aclsparseSpMMOpDescr* d = plan->descr;
    if (d == nullptr || d->signature != aclsp::kSpMMOpDescrSignature) return ACL_SPARSE_STATUS_INVALID_VALUE;
    if (alpha == nullptr || beta == nullptr) return ACL_SPARSE_STATUS_INVALID_VALUE;
    aclsparseStatus_t st = ValidateDnMats(d, matB, matC);
    if (st != ACL_SPARSE_STATUS_SUCCESS) return st;
    if (d->m > static_cast<uint64_t>(INT32_MAX)) return ACL_SPARSE_STATUS_NOT_SUPPORTED;
    if (d->m == 0 || matC->cols == 0) return ACL_SPARSE_STATUS_SUCCESS;
    if (d->alg == ACL_SPARSE_SPMMOP_ALG2 && d->num_bins == 0) return ACL_SPARSE_STATUS_INVALID_VALUE;
    const bool deviceScalars = handle->pointer_mode == ACL_SPARSE_POINTER_MODE_DEVICE;
    aclsp::SpmmLaunch l{};
    l.row_offsets = d->row_offsets;
    l.col_ind = d->col_ind;
    l.values = d->values;
    l.b = matB->values;
    l.c = matC->values;
    l.m = static_cast<int64_t>(d->m);
    l.k = static_cast<int64_t>(d->k);
    l.n = matC->cols;
    l.ldb = matB->ld;
    l.ldc = matC->ld;
    l.nnz = static_cast<int64_t>(d->nnz);
    l.base = d->base == ACL_SPARSE_INDEX_BASE_ONE ? 1 : 0;
    l.rowptr64 = d->row_type == ACL_SPARSE_INDEX_64I ? 1 : 0;
    l.fp16 = d->value_type == ACL_FLOAT16 ? 1 : 0;
    l.high_precision = d->alg == ACL_SPARSE_SPMMOP_ALG1_HIGH_PRECISION && d->value_type == ACL_FLOAT ? 1 : 0;
    l.b_trans = d->op_b == ACL_SPARSE_OP_TRANSPOSE ? 1 : 0;
    l.b_row_major = matB->order == ACL_SPARSE_ORDER_ROW ? 1 : 0;
    l.c_row_major = matC->order == ACL_SPARSE_ORDER_ROW ? 1 : 0;
    if (deviceScalars) {
        l.alpha_ptr = static_cast<const float*>(alpha);
        l.beta_ptr = static_cast<const float*>(beta);
    } else {
        std::memcpy(&l.alpha, alpha, sizeof(float));
        std::memcpy(&l.beta, beta, sizeof(float));
    }
    (void)hipGetLastError();
    if (aclsp::LaunchSpmmOp(l, StreamOf(handle)) != 0 || hipGetLastError() != hipSuccess) {
        return ACL_SPARSE_STATUS_EXECUTION_FAILED;
    }
    return ACL_SPARSE_STATUS_SUCCESS;
}

}  // extern "C"
