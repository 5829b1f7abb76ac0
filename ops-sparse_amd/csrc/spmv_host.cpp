// aclsparseSpMVGetBufferSize / aclsparseSpMVPreprocess / aclsparseSpMV.
//
// Validation order and status codes restate sparse/spmv/arch35/spmv_host.cpp:
//   handle (:109-126) -> descriptors (:175-183) -> op (:187-190) ->
//   compute type / alg (:191-196) -> pointer mode + scalar alignment (:142-163)
//   -> format (:220-233) -> shape (:235-261) -> dtype combo (:44-66, :274-281)
//   -> strides (:282-292) -> vector sizes (:315-329); execution adds storage
//   binding + aliasing (:331-355) and the workspace check (:357-368).
// Deviation: CSR row offsets may be ACL_SPARSE_INDEX_64I (the reference
// rejects them in SpMV); column indices stay 32-bit.
#include <hip/hip_runtime.h>

#include <cstring>
#include <limits>
#include <mutex>
#include <vector>

#include "aclsparse_internal.h"

namespace {

using aclsp::SpmvLayout;

bool IsTranspose(aclsparseOperation_t op)
{
    return op == ACL_SPARSE_OP_TRANSPOSE || op == ACL_SPARSE_OP_CONJUGATE_TRANSPOSE;
}

bool IsScalarType(aclDataType t) { return t == ACL_INT32 || t == ACL_FLOAT || t == ACL_COMPLEX64; }

bool IsSupportedAlg(aclsparseSpMVAlg_t alg)
{
    return alg == ACL_SPARSE_SPMV_ALG_DEFAULT || alg == ACL_SPARSE_SPMV_CSR_ALG1 || alg == ACL_SPARSE_SPMV_CSR_ALG2;
}

// Supported (A, x, y, compute) combinations (sparse/spmv/arch35/spmv_host.cpp:44-66).
bool IsSupportedCombo(aclDataType v, aclDataType x, aclDataType y, aclDataType c)
{
    if (v != x) return false;
    if (c == ACL_INT32) return v == ACL_INT8 && y == ACL_INT32;
    if (c == ACL_COMPLEX64) return (v == ACL_COMPLEX64 || v == ACL_FLOAT) && y == ACL_COMPLEX64;
    if (c != ACL_FLOAT) return false;
    return (v == ACL_INT8 && y == ACL_FLOAT) || (v == ACL_FLOAT16 && (y == ACL_FLOAT16 || y == ACL_FLOAT)) ||
           (v == ACL_BF16 && (y == ACL_BF16 || y == ACL_FLOAT)) || (v == ACL_FLOAT && y == ACL_FLOAT);
}

size_t ElementBytes(aclDataType t)
{
    return t == ACL_INT8 ? 1U : (t == ACL_FLOAT16 || t == ACL_BF16) ? 2U : t == ACL_COMPLEX64 ? 8U : 4U;
}

size_t ScalarAlignment(aclDataType c)
{
    return c == ACL_INT32 ? alignof(int32_t) : c == ACL_COMPLEX64 ? alignof(aclsparseComplex)
                                              : c == ACL_FLOAT ? alignof(float) : 0U;
}

bool StrideFits(uint64_t length, int64_t stride, size_t elementBytes)
{
    if (stride <= 0 || elementBytes == 0U) return false;
    const uint64_t maxOffset = static_cast<uint64_t>(std::numeric_limits<int64_t>::max()) / elementBytes;
    return length <= 1U || static_cast<uint64_t>(stride) <= maxOffset / (length - 1U);
}

aclsparseStatus_t ValidateHandle(aclsparseHandle_t h)
{
    if (h == nullptr) return ACL_SPARSE_STATUS_HANDLE_IS_NULLPTR;
    if (h->signature != aclsp::kHandleSignature) return ACL_SPARSE_STATUS_INVALID_VALUE;
    if (h->stream == nullptr) return ACL_SPARSE_STATUS_INVALID_VALUE;  // stream must be set
    return ACL_SPARSE_STATUS_SUCCESS;
}

aclsparseStatus_t ValidateSetup(aclsparseHandle_t h, aclsparseOperation_t op, const void* alpha,
                                aclsparseConstSpMatDescr_t A, aclsparseConstDnVecDescr_t x, const void* beta,
                                aclsparseConstDnVecDescr_t y, aclDataType c, aclsparseSpMVAlg_t alg)
{
    aclsparseStatus_t st = ValidateHandle(h);
    if (st != ACL_SPARSE_STATUS_SUCCESS) return st;
    if (A == nullptr || x == nullptr || y == nullptr) return ACL_SPARSE_STATUS_INVALID_VALUE;
    if (A->signature != aclsp::kSpMatSignature || x->signature != aclsp::kDnVecSignature ||
        y->signature != aclsp::kDnVecSignature) {
        return ACL_SPARSE_STATUS_INVALID_VALUE;
    }
    if (op != ACL_SPARSE_OP_NON_TRANSPOSE && !IsTranspose(op)) return ACL_SPARSE_STATUS_NOT_SUPPORTED;
    if (!IsScalarType(c) || !IsSupportedAlg(alg)) return ACL_SPARSE_STATUS_NOT_SUPPORTED;
    if (h->pointer_mode != ACL_SPARSE_POINTER_MODE_HOST && h->pointer_mode != ACL_SPARSE_POINTER_MODE_DEVICE) {
        return ACL_SPARSE_STATUS_INVALID_VALUE;
    }
    if (alpha == nullptr || beta == nullptr) return ACL_SPARSE_STATUS_INVALID_VALUE;
    const size_t a = ScalarAlignment(c);
    if (a == 0U || reinterpret_cast<uintptr_t>(alpha) % a != 0U || reinterpret_cast<uintptr_t>(beta) % a != 0U) {
        return ACL_SPARSE_STATUS_INVALID_VALUE;
    }
    return ACL_SPARSE_STATUS_SUCCESS;
}

aclsparseStatus_t ValidateMetadata(const aclsparseSpMatDescr* m, const aclsparseDnVecDescr* x,
                                   const aclsparseDnVecDescr* y, aclDataType c)
{
    if (m->format != ACL_SPARSE_FORMAT_CSR ||
        (m->ptr_type != ACL_SPARSE_INDEX_32I && m->ptr_type != ACL_SPARSE_INDEX_64I) ||
        m->idx_type != ACL_SPARSE_INDEX_32I ||
        (m->base != ACL_SPARSE_INDEX_BASE_ZERO && m->base != ACL_SPARSE_INDEX_BASE_ONE)) {
        return ACL_SPARSE_STATUS_NOT_SUPPORTED;
    }
    if (m->nnz > 0U && (m->rows == 0U || m->cols == 0U)) return ACL_SPARSE_STATUS_INVALID_VALUE;
    const uint64_t maxI32 = static_cast<uint64_t>(std::numeric_limits<int32_t>::max());
    const uint64_t baseOffset = m->base == ACL_SPARSE_INDEX_BASE_ONE ? 1U : 0U;
    // I32 row offsets must hold nnz+base; I64 row offsets are limited by the
    // 2^40 element bound of this build (block-relative offsets are 32-bit and
    // every row must stay below 2^31 entries).
    const uint64_t maxNnz = m->ptr_type == ACL_SPARSE_INDEX_32I ? maxI32 - baseOffset : (uint64_t{1} << 40);
    if (m->rows > maxI32 || m->cols > maxI32 || m->nnz > maxNnz) return ACL_SPARSE_STATUS_NOT_SUPPORTED;
    if (m->rows != 0U && m->cols > UINT64_MAX / m->rows) return ACL_SPARSE_STATUS_INVALID_VALUE;
    if (!IsSupportedCombo(m->value_type, x->value_type, y->value_type, c)) return ACL_SPARSE_STATUS_NOT_SUPPORTED;
    const size_t ptrBytes = m->ptr_type == ACL_SPARSE_INDEX_64I ? 8U : 4U;
    if (!StrideFits(m->rows + 1U, m->ptr_stride, ptrBytes) || !StrideFits(m->nnz, m->idx_stride, 4U) ||
        !StrideFits(m->nnz, m->value_stride, ElementBytes(m->value_type)) ||
        !StrideFits(x->nums, x->stride, ElementBytes(x->value_type)) ||
        !StrideFits(y->nums, y->stride, ElementBytes(y->value_type))) {
        return ACL_SPARSE_STATUS_INVALID_VALUE;
    }
    return ACL_SPARSE_STATUS_SUCCESS;
}

aclsparseStatus_t ValidateVectorSizes(aclsparseOperation_t op, const aclsparseSpMatDescr* m,
                                      const aclsparseDnVecDescr* x, const aclsparseDnVecDescr* y)
{
    const uint64_t xr = IsTranspose(op) ? m->rows : m->cols;
    const uint64_t yr = IsTranspose(op) ? m->cols : m->rows;
    return (x->nums != xr || y->nums != yr) ? ACL_SPARSE_STATUS_INVALID_VALUE : ACL_SPARSE_STATUS_SUCCESS;
}

aclsparseStatus_t ValidateInputs(aclsparseHandle_t h, aclsparseOperation_t op, const void* alpha,
                                 aclsparseConstSpMatDescr_t A, aclsparseConstDnVecDescr_t x, const void* beta,
                                 aclsparseConstDnVecDescr_t y, aclDataType c, aclsparseSpMVAlg_t alg)
{
    aclsparseStatus_t st = ValidateSetup(h, op, alpha, A, x, beta, y, c, alg);
    if (st != ACL_SPARSE_STATUS_SUCCESS) return st;
    st = ValidateMetadata(A, x, y, c);
    if (st != ACL_SPARSE_STATUS_SUCCESS) return st;
    // The transpose sums every column in CSR order through a CSC pattern
    // whose sort is limited to INT32_MAX entries (the reference's own nnz
    // limit, sparse/spmv/README.md "nnz 不超过 INT32_MAX"); larger transposes
    // (possible only with this build's 64-bit row offsets) are not supported.
    if (IsTranspose(op) && A->nnz > static_cast<uint64_t>(std::numeric_limits<int32_t>::max())) {
        return ACL_SPARSE_STATUS_NOT_SUPPORTED;
    }
    return ValidateVectorSizes(op, A, x, y);
}

bool HasAliases(const aclsparseSpMatDescr* m, const aclsparseDnVecDescr* x, const aclsparseDnVecDescr* y)
{
    if (m->ptrs != nullptr &&
        (m->ptrs == m->idxs || m->ptrs == m->values || m->ptrs == x->values || m->ptrs == y->values)) {
        return true;
    }
    if (m->idxs != nullptr && (m->idxs == m->values || m->idxs == x->values || m->idxs == y->values)) return true;
    return (m->values != nullptr && (m->values == x->values || m->values == y->values)) ||
           (x->values != nullptr && x->values == y->values);
}

aclsparseStatus_t ValidateStorage(aclsparseOperation_t op, const aclsparseSpMatDescr* m,
                                  const aclsparseDnVecDescr* x, const aclsparseDnVecDescr* y)
{
    const uint64_t xr = IsTranspose(op) ? m->rows : m->cols;
    const uint64_t yr = IsTranspose(op) ? m->cols : m->rows;
    if ((m->rows > 0U && m->ptrs == nullptr) || (m->nnz > 0U && (m->idxs == nullptr || m->values == nullptr)) ||
        (xr > 0U && x->values == nullptr) || (yr > 0U && y->values == nullptr)) {
        return ACL_SPARSE_STATUS_INVALID_VALUE;
    }
    return HasAliases(m, x, y) ? ACL_SPARSE_STATUS_INVALID_VALUE : ACL_SPARSE_STATUS_SUCCESS;
}

aclsparseStatus_t ValidateWorkspace(void* buffer)
{
    if (buffer == nullptr) return ACL_SPARSE_STATUS_INSUFFICIENT_RESOURCES;
    if (reinterpret_cast<uintptr_t>(buffer) % aclsp::kWsAlign != 0U) return ACL_SPARSE_STATUS_INVALID_VALUE;
    return ACL_SPARSE_STATUS_SUCCESS;
}

// CSR_ALG1 takes the reference-sized workspace (sparse/spmv/arch35/
// spmv_tiling_data.h:104-141: the normalised row offsets, plus a cols-long
// accumulator for a transpose) and the kernels that need nothing more: the row
// kernels for opA = N, the atomic scatter for T and H.  DEFAULT and CSR_ALG2
// take the larger workspace of the staged, narrow-column and CSC tables.
bool LeanAlg(aclsparseSpMVAlg_t alg) { return alg == ACL_SPARSE_SPMV_CSR_ALG1; }

SpmvLayout LayoutFor(const aclsparseSpMatDescr* m, aclsparseOperation_t op, aclDataType c, aclsparseSpMVAlg_t alg)
{
    return aclsp::ComputeLayout(m->rows, m->cols, m->nnz, m->ptr_type, c, IsTranspose(op), true,
                                aclsp::StageValueBytes(m->value_type, c), aclsp::NarrowTypes(m->value_type, c),
                                aclsp::CbandTypes(m->value_type, c), LeanAlg(alg));
}

bool Aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15U) == 0U; }

// The staged-gather tables are built when the layout has them and the
// operands are what its kernels (and the row kernel it falls back to) read:
// bound, unit-stride, 16-byte aligned column indices and values.
bool StageUsable(const SpmvLayout& l, const aclsparseSpMatDescr* m, const aclsparseDnVecDescr* x,
                 const aclsparseDnVecDescr* y)
{
    return l.staged && m->idxs != nullptr && m->values != nullptr && m->idx_stride == 1 && m->value_stride == 1 &&
           x->stride == 1 && y->stride == 1 && Aligned16(m->idxs) && Aligned16(m->values);
}

// The narrow column copy is built when the layout has it and the row kernel
// would stream this matrix: unit strides, 16-byte aligned column indices and
// values, x addressable with 32-bit byte offsets.
bool NarrowUsable(const SpmvLayout& l, const aclsparseSpMatDescr* m, const aclsparseDnVecDescr* x,
                  const aclsparseDnVecDescr* y)
{
    const uint64_t xBytes = m->value_type == ACL_FLOAT16 || m->value_type == ACL_BF16 ? 2U
                            : m->value_type == ACL_INT8                                 ? 1U
                            : m->value_type == ACL_COMPLEX64                            ? 8U
                                                                                        : 4U;
    return l.narrow && m->idxs != nullptr && m->values != nullptr && m->idx_stride == 1 && m->value_stride == 1 &&
           x->stride == 1 && y->stride == 1 && Aligned16(m->idxs) && Aligned16(m->values) &&
           m->cols * xBytes <= 0x7FFFFFFFULL;
}

// The complex banded transpose's rows and decision are built when the layout
// has room for them and its kernel would read this matrix: unit strides,
// bound column indices and values, x and y addressable with 32-bit byte
// offsets.
bool CbandUsable(const SpmvLayout& l, const aclsparseSpMatDescr* m, const aclsparseDnVecDescr* x,
                 const aclsparseDnVecDescr* y)
{
    return l.cband && m->idxs != nullptr && m->values != nullptr && m->idx_stride == 1 && m->value_stride == 1 &&
           x->stride == 1 && y->stride == 1 && m->rows * 8U <= 0x7FFFFFFFULL && m->nnz * 8U <= 0x7FFFFFFFULL;
}

// After a staged or narrow Preprocess: publish the path flag it leaves in the
// workspace header to the host (a pooled pinned slot, no wait); any failure
// leaves the choice unknown (SpMV then launches every kernel set, each reading
// the device flag).
void PublishStagedChoice(aclsparseSpMatDescr* m, void* ws, void* stream)
{
    aclsp::PublishPathChoice(m->staged_choice, ws, stream);
}

// The path of the matching staged Preprocess if its copy has completed, else -1.
int32_t StagedChoice(const aclsparseSpMatDescr* m, void* stream)
{
    return aclsp::QueryPathChoice(m->staged_choice, stream);
}

SpmvPlan MakePlan(const aclsparseSpMatDescr* m, const aclsparseDnVecDescr* x, const aclsparseDnVecDescr* y,
                  aclsparseOperation_t op, aclDataType c, aclsparseSpMVAlg_t alg, const void* buffer,
                  const aclsparseContext* h)
{
    SpmvPlan p;
    p.buffer = buffer;
    p.row_offsets = m->ptrs;
    p.col_ind = m->idxs;
    p.values = m->values;
    p.row_stride = m->ptr_stride;
    p.col_stride = m->idx_stride;
    p.val_stride = m->value_stride;
    p.x_stride = x->stride;
    p.y_stride = y->stride;
    p.rows = m->rows;
    p.cols = m->cols;
    p.nnz = m->nnz;
    p.base = m->base;
    p.ptr_type = m->ptr_type;
    p.value_type = m->value_type;
    p.x_type = x->value_type;
    p.y_type = y->value_type;
    p.compute_type = c;
    p.op = op;
    p.alg = static_cast<int32_t>(alg);
    p.stream = h->stream;
    p.stream_epoch = h->stream_epoch;
    return p;
}

bool PlanMatches(const SpmvPlan& a, const SpmvPlan& b)
{
    return a.buffer != nullptr && a.buffer == b.buffer && a.row_offsets == b.row_offsets &&
           a.col_ind == b.col_ind && a.values == b.values && a.row_stride == b.row_stride &&
           a.col_stride == b.col_stride && a.val_stride == b.val_stride && a.x_stride == b.x_stride &&
           a.y_stride == b.y_stride && a.rows == b.rows && a.cols == b.cols && a.nnz == b.nnz &&
           a.base == b.base && a.ptr_type == b.ptr_type && a.value_type == b.value_type &&
           a.x_type == b.x_type && a.y_type == b.y_type && a.compute_type == b.compute_type && a.op == b.op &&
           a.alg == b.alg && a.stream == b.stream && a.stream_epoch == b.stream_epoch;
}

void* HipStreamOf(const aclsparseContext* h)
{
    return h->stream == ACL_SPARSE_HIP_NULL_STREAM ? nullptr : h->stream;
}

aclsp::SpmvLaunch MakeLaunch(const aclsparseContext* h, aclsparseOperation_t op, const void* alpha,
                             const aclsparseSpMatDescr* m, const aclsparseDnVecDescr* x, const void* beta,
                             const aclsparseDnVecDescr* y, aclDataType c, aclsparseSpMVAlg_t alg, void* ws)
{
    aclsp::SpmvLaunch l{};
    l.row_ptr = m->ptrs;
    l.row_stride = m->ptr_stride;
    l.col = static_cast<const int32_t*>(m->idxs);
    l.col_stride = m->idx_stride;
    l.val = m->values;
    l.val_stride = m->value_stride;
    l.x = x->values;
    l.x_stride = x->stride;
    l.y = y->values;
    l.y_stride = y->stride;
    l.rows = static_cast<int64_t>(m->rows);
    l.cols = static_cast<int64_t>(m->cols);
    l.nnz = static_cast<int64_t>(m->nnz);
    l.base = m->base == ACL_SPARSE_INDEX_BASE_ONE ? 1 : 0;
    l.rowptr64 = m->ptr_type == ACL_SPARSE_INDEX_64I ? 1 : 0;
    switch (m->value_type) {
        case ACL_FLOAT16: l.val_kind = aclsp::ValKind::F16; break;
        case ACL_BF16: l.val_kind = aclsp::ValKind::BF16; break;
        case ACL_INT8: l.val_kind = aclsp::ValKind::I8; break;
        case ACL_COMPLEX64: l.val_kind = aclsp::ValKind::C64; break;
        default: l.val_kind = aclsp::ValKind::F32; break;
    }
    switch (y->value_type) {
        case ACL_FLOAT16: l.out_kind = aclsp::OutKind::F16; break;
        case ACL_BF16: l.out_kind = aclsp::OutKind::BF16; break;
        case ACL_INT32: l.out_kind = aclsp::OutKind::I32; break;
        case ACL_COMPLEX64: l.out_kind = aclsp::OutKind::C64; break;
        default: l.out_kind = aclsp::OutKind::F32; break;
    }
    l.acc_kind = c == ACL_INT32 ? aclsp::AccKind::I64 : c == ACL_COMPLEX64 ? aclsp::AccKind::C64
                                                                           : aclsp::AccKind::F32;
    l.op = static_cast<int32_t>(op);
    l.alg = static_cast<int32_t>(alg);
    l.device_scalars = h->pointer_mode == ACL_SPARSE_POINTER_MODE_DEVICE ? 1 : 0;
    if (l.device_scalars) {
        l.alpha_ptr = alpha;
        l.beta_ptr = beta;
    } else if (c == ACL_INT32) {
        std::memcpy(&l.alpha_i, alpha, sizeof(int32_t));
        std::memcpy(&l.beta_i, beta, sizeof(int32_t));
    } else if (c == ACL_COMPLEX64) {
        aclsparseComplex a, b;
        std::memcpy(&a, alpha, sizeof(a));
        std::memcpy(&b, beta, sizeof(b));
        l.alpha_re = a.x;
        l.alpha_im = a.y;
        l.beta_re = b.x;
        l.beta_im = b.y;
    } else {
        std::memcpy(&l.alpha_re, alpha, sizeof(float));
        std::memcpy(&l.beta_re, beta, sizeof(float));
    }
    l.ws = ws;
    l.layout = LayoutFor(m, op, c, alg);
    return l;
}

}  // namespace

extern "C" {

aclsparseStatus_t aclsparseSpMVGetBufferSize(aclsparseHandle_t handle, aclsparseOperation_t opA, const void* alpha,
                                             aclsparseConstSpMatDescr_t matA, aclsparseConstDnVecDescr_t vecX,
                                             const void* beta, aclsparseDnVecDescr_t vecY, aclDataType computeType,
                                             aclsparseSpMVAlg_t alg, size_t* bufferSize)
{
    if (bufferSize == nullptr) return ACL_SPARSE_STATUS_INVALID_VALUE;
    *bufferSize = 0U;
    aclsparseStatus_t st = ValidateInputs(handle, opA, alpha, matA, vecX, beta, vecY, computeType, alg);
    if (st != ACL_SPARSE_STATUS_SUCCESS) return st;
    *bufferSize = LayoutFor(matA, opA, computeType, alg).total;
    return ACL_SPARSE_STATUS_SUCCESS;
}

aclsparseStatus_t aclsparseSpMVPreprocess(aclsparseHandle_t handle, aclsparseOperation_t opA, const void* alpha,
                                          aclsparseConstSpMatDescr_t matA, aclsparseConstDnVecDescr_t vecX,
                                          const void* beta, aclsparseDnVecDescr_t vecY, aclDataType computeType,
                                          aclsparseSpMVAlg_t alg, void* externalBuffer)
{
    aclsparseStatus_t st = ValidateInputs(handle, opA, alpha, matA, vecX, beta, vecY, computeType, alg);
    if (st != ACL_SPARSE_STATUS_SUCCESS) return st;
    auto* m = const_cast<aclsparseSpMatDescr*>(matA);
    // Preprocess reads only the row offsets; values and vectors may be bound later.
    if (m->rows > 0U && m->ptrs == nullptr) return ACL_SPARSE_STATUS_INVALID_VALUE;
    st = ValidateWorkspace(externalBuffer);
    if (st != ACL_SPARSE_STATUS_SUCCESS) return st;
    bool staged = false, narrow = false, cband = false;
    if (m->rows > 0U) {
        (void)hipGetLastError();
        aclsp::SpmvLaunch l = MakeLaunch(handle, opA, alpha, m, vecX, beta, vecY, computeType, alg, externalBuffer);
        staged = StageUsable(l.layout, m, vecX, vecY);
        narrow = NarrowUsable(l.layout, m, vecX, vecY);
        cband = IsTranspose(opA) && CbandUsable(l.layout, m, vecX, vecY);
        l.staged = staged ? 1 : 0;
        l.narrow = narrow ? 1 : 0;
        l.cband = cband ? 1 : 0;
        if (aclsp::LaunchSpmvPreprocess(l, HipStreamOf(handle)) != 0 || hipGetLastError() != hipSuccess) {
            m->plan = SpmvPlan{};
            return ACL_SPARSE_STATUS_EXECUTION_FAILED;
        }
        if (staged || narrow || cband) PublishStagedChoice(m, externalBuffer, HipStreamOf(handle));
        else aclsp::ReleasePathChoice(m->staged_choice);
    }
    m->plan = MakePlan(m, vecX, vecY, opA, computeType, alg, externalBuffer, handle);
    m->plan.staged = staged;
    m->plan.narrow = narrow;
    m->plan.cband = cband;
    return ACL_SPARSE_STATUS_SUCCESS;
}

aclsparseStatus_t aclsparseSpMV(aclsparseHandle_t handle, aclsparseOperation_t opA, const void* alpha,
                                aclsparseConstSpMatDescr_t matA, aclsparseConstDnVecDescr_t vecX, const void* beta,
                                aclsparseDnVecDescr_t vecY, aclDataType computeType, aclsparseSpMVAlg_t alg,
                                void* externalBuffer)
{
    aclsparseStatus_t st = ValidateInputs(handle, opA, alpha, matA, vecX, beta, vecY, computeType, alg);
    if (st != ACL_SPARSE_STATUS_SUCCESS) return st;
    st = ValidateStorage(opA, matA, vecX, vecY);
    if (st != ACL_SPARSE_STATUS_SUCCESS) return st;
    st = ValidateWorkspace(externalBuffer);
    if (st != ACL_SPARSE_STATUS_SUCCESS) return st;
    const uint64_t outLen = IsTranspose(opA) ? matA->cols : matA->rows;
    if (outLen == 0U) return ACL_SPARSE_STATUS_SUCCESS;

    auto* m = const_cast<aclsparseSpMatDescr*>(matA);
    aclsp::SpmvLaunch l = MakeLaunch(handle, opA, alpha, m, vecX, beta, vecY, computeType, alg, externalBuffer);
    void* stream = HipStreamOf(handle);
    (void)hipGetLastError();
    // The partition is rebuilt unless a matching Preprocess already wrote it
    // into this very buffer.  A zero-row matrix has no partition to build.
    // Without a matching plan the row kernels run (the staged tables are
    // built only by Preprocess).
    const bool planned = m->rows == 0U ||
                         PlanMatches(m->plan, MakePlan(m, vecX, vecY, opA, computeType, alg, externalBuffer, handle));
    if (!planned && aclsp::LaunchSpmvPreprocess(l, stream) != 0) return ACL_SPARSE_STATUS_EXECUTION_FAILED;
    // pass A reads x as 16-byte vectors
    l.staged = planned && m->rows > 0U && m->plan.staged && Aligned16(vecX->values) ? 1 : 0;
    l.narrow = planned && m->rows > 0U && m->plan.narrow ? 1 : 0;
    l.cband = planned && m->rows > 0U && m->plan.cband ? 1 : 0;
    l.staged_choice = l.staged || l.narrow || l.cband ? StagedChoice(m, stream) : -1;
    if (aclsp::LaunchSpmvCompute(l, stream) != 0 || hipGetLastError() != hipSuccess) {
        return ACL_SPARSE_STATUS_EXECUTION_FAILED;
    }
    return ACL_SPARSE_STATUS_SUCCESS;
}

}  // extern "C"

namespace aclsp {

aclsparseStatus_t SpmvWithScratch(aclsparseHandle_t handle, aclsparseOperation_t opA, const void* alpha,
                                  aclsparseConstSpMatDescr_t matA, aclsparseConstDnVecDescr_t vecX, const void* beta,
                                  aclsparseDnVecDescr_t vecY, aclDataType computeType, aclsparseSpMVAlg_t alg,
                                  void* (*scratch)(), size_t scratchBytes)
{
    aclsparseStatus_t st = ValidateInputs(handle, opA, alpha, matA, vecX, beta, vecY, computeType, alg);
    if (st != ACL_SPARSE_STATUS_SUCCESS) return st;
    st = ValidateStorage(opA, matA, vecX, vecY);
    if (st != ACL_SPARSE_STATUS_SUCCESS) return st;
    const uint64_t outLen = IsTranspose(opA) ? matA->cols : matA->rows;
    if (outLen == 0U) return ACL_SPARSE_STATUS_SUCCESS;
    // the layout without the staged-gather tables (they need Preprocess)
    const SpmvLayout layout = ComputeLayout(matA->rows, matA->cols, matA->nnz, matA->ptr_type, computeType,
                                            IsTranspose(opA), true, 0U);
    if (layout.total > scratchBytes) return ACL_SPARSE_STATUS_INSUFFICIENT_RESOURCES;
    void* ws = scratch();
    if (ws == nullptr) return ACL_SPARSE_STATUS_EXECUTION_FAILED;
    SpmvLaunch l = MakeLaunch(handle, opA, alpha, matA, vecX, beta, vecY, computeType, alg, ws);
    l.layout = layout;
    l.staged = 0;
    l.narrow = 0;
    void* stream = HipStreamOf(handle);
    (void)hipGetLastError();
    if (matA->rows > 0U && LaunchSpmvPreprocess(l, stream) != 0) return ACL_SPARSE_STATUS_EXECUTION_FAILED;
    if (LaunchSpmvCompute(l, stream) != 0 || hipGetLastError() != hipSuccess) {
        return ACL_SPARSE_STATUS_EXECUTION_FAILED;
    }
    return ACL_SPARSE_STATUS_SUCCESS;
}

// Pool of path-choice slots.  Preprocess takes a slot, copies the header's
// flag into it asynchronously and records the slot's event after the copy.
// A slot handed back (by the next Preprocess of the same descriptor or by its
// destruction) may still have that copy in flight, so it is reused only once
// its event reports completion (hipEventQuery, never a wait).  Slots are
// allocated in batches of pinned memory and kept for the life of the process,
// so a late copy always lands in memory the pool owns.
struct ChoiceSlot {
    uint32_t* host;
    hipEvent_t event;
    bool recorded;  // an event record (and the copy before it) was enqueued
};

namespace {

constexpr uint32_t kChoiceUnknown = 0xFFFFFFFFU;
constexpr int kSlotBatch = 64;

std::mutex gSlotMutex;
std::vector<ChoiceSlot*> gFreeSlots;
std::vector<ChoiceSlot*> gPendingSlots;  // handed back, copy possibly in flight

// A slot ready for a new copy, or nullptr.  Called with gSlotMutex held.
ChoiceSlot* TakeSlotLocked()
{
    for (size_t i = 0; i < gPendingSlots.size();) {
        ChoiceSlot* c = gPendingSlots[i];
        const hipError_t e = c->recorded ? hipEventQuery(c->event) : hipSuccess;
        if (e == hipSuccess) {
            gFreeSlots.push_back(c);
            gPendingSlots[i] = gPendingSlots.back();
            gPendingSlots.pop_back();
        } else {
            if (e != hipErrorNotReady) (void)hipGetLastError();
            ++i;
        }
    }
    if (gFreeSlots.empty()) {
        void* p = nullptr;
        if (hipHostMalloc(&p, kSlotBatch * sizeof(uint32_t), hipHostMallocDefault) != hipSuccess) {
            (void)hipGetLastError();
            return nullptr;
        }
        auto* words = static_cast<uint32_t*>(p);
        for (int k = 0; k < kSlotBatch; ++k) {
            hipEvent_t e = nullptr;
            if (hipEventCreateWithFlags(&e, hipEventDisableTiming) != hipSuccess) {
                (void)hipGetLastError();
                break;  // the remaining words stay unused
            }
            gFreeSlots.push_back(new ChoiceSlot{words + k, e, false});
        }
        if (gFreeSlots.empty()) return nullptr;
    }
    ChoiceSlot* c = gFreeSlots.back();
    gFreeSlots.pop_back();
    return c;
}

bool Capturing(hipStream_t s)
{
    hipStreamCaptureStatus st = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing(s, &st) != hipSuccess) {
        (void)hipGetLastError();
        return true;  // unknown: take the path that needs no host call
    }
    return st != hipStreamCaptureStatusNone;
}

}  // namespace

// Hand a slot back to the pool (its copy may still be in flight).
void ReleasePathChoice(ChoiceSlot*& slot)
{
    if (slot == nullptr) return;
    std::lock_guard<std::mutex> lock(gSlotMutex);
    gPendingSlots.push_back(slot);
    slot = nullptr;
}

// After a Preprocess that may choose a path on the device: hand back the
// previous slot, take a fresh one, set it to the "unknown" sentinel, copy the
// header's flag into it and record its event after the copy.  Nothing waits
// for the device.  Under stream capture no copy is made and the choice stays
// unknown (the captured SpMVs read the device flag).
void PublishPathChoice(ChoiceSlot*& slot, void* ws, void* stream)
{
    ReleasePathChoice(slot);
    hipStream_t s = static_cast<hipStream_t>(stream);
    if (Capturing(s)) return;
    ChoiceSlot* c = nullptr;
    {
        std::lock_guard<std::mutex> lock(gSlotMutex);
        c = TakeSlotLocked();
    }
    if (c == nullptr) return;
    *static_cast<volatile uint32_t*>(c->host) = kChoiceUnknown;
    c->recorded = false;
    const auto* header = static_cast<const SpmvWsHeader*>(ws);
    if (hipMemcpyAsync(c->host, &header->staged_flag, sizeof(uint32_t), hipMemcpyDeviceToHost, s) != hipSuccess) {
        (void)hipGetLastError();
        ReleasePathChoice(c);  // nothing was enqueued: free at once
        return;
    }
    c->recorded = true;  // a copy is enqueued: the slot is reused only after its event
    if (hipEventRecord(c->event, s) != hipSuccess) {
        (void)hipGetLastError();
        // without the event the copy's completion cannot be observed: the
        // slot is retired for good (its word may still be written)
        return;
    }
    slot = c;
}

// The published path (0 the row / CSC kernels, 1 the staged or column-bucketed
// kernels, 2 the banded transpose kernel, 3 the narrow-column row kernel, 4
// the banded transpose kernel on 16-bit copies, 5 the narrow-column row kernel
// on entry-aligned blocks, 6 the packed banded transpose) if its copy has
// completed, else -1.  Always -1 under stream capture: a captured graph then
// holds every kernel set, each gated on the device flag, so that it stays
// correct when a later Preprocess into the same workspace chooses another path.
int32_t QueryPathChoice(const ChoiceSlot* slot, void* stream)
{
    if (slot == nullptr) return -1;
    hipStream_t s = static_cast<hipStream_t>(stream);
    if (Capturing(s)) return -1;
    // The copy is one aligned 4-byte write over the sentinel stored before it
    // was enqueued: a value other than the sentinel is the final one.
    uint32_t v = *static_cast<volatile const uint32_t*>(slot->host);
    if (v == kChoiceUnknown) {
        if (hipEventQuery(slot->event) != hipSuccess) {
            (void)hipGetLastError();
            return -1;
        }
        v = *static_cast<volatile const uint32_t*>(slot->host);
    }
    return v <= static_cast<uint32_t>(kMaxPathFlag) ? static_cast<int32_t>(v) : -1;
}

}  // namespace aclsp
