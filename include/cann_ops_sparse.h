/*
 * cann_ops_sparse.h — C ABI of the MI355X (gfx950) CSR SpMV library.
 *
 * This header declares exactly the entry points of the reference's SpMV path
 * (plus the SpMVOp family and the descriptor/handle calls that path needs),
 * with the same names, argument order, enum values and status semantics, so a
 * caller written against Atlas-Ascend-Fork/ops-sparse links against
 * libaclsparse_hip.so unchanged.  Each declaration cites the reference
 * declaration it replaces (paths relative to the reference repository).
 *
 * Differences that are part of the contract:
 *   - aclrtStream is a hipStream_t passed as void* (no HIP headers needed by
 *     callers); a null stream means "not set" exactly as in the reference
 *     (aclsparseSpMV* reject it); callers that want the HIP null stream pass
 *     ACL_SPARSE_HIP_NULL_STREAM (below) to aclsparseSetStream.
 *   - aclsparseSpMV accepts ACL_SPARSE_INDEX_64I row offsets (column indices
 *     stay 32-bit).  The reference rejects I64 in SpMV
 *     (sparse/spmv/arch35/spmv_host.cpp:220-231); this build extends it.
 *   - The workspace returned by aclsparseSpMVGetBufferSize is larger than the
 *     reference formula (it also holds the row-block partition); only
 *     "non-zero, multiple of 64 bytes" is contractual, as in the reference
 *     tests (test/spmv/arch35/spmv_test.cpp:124-128).
 */
#ifndef CANN_OPS_SPARSE_H_
#define CANN_OPS_SPARSE_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* CANN acl_base_rt.h data types, same numeric values
 * (mirrored at test/spmm/python/algorithm_mock/acl/acl_base_rt.h:14-17). */
typedef enum aclDataType {
    ACL_DT_UNDEFINED = -1,
    ACL_FLOAT = 0,
    ACL_FLOAT16 = 1,
    ACL_INT8 = 2,
    ACL_INT32 = 3,
    ACL_UINT8 = 4,
    ACL_INT16 = 6,
    ACL_UINT16 = 7,
    ACL_UINT32 = 8,
    ACL_INT64 = 9,
    ACL_UINT64 = 10,
    ACL_DOUBLE = 11,
    ACL_BOOL = 12,
    ACL_COMPLEX64 = 16,
    ACL_BF16 = 27
} aclDataType;

/* hipStream_t, opaque to callers. */
typedef void* aclrtStream;

/* The HIP null stream is a valid stream, but a null aclrtStream means "unset"
 * in this API (sparse/spmv/arch35/spmv_host.cpp:119-122).  Pass this sentinel
 * to aclsparseSetStream to run on the HIP null stream. */
#define ACL_SPARSE_HIP_NULL_STREAM ((aclrtStream)(uintptr_t)1)

/* include/cann_ops_sparse.h:32-36 */
typedef enum aclsparseOperation_t {
    ACL_SPARSE_OP_NON_TRANSPOSE = 0,
    ACL_SPARSE_OP_TRANSPOSE = 1,
    ACL_SPARSE_OP_CONJUGATE_TRANSPOSE = 2
} aclsparseOperation_t;

struct aclsparseContext;
struct aclsparseSpMatDescr;
struct aclsparseDnVecDescr;
typedef struct aclsparseContext* aclsparseHandle_t;
typedef struct aclsparseSpMatDescr* aclsparseSpMatDescr_t;
typedef struct aclsparseDnVecDescr* aclsparseDnVecDescr_t;
typedef struct aclsparseSpMatDescr const* aclsparseConstSpMatDescr_t;
typedef struct aclsparseDnVecDescr const* aclsparseConstDnVecDescr_t;

/* include/cann_ops_sparse.h:63-66 */
typedef enum aclsparseOrder_t {
    ACL_SPARSE_ORDER_ROW = 0,
    ACL_SPARSE_ORDER_COL = 1
} aclsparseOrder_t;

struct aclsparseDnMatDescr;
typedef struct aclsparseDnMatDescr* aclsparseDnMatDescr_t;
typedef struct aclsparseDnMatDescr const* aclsparseConstDnMatDescr_t;

/* include/cann_ops_sparse.h:2412-2417 */
typedef enum aclsparseSpMMOpAlg_t {
    ACL_SPARSE_SPMMOP_ALG_DEFAULT = 0,
    ACL_SPARSE_SPMMOP_ALG1 = 1,
    ACL_SPARSE_SPMMOP_ALG2 = 2,
    ACL_SPARSE_SPMMOP_ALG1_HIGH_PRECISION = 3
} aclsparseSpMMOpAlg_t;

struct aclsparseSpMMOpDescr;
struct aclsparseSpMMOpPlan;
typedef struct aclsparseSpMMOpDescr* aclsparseSpMMOpDescr_t;
typedef struct aclsparseSpMMOpDescr const* aclsparseConstSpMMOpDescr_t;
typedef struct aclsparseSpMMOpPlan* aclsparseSpMMOpPlan_t;

/* include/cann_ops_sparse.h:69-83 */
typedef enum aclsparseSpMVOpAlg_t {
    ACL_SPARSE_SPMVOP_ALG_DEFAULT = 0,
    ACL_SPARSE_SPMVOP_ALG1 = 1,
    ACL_SPARSE_SPMVOP_ALG2 = 2
} aclsparseSpMVOpAlg_t;

struct aclsparseSpMVOpDescr;
struct aclsparseSpMVOpPlan;
typedef struct aclsparseSpMVOpDescr* aclsparseSpMVOpDescr_t;
typedef struct aclsparseSpMVOpDescr const* aclsparseConstSpMVOpDescr_t;
typedef struct aclsparseSpMVOpPlan* aclsparseSpMVOpPlan_t;

/* include/cann_ops_sparse.h:124-174 */
typedef enum aclsparseStatus_t {
    ACL_SPARSE_STATUS_SUCCESS = 0,
    ACL_SPARSE_STATUS_NOT_INITIALIZED = 1,
    ACL_SPARSE_STATUS_ALLOC_FAILED = 2,
    ACL_SPARSE_STATUS_INVALID_VALUE = 3,
    ACL_SPARSE_STATUS_ARCH_MISMATCH = 4,
    ACL_SPARSE_STATUS_EXECUTION_FAILED = 5,
    ACL_SPARSE_STATUS_INTERNAL_ERROR = 6,
    ACL_SPARSE_STATUS_MATRIX_TYPE_NOT_SUPPORTED = 7,
    ACL_SPARSE_STATUS_NOT_SUPPORTED = 8,
    ACL_SPARSE_STATUS_INSUFFICIENT_RESOURCES = 9,
    ACL_SPARSE_STATUS_HANDLE_IS_NULLPTR = 10
} aclsparseStatus_t;

/* include/cann_ops_sparse.h:176-201 */
typedef enum aclsparseSpMVAlg_t {
    ACL_SPARSE_SPMV_ALG_DEFAULT = 0,
    ACL_SPARSE_SPMV_COO_ALG1 = 1,
    ACL_SPARSE_SPMV_COO_ALG2 = 2,
    ACL_SPARSE_SPMV_CSR_ALG1 = 3,
    ACL_SPARSE_SPMV_CSR_ALG2 = 4,
    ACL_SPARSE_SPMV_SELL_ALG1 = 5,
    ACL_SPARSE_SPMV_CSR_ALG_CUBE = 6
} aclsparseSpMVAlg_t;

/* include/cann_ops_sparse.h:205-208 */
typedef struct aclsparseComplex {
    float x;
    float y;
} aclsparseComplex;

/* include/cann_ops_sparse.h:244-246 */
typedef enum aclsparseIndexType_t {
    ACL_SPARSE_INDEX_32I = 0,
    ACL_SPARSE_INDEX_64I = 1
} aclsparseIndexType_t;

/* include/cann_ops_sparse.h:258-260 */
typedef enum aclsparseIndexBase_t {
    ACL_SPARSE_INDEX_BASE_ZERO = 0,
    ACL_SPARSE_INDEX_BASE_ONE = 1
} aclsparseIndexBase_t;

/* include/cann_ops_sparse.h:263-276 */
typedef enum aclsparseFormat_t {
    ACL_SPARSE_FORMAT_COO = 0,
    ACL_SPARSE_FORMAT_CSR = 1,
    ACL_SPARSE_FORMAT_CSC = 2,
    ACL_SPARSE_FORMAT_BLOCKED_ELL = 3,
    ACL_SPARSE_FORMAT_SLICED_ELL = 4,
    ACL_SPARSE_FORMAT_BSR = 5
} aclsparseFormat_t;

/* include/cann_ops_sparse.h:1623-1625 */
typedef enum aclsparsePointerMode_t {
    ACL_SPARSE_POINTER_MODE_HOST = 0,
    ACL_SPARSE_POINTER_MODE_DEVICE = 1
} aclsparsePointerMode_t;

/* ---------------- handle (include/cann_ops_sparse.h:1542-1647) ---------------- */

/* replaces include/cann_ops_sparse.h:1542 aclsparseCreate */
aclsparseStatus_t aclsparseCreate(aclsparseHandle_t* handle);
/* replaces include/cann_ops_sparse.h:1553 aclsparseDestroy */
aclsparseStatus_t aclsparseDestroy(aclsparseHandle_t handle);
/* replaces include/cann_ops_sparse.h:1562 aclsparseSetStream */
aclsparseStatus_t aclsparseSetStream(aclsparseHandle_t handle, aclrtStream stream);
/* replaces include/cann_ops_sparse.h:1572 aclsparseGetStream */
aclsparseStatus_t aclsparseGetStream(aclsparseHandle_t handle, aclrtStream* stream);
/* replaces include/cann_ops_sparse.h:1591 aclsparseSetWorkspace */
aclsparseStatus_t aclsparseSetWorkspace(aclsparseHandle_t handle, void* workspace, size_t workspaceSize);
/* replaces include/cann_ops_sparse.h:1605 aclsparseGetWorkspace */
aclsparseStatus_t aclsparseGetWorkspace(aclsparseHandle_t handle, void** workspace, size_t* workspaceSize);
/* No counterpart in the reference: the build id of this library (the first 32
 * hex digits of a SHA-256 over its native sources, this header and the
 * compiler flags), for loaders that refuse a library built from other
 * sources.  The returned string is static. */
const char* aclsparseHipBuildId(void);
/* replaces include/cann_ops_sparse.h:1617 aclsparseGetVersion */
aclsparseStatus_t aclsparseGetVersion(aclsparseHandle_t handle, int* version);
/* replaces include/cann_ops_sparse.h:1637 aclsparseSetPointerMode */
aclsparseStatus_t aclsparseSetPointerMode(aclsparseHandle_t handle, aclsparsePointerMode_t mode);
/* replaces include/cann_ops_sparse.h:1647 aclsparseGetPointerMode */
aclsparseStatus_t aclsparseGetPointerMode(aclsparseHandle_t handle, aclsparsePointerMode_t* mode);

/* ---------------- dense vector descriptor ---------------- */

/* replaces include/cann_ops_sparse.h:288 */
aclsparseStatus_t aclsparseCreateDnVec(aclsparseDnVecDescr_t* dnVecDescr, int64_t size, void* values,
                                       aclDataType valueType);
/* replaces include/cann_ops_sparse.h:294 */
aclsparseStatus_t aclsparseCreateConstDnVec(aclsparseConstDnVecDescr_t* dnVecDescr, int64_t size,
                                            const void* values, aclDataType valueType);
/* replaces include/cann_ops_sparse.h:304 */
aclsparseStatus_t aclsparseDestroyDnVec(aclsparseConstDnVecDescr_t dnVecDescr);
/* replaces include/cann_ops_sparse.h:455 */
aclsparseStatus_t aclsparseDnVecGet(aclsparseDnVecDescr_t dnVecDescr, int64_t* size, void** values,
                                    aclDataType* valueType);
/* replaces include/cann_ops_sparse.h:474 */
aclsparseStatus_t aclsparseDnVecGetValues(aclsparseDnVecDescr_t dnVecDescr, void** values);
/* replaces include/cann_ops_sparse.h:488 */
aclsparseStatus_t aclsparseDnVecSetValues(aclsparseDnVecDescr_t dnVecDescr, void* values);
/* replaces include/cann_ops_sparse.h:497 */
aclsparseStatus_t aclsparseDnVecSetStride(aclsparseDnVecDescr_t dnVecDescr, int64_t stride);
/* replaces include/cann_ops_sparse.h:502 */
aclsparseStatus_t aclsparseDnVecGetStride(aclsparseConstDnVecDescr_t dnVecDescr, int64_t* stride);

/* ---------------- CSR sparse matrix descriptor ---------------- */

/* replaces include/cann_ops_sparse.h:529 */
aclsparseStatus_t aclsparseCreateCsr(aclsparseSpMatDescr_t* spMatDescr, int64_t rows, int64_t cols, int64_t nnz,
                                     void* csrRowOffsets, void* csrColInd, void* csrValues,
                                     aclsparseIndexType_t csrRowOffsetsType, aclsparseIndexType_t csrColIndType,
                                     aclsparseIndexBase_t idxBase, aclDataType valueType);
/* replaces include/cann_ops_sparse.h:535 */
aclsparseStatus_t aclsparseCreateConstCsr(aclsparseConstSpMatDescr_t* spMatDescr, int64_t rows, int64_t cols,
                                          int64_t nnz, const void* csrRowOffsets, const void* csrColInd,
                                          const void* csrValues, aclsparseIndexType_t csrRowOffsetsType,
                                          aclsparseIndexType_t csrColIndType, aclsparseIndexBase_t idxBase,
                                          aclDataType valueType);
/* replaces include/cann_ops_sparse.h:797 */
aclsparseStatus_t aclsparseCsrSetPointers(aclsparseSpMatDescr_t descr, void* rowOffsets, void* colIndices,
                                          void* values);
/* replaces include/cann_ops_sparse.h:804 */
aclsparseStatus_t aclsparseCsrSetStrides(aclsparseSpMatDescr_t descr, int64_t rowOffsetsStride,
                                         int64_t colIndStride, int64_t valuesStride);
/* replaces include/cann_ops_sparse.h:811 */
aclsparseStatus_t aclsparseCsrGetStrides(aclsparseConstSpMatDescr_t descr, int64_t* rowOffsetsStride,
                                         int64_t* colIndStride, int64_t* valuesStride);
/* replaces include/cann_ops_sparse.h:872 */
aclsparseStatus_t aclsparseDestroySpMat(aclsparseConstSpMatDescr_t spMatDescr);
/* replaces include/cann_ops_sparse.h:885 */
aclsparseStatus_t aclsparseSpMatGetFormat(aclsparseConstSpMatDescr_t spMatDescr, aclsparseFormat_t* format);
/* replaces include/cann_ops_sparse.h:893 */
aclsparseStatus_t aclsparseSpMatGetIndexBase(aclsparseConstSpMatDescr_t spMatDescr,
                                             aclsparseIndexBase_t* idxBase);
/* replaces include/cann_ops_sparse.h:903 */
aclsparseStatus_t aclsparseSpMatGetValues(aclsparseSpMatDescr_t spMatDescr, void** values);
/* replaces include/cann_ops_sparse.h:920 */
aclsparseStatus_t aclsparseSpMatSetValues(aclsparseSpMatDescr_t spMatDescr, void* values);
/* replaces include/cann_ops_sparse.h:927 */
aclsparseStatus_t aclsparseSpMatGetSize(aclsparseConstSpMatDescr_t spMatDescr, int64_t* rows, int64_t* cols,
                                        int64_t* nnz);
/* replaces include/cann_ops_sparse.h:2736 aclsparseCsrGet */
aclsparseStatus_t aclsparseCsrGet(aclsparseSpMatDescr_t spMatDescr, int64_t* rows, int64_t* cols, int64_t* nnz,
                                  void** csrRowOffsets, void** csrColInd, void** csrValues,
                                  aclsparseIndexType_t* csrRowOffsetsType, aclsparseIndexType_t* csrColIndType,
                                  aclsparseIndexBase_t* idxBase, aclDataType* valueType);

/* ---------------- SpMV (include/cann_ops_sparse.h:960-1006) ---------------- */

/* replaces include/cann_ops_sparse.h:960 (sparse/spmv/arch35/spmv_host.cpp:636-658) */
aclsparseStatus_t aclsparseSpMVGetBufferSize(aclsparseHandle_t handle, aclsparseOperation_t opA, const void* alpha,
                                             aclsparseConstSpMatDescr_t matA, aclsparseConstDnVecDescr_t vecX,
                                             const void* beta, aclsparseDnVecDescr_t vecY, aclDataType computeType,
                                             aclsparseSpMVAlg_t alg, size_t* bufferSize);
/* replaces include/cann_ops_sparse.h:983 (sparse/spmv/arch35/spmv_host.cpp:660-668) */
aclsparseStatus_t aclsparseSpMVPreprocess(aclsparseHandle_t handle, aclsparseOperation_t opA, const void* alpha,
                                          aclsparseConstSpMatDescr_t matA, aclsparseConstDnVecDescr_t vecX,
                                          const void* beta, aclsparseDnVecDescr_t vecY, aclDataType computeType,
                                          aclsparseSpMVAlg_t alg, void* externalBuffer);
/* replaces include/cann_ops_sparse.h:1003 (sparse/spmv/arch35/spmv_host.cpp:670-678) */
aclsparseStatus_t aclsparseSpMV(aclsparseHandle_t handle, aclsparseOperation_t opA, const void* alpha,
                                aclsparseConstSpMatDescr_t matA, aclsparseConstDnVecDescr_t vecX, const void* beta,
                                aclsparseDnVecDescr_t vecY, aclDataType computeType, aclsparseSpMVAlg_t alg,
                                void* externalBuffer);
/* No counterpart in the reference: aclsparseSpMV without a caller workspace,
 * for callers that cannot allocate device memory (code under HIP graph
 * capture, serving loops, harnesses that forbid allocation).  It calls no
 * allocator: its partition tables live in a static device array of
 * ACL_SPARSE_SPMV_NO_ALLOC_MAX_BYTES per GPU, held from library load to process
 * exit.  Every call rebuilds the row partition (as aclsparseSpMV does without
 * a matching Preprocess) and runs the row kernels or the transpose path; the
 * staged-gather path is not used (its tables need Preprocess).  A matrix whose
 * tables exceed the array returns ACL_SPARSE_STATUS_INSUFFICIENT_RESOURCES.
 * Calls on one GPU share the array: calls that overlap in time on one GPU
 * (other streams, other threads) race and must be ordered by the caller.
 * Launches go to the handle's stream, which must belong to the current device. */
#define ACL_SPARSE_SPMV_NO_ALLOC_MAX_BYTES (32u * 1024u * 1024u)
aclsparseStatus_t aclsparseSpMVNoAlloc(aclsparseHandle_t handle, aclsparseOperation_t opA, const void* alpha,
                                       aclsparseConstSpMatDescr_t matA, aclsparseConstDnVecDescr_t vecX,
                                       const void* beta, aclsparseDnVecDescr_t vecY, aclDataType computeType,
                                       aclsparseSpMVAlg_t alg);

/* ---------------- SpMVOp (include/cann_ops_sparse.h:2338-2396) ---------------- */

/* replaces include/cann_ops_sparse.h:2345 (sparse/spmv_op/arch35/spmv_op_host.cpp:515-560) */
aclsparseStatus_t aclsparseSpMVOp_bufferSize(aclsparseHandle_t handle, aclsparseOperation_t opA,
                                             aclsparseConstSpMatDescr_t matA, aclsparseConstDnVecDescr_t vecX,
                                             aclsparseConstDnVecDescr_t vecY, aclsparseDnVecDescr_t vecZ,
                                             aclDataType computeType, aclsparseSpMVOpAlg_t alg, size_t* bufferSize);
/* replaces include/cann_ops_sparse.h:2355 (sparse/spmv_op/arch35/spmv_op_host.cpp:631-674) */
aclsparseStatus_t aclsparseSpMVOp_createDescr(aclsparseHandle_t handle, aclsparseSpMVOpDescr_t* descr,
                                              aclsparseOperation_t opA, aclsparseConstSpMatDescr_t matA,
                                              aclsparseConstDnVecDescr_t vecX, aclsparseConstDnVecDescr_t vecY,
                                              aclsparseDnVecDescr_t vecZ, aclDataType computeType,
                                              aclsparseSpMVOpAlg_t alg, void* buffer);
/* replaces include/cann_ops_sparse.h:2365 (sparse/spmv_op/arch35/spmv_op_host.cpp:677-684) */
aclsparseStatus_t aclsparseSpMVOp_destroyDescr(aclsparseSpMVOpDescr_t descr);
/* replaces include/cann_ops_sparse.h:2371 (sparse/spmv_op/arch35/spmv_op_host.cpp:687-713) */
aclsparseStatus_t aclsparseSpMVOp_createPlan(aclsparseHandle_t handle, aclsparseSpMVOpDescr_t descr,
                                             aclsparseSpMVOpPlan_t* plan, const void* epilogueLTOBuffer,
                                             size_t epilogueLTOBufferSize);
/* replaces include/cann_ops_sparse.h:2380 (sparse/spmv_op/arch35/spmv_op_host.cpp:716-723) */
aclsparseStatus_t aclsparseSpMVOp_destroyPlan(aclsparseSpMVOpPlan_t plan);
/* replaces include/cann_ops_sparse.h:2386 (sparse/spmv_op/arch35/spmv_op_host.cpp:726-750) */
aclsparseStatus_t aclsparseSpMVOp_setGlobalUserData(aclsparseHandle_t handle, aclsparseSpMVOpPlan_t plan,
                                                    const char* epilogueDataName, void* epilogueData,
                                                    size_t epilogueDataSize);
/* replaces include/cann_ops_sparse.h:2394 (sparse/spmv_op/arch35/spmv_op_host.cpp:753-773) */
aclsparseStatus_t aclsparseSpMVOp(aclsparseHandle_t handle, aclsparseSpMVOpPlan_t plan, const void* alpha,
                                  const void* beta, aclsparseConstDnVecDescr_t vecX, aclsparseConstDnVecDescr_t vecY,
                                  aclsparseDnVecDescr_t vecZ);

/* ---------------- dense matrix descriptor (sparse/common/aclsparse_descr.cpp:1102-1302) ---------------- */

/* replaces include/cann_ops_sparse.h:1028 */
aclsparseStatus_t aclsparseCreateDnMat(aclsparseDnMatDescr_t* dnMatDescr, int64_t rows, int64_t cols, int64_t ld,
                                       void* values, aclDataType valueType, aclsparseOrder_t order);
/* replaces include/cann_ops_sparse.h:1036 */
aclsparseStatus_t aclsparseCreateConstDnMat(aclsparseConstDnMatDescr_t* dnMatDescr, int64_t rows, int64_t cols,
                                            int64_t ld, const void* values, aclDataType valueType,
                                            aclsparseOrder_t order);
/* replaces include/cann_ops_sparse.h:1045 */
aclsparseStatus_t aclsparseDestroyDnMat(aclsparseConstDnMatDescr_t dnMatDescr);
/* replaces include/cann_ops_sparse.h:1061 */
aclsparseStatus_t aclsparseDnMatGet(aclsparseDnMatDescr_t dnMatDescr, int64_t* rows, int64_t* cols, int64_t* ld,
                                    void** values, aclDataType* valueType, aclsparseOrder_t* order);
/* replaces include/cann_ops_sparse.h:1070 */
aclsparseStatus_t aclsparseConstDnMatGet(aclsparseConstDnMatDescr_t dnMatDescr, int64_t* rows, int64_t* cols,
                                         int64_t* ld, const void** values, aclDataType* valueType,
                                         aclsparseOrder_t* order);
/* replaces include/cann_ops_sparse.h:1081 */
aclsparseStatus_t aclsparseDnMatGetValues(aclsparseDnMatDescr_t dnMatDescr, void** values);
/* replaces include/cann_ops_sparse.h:1086 */
aclsparseStatus_t aclsparseConstDnMatGetValues(aclsparseConstDnMatDescr_t dnMatDescr, const void** values);
/* replaces include/cann_ops_sparse.h:1095 */
aclsparseStatus_t aclsparseDnMatSetValues(aclsparseDnMatDescr_t dnMatDescr, void* values);

/* ---------------- SpMMOp (include/cann_ops_sparse.h:2399-2497) ---------------- */

/* replaces include/cann_ops_sparse.h:2431 (sparse/spmm_op/arch35/spmm_op_host.cpp:695-740) */
aclsparseStatus_t aclsparseSpMMOp_bufferSize(aclsparseHandle_t handle, aclsparseOperation_t opA,
                                             aclsparseOperation_t opB, aclsparseConstSpMatDescr_t matA,
                                             aclsparseConstDnMatDescr_t matB, aclsparseDnMatDescr_t matC,
                                             aclDataType computeType, aclsparseSpMMOpAlg_t alg, size_t* bufferSize);
/* replaces include/cann_ops_sparse.h:2442 (sparse/spmm_op/arch35/spmm_op_host.cpp:961-1002) */
aclsparseStatus_t aclsparseSpMMOp_createDescr(aclsparseHandle_t handle, aclsparseSpMMOpDescr_t* descr,
                                              aclsparseOperation_t opA, aclsparseOperation_t opB,
                                              aclsparseConstSpMatDescr_t matA, aclsparseConstDnMatDescr_t matB,
                                              aclsparseDnMatDescr_t matC, aclDataType computeType,
                                              aclsparseSpMMOpAlg_t alg, void* buffer);
/* replaces include/cann_ops_sparse.h:2452 (sparse/spmm_op/arch35/spmm_op_host.cpp:1005-1012) */
aclsparseStatus_t aclsparseSpMMOp_destroyDescr(aclsparseSpMMOpDescr_t descr);
/* replaces include/cann_ops_sparse.h:2458 (sparse/spmm_op/arch35/spmm_op_host.cpp:1015-1043) */
aclsparseStatus_t aclsparseSpMMOp_createPlan(aclsparseHandle_t handle, aclsparseSpMMOpDescr_t descr,
                                             aclsparseSpMMOpPlan_t* plan, const void* epilogueLTOBuffer,
                                             size_t epilogueLTOBufferSize);
/* replaces include/cann_ops_sparse.h:2467 (sparse/spmm_op/arch35/spmm_op_host.cpp:1046-1053) */
aclsparseStatus_t aclsparseSpMMOp_destroyPlan(aclsparseSpMMOpPlan_t plan);
/* replaces include/cann_ops_sparse.h:2473 (sparse/spmm_op/arch35/spmm_op_host.cpp:1056-1080) */
aclsparseStatus_t aclsparseSpMMOp_setGlobalUserData(aclsparseHandle_t handle, aclsparseSpMMOpPlan_t plan,
                                                    const char* epilogueDataName, void* epilogueData,
                                                    size_t epilogueDataSize);
/* replaces include/cann_ops_sparse.h:2484 (sparse/spmm_op/arch35/spmm_op_host.cpp:1083-1102) */
aclsparseStatus_t aclsparseSpMMOp(aclsparseHandle_t handle, aclsparseSpMMOpPlan_t plan, const void* alpha,
                                  const void* beta, aclsparseConstDnMatDescr_t matB, aclsparseDnMatDescr_t matC);

#ifdef __cplusplus
}
#endif

#endif /* CANN_OPS_SPARSE_H_ */
