// aclsparseSpMVNoAlloc: aclsparseSpMV for callers that cannot allocate device
// memory (code under HIP graph capture, serving loops, harnesses that forbid
// allocation).  The reference has no such entry point.
//
// The SpMV workspace (header, normalised row offsets, row-block partition,
// task tables; for a transpose the CSC pattern and its sort storage) lives in
// `scratch`, a static device array of ACL_SPARSE_SPMV_NO_ALLOC_MAX_BYTES that
// every GPU the library runs on holds from the library's load to the end of
// the process.  In host code `scratch` names a host-side stand-in, not device
// memory: its device address is resolved with hipGetSymbolAddress once per
// device, with that device current, on the entry point's first call there,
// and only that address is passed to kernels.  No allocator is called.
//
// Every call rebuilds all tables it reads, so nothing in the array has to
// start at zero and what the previous call left there is never used.  Calls
// that overlap in time on one GPU share the array and race; the caller
// orders them (one stream, or events between streams).
#include <hip/hip_runtime.h>

#include <mutex>

#include "aclsparse_internal.h"
#include "cann_ops_sparse.h"

namespace {

constexpr size_t kScratchBytes = ACL_SPARSE_SPMV_NO_ALLOC_MAX_BYTES;
constexpr int kMaxDevices = 64;

__device__ __align__(256) uint8_t scratch[kScratchBytes];

std::mutex gScratchMutex;
void* gScratchPtr[kMaxDevices] = {};

// Device address of `scratch` on the current device (nullptr on failure).
void* ScratchOfCurrentDevice()
{
    int dev = -1;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return nullptr;
    std::lock_guard<std::mutex> lock(gScratchMutex);
    if (gScratchPtr[dev] == nullptr) {
        void* p = nullptr;
        if (hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)) != hipSuccess || p == nullptr) return nullptr;
        gScratchPtr[dev] = p;
    }
    return gScratchPtr[dev];
}

}  // namespace

extern "C" aclsparseStatus_t aclsparseSpMVNoAlloc(aclsparseHandle_t handle, aclsparseOperation_t opA,
                                                  const void* alpha, aclsparseConstSpMatDescr_t matA,
                                                  aclsparseConstDnVecDescr_t vecX, const void* beta,
                                                  aclsparseDnVecDescr_t vecY, aclDataType computeType,
                                                  aclsparseSpMVAlg_t alg)
{
    return aclsp::SpmvWithScratch(handle, opA, alpha, matA, vecX, beta, vecY, computeType, alg,
                                  ScratchOfCurrentDevice, kScratchBytes);
}
