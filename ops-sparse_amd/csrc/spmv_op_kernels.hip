// gfx950 kernels of aclsparseSpMVOp: Z = alpha*A*X + beta*Y (fp32) with a
// doubly compensated dot product per row.
//
// The reference runs one scalar thread per row with Priest's accumulator
// (TwoProduct by FMA + two TwoSum stages, sparse/spmv_op/arch35/spmv_op_kernel.cpp:87-128)
// and builds the ALG2 tables with one scalar thread (:425-540).  Here:
//  * ALG1 (no buffer): the SpMV stream kernel with the compensated
//    accumulator (SpmvOpStreamKernel in spmv_kernels.hip) on row blocks of a
//    fixed row count (about 500 non-zeros each) read straight from the
//    caller's row offsets.
//  * ALG2 (buffer): createDescr builds the reference's tables in parallel
//    (row lengths, a stable descending radix sort (hipCUB), an int64
//    inclusive scan, the bin edges by binary search plus the reference's
//    one-edge-per-row rule; reorder, scratch and bin_edge are bit-identical
//    to the reference's serial tables) and, after them, the SpMV row-block
//    partition; execution runs the SpMV stream kernel with the compensated
//    accumulator (SpmvOpStreamKernel in spmv_kernels.hip).
//  Summation orders depend only on the matrix: results are bit-reproducible
//  run to run.
#include <hip/hip_runtime.h>
#include <hipcub/hipcub.hpp>

#include <cstdint>

#include "aclsparse_internal.h"
#include "compensated.h"

// The error-free transformations below (TwoSum, TwoProduct) rely on every
// operation being rounded as written: no contraction of a*b + c into FMA.
#pragma clang fp contract(off)

namespace aclsp {
namespace {

constexpr int kThreads = 256;



struct OpParams {
    const void* rp;
    const int32_t* col;
    const float* val;
    const float* x;
    const float* y;
    float* z;
    int64_t m, n, nnz;
    int32_t base;
    float alpha, beta;
    const float* alpha_ptr;
    const float* beta_ptr;
    int32_t device_scalars;
};

__device__ __forceinline__ void Scalars(const OpParams& p, float& a, float& b)
{
    a = p.device_scalars ? *p.alpha_ptr : p.alpha;
    b = p.device_scalars ? *p.beta_ptr : p.beta;
}

// nnz == 0: Z = beta*Y; Y is not read when beta == 0.
__global__ __launch_bounds__(kThreads) void SpmvOpBetaYKernel(OpParams p)
{
    float a, b;
    Scalars(p, a, b);
    for (int64_t i = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x; i < p.m;
         i += static_cast<int64_t>(gridDim.x) * kThreads) {
        const float yv = b == 0.0f ? 0.0f : p.y[i];
        p.z[i] = b * yv;
    }
}

// ---------------------------- ALG2 preprocess -----------------------------

template <typename RowT>
__global__ __launch_bounds__(kThreads) void OpLengthsKernel(const RowT* rp, int64_t m, int32_t* len, int32_t* iota)
{
    for (int64_t i = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x; i < m;
         i += static_cast<int64_t>(gridDim.x) * kThreads) {
        len[i] = static_cast<int32_t>(rp[i + 1] - rp[i]);
        iota[i] = static_cast<int32_t>(i);
    }
}

__global__ __launch_bounds__(kThreads) void OpWidenKernel(const int32_t* sortedLen, int64_t m, int32_t* scratch,
                                                          int64_t* running)
{
    for (int64_t i = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x; i < m;
         i += static_cast<int64_t>(gridDim.x) * kThreads) {
        scratch[i] = sortedLen[i];
        running[i] = sortedLen[i];
    }
}

// bin_edge[b] for b in [1, bins): the first sorted position i whose running
// sum reaches b*ceil(total/bins), but never the same position as the
// previous edge (the reference advances one edge per row); edges past the
// last row are m (spmv_op_kernel.cpp:505-528).
__global__ __launch_bounds__(kThreads) void OpBinEdgeKernel(const int64_t* running, int64_t m, uint32_t bins,
                                                            int32_t* binEdge)
{
    __shared__ int64_t lb[kThreads + 1];
    const int64_t total = running[m - 1];
    const int64_t perBin = (total > 0 && bins > 0) ? (total + bins - 1) / bins : 0;
    for (uint32_t b = threadIdx.x + 1; b < bins; b += kThreads) {
        const int64_t target = perBin * static_cast<int64_t>(b);
        int64_t lo = 0, hi = m;
        while (lo < hi) {
            const int64_t mid = (lo + hi) >> 1;
            if (running[mid] >= target) hi = mid;
            else lo = mid + 1;
        }
        lb[b] = lo;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        binEdge[0] = 0;
        uint32_t b = 1;
        int64_t prev = -1;
        for (; b < bins; ++b) {
            const int64_t i = lb[b] > prev + 1 ? lb[b] : prev + 1;
            if (i >= m) break;
            binEdge[b] = static_cast<int32_t>(i + 1);
            prev = i;
        }
        for (; b <= bins; ++b) binEdge[b] = static_cast<int32_t>(m);
    }
}

int CuCount()
{
    int dev = 0, n = 0;
    if (hipGetDevice(&dev) != hipSuccess) return 256;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) return 256;
    return n;
}

size_t SortScanTempBytes(int64_t m)
{
    size_t sortBytes = 0, scanBytes = 0;
    const int items = static_cast<int>(m);
    if (hipcub::DeviceRadixSort::SortPairsDescending(nullptr, sortBytes, static_cast<int32_t*>(nullptr),
                                                     static_cast<int32_t*>(nullptr), static_cast<int32_t*>(nullptr),
                                                     static_cast<int32_t*>(nullptr), items) != hipSuccess) {
        sortBytes = static_cast<size_t>(m) * 16 + (1 << 20);
    }
    if (hipcub::DeviceScan::InclusiveSum(nullptr, scanBytes, static_cast<int64_t*>(nullptr),
                                         static_cast<int64_t*>(nullptr), items) != hipSuccess) {
        scanBytes = static_cast<size_t>(m) * 8 + (1 << 20);
    }
    return sortBytes > scanBytes ? sortBytes : scanBytes;
}

int GridFor(int64_t n)
{
    int64_t g = (n + kThreads - 1) / kThreads;
    return static_cast<int>(g < 1 ? 1 : g > 65536 ? 65536 : g);
}

}  // namespace

uint32_t SpmvOpNumBins(int64_t m)
{
    if (m <= 0) return 0;
    const int64_t need = (m + kOpRowsPerBin - 1) / kOpRowsPerBin;
    const int64_t cus = CuCount();
    const int64_t bins = need < cus ? need : cus;
    return static_cast<uint32_t>(bins < 1 ? 1 : bins);
}

SpmvOpLayout SpmvOpComputeLayout(int64_t m, int64_t n, int64_t nnz, aclsparseIndexType_t rowType, uint32_t bins)
{
    SpmvOpLayout l;
    const size_t rb = static_cast<size_t>(m) * sizeof(int32_t);
    l.reorder = kOpHeaderBytes;
    l.tmp_reorder = AlignUp(l.reorder + rb);
    l.scratch = AlignUp(l.tmp_reorder + rb);
    l.tmp_scratch = AlignUp(l.scratch + rb);
    l.bin_edge = AlignUp(l.tmp_scratch + rb);
    l.running = AlignUp(l.bin_edge + static_cast<size_t>(bins + 1) * sizeof(int32_t));
    l.temp = AlignUp(l.running + static_cast<size_t>(m) * sizeof(int64_t));
    l.temp_bytes = m > 0 ? SortScanTempBytes(m) : 0;
    l.spmv = AlignUp(l.temp + l.temp_bytes + 256);  // +256: the temp area is re-aligned to 256 bytes
    // (with the narrow column copy for matrices that can have one)
    l.sl = ComputeLayout(static_cast<uint64_t>(m), static_cast<uint64_t>(n), static_cast<uint64_t>(nnz), rowType,
                         ACL_FLOAT, false, false, 0U, true);
    l.total = AlignUp(l.spmv + l.sl.total);
    return l;
}

namespace {

SpmvOpLayout LayoutOf(const aclsparseSpMVOpDescr& d)
{
    return SpmvOpComputeLayout(static_cast<int64_t>(d.m), static_cast<int64_t>(d.n), static_cast<int64_t>(d.nnz),
                               d.row_type, d.num_bins);
}

// The SpMV launch description of the execution kernel's partition, which
// sits in the ALG2 buffer after the reference's tables.
SpmvLaunch OpLaunch(const aclsparseSpMVOpDescr& d, const SpmvOpLayout& l)
{
    SpmvLaunch sl{};
    sl.row_ptr = d.row_offsets;
    sl.row_stride = 1;
    sl.col = d.col_ind;
    sl.col_stride = 1;
    sl.val = d.values;
    sl.val_stride = 1;
    sl.x_stride = 1;
    sl.y_stride = 1;
    sl.rows = static_cast<int64_t>(d.m);
    sl.cols = static_cast<int64_t>(d.n);
    sl.nnz = static_cast<int64_t>(d.nnz);
    sl.base = d.base == ACL_SPARSE_INDEX_BASE_ONE ? 1 : 0;
    sl.rowptr64 = d.row_type == ACL_SPARSE_INDEX_64I ? 1 : 0;
    sl.val_kind = ValKind::F32;
    sl.out_kind = OutKind::F32;
    sl.acc_kind = AccKind::F32;
    sl.op = ACL_SPARSE_OP_NON_TRANSPOSE;
    sl.ws = static_cast<uint8_t*>(d.buffer) + l.spmv;
    sl.layout = l.sl;
    sl.staged_choice = -1;
    return sl;
}

bool Aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15U) == 0U; }

}  // namespace

// ALG2: the narrow column copy is built when the layout has it and the
// stream kernel reads these operands (16-byte aligned columns and values, x
// addressable with 32-bit byte offsets).
bool SpmvOpNarrowUsable(const aclsparseSpMVOpDescr& d)
{
    return d.alg == ACL_SPARSE_SPMVOP_ALG2 && LayoutOf(d).sl.narrow && d.col_ind != nullptr && d.values != nullptr &&
           Aligned16(d.col_ind) && Aligned16(d.values) && d.nnz >= 4 && d.n * 4ULL <= 0x7FFFFFFFULL;
}

void* SpmvOpSpmvWorkspace(const aclsparseSpMVOpDescr& d)
{
    return static_cast<uint8_t*>(d.buffer) + LayoutOf(d).spmv;
}

namespace {


}  // namespace

int LaunchLengthTables(const LengthTables& t, void* stream)
{
    const int64_t m = t.m;
    if (m <= 0) return 0;
    hipStream_t s = static_cast<hipStream_t>(stream);
    if (t.rowptr64) {
        hipLaunchKernelGGL(OpLengthsKernel<int64_t>, dim3(GridFor(m)), dim3(kThreads), 0, s,
                           static_cast<const int64_t*>(t.row_offsets), m, t.scratch, t.tmp_reorder);
    } else {
        hipLaunchKernelGGL(OpLengthsKernel<int32_t>, dim3(GridFor(m)), dim3(kThreads), 0, s,
                           static_cast<const int32_t*>(t.row_offsets), m, t.scratch, t.tmp_reorder);
    }
    // device sort/scan temporary storage, aligned to 256 bytes in absolute terms
    void* temp = reinterpret_cast<void*>((reinterpret_cast<uintptr_t>(t.temp) + 255) & ~uintptr_t{255});
    size_t tempBytes = t.temp_bytes;
    // Stable: equal lengths keep ascending row order, as the reference's
    // merge that takes the left run on ties.
    if (hipcub::DeviceRadixSort::SortPairsDescending(temp, tempBytes, t.scratch, t.tmp_scratch, t.tmp_reorder,
                                                     t.reorder, static_cast<int>(m), 0, 32, s) != hipSuccess) {
        return 1;
    }
    hipLaunchKernelGGL(OpWidenKernel, dim3(GridFor(m)), dim3(kThreads), 0, s, t.tmp_scratch, m, t.scratch, t.running);
    tempBytes = t.temp_bytes;
    if (hipcub::DeviceScan::InclusiveSum(temp, tempBytes, t.running, t.running, static_cast<int>(m), s) != hipSuccess) {
        return 1;
    }
    hipLaunchKernelGGL(OpBinEdgeKernel, dim3(1), dim3(kThreads), 0, s, t.running, m, t.bins, t.bin_edge);
    return 0;
}

SpmmOpLayout SpmmOpComputeLayout(int64_t m, uint32_t bins)
{
    SpmmOpLayout l;
    const size_t rb = static_cast<size_t>(m) * sizeof(int32_t);
    l.reorder = kOpHeaderBytes;
    l.bin_edge = AlignUp(l.reorder + rb);
    l.ref_total = AlignUp(l.bin_edge + static_cast<size_t>(bins + 1) * sizeof(int32_t));
    l.tmp_reorder = l.ref_total;
    l.scratch = AlignUp(l.tmp_reorder + rb);
    l.tmp_scratch = AlignUp(l.scratch + rb);
    l.running = AlignUp(l.tmp_scratch + rb);
    l.temp = AlignUp(l.running + static_cast<size_t>(m) * sizeof(int64_t));
    l.temp_bytes = m > 0 ? SortScanTempBytes(m) : 0;
    l.total = AlignUp(l.temp + l.temp_bytes + 256);  // +256: the temp area is re-aligned to 256 bytes
    return l;
}

int LaunchSpmvOpPreprocess(const aclsparseSpMVOpDescr& d, void* stream)
{
    const int64_t m = static_cast<int64_t>(d.m);
    if (m <= 0) return 0;
    const SpmvOpLayout l = LayoutOf(d);
    uint8_t* ws = static_cast<uint8_t*>(d.buffer);
    LengthTables t{};
    t.row_offsets = d.row_offsets;
    t.rowptr64 = d.row_type == ACL_SPARSE_INDEX_64I;
    t.m = m;
    t.bins = d.num_bins;
    t.reorder = reinterpret_cast<int32_t*>(ws + l.reorder);
    t.tmp_reorder = reinterpret_cast<int32_t*>(ws + l.tmp_reorder);
    t.scratch = reinterpret_cast<int32_t*>(ws + l.scratch);
    t.tmp_scratch = reinterpret_cast<int32_t*>(ws + l.tmp_scratch);
    t.bin_edge = reinterpret_cast<int32_t*>(ws + l.bin_edge);
    t.running = reinterpret_cast<int64_t*>(ws + l.running);
    t.temp = ws + l.temp;
    t.temp_bytes = l.temp_bytes;
    if (LaunchLengthTables(t, stream) != 0) return 1;
    // the execution kernel's row-block partition (and the narrow column copy)
    SpmvLaunch sl = OpLaunch(d, l);
    sl.narrow = d.narrow ? 1 : 0;
    return LaunchSpmvPreprocess(sl, stream);
}

int LaunchSpmvOpExecute(const aclsparseSpMVOpDescr& d, const void* x, const void* y, void* z, float alpha,
                        float beta, const void* alphaPtr, const void* betaPtr, bool deviceScalars, void* stream)
{
    hipStream_t s = static_cast<hipStream_t>(stream);
    OpParams p{};
    p.rp = d.row_offsets;
    p.col = d.col_ind;
    p.val = d.values;
    p.x = static_cast<const float*>(x);
    p.y = static_cast<const float*>(y);
    p.z = static_cast<float*>(z);
    p.m = static_cast<int64_t>(d.m);
    p.n = static_cast<int64_t>(d.n);
    p.nnz = static_cast<int64_t>(d.nnz);
    p.base = d.base == ACL_SPARSE_INDEX_BASE_ONE ? 1 : 0;
    p.alpha = alpha;
    p.beta = beta;
    p.alpha_ptr = static_cast<const float*>(alphaPtr);
    p.beta_ptr = static_cast<const float*>(betaPtr);
    p.device_scalars = deviceScalars ? 1 : 0;
    if (p.nnz == 0) {
        hipLaunchKernelGGL(SpmvOpBetaYKernel, dim3(GridFor(p.m)), dim3(kThreads), 0, s, p);
        return 0;
    }
    const bool i64 = d.row_type == ACL_SPARSE_INDEX_64I;
    if (d.alg == ACL_SPARSE_SPMVOP_ALG2) {
        // ALG2 has a buffer: it runs on the row-block partition that
        // createDescr built there, with the stream kernel's coalesced chunk
        // loads (the length-sorted tables are the reference's load balance
        // for its cores; the merge-path row blocks balance any row-length
        // distribution without them).
        SpmvLaunch sl = OpLaunch(d, LayoutOf(d));
        sl.narrow = d.narrow ? 1 : 0;
        sl.staged_choice = d.narrow ? QueryPathChoice(d.choice, stream) : -1;
        sl.x = x;
        sl.y = const_cast<void*>(y);
        sl.device_scalars = deviceScalars ? 1 : 0;
        sl.alpha_re = alpha;
        sl.beta_re = beta;
        sl.alpha_ptr = alphaPtr;
        sl.beta_ptr = betaPtr;
        return LaunchSpmvOpStream(sl, static_cast<float*>(z), stream);
    }
    // ALG1 has no buffer: the stream kernel on fixed-size row blocks read
    // straight from the caller's row offsets.
    {
        SpmvLaunch sl{};
        sl.row_ptr = d.row_offsets;
        sl.col = d.col_ind;
        sl.val = d.values;
        sl.x = x;
        sl.y = const_cast<void*>(y);
        sl.rows = p.m;
        sl.cols = p.n;
        sl.nnz = p.nnz;
        sl.base = p.base;
        sl.rowptr64 = i64 ? 1 : 0;
        sl.device_scalars = deviceScalars ? 1 : 0;
        sl.alpha_re = alpha;
        sl.beta_re = beta;
        sl.alpha_ptr = alphaPtr;
        sl.beta_ptr = betaPtr;
        return LaunchSpmvOpStreamFixed(sl, static_cast<float*>(z), stream);
    }
}

}  // namespace aclsp
