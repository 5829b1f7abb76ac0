// Staged-gather SpMV on gfx950: y = alpha*A*x + beta*y for matrices whose x
// does not fit an XCD's L2 and whose columns are scattered.
//
// The row kernels (spmv_kernels.hip) gather x[col] straight from memory: for
// a random column pattern over a 33.5 MB x every 2- or 4-byte value costs a
// 128-byte line from the MALL, and the gathers cap the kernel at the MALL's
// line rate (about 64 G lines/s), 5% of HBM bandwidth.  This path moves the
// same data with streaming accesses only:
//
//  * Preprocess (pattern only; values, x and y may change between calls, the
//    reference's contract, sparse/spmv/README.md aclsparseSpMVPreprocess):
//    merge-path tiles of kStageTileItems rows+entries; every entry goes to the
//    bucket of its column's x segment (128 KiB of x); per tile, a stable
//    counting rank by bucket (StageRankKernel) gives each entry its slot in the
//    tile's bucket-ordered runs (st_perm) and, in bucket order, its column
//    within the bucket (st_cl).  A per-tile estimate of the distinct x lines
//    decides the path: when the lines are few (banded matrices) the row
//    kernels keep the matrix.
//  * Pass A (StageGatherKernel), one workgroup per slice of the bucket-ordered
//    slots: loads the slice's x segment into LDS (128 KiB) and writes
//    xg[j] = segment[cl[j]]: a sequential read of cl and a sequential write.
//  * Pass B (StageTileKernel), one workgroup per tile: copies the tile's run
//    of every bucket from xg into LDS (runs of neighbouring tiles are
//    adjacent, so their lines are shared through L2; a bit map of run starts
//    gives every slot its run without a search), multiplies each value a_k
//    (CSR order, coalesced) by its staged x value, and sums the tile's rows
//    from LDS: short rows one thread each, long rows a wave each.  Rows
//    crossing tile ends leave partial sums (st_head / st_tail).  The kernel
//    is bound by instruction issue as much as by memory, so the per-slot
//    and per-entry work is kept to a few integer operations.
//  * Fix-up (StageFixupKernel): one thread per tile whose first row ends in
//    it combines that row's partial sums in tile order.
//
// Every row is summed in an order fixed by the pattern, so results are
// reproducible bit for bit.  Reference counterpart of the whole path: the
// warp-per-row kernels of sparse/spmv/arch35/spmv_kernel.cpp:501-577, which
// gather x from global memory.
#include <hip/hip_runtime.h>
#include <hipcub/hipcub.hpp>

#include <cstdint>
#include <type_traits>

#include "aclsparse_internal.h"
#include "spmv_device.h"

namespace aclsp {
namespace {

using namespace dev;

constexpr int kXcds = 8;
constexpr int kWave = 64;
constexpr int kSortThreads = 512;                       // per-tile preprocess kernels
constexpr int kTileThreads = 512;                       // pass B (768 and 1024 measured no faster)
constexpr int kTileWaves = kTileThreads / kWave;
constexpr int kGatherThreads = 1024;                    // pass A
constexpr int kGatherBatch = 4;                         // pass A: groups of 8 slots per thread per round
constexpr int kLongRow = 32;                            // in-tile rows longer than this are summed by a wave
constexpr int CeilDiv(int a, int b) { return (a + b - 1) / b; }
constexpr int kScanIpt = CeilDiv(kStageMaxBuckets + 1, kTileThreads);         // run lengths per thread
constexpr int kNarrow = static_cast<int>(kStageTileItemsNarrow);
constexpr int kWide = static_cast<int>(kStageTileItemsWide);

// Per-tile shapes of a tile of kItems rows + entries.
template <int kItems>
struct Tile {
    static constexpr int kMaxLong = kItems / kLongRow + 1;                          // long rows of a tile
    static constexpr int kGroupSlots = CeilDiv((kItems + 3) / 4 + 1, kTileThreads);  // groups of 4 entries per thread
    static constexpr int kStageLanes = CeilDiv(kItems, kTileThreads);               // 64-slot windows per wave
    static constexpr int kWindows = (kItems + 63) / 64;                             // 64-slot windows of a tile
    static_assert(kTileWaves * kStageLanes * kWave >= kItems, "staging capacity");
    static_assert(kItems + 7 * (kStageMaxBuckets + 1) < 65536, "uint16 slot numbers");
};

struct StageParams {
    const void* norm;  // normalised row offsets, RowT[rows+2]
    const int32_t* col;
    int32_t base;
    int32_t buckets;  // S; bucket S collects columns outside [0, cols)
    int32_t wshift;   // log2 of the columns per bucket
    int32_t line_shift;  // log2 of the x values per 128-byte line
    const void* val;
    const void* x;
    void* y;
    int64_t rows, cols, nnz;
    int64_t tiles;  // T
    int64_t tile_items;  // rows + entries per tile
    int32_t* tile_row;
    int64_t* tile_nnz;
    uint32_t* counts;
    uint32_t* start_bm;
    uint32_t* start;
    uint16_t* perm;
    uint16_t* cl;
    void* xg;
    float* head;
    float* tail;
    unsigned long long* metric;
    uint32_t* flag;
    const uint16_t* rp16;  // low 16 bits of the normalised row offsets (the narrow copy's), or null
    int64_t part;  // pass A: bucket-ordered slots per workgroup
    int32_t chunk; // staged slots per 8-byte chunk: runs are padded to a multiple
    int32_t banded_ok;  // bucketed transpose: the one-pass banded kernel exists for this matrix
    // column-bucketed transpose
    const void* colptr;   // RowT[cols+1], column offsets of the CSC pattern
    const void* csc_pos;  // RowT[nnz], CSR index of each entry in column order
    int32_t* inv;         // int32[nnz], column-order place of each CSR entry, then (after
                          // the sort) csc_row: the row of each entry in column order
    const int32_t* entry_row;  // int32[nnz], the row of each entry in CSR order
    float* prod;          // float[nnz+8], products in bucket order
    Scalars s;
};

// Workgroup -> tile of pass B (and slice of pass A): tiles in chunks of
// kTileChunk per XCD, the chunks dealt to the XCDs round-robin, so that the
// tiles in flight at any time are consecutive over the whole chip (their
// staged runs lie close together in every bucket of xg, which HBM serves
// better than eight separate stretches), while neighbouring tiles, whose
// runs share cache lines, mostly stay on one XCD.  The grid is a multiple of
// 8; a last, partial round is split evenly over the XCDs.
constexpr int64_t kTileChunk = 32;
__device__ __forceinline__ int64_t ChunkedXcdIndex()
{
    constexpr int64_t kRound = kXcds * kTileChunk;
    const int64_t bx = blockIdx.x;
    const int64_t r0 = bx / kRound * kRound;
    const int64_t per = r0 + kRound <= static_cast<int64_t>(gridDim.x) ? kTileChunk
                                                                      : (static_cast<int64_t>(gridDim.x) - r0) / kXcds;
    const int64_t within = bx - r0;
    return r0 + (within % kXcds) * per + within / kXcds;
}

__device__ __forceinline__ uint32_t FlagSet(const uint32_t* flag)
{
    typedef const __attribute__((address_space(4))) uint32_t* CPtr;  // scalar load: written by Preprocess
    return *reinterpret_cast<CPtr>(reinterpret_cast<uintptr_t>(flag));
}

template <typename RowT>
__device__ __forceinline__ int64_t Norm(const StageParams& q, int64_t i)
{
    return static_cast<int64_t>(static_cast<const RowT*>(q.norm)[i]);
}

// Sort key of an entry: its column (bucket = key >> wshift), or the first
// column of the bucket S when the column is outside the matrix.
__device__ __forceinline__ uint32_t KeyOf(const StageParams& q, int32_t rawCol)
{
    const int64_t c = static_cast<int64_t>(rawCol) - q.base;
    if (c < 0 || c >= q.cols) return static_cast<uint32_t>(q.buckets) << q.wshift;
    return static_cast<uint32_t>(c);
}

// ------------------------------- preprocess ---------------------------------

// Corner (row, entry) of every tile on the merge path of row ends and
// entries (Merrill & Garland, SC'16): tile t starts at diagonal t*tile_items.
template <typename RowT>
__global__ __launch_bounds__(256) void StageTileSplitKernel(StageParams q)
{
    const int64_t t = blockIdx.x * int64_t{256} + threadIdx.x;
    if (t == 0) *q.metric = 0ULL;
    if (t > q.tiles) return;
    const int64_t total = q.rows + q.nnz;
    const int64_t d = t * q.tile_items < total ? t * q.tile_items : total;
    int64_t lo = d - q.nnz > 0 ? d - q.nnz : 0;
    int64_t hi = d < q.rows ? d : q.rows;
    while (lo < hi) {
        const int64_t mid = (lo + hi) >> 1;
        if (Norm<RowT>(q, mid + 1) <= d - 1 - mid) lo = mid + 1;
        else hi = mid;
    }
    q.tile_row[t] = static_cast<int32_t>(lo);
    q.tile_nnz[t] = d - lo;
}

// A tile's column indices (entries e0 .. e0+n-1, n at most the wide tile's
// items) by 16-byte buffer loads of 4 from any 4-byte boundary, all issued
// before the first is used: thread tid holds entries (u*kSortThreads+tid)*4
// .. +3 in raw[u] (zero past the array's end; entries past n are the next
// tile's, which the caller skips).
constexpr int kColGroups = CeilDiv(static_cast<int>(kStageTileItemsWide), 4 * kSortThreads);
__device__ __forceinline__ uint32_t WordOf(const uint4& v, int i)
{
    return i == 0 ? v.x : i == 1 ? v.y : i == 2 ? v.z : v.w;
}
__device__ __forceinline__ void LoadTileCols(const StageParams& q, int64_t e0, int n, uint4 (&raw)[kColGroups])
{
    const int64_t cBytes = (q.nnz - e0) * 4;
    const __amdgpu_buffer_rsrc_t rc = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<int32_t*>(q.col + e0), 0, static_cast<int>(cBytes < 0x7FFFFFFFLL ? cBytes : 0x7FFFFFFFLL),
        0x00020000);
#pragma unroll
    for (int u = 0; u < kColGroups; ++u) {
        if (u * 4 * kSortThreads >= n) break;  // uniform over the workgroup
        const int i = (u * kSortThreads + static_cast<int>(threadIdx.x)) * 4;
        raw[u] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(rc, i * 4, 0, 0));
    }
    asm volatile("" ::: "memory");
}

// counts[s*(T+1) + t] = staged slots of tile t in bucket s: its entries,
// padded to a multiple of q.chunk (column T is zero).  Also the path
// decision's metric: the tile's distinct x lines, estimated by linear
// counting over a 2^15-bit LDS bitmap of hashed lines (order-independent,
// hence the same on every run), added to q.metric.  The decision follows
// this kernel, so a matrix that keeps the row kernels skips the rest.
constexpr int kMapBits = 1 << 15;
constexpr int kMapWords = kMapBits / 32;
__global__ __launch_bounds__(kSortThreads) void StageCountKernel(StageParams q)
{
    __shared__ uint32_t hist[kStageMaxBuckets + 1];
    __shared__ uint32_t map[kMapWords];
    __shared__ uint32_t mapSet;
    const int64_t t = blockIdx.x;
    const int nb = q.buckets + 1;
    for (int s = threadIdx.x; s < nb; s += kSortThreads) hist[s] = 0U;
    for (int i = threadIdx.x; i < kMapWords; i += kSortThreads) map[i] = 0U;
    if (threadIdx.x == 0) mapSet = 0U;
    __syncthreads();
    int n = 0;
    if (t < q.tiles) {
        // all of the tile's column indices in one round trip (16-byte loads of
        // 4), then the atomics
        const int64_t e0 = q.tile_nnz[t], e1 = q.tile_nnz[t + 1];
        n = static_cast<int>(e1 - e0);
        uint4 raw[kColGroups];
        LoadTileCols(q, e0, n, raw);
        const uint32_t nullBucket = static_cast<uint32_t>(q.buckets);
        // Banded tiles put most of their entries in one bucket and many on the
        // same x lines: a group of 4 whose entries share a bucket counts once,
        // and an entry on the same line as the one before it sets no bit, so
        // that fewer LDS atomics pile up on one address.
#pragma unroll
        for (int u = 0; u < kColGroups; ++u) {
            if (u * 4 * kSortThreads >= n) break;  // uniform
            const int i = (u * kSortThreads + static_cast<int>(threadIdx.x)) * 4;
            uint32_t key[4];
#pragma unroll
            for (int k = 0; k < 4; ++k) key[k] = KeyOf(q, static_cast<int32_t>(WordOf(raw[u], k)));
            const uint32_t b0 = key[0] >> q.wshift;
            const bool whole = i + 4 <= n && (key[1] >> q.wshift) == b0 && (key[2] >> q.wshift) == b0 &&
                               (key[3] >> q.wshift) == b0;
            if (whole) {
                atomicAdd(&hist[b0], 4U);
            } else {
#pragma unroll
                for (int k = 0; k < 4; ++k) {
                    if (i + k < n) atomicAdd(&hist[key[k] >> q.wshift], 1U);
                }
            }
            uint32_t prevLine = 0xFFFFFFFFU;
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                const uint32_t line = key[k] >> q.line_shift;
                if (i + k < n && (key[k] >> q.wshift) != nullBucket && line != prevLine) {
                    const uint32_t h = (line * 2654435761U) >> 17;
                    atomicOr(&map[h >> 5], 1U << (h & 31U));
                }
                prevLine = line;
            }
        }
    }
    __syncthreads();
    {
        uint32_t z = 0U;
        for (int i = threadIdx.x; i < kMapWords; i += kSortThreads) z += static_cast<uint32_t>(__builtin_popcount(map[i]));
        if (z != 0U) atomicAdd(&mapSet, z);
    }
    // padded to whole 8-byte chunks of staged x
    const uint32_t m = static_cast<uint32_t>(q.chunk) - 1U;
    for (int s = threadIdx.x; s < nb; s += kSortThreads) q.counts[s * (q.tiles + 1) + t] = (hist[s] + m) & ~m;
    __syncthreads();
    if (threadIdx.x == 0 && t < q.tiles) {
        const uint32_t z = mapSet;
        const double mb = static_cast<double>(kMapBits);
        const double est = z >= static_cast<uint32_t>(kMapBits) ? static_cast<double>(n)
                                                                  : -mb * log1p(-static_cast<double>(z) / mb);
        const unsigned long long lines = static_cast<unsigned long long>(est + 0.5);
        if (lines != 0ULL) atomicAdd(q.metric, lines);
    }
}

// start[t*(S+1) + s] = start_bm[s*(T+1) + t].
__global__ __launch_bounds__(256) void StageTransposeKernel(StageParams q)
{
    __shared__ uint32_t tile[32][33];
    const int64_t nt = q.tiles + 1;
    const int nb = q.buckets + 1;
    const int64_t t0 = blockIdx.x * int64_t{32};
    const int s0 = blockIdx.y * 32;
    for (int i = threadIdx.y; i < 32; i += 8) {
        const int s = s0 + i;
        const int64_t t = t0 + threadIdx.x;
        if (s < nb && t < nt) tile[i][threadIdx.x] = q.start_bm[s * nt + t];
    }
    __syncthreads();
    for (int i = threadIdx.y; i < 32; i += 8) {
        const int64_t t = t0 + i;
        const int s = s0 + threadIdx.x;
        if (s < nb && t < nt) q.start[t * nb + s] = tile[threadIdx.x][i];
    }
}

// Per tile, without a sort: every entry's slot in the tile's bucket-ordered
// runs (st_perm) and, in bucket order, its column within the bucket (st_cl).
// Each entry takes the next place of its bucket's run with an LDS atomic, so
// the order of the entries inside a run is the order the atomics landed in.
// That order is free: pass A fills each slot from its own column and pass B
// looks each entry's x value up by its own slot, while every row is still
// summed in CSR order, so SpMV results do not depend on it.  The columns are
// placed at their slots in LDS (run padding stays zero) and every run is
// copied out whole.  Runs only when the path decision chose the staged
// kernels.
template <int kItems, int kThr>
__global__ __launch_bounds__(kThr) void StageRankKernel(StageParams q)
{
    static_assert(kThr == kSortThreads, "the column loads assume kSortThreads threads");
    static_assert(kItems <= kColGroups * 4 * kSortThreads, "a tile's entries fit the column loads");
    constexpr int kNb = kStageMaxBuckets + 1;
    constexpr int kMaxChunk = static_cast<int>(kStageChunkBytes) / 2;  // slots per chunk, at most (2-byte x)
    constexpr int kSlotCap = kItems + (kMaxChunk - 1) * kNb;           // padded slots of a tile
    constexpr int kStageWords = (kSlotCap + 1) / 2;
    constexpr int kRunIpt = CeilDiv(kNb, kThr);
    using Scan = hipcub::BlockScan<uint32_t, kThr>;
    __shared__ uint32_t stagedW[kStageWords];
    __shared__ uint32_t cnt[kNb];       // next place in each bucket's run
    __shared__ uint32_t padOff[kNb + 1];
    __shared__ uint32_t runStart[kNb];  // first st_cl slot of each bucket's run of this tile
    __shared__ typename Scan::TempStorage scanStorage;
    uint16_t* staged = reinterpret_cast<uint16_t*>(stagedW);

    if (FlagSet(q.flag) != 1U) return;
    const int64_t t = blockIdx.x;
    const int tid = threadIdx.x;
    const int64_t e0 = q.tile_nnz[t], e1 = q.tile_nnz[t + 1];
    const int n = static_cast<int>(e1 - e0);
    const int nb = q.buckets + 1;
    const uint32_t* startRow = q.start + t * nb;  // first slot of each bucket's run: this tile, then the next

    // the tile's run offsets in padded slots (run lengths from two tile-major rows of the scan)
    uint32_t pc[kRunIpt];
#pragma unroll
    for (int u = 0; u < kRunIpt; ++u) {
        const int sb = tid * kRunIpt + u;
        const uint32_t a = sb < nb ? startRow[sb] : 0U;
        pc[u] = sb < nb ? startRow[nb + sb] - a : 0U;
        if (sb < nb) runStart[sb] = a;
    }
    uint32_t total;
    Scan(scanStorage).ExclusiveSum(pc, pc, total);
#pragma unroll
    for (int u = 0; u < kRunIpt; ++u) {
        const int sb = tid * kRunIpt + u;
        if (sb < nb) {
            padOff[sb] = pc[u];
            cnt[sb] = pc[u];
        }
    }
    if (tid == 0) padOff[nb] = total;
    for (int i = tid; i < kStageWords; i += kThr) stagedW[i] = 0U;
    __syncthreads();

    const uint32_t nullBucket = static_cast<uint32_t>(q.buckets);
    const uint32_t inMask = (1U << q.wshift) - 1U;
    // the tile's column indices in one round trip, then per entry its slot
    uint4 raw[kColGroups];
    LoadTileCols(q, e0, n, raw);
#pragma unroll
    for (int u = 0; u < kColGroups; ++u) {
        if (u * 4 * kThr >= n) break;  // uniform
        const int i4 = (u * kThr + tid) * 4;
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const int i = i4 + k;
            if (i < n) {
                const uint32_t key = KeyOf(q, static_cast<int32_t>(WordOf(raw[u], k)));
                const uint32_t b = key >> q.wshift;
                const uint32_t slot = atomicAdd(&cnt[b], 1U);
                q.perm[e0 + i] = static_cast<uint16_t>(slot);
                if (b != nullBucket) staged[slot] = static_cast<uint16_t>(key & inMask);
            }
        }
    }
    __syncthreads();
    // every run out whole, two slots per store (runs and their starts are
    // padded to whole chunks of at least two slots), one wave per bucket
    const int lane = tid & (kWave - 1);
    for (int sb = tid / kWave; sb < nb; sb += kThr / kWave) {
        const uint32_t a = padOff[sb], len = padOff[sb + 1] - a;
        uint32_t* dst = reinterpret_cast<uint32_t*>(q.cl + runStart[sb]);
        const uint32_t* src = stagedW + a / 2;
        for (uint32_t j = lane; j < len / 2; j += kWave) dst[j] = src[j];
    }
}

// The path decision: staged when the tiles' distinct x lines exceed
// nnz / kStageLinesPerEntryDen.
__global__ void StageDecideKernel(StageParams q)
{
    const unsigned long long lines = *q.metric;
    *q.flag = lines * static_cast<unsigned long long>(kStageLinesPerEntryDen) >
                      static_cast<unsigned long long>(q.nnz)
                  ? 1U
                  : 0U;
}

// --------------------------------- pass A -----------------------------------

template <typename XT>
__device__ __forceinline__ void StoreGroup(XT* dst, const XT (&o)[8]);

template <>
__device__ __forceinline__ void StoreGroup<uint16_t>(uint16_t* dst, const uint16_t (&o)[8])
{
    uint4 v;
    v.x = static_cast<uint32_t>(o[0]) | (static_cast<uint32_t>(o[1]) << 16);
    v.y = static_cast<uint32_t>(o[2]) | (static_cast<uint32_t>(o[3]) << 16);
    v.z = static_cast<uint32_t>(o[4]) | (static_cast<uint32_t>(o[5]) << 16);
    v.w = static_cast<uint32_t>(o[6]) | (static_cast<uint32_t>(o[7]) << 16);
    *reinterpret_cast<uint4*>(dst) = v;
}

template <>
__device__ __forceinline__ void StoreGroup<uint32_t>(uint32_t* dst, const uint32_t (&o)[8])
{
    reinterpret_cast<uint4*>(dst)[0] = make_uint4(o[0], o[1], o[2], o[3]);
    reinterpret_cast<uint4*>(dst)[1] = make_uint4(o[4], o[5], o[6], o[7]);
}

// Workgroup w fills the bucket-ordered slots [w*part, (w+1)*part): for every
// bucket overlapping them, the bucket's x segment is loaded into LDS and each
// slot j gets xg[j] = segment[cl[j]] (0 for the out-of-range bucket).  XT is
// the raw x element (uint16_t for fp16 / bf16, uint32_t for fp32).
template <typename XT>
__global__ __launch_bounds__(kGatherThreads) void StageGatherKernel(StageParams q)
{
    extern __shared__ uint4 segRaw[];
    XT* seg = reinterpret_cast<XT*>(segRaw);
    if (FlagSet(q.flag) != 1U) return;
    const int64_t w = ChunkedXcdIndex();
    const int nb = q.buckets + 1;
    const uint32_t* base = q.start;                  // row 0: first slot of every bucket
    const uint32_t* ends = q.start + q.tiles * nb;   // row T: end of every bucket
    const int64_t total = ends[nb - 1];              // staged slots, padding included
    const int64_t a = w * q.part;
    if (a >= total) return;
    const int64_t b = a + q.part < total ? a + q.part : total;
    // first bucket that ends after a
    int lo = 0, hi = nb - 1;
    while (lo < hi) {
        const int mid = (lo + hi) >> 1;
        if (static_cast<int64_t>(ends[mid]) <= a) lo = mid + 1;
        else hi = mid;
    }
    const int64_t segLen = int64_t{1} << q.wshift;
    const XT* x = static_cast<const XT*>(q.x);
    XT* xg = static_cast<XT*>(q.xg);
    constexpr int kVec = 16 / sizeof(XT);
    for (int s = lo; s < nb; ++s) {
        const int64_t sb = base[s], se = ends[s];
        if (sb >= b) break;
        const int64_t j0 = sb > a ? sb : a;
        const int64_t j1 = se < b ? se : b;
        if (j0 >= j1) continue;
        const bool real = s < q.buckets;
        if (real) {
            const int64_t c0 = static_cast<int64_t>(s) << q.wshift;
            const int64_t n = q.cols - c0 < segLen ? q.cols - c0 : segLen;
            const int64_t nv = n / kVec;
            // the segment in one round trip: all of a thread's 16-byte loads,
            // then its LDS stores
            constexpr int kSegIters = static_cast<int>(kStageSegmentBytes) / 16 / kGatherThreads;
            const uint4* xs = reinterpret_cast<const uint4*>(x + c0);
            uint4 sv[kSegIters];
#pragma unroll
            for (int it = 0; it < kSegIters; ++it) {
                const int64_t i = it * kGatherThreads + threadIdx.x;
                sv[it] = i < nv ? xs[i] : uint4{};
            }
#pragma unroll
            for (int it = 0; it < kSegIters; ++it) {
                const int64_t i = it * kGatherThreads + threadIdx.x;
                if (i < nv) segRaw[i] = sv[it];
            }
            for (int64_t i = nv * kVec + threadIdx.x; i < n; i += kGatherThreads) seg[i] = x[c0 + i];
            __syncthreads();
        }
        // groups of 8 slots, kGatherBatch groups per thread per round: the
        // round's column loads are all issued before its first LDS read
        const int64_t gEnd = (j1 + 7) >> 3;
        for (int64_t g0 = (j0 >> 3) + threadIdx.x; g0 < gEnd; g0 += kGatherBatch * kGatherThreads) {
            uint4 c[kGatherBatch];
#pragma unroll
            for (int u = 0; u < kGatherBatch; ++u) {
                const int64_t g = g0 + u * kGatherThreads;
                c[u] = *reinterpret_cast<const uint4*>(q.cl + (g < gEnd ? g : g0) * 8);
            }
            asm volatile("" ::: "memory");
#pragma unroll
            for (int u = 0; u < kGatherBatch; ++u) {
                const int64_t g = g0 + u * kGatherThreads;
                const uint32_t cw[4] = {c[u].x, c[u].y, c[u].z, c[u].w};
                XT o[8];
#pragma unroll
                for (int k = 0; k < 8; ++k) {
                    const uint32_t ci = (cw[k >> 1] >> ((k & 1) * 16)) & 0xFFFFU;
                    o[k] = real ? seg[ci] : XT{0};
                }
                const int64_t j = g * 8;
                if (g >= gEnd) continue;
                if (j >= j0 && j + 8 <= j1) {
                    StoreGroup<XT>(xg + j, o);
                } else {
                    for (int k = 0; k < 8; ++k) {
                        if (j + k >= j0 && j + k < j1) xg[j + k] = o[k];
                    }
                }
            }
        }
        __syncthreads();
    }
}

// --------------------------------- pass B -----------------------------------

template <ValKind V>
struct StageVal;
template <>
struct StageVal<ValKind::F32> {
    using Raw = uint32_t;
    using Group = uint4;  // 4 values
    __device__ static float ToF(uint32_t r) { return __uint_as_float(r); }
    __device__ static uint32_t Get(const uint4& g, int u) { return u == 0 ? g.x : u == 1 ? g.y : u == 2 ? g.z : g.w; }
};
template <>
struct StageVal<ValKind::F16> {
    using Raw = uint16_t;
    using Group = uint2;
    __device__ static float ToF(uint16_t r) { return HalfToFloat(r); }
    __device__ static uint16_t Get(const uint2& g, int u)
    {
        const uint32_t w = u < 2 ? g.x : g.y;
        return static_cast<uint16_t>(w >> ((u & 1) * 16));
    }
};
template <>
struct StageVal<ValKind::BF16> {
    using Raw = uint16_t;
    using Group = uint2;
    __device__ static float ToF(uint16_t r) { return Bf16ToFloat(r); }
    __device__ static uint16_t Get(const uint2& g, int u)
    {
        const uint32_t w = u < 2 ? g.x : g.y;
        return static_cast<uint16_t>(w >> ((u & 1) * 16));
    }
};

// Word i of a 2- or 4-word vector (0 past its end).
template <int I, typename T>
__device__ __forceinline__ uint32_t GetW(const T& v)
{
    if constexpr (sizeof(T) == 16) return I == 0 ? v.x : I == 1 ? v.y : I == 2 ? v.z : v.w;
    else return I == 0 ? v.x : I == 1 ? v.y : 0U;
}

__device__ __forceinline__ float WaveSum(float v)
{
    for (int m = kWave / 2; m >= 1; m >>= 1) v += __shfl_xor(v, m, kWave);
    return v;
}

// Sum of elements lo..hi (0 <= lo, hi <= 3) of a group of 4 products.
__device__ __forceinline__ float GroupPart(const float4& f, int lo, int hi)
{
    const float x0 = lo == 0 ? f.x : 0.0f;
    const float x1 = lo <= 1 && hi >= 1 ? f.y : 0.0f;
    const float x2 = lo <= 2 && hi >= 2 ? f.z : 0.0f;
    const float x3 = hi == 3 ? f.w : 0.0f;
    return (x0 + x1) + (x2 + x3);
}

// Sum of the products [a, b) of a row of at most kLongRow entries, read from
// LDS as groups of 4: the first and last group masked, the whole groups
// between them (at most 7) in an order rotated by the lane, so that the
// lanes of rows of equal length (which start a multiple of the length apart)
// spread over the LDS banks.  A fixed order per row and lane: the same row
// always has the same lane.  kMidUnroll: how many of the middle groups' loads
// may be in flight at once (1 keeps the registers of a caller that holds
// many live values down; the sum is the same either way).
template <int kMidUnroll = 7>
__device__ __forceinline__ float ShortRowSum(const float4* areaV, int a, int b, int lane)
{
    if (b <= a) return 0.0f;
    const int q0 = a >> 2, q1 = (b - 1) >> 2;
    const float4 f = areaV[q0];
    const float4 g = areaV[q1];
    float sum = GroupPart(f, a & 3, q1 == q0 ? (b - 1) & 3 : 3);
    const int m = q1 - q0 - 1;  // whole groups between the two ends
    if (__ballot(m > 0) != 0) {
        // rotation start: the lane's low bits, below the largest power of 2 <= m
        const int p = m > 0 ? 1 << (31 - __builtin_clz(static_cast<uint32_t>(m))) : 1;
        const int r = (lane & 7) & (p - 1);
        float mid[2] = {0.0f, 0.0f};
        if (__ballot(m > 3) != 0) {
#pragma unroll kMidUnroll
            for (int c = 0; c < 7; ++c) {
                int u = r + c;
                u = u >= m ? u - m : u;
                const float4 v = areaV[q0 + 1 + (c < m ? u : 0)];
                const float s4 = (v.x + v.y) + (v.z + v.w);
                mid[c & 1] += c < m ? s4 : 0.0f;
            }
        } else {
#pragma unroll
            for (int c = 0; c < 3; ++c) {
                int u = r + c;
                u = u >= m ? u - m : u;
                const float4 v = areaV[q0 + 1 + (c < m ? u : 0)];
                const float s4 = (v.x + v.y) + (v.z + v.w);
                mid[c & 1] += c < m ? s4 : 0.0f;
            }
        }
        sum += mid[0] + mid[1];
    }
    if (q1 != q0) sum += GroupPart(g, 0, (b - 1) & 3);
    return sum;
}

// Row end of a tile's row: y, or the tile's head / tail partial sum.
template <OutKind O>
__device__ __forceinline__ void FinishRow(const StageParams& q, int64_t t, int loc, int nRowsDone, bool headRow,
                                          bool tailHasEntries, float sum, float alpha, float beta, bool betaNz,
                                          int64_t r0)
{
    using OutT = typename OutOf<O>::T;
    if (loc < nRowsDone) {
        if (loc == 0 && headRow) q.head[t] = sum;
        else StoreRow<O, AccKind::F32>(static_cast<OutT*>(q.y), r0 + loc, sum, alpha, beta, betaNz);
    } else if (tailHasEntries) {
        if (nRowsDone == 0 && headRow) q.head[t] = sum;
        else q.tail[t] = sum;
    }
}

// Pass B's LDS that depends on the bucket count (nb = S + 1), sized at
// launch: the run map's first chunks (nb words), then the area of staged x
// chunks / row ends and products (both in words, rounded to 16 bytes).
template <int kItems, typename Raw>
struct TileLds {
    static constexpr int kG = sizeof(Raw) == 2 ? 8 : 4;  // entries per group
    static constexpr int kP = static_cast<int>(kStageChunkBytes) / static_cast<int>(sizeof(Raw));
    static constexpr int kPhases = kItems == kWide ? 2 : 1;
    // products of one phase (a half of the tile's groups for the wide tiles)
    // after the 16-bit row ends: at most R/2 + 8 words of row ends and
    // E/kPhases + 1.5 kG words of products, R + E = kItems
    static constexpr int kProdFloats = kItems / kPhases + 2 * kG + 8;
    __host__ __device__ static constexpr int ChunkCap(int nb) { return (kItems + (kP - 1) * nb + kP - 1) / kP; }
    __host__ __device__ static constexpr int RunWords(int nb) { return (nb + 3) & ~3; }
    __host__ __device__ static constexpr int AreaWords(int nb)
    {
        const int staged = static_cast<int>(kStageChunkBytes) / 4 * ChunkCap(nb);
        return ((staged > kProdFloats ? staged : kProdFloats) + 3) & ~3;
    }
    __host__ __device__ static constexpr int DynBytes(int nb) { return 4 * (RunWords(nb) + AreaWords(nb)); }
};

// One workgroup per tile (tiles dealt to the XCDs in chunks).  LDS: the run
// map (runDelta, sized at launch for the matrix's buckets, startBits,
// firstRank), then one area that holds the staged x values, then (in place)
// the tile's row ends relative to the first group (uint16) followed by the
// products by groups of kG entries.  The wide tiles write and sum their
// products in two phases of half the groups each, so that the area is no
// larger than the staged x.  For x of 32 MB (257 buckets) that is 37 KB per
// workgroup: four workgroups per CU, eight waves per SIMD, for both tile
// sizes.  The wide tiles fit eight waves' registers (63 VGPRs) by loading
// their slots after the staging stores and by summing a row's middle groups
// in a loop rather than seven loads at once (with either one missing, 4-12
// VGPRs spill and pass B is slower than at six waves).  On the 16.8 M-row
// fp16 matrix with 32 random columns per row pass B took 747 µs with two
// workgroups of 75 KB per CU (every product in LDS at once), 691-698 µs with
// three, 647 µs with four; on the c3-like fp32 matrix 364 -> 334 µs from
// three workgroups (room for 1025 buckets) to four.
template <int kItems, typename RowT, ValKind V, OutKind O, bool kRows16>
__global__ __launch_bounds__(kTileThreads) __attribute__((amdgpu_waves_per_eu(8))) void StageTileKernel(StageParams q)
{
    constexpr int kTileItems = kItems;
    constexpr int kMaxLong = Tile<kItems>::kMaxLong;
    // entries per group: one 16-byte load of values (4 fp32, or 8 fp16 / bf16)
    // and of slots (8) where it fits: half the load instructions of groups of
    // 4 for 16-bit values (pass B 762 -> 748 µs on c4)
    constexpr int kG = sizeof(typename StageVal<V>::Raw) == 2 ? 8 : 4;
    constexpr int kGroupSlots = CeilDiv((kItems + kG - 1) / kG + 1, kTileThreads);  // groups per thread
    using SV = StageVal<V>;
    using Raw = typename SV::Raw;
    using Scan = hipcub::BlockScan<uint32_t, kTileThreads>;
    // staged x moves in chunks of kP slots (runs are padded to whole chunks)
    constexpr int kCB = static_cast<int>(kStageChunkBytes);
    using ChunkT = typename std::conditional<kCB == 16, uint4, uint2>::type;
    static_assert(kCB == 8 || kCB == 16, "8- or 16-byte chunks");
    constexpr int kP = kCB / static_cast<int>(sizeof(Raw));
    constexpr int kChunkCap = (kTileItems + (kP - 1) * (kStageMaxBuckets + 1) + kP - 1) / kP;
    constexpr int kChunkIters = (kChunkCap + kTileThreads - 1) / kTileThreads;  // 64-chunk windows per wave
    constexpr int kChunkWindows = kTileWaves * kChunkIters;
    using Lds = TileLds<kItems, Raw>;
    constexpr int kPhases = Lds::kPhases;
    constexpr bool kLateSlots = kItems == kWide;
    extern __shared__ float4 tileDyn[];  // Lds::DynBytes(nb) bytes
    uint32_t* runDelta = reinterpret_cast<uint32_t*>(tileDyn);
    float4* areaV = tileDyn + Lds::RunWords(q.buckets + 1) / 4;
    __shared__ uint32_t startBits[2 * kChunkWindows];
    __shared__ uint32_t firstRank[kChunkWindows];
    __shared__ uint16_t longRows[kMaxLong];
    __shared__ int longCount;
    __shared__ int headFlag;
    float* area = reinterpret_cast<float*>(areaV);
    __shared__ typename Scan::TempStorage scanStorage;

    const int64_t t = ChunkedXcdIndex();
    if (t >= q.tiles) return;
    const int tid = threadIdx.x;
    const int lane = tid & (kWave - 1);
    const int wv = tid / kWave;
    const int nb = q.buckets + 1;

    // The tile's loads are ordered by what they depend on, so that only two
    // memory round trips separate the launch from the first product:
    //   1. the path flag and the tile's corners (scalar loads), and the
    //      tile's two rows of the run table (first slot of every bucket's run
    //      in this tile and in the next), which depend on t alone;
    //   2. row offsets, values and slots (need the corners), then the staged
    //      x runs (need the run table's scan); the wave waits for the row
    //      offsets, then for the runs, while the values are still arriving.
    //      The wide tiles issue their slots after the staging instead, so
    //      that fewer registers are live at once (kLateSlots).
    // Vector loads are buffer loads under no lane-divergent branch (a load
    // under such a branch makes the wave wait for it where the branches
    // join): addresses outside a buffer read zero, and lanes with nothing to
    // load are masked afterwards.  Whole waves skip the loads that lie
    // entirely past their data (wave-uniform branches: the run table past the
    // last bucket, row offsets past the tile's rows, staging windows past the
    // wave's chunks), which keeps those instructions out of the address unit's
    // queue (3% of pass B on c4).  Compiler barriers keep the issue order.
    const uint32_t* startRow = q.start + t * nb;
    asm volatile("" ::"s"(startRow) : "memory");  // the kernel arguments the run loads need, first
    const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint32_t*>(startRow), 0, static_cast<int>(2 * nb * sizeof(uint32_t)), 0x00020000);
    uint32_t runA[kScanIpt], runB[kScanIpt];
    // waves whose run-table entries all lie past the last bucket issue no loads
    if (__builtin_amdgcn_readfirstlane(wv) * kWave * kScanIpt < nb) {
#pragma unroll
        for (int u = 0; u < kScanIpt; ++u) {
            const int s = tid * kScanIpt + u;
            runA[u] = __builtin_amdgcn_raw_buffer_load_b32(rs, s * 4, 0, 0);
            runB[u] = __builtin_amdgcn_raw_buffer_load_b32(rs, (nb + s) * 4, 0, 0);
        }
    } else {
#pragma unroll
        for (int u = 0; u < kScanIpt; ++u) runA[u] = runB[u] = 0U;
    }
    asm volatile("" ::: "memory");
    typedef const __attribute__((address_space(4))) int32_t* CI32;
    typedef const __attribute__((address_space(4))) int64_t* CI64;
    const uint32_t flag = FlagSet(q.flag);
    const int64_t r0 = reinterpret_cast<CI32>(reinterpret_cast<uintptr_t>(q.tile_row))[t];
    const int64_t r1 = reinterpret_cast<CI32>(reinterpret_cast<uintptr_t>(q.tile_row))[t + 1];
    const int64_t e0 = reinterpret_cast<CI64>(reinterpret_cast<uintptr_t>(q.tile_nnz))[t];
    const int64_t e1 = reinterpret_cast<CI64>(reinterpret_cast<uintptr_t>(q.tile_nnz))[t + 1];
    float alpha, beta;
    LoadScalars<AccKind::F32>(q.s, alpha, beta);
    asm volatile("" ::: "memory");
    if (flag != 1U) return;
    const int E = static_cast<int>(e1 - e0);
    const int R = static_cast<int>(r1 - r0);

    // 2a. row offsets of the tile's first 2*kTileThreads+1 rows.  kRows16:
    //     their low 16 bits only (2 bytes per row): rows 1..R of the tile
    //     start inside it, so offset - e0 lies in [0, E] (E < 2^16) and
    //     follows from the low halves; row 0 is clamped to the tile anyway
    const int64_t nBytes = (q.rows + 2 - r0) * static_cast<int64_t>(kRows16 ? 2 : sizeof(RowT));
    const __amdgpu_buffer_rsrc_t rn = __builtin_amdgcn_make_buffer_rsrc(
        kRows16 ? static_cast<void*>(const_cast<uint16_t*>(q.rp16 + r0))
                : static_cast<void*>(const_cast<RowT*>(static_cast<const RowT*>(q.norm) + r0)),
        0, static_cast<int>(nBytes < 0x7FFFFFFFLL ? nBytes : 0x7FFFFFFFLL), 0x00020000);
    int64_t rowOff[2];
#pragma unroll
    for (int u = 0; u < 2; ++u) {
        const int i = tid + u * kTileThreads;
        if (u == 1 && R < kTileThreads) {  // the second half of the offsets is past the tile's rows
            rowOff[u] = 0;
            continue;
        }
        if constexpr (kRows16) {
            rowOff[u] = static_cast<int64_t>(__builtin_amdgcn_raw_buffer_load_b16(rn, i * 2, 0, 0));
        } else if constexpr (sizeof(RowT) == 8) {
            rowOff[u] = static_cast<int64_t>(
                __builtin_bit_cast(uint64_t, __builtin_amdgcn_raw_buffer_load_b64(rn, i * 8, 0, 0)));
        } else {
            rowOff[u] = static_cast<int32_t>(__builtin_amdgcn_raw_buffer_load_b32(rn, i * 4, 0, 0));
        }
    }
    asm volatile("" ::: "memory");
    // 2b. values and slots of this thread's groups of kG entries (CSR order),
    //     from the tile's first group; loads past an array's last dword read
    //     zero (byte counts are rounded up to a dword, which never leaves the
    //     array's 16-byte block; st_perm is padded by 8 slots)
    const int64_t g0 = e0 / kG;
    const int a0 = static_cast<int>(e0 - g0 * kG);  // entry e0's place in its group
    const int ng = (a0 + E + kG - 1) / kG;          // groups of kG entries touching the tile
    const int64_t vBytes = ((q.nnz - g0 * kG) * static_cast<int64_t>(sizeof(Raw)) + 3) & ~int64_t{3};
    const __amdgpu_buffer_rsrc_t rv = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<Raw*>(static_cast<const Raw*>(q.val) + g0 * kG), 0,
        static_cast<int>(vBytes < 0x7FFFFFFFLL ? vBytes : 0x7FFFFFFFLL), 0x00020000);
    const int64_t pBytes = (q.nnz + 8 - g0 * kG) * 2;
    const __amdgpu_buffer_rsrc_t rp = __builtin_amdgcn_make_buffer_rsrc(
        q.perm + g0 * kG, 0, static_cast<int>(pBytes < 0x7FFFFFFFLL ? pBytes : 0x7FFFFFFFLL), 0x00020000);
    using GroupT = typename std::conditional<kG == 8 || sizeof(Raw) == 4, uint4, uint2>::type;
    using SlotsT = typename std::conditional<kG == 8, uint4, uint2>::type;
    GroupT gv[kGroupSlots];
    SlotsT gp[kGroupSlots];
#pragma unroll
    for (int u = 0; u < kGroupSlots; ++u) {
        const int gi = tid + u * kTileThreads;
        if constexpr (sizeof(GroupT) == 16) {
            gv[u] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(rv, gi * 16, 0, 0));
        } else {
            gv[u] = __builtin_bit_cast(uint2, __builtin_amdgcn_raw_buffer_load_b64(rv, gi * 8, 0, 0));
        }
        if constexpr (!kLateSlots) {
            if constexpr (kG == 8) {
                gp[u] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(rp, gi * 16, 0, 0));
            } else {
                gp[u] = __builtin_bit_cast(uint2, __builtin_amdgcn_raw_buffer_load_b64(rp, gi * 8, 0, 0));
            }
        }
    }
    asm volatile("" ::: "memory");

    // 3. the chunk -> run map of the tile's bucket-ordered staged slots, from
    //    an exclusive scan of the run lengths in chunks (waits for the run
    //    table only).  Each scanned word packs (non-empty runs before, chunks
    //    before); for every non-empty run of rank r starting at chunk o:
    //    runDelta[r] = its first xg chunk - o, bit o of startBits, and
    //    firstRank of each 64-chunk window whose first chunk it holds.  The
    //    run of chunk i = 64*W + l then has rank firstRank[W] + (bits 1..l
    //    of the window's 64 start bits).
    for (int w = tid; w < 2 * kChunkWindows; w += kTileThreads) {
        startBits[w] = 0U;
        if (w < kChunkWindows) firstRank[w] = 0U;
    }
    uint32_t cnt[kScanIpt];
#pragma unroll
    for (int u = 0; u < kScanIpt; ++u) {
        const int s = tid * kScanIpt + u;
        const uint32_t c = s < nb ? (runB[u] - runA[u]) / kP : 0U;
        cnt[u] = c | (c != 0U ? 0x10000U : 0U);
    }
    uint32_t packedTotal;
    Scan(scanStorage).ExclusiveSum(cnt, cnt, packedTotal);  // its barriers also order the clearing above
    const int C = static_cast<int>(packedTotal & 0xFFFFU);  // staged chunks of the tile
#pragma unroll
    for (int u = 0; u < kScanIpt; ++u) {
        const int s = tid * kScanIpt + u;
        const uint32_t c = s < nb ? (runB[u] - runA[u]) / kP : 0U;
        if (c != 0U) {
            const uint32_t o = cnt[u] & 0xFFFFU, r = cnt[u] >> 16;
            runDelta[r] = runA[u] / kP - o;
            atomicOr(&startBits[o >> 5], 1U << (o & 31U));
            for (uint32_t w = (o + 63U) >> 6; w * 64U < o + c; ++w) firstRank[w] = r;
        }
    }
    if (tid == 0) longCount = 0;
    const bool lastRowInside = r1 < q.rows;
    const int nLoc = R + (lastRowInside ? 1 : 0);
    __syncthreads();

    // 4. stage the runs, 8 bytes per lane.  Wave w fills the 64-chunk
    //    windows of chunks [w*span, (w+1)*span), lanes on consecutive chunks,
    //    so the loads of one run are coalesced.  The source chunk of each of
    //    the lane's loads comes first (independent LDS lookups; the window's
    //    words are the same for the whole wave), the loads after it; lanes
    //    past the range load chunk 0 and discard it.
    {
        const ChunkT* xg = static_cast<const ChunkT*>(q.xg);
        ChunkT* xl = reinterpret_cast<ChunkT*>(area);
        const int span = (C + kTileWaves * kWave - 1) / (kTileWaves * kWave) * kWave;
        const int i0 = __builtin_amdgcn_readfirstlane(wv) * span;  // wave-uniform
        const int i1 = i0 + span < C ? i0 + span : C;
        const uint32_t maskLo = lane < 32 ? (2U << lane) - 2U : 0xFFFFFFFEU;   // bits 1..l
        const uint32_t maskHi = lane < 32 ? 0U : (2U << (lane - 32)) - 1U;
        uint32_t src[kChunkIters];
#pragma unroll
        for (int m = 0; m < kChunkIters; ++m) {
            const int w = (i0 >> 6) + m;
            const int i = (w << 6) + lane;
            const uint32_t fr = firstRank[w];
            const uint32_t bLo = startBits[2 * w], bHi = startBits[2 * w + 1];
            const uint32_t r = fr + static_cast<uint32_t>(__builtin_popcount(bLo & maskLo)) +
                               static_cast<uint32_t>(__builtin_popcount(bHi & maskHi));
            const uint32_t d = runDelta[r];  // read by every lane: no load under a branch
            src[m] = i < i1 ? d + static_cast<uint32_t>(i) : 0U;
        }
        ChunkT v[kChunkIters];
#pragma unroll
        for (int m = 0; m < kChunkIters; ++m) {  // xg holds fewer than 2^32 slots
            if (i0 + m * kWave >= i1) {  // a 64-chunk window wholly past the wave's range: no load
                v[m] = ChunkT{};
                continue;
            }
            v[m] = xg[src[m]];
        }
        asm volatile("" ::: "memory");  // all loads before the first store
        if (tid == 0) {  // the tile's first row started in an earlier tile
            headFlag = (kRows16 ? Norm<RowT>(q, r0) : rowOff[0]) < e0 ? 1 : 0;
        }
#pragma unroll
        for (int m = 0; m < kChunkIters; ++m) {
            const int i = i0 + m * kWave + lane;
            if (i < i1) xl[i] = v[m];
        }
    }
    if constexpr (kLateSlots) {  // the slots after the staging: fewer registers live at once
#pragma unroll
        for (int u = 0; u < kGroupSlots; ++u) {
            const int gi = tid + u * kTileThreads;
            if constexpr (kG == 8) {
                gp[u] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(rp, gi * 16, 0, 0));
            } else {
                gp[u] = __builtin_bit_cast(uint2, __builtin_amdgcn_raw_buffer_load_b64(rp, gi * 8, 0, 0));
            }
        }
    }
    __syncthreads();
    const bool headRow = headFlag != 0;

    // 5. products a_k * x(slot_k) in registers, then into the area by groups
    //    of kG (entry e0 at a0), with the tile's row offsets relative to the
    //    first group (clamped to the tile) after them.  The tile's two edge
    //    groups also hold entries of the neighbouring tiles: their slots are
    //    other tiles' (still inside the staged area) and their products are
    //    replaced by zero.
    float4 prod[kGroupSlots][kG / 4];
    {
        const Raw* xlr = reinterpret_cast<const Raw*>(area);
#pragma unroll
        for (int u = 0; u < kGroupSlots; ++u) {
            const int gi = tid + u * kTileThreads;
            float pr[kG];
            const uint32_t pws[4] = {gp[u].x, gp[u].y, kG == 8 ? GetW<2>(gp[u]) : 0U, kG == 8 ? GetW<3>(gp[u]) : 0U};
            const uint32_t vws[4] = {gv[u].x, gv[u].y, sizeof(GroupT) == 16 ? GetW<2>(gv[u]) : 0U,
                                     sizeof(GroupT) == 16 ? GetW<3>(gv[u]) : 0U};
#pragma unroll
            for (int k = 0; k < kG; ++k) {
                const int slot = static_cast<int>((pws[k >> 1] >> ((k & 1) * 16)) & 0xFFFFU);
                Raw a;
                if constexpr (sizeof(Raw) == 4) {
                    a = vws[k];
                } else {
                    a = static_cast<Raw>(vws[k >> 1] >> ((k & 1) * 16));
                }
                pr[k] = SV::ToF(a) * SV::ToF(xlr[slot]);
            }
            const int lo = a0 - gi * kG, hi = a0 + E - gi * kG;  // entries [lo, hi) of the group are the tile's
            if (lo > 0 || hi < kG) {
#pragma unroll
                for (int k = 0; k < kG; ++k) pr[k] = k >= lo && k < hi ? pr[k] : 0.0f;
            }
#pragma unroll
            for (int h = 0; h < kG / 4; ++h) {
                prod[u][h] = make_float4(pr[4 * h], pr[4 * h + 1], pr[4 * h + 2], pr[4 * h + 3]);
            }
        }
    }
    __syncthreads();
    // row ends relative to the first group (uint16: at most a0 + E < 2^16),
    // at the start of the area, the products of the current phase after them
    uint16_t* rel = reinterpret_cast<uint16_t*>(area);
    const int relWords = ((R + 2 + 1) / 2 + 3) & ~3;
    float4* prodV = areaV + relWords / 4;
    const auto relOf = [&](int i, int64_t off) {
        if constexpr (kRows16) {
            if (i == 0) return a0;
            const int32_t d = static_cast<int32_t>((static_cast<uint32_t>(off) - static_cast<uint32_t>(e0)) & 0xFFFFU);
            return a0 + (d > E ? E : d);
        } else {
            const int64_t d = off - e0;
            return a0 + static_cast<int32_t>(d < 0 ? 0 : d > E ? E : d);
        }
    };
#pragma unroll
    for (int u = 0; u < 2; ++u) {
        const int i = tid + u * kTileThreads;
        if (i <= R) rel[i] = static_cast<uint16_t>(relOf(i, rowOff[u]));
    }
    if (tid == 0) rel[R + 1] = static_cast<uint16_t>(a0 + E);
    for (int i = tid + 2 * kTileThreads; i <= R; i += kTileThreads) {  // tiles of many short rows
        rel[i] = static_cast<uint16_t>(relOf(i, kRows16 ? static_cast<int64_t>(q.rp16[r0 + i]) : Norm<RowT>(q, r0 + i)));
    }

    // 6. rows, by phases: phase p holds the products of groups [p*gs, ...)
    //    (entries [p*em, ...) relative to the first group).  A row is summed
    //    over its part in each phase it touches, the phase where it ends
    //    finishes it; the one row that crosses em carries its first part in
    //    crossPart.  Short parts by one thread, long ones queued for a wave.
    const bool betaNz = beta != 0.0f;  // y is not read when beta == 0, wherever beta lives
    const int gs = kPhases == 1 ? ng : ng / 2;
    const int em = gs * kG;
    __shared__ float crossPart;
#pragma unroll
    for (int ph = 0; ph < kPhases; ++ph) {
        const int g1 = ph + 1 == kPhases ? ng : gs;
        const int off = ph == 0 ? 0 : em;
#pragma unroll
        for (int u = 0; u < kGroupSlots; ++u) {
            const int gi = tid + u * kTileThreads;
            if (gi >= ph * gs && gi < g1) {
#pragma unroll
                for (int h = 0; h < kG / 4; ++h) prodV[(gi - ph * gs) * (kG / 4) + h] = prod[u][h];
            }
        }
        if (tid == 0) longCount = 0;
        __syncthreads();
        const bool tailHasEntries = lastRowInside && rel[R] < a0 + E;
        for (int loc = tid; loc < nLoc; loc += kTileThreads) {
            int a = rel[loc], b = rel[loc + 1];
            bool finish = true, carry = false;
            if constexpr (kPhases == 2) {
                if (ph == 0) {
                    if (a >= em) continue;
                    if (b > em) { b = em; finish = false; }
                } else {
                    if (a < em && b <= em) continue;
                    if (a < em) { a = em; carry = true; }
                }
            }
            if (b - a > kLongRow) {
                longRows[atomicAdd(&longCount, 1)] = static_cast<uint16_t>(loc);
                continue;
            }
            float sum = ShortRowSum<kPhases == 2 ? 1 : 7>(prodV, a - off, b - off, lane);
            if (carry) sum = crossPart + sum;
            if (finish) FinishRow<O>(q, t, loc, R, headRow, tailHasEntries, sum, alpha, beta, betaNz, r0);
            else crossPart = sum;
        }
        __syncthreads();
        const int nLong = longCount;
        for (int li = wv; li < nLong; li += kTileWaves) {
            const int loc = longRows[li];
            int a = rel[loc], b = rel[loc + 1];
            bool finish = true, carry = false;
            if constexpr (kPhases == 2) {
                if (ph == 0) {
                    if (b > em) { b = em; finish = false; }
                } else if (a < em) {
                    a = em;
                    carry = true;
                }
            }
            float part = 0.0f;
            for (int k = a + lane; k < b; k += kWave) part += area[relWords + k - off];
            float sum = WaveSum(part);
            if (carry) sum = crossPart + sum;
            if (lane == 0) {
                if (finish) FinishRow<O>(q, t, loc, R, headRow, tailHasEntries, sum, alpha, beta, betaNz, r0);
                else crossPart = sum;
            }
        }
        if (ph + 1 < kPhases) __syncthreads();  // the first half's products are read before the second half overwrites them
    }
}

// Rows that cross tile ends: the tile where such a row ends adds, in tile
// order, the tail partial of the tile where it starts and the head partials
// of every tile after it, then stores y.  The tile where row r starts
// follows from the merge path: its first entry s is item r + s of the
// merged sequence (the ends of rows 0..r-1 and entries 0..s-1 come before
// it), so it lies in tile (r + s) / tile_items; the partials are then read
// with independent loads, however many tiles the row spans.
template <typename RowT, OutKind O>
__global__ __launch_bounds__(256) void StageFixupKernel(StageParams q)
{
    using OutT = typename OutOf<O>::T;
    if (FlagSet(q.flag) != 1U) return;
    const int64_t t = blockIdx.x * int64_t{256} + threadIdx.x;
    if (t >= q.tiles) return;
    const int64_t r0 = q.tile_row[t];
    if (q.tile_row[t + 1] == r0) return;                 // no row ends in tile t
    const int64_t start = Norm<RowT>(q, r0);
    if (start >= q.tile_nnz[t]) return;                  // its first row starts inside it
    const int64_t u = (r0 + start) / q.tile_items;       // the tile where that row starts (< t)
    float sum = q.tail[u];
    for (int64_t v = u + 1; v <= t; ++v) sum += q.head[v];
    float alpha, beta;
    LoadScalars<AccKind::F32>(q.s, alpha, beta);
    const bool betaNz = beta != 0.0f;  // y is not read when beta == 0, wherever beta lives
    StoreRow<O, AccKind::F32>(static_cast<OutT*>(q.y), r0, sum, alpha, beta, betaNz);
}

// ----------------------- column-bucketed transpose ---------------------------
//
// y = alpha * A^T x + beta * y, fp32 values and compute (BtEligible).  The
// tiles are the staged path's merge-path tiles; bucket b holds the columns
// [b*W, (b+1)*W), bucket S the entries outside the rows' range or whose
// column is outside [0, cols).  Preprocess (pattern only, after the CSC
// build): per (bucket, tile) counts and their bucket-major scan, each entry's
// slot in its tile's bucket-ordered runs (st_perm), and, for each slot, its
// place among its bucket's entries in column order (st_cl, from the CSC
// pattern).  The bucket-major scan gives bucket b the slots
// [colptr[b*W], colptr[(b+1)*W]): the same count, and the same start, as its
// columns' CSC range.
//  * Pass 1 (BtScatterKernel), one workgroup per tile: the products
//    a_k * x[row(k)] (values in CSR order, coalesced; each row's x spread
//    over its entries in LDS, half a tile at a time), placed in LDS at their
//    slots (again by halves), then written as the tile's runs; runs of
//    neighbouring tiles are adjacent, so their partial lines merge in L2.
//  * Pass 2 (BtColumnKernel), one workgroup per CU looping over the buckets
//    (each bucket's region of up to kBtRegionCap products takes most of a
//    CU's LDS; the next bucket's loads fly while the current one is summed):
//    its products (sequential) go to LDS at their column-order places, then every column
//    is summed in row order, the order the reference's ALG2 accumulates in
//    (sparse/spmv/README.md:252), and y = alpha*sum + beta*y.
// Counterpart: the transpose of sparse/spmv/arch35/spmv_kernel.cpp:579-668,
// which scatters a_k * x[row] into y with atomics.

constexpr int kBtScanIpt = CeilDiv(kBtMaxBuckets + 1, kTileThreads);  // run lengths per thread
constexpr int kBtColThreads = 1024;                                    // pass 2
constexpr int kBtLongCol = 64;  // columns longer than this are summed by a wave
constexpr int kBtRunEntries = 64;  // mean run length (entries) below which the bucketed kernels are chosen
constexpr int kBtMaxLongCols = static_cast<int>(kBtRegionCap) / (kBtLongCol + 1) + 1;

// Bucket of entry k (S: outside the rows' range or a column outside [0, cols)).
__device__ __forceinline__ uint32_t BtKey(const StageParams& q, int64_t k, int64_t first, int64_t last, int32_t col)
{
    if (k < first || k >= last) return static_cast<uint32_t>(q.buckets);
    return KeyOf(q, col) >> q.wshift;
}

// inv[csc_pos[j]] = j.
template <typename RowT>
__global__ __launch_bounds__(256) void BtInvertKernel(StageParams q)
{
    const int64_t j = blockIdx.x * int64_t{256} + threadIdx.x;
    if (j >= q.nnz) return;
    q.inv[static_cast<int64_t>(static_cast<const RowT*>(q.csc_pos)[j])] = static_cast<int32_t>(j);
}

// counts[s*(T+1) + t] = entries of tile t in bucket s (column T is zero).
template <typename RowT>
__global__ __launch_bounds__(kSortThreads) void BtCountKernel(StageParams q)
{
    __shared__ uint32_t hist[kBtMaxBuckets + 1];
    const int64_t t = blockIdx.x;
    const int nb = q.buckets + 1;
    for (int s = threadIdx.x; s < nb; s += kSortThreads) hist[s] = 0U;
    __syncthreads();
    if (t < q.tiles) {
        const int64_t first = Norm<RowT>(q, 0), last = Norm<RowT>(q, q.rows);
        const int64_t e0 = q.tile_nnz[t], e1 = q.tile_nnz[t + 1];
        const int n = static_cast<int>(e1 - e0);
        uint4 raw[kColGroups];
        LoadTileCols(q, e0, n, raw);  // one round trip
#pragma unroll
        for (int u = 0; u < kColGroups; ++u) {
            if (u * 4 * kSortThreads >= n) break;  // uniform
            const int i = (u * kSortThreads + static_cast<int>(threadIdx.x)) * 4;
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                if (i + k < n) {
                    atomicAdd(&hist[BtKey(q, e0 + i + k, first, last, static_cast<int32_t>(WordOf(raw[u], k)))], 1U);
                }
            }
        }
    }
    __syncthreads();
    for (int s = threadIdx.x; s < nb; s += kSortThreads) q.counts[s * (q.tiles + 1) + t] = hist[s];
}

// Per tile: perm[k] = slot of entry k in the tile's bucket-ordered runs;
// cl[start(t,b) + (slot - run start)] = the entry's place in bucket b's
// column-ordered products.  Each entry takes the next place of its bucket's
// run with an LDS atomic: the order inside a run is free, because pass 1 puts
// every product at its own slot and pass 2 moves it to its own column-order
// place before the columns are summed in row order, so results do not depend
// on it.  Adds the tile's count of non-empty runs (the path metric).
template <int kItems, typename RowT>
__global__ __launch_bounds__(kSortThreads) void BtRankKernel(StageParams q)
{
    constexpr int kNb = kBtMaxBuckets + 1;
    constexpr int kRunIpt = CeilDiv(kNb, kSortThreads);
    static_assert(kItems <= kColGroups * 4 * kSortThreads, "a tile's entries fit the column loads");
    using Scan = hipcub::BlockScan<uint32_t, kSortThreads>;
    __shared__ uint32_t cnt[kNb];       // next slot of each bucket's run (tile-local)
    __shared__ uint32_t runBase[kNb];   // st_cl slot of each run's first entry minus its tile-local first slot
    __shared__ uint32_t colBase[kNb];   // CSC index of each bucket's first entry
    __shared__ typename Scan::TempStorage scanStorage;
    __shared__ uint32_t runCount;
    const int64_t t = blockIdx.x;
    const int tid = threadIdx.x;
    const int64_t e0 = q.tile_nnz[t], e1 = q.tile_nnz[t + 1];
    const int n = static_cast<int>(e1 - e0);
    const int nb = q.buckets + 1;
    const int64_t first = Norm<RowT>(q, 0), last = Norm<RowT>(q, q.rows);
    const uint32_t* startRow = q.start + t * nb;
    const RowT* colptr = static_cast<const RowT*>(q.colptr);
    if (tid == 0) runCount = 0U;
    uint32_t pc[kRunIpt], a[kRunIpt];
    uint32_t runs = 0U;
#pragma unroll
    for (int u = 0; u < kRunIpt; ++u) {
        const int sb = tid * kRunIpt + u;
        a[u] = sb < nb ? startRow[sb] : 0U;
        pc[u] = sb < nb ? startRow[nb + sb] - a[u] : 0U;
        if (sb < q.buckets && pc[u] != 0U) ++runs;
        if (sb < q.buckets) colBase[sb] = static_cast<uint32_t>(colptr[static_cast<int64_t>(sb) << q.wshift]);
    }
    Scan(scanStorage).ExclusiveSum(pc, pc);
#pragma unroll
    for (int u = 0; u < kRunIpt; ++u) {
        const int sb = tid * kRunIpt + u;
        if (sb < nb) {
            cnt[sb] = pc[u];
            runBase[sb] = a[u] - pc[u];
        }
    }
    if (runs != 0U) atomicAdd(&runCount, runs);
    __syncthreads();
    // the tile's column indices and CSC indices (inv) in one round trip of
    // 16-byte loads, then per entry its slot and place
    uint4 raw[kColGroups], rinv[kColGroups];
    LoadTileCols(q, e0, n, raw);
    {
        const int64_t iBytes = (q.nnz - e0) * 4;
        const __amdgpu_buffer_rsrc_t ri = __builtin_amdgcn_make_buffer_rsrc(
            q.inv + e0, 0, static_cast<int>(iBytes < 0x7FFFFFFFLL ? iBytes : 0x7FFFFFFFLL), 0x00020000);
#pragma unroll
        for (int u = 0; u < kColGroups; ++u) {
            if (u * 4 * kSortThreads >= n) break;  // uniform
            const int i = (u * kSortThreads + tid) * 4;
            rinv[u] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(ri, i * 4, 0, 0));
        }
        asm volatile("" ::: "memory");
    }
#pragma unroll
    for (int u = 0; u < kColGroups; ++u) {
        if (u * 4 * kSortThreads >= n) break;
        const int i4 = (u * kSortThreads + tid) * 4;
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const int i = i4 + k;
            if (i < n) {
                const uint32_t b = BtKey(q, e0 + i, first, last, static_cast<int32_t>(WordOf(raw[u], k)));
                const uint32_t slot = atomicAdd(&cnt[b], 1U);
                q.perm[e0 + i] = static_cast<uint16_t>(slot);
                const uint32_t place =
                    b < static_cast<uint32_t>(q.buckets) ? WordOf(rinv[u], k) - colBase[b] : 0U;
                q.cl[runBase[b] + slot] = static_cast<uint16_t>(place);
            }
        }
    }
    __syncthreads();
    if (tid == 0 && runCount != 0U) atomicAdd(q.metric, static_cast<unsigned long long>(runCount));
}

// csc_row[j] = entry_row[csc_pos[j]] (into the inv array, no longer
// needed), for the one-pass banded kernel only: launched after the path
// decision, it does nothing unless that kernel was chosen (a gather of one
// line per entry, which the other paths would pay for nothing).
template <typename RowT>
__global__ __launch_bounds__(256) void BtCscRowKernel(StageParams q)
{
    const int64_t j = blockIdx.x * int64_t{256} + threadIdx.x;
    if (j >= q.nnz || FlagSet(q.flag) != 2U) return;
    q.inv[j] = q.entry_row[static_cast<int64_t>(static_cast<const RowT*>(q.csc_pos)[j])];
}

// The path decision (header flag): 1, the column-bucketed kernels, when the
// entries are scattered over the columns and every bucket's entries fit pass
// 2's LDS; 2, the one-pass banded column kernel, when they are not (the
// values and x an entry needs are then near those of its neighbours in
// column order); 0, the CSC product and column passes.  Scattered: the
// tiles' runs are short (mean below kBtRunEntries entries), or, from
// kBtWideNnz entries on, a tile has a run in at least half of the buckets on
// average (a random pattern with few, wide buckets has long runs too; a
// banded one touches a few buckets per tile).  Measured on random patterns
// (banded kernel -> bucketed kernels, µs per SpMV): 1 M entries 22 -> 34,
// 2 M 40 -> 27-30, 4 M 78 (CSC kernels) -> 38.
constexpr int64_t kBtWideNnz = int64_t{1} << 21;
template <typename RowT>
__global__ __launch_bounds__(256) void BtDecideKernel(StageParams q)
{
    __shared__ int ok;
    const unsigned long long runs = *q.metric;
    const bool scattered =
        runs * static_cast<unsigned long long>(kBtRunEntries) > static_cast<unsigned long long>(q.nnz) ||
        (q.nnz >= kBtWideNnz && 2ULL * runs >= static_cast<unsigned long long>(q.tiles) *
                                                     static_cast<unsigned long long>(q.buckets));
    if (threadIdx.x == 0) ok = 1;
    __syncthreads();
    const RowT* colptr = static_cast<const RowT*>(q.colptr);
    const int64_t w = int64_t{1} << q.wshift;
    for (int64_t b = threadIdx.x; b < q.buckets; b += 256) {
        const int64_t c0 = b * w;
        const int64_t c1 = c0 + w < q.cols ? c0 + w : q.cols;
        if (static_cast<int64_t>(colptr[c1]) - static_cast<int64_t>(colptr[c0]) > kBtRegionCap) ok = 0;
    }
    __syncthreads();
    if (threadIdx.x == 0) *q.flag = scattered ? (ok != 0 ? 1U : 0U) : (q.banded_ok != 0 ? 2U : 0U);
}

// Pass 1's LDS sized at launch: the run map's first slots (nb words), then
// an area for the 16-bit row ends plus x over half the tile's entries, or
// half the tile's products at their slots (kWide/2 + 80 words either way).
constexpr unsigned BtScatterLdsBytes(int64_t nb)
{
    return static_cast<unsigned>(4 * (((nb + 3) & ~int64_t{3}) + ((kWide / 2 + 80 + 3) & ~3)));
}

// Pass 1: products of one tile into its runs (see above).  The row offsets
// and x of the tile's first kBtPreRows*kTileThreads rows are loaded with the
// values (tiles of the Poisson-like c5 pattern hold about 1400 rows); rows
// past them, in tiles of many short rows, are read after.  The x spread and
// the slot placement each go in two halves, so that the LDS area is half a
// tile (43 KB per workgroup with 1025 buckets: three workgroups per CU, six
// waves per SIMD at 77 VGPRs, the products taking the values' registers and
// the slots loaded after the products): c5 pass 1 66.4 -> 62.3 µs against two
// workgroups of 81 KB.  Eight waves per SIMD spill 25-30 VGPRs.
constexpr int kBtPreRows = 4;

template <int kItems, typename RowT>
__global__ __launch_bounds__(kTileThreads) __attribute__((amdgpu_waves_per_eu(6))) void BtScatterKernel(StageParams q)
{
    constexpr int kTileItems = kItems;
    constexpr int kMaxLong = Tile<kItems>::kMaxLong;
    constexpr int kGroupSlots = Tile<kItems>::kGroupSlots;
    constexpr int kStageLanes = Tile<kItems>::kStageLanes;
    constexpr int kWindows = Tile<kItems>::kWindows;
    using Scan = hipcub::BlockScan<uint32_t, kTileThreads>;
    extern __shared__ float4 btDyn[];  // BtScatterLdsBytes(nb) bytes: the run map's first slots, then the area
    uint32_t* runDelta = reinterpret_cast<uint32_t*>(btDyn);
    float4* areaV = btDyn + ((q.buckets + 1 + 3) & ~3) / 4;
    __shared__ uint32_t startBits[2 * kWindows];
    __shared__ uint32_t firstRank[kWindows];
    __shared__ uint16_t longRows[kMaxLong];
    __shared__ int longCount[2];
    __shared__ typename Scan::TempStorage scanStorage;
    float* area = reinterpret_cast<float*>(areaV);

    const int64_t t = ChunkedXcdIndex();  // as pass B: tiles in flight consecutive chip-wide
    if (t >= q.tiles) return;
    const int tid = threadIdx.x;
    const int lane = tid & (kWave - 1);
    const int wv = tid / kWave;
    const int nb = q.buckets + 1;

    // 1. the tile's two rows of the run table (depend on t alone), then the
    //    flag and the tile's corners (scalar loads)
    const uint32_t* startRow = q.start + t * nb;
    asm volatile("" ::"s"(startRow) : "memory");
    const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint32_t*>(startRow), 0, static_cast<int>(2 * nb * sizeof(uint32_t)), 0x00020000);
    uint32_t runA[kBtScanIpt], runB[kBtScanIpt];
#pragma unroll
    for (int u = 0; u < kBtScanIpt; ++u) {
        const int s = tid * kBtScanIpt + u;
        runA[u] = __builtin_amdgcn_raw_buffer_load_b32(rs, s * 4, 0, 0);
        runB[u] = __builtin_amdgcn_raw_buffer_load_b32(rs, (nb + s) * 4, 0, 0);
    }
    asm volatile("" ::: "memory");
    typedef const __attribute__((address_space(4))) int32_t* CI32;
    typedef const __attribute__((address_space(4))) int64_t* CI64;
    const uint32_t flag = FlagSet(q.flag);
    const int64_t r0 = reinterpret_cast<CI32>(reinterpret_cast<uintptr_t>(q.tile_row))[t];
    const int64_t r1 = reinterpret_cast<CI32>(reinterpret_cast<uintptr_t>(q.tile_row))[t + 1];
    const int64_t e0 = reinterpret_cast<CI64>(reinterpret_cast<uintptr_t>(q.tile_nnz))[t];
    const int64_t e1 = reinterpret_cast<CI64>(reinterpret_cast<uintptr_t>(q.tile_nnz))[t + 1];
    asm volatile("" ::: "memory");
    if (flag != 1U) return;
    const int E = static_cast<int>(e1 - e0);
    const int R = static_cast<int>(r1 - r0);
    const bool lastRowInside = r1 < q.rows;
    const int nLoc = R + (lastRowInside ? 1 : 0);  // rows with entries in the tile (the last may continue)

    // 2. row offsets and x of the tile's first 2*kTileThreads rows, values
    //    and slots of this thread's groups of 4 entries (unconditional buffer
    //    loads; out-of-range addresses read zero)
    const int64_t nBytes = (q.rows + 2 - r0) * static_cast<int64_t>(sizeof(RowT));
    const __amdgpu_buffer_rsrc_t rn = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<RowT*>(static_cast<const RowT*>(q.norm) + r0), 0,
        static_cast<int>(nBytes < 0x7FFFFFFFLL ? nBytes : 0x7FFFFFFFLL), 0x00020000);
    const int64_t xBytes = (q.rows - r0) * 4;
    const __amdgpu_buffer_rsrc_t rx = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<float*>(static_cast<const float*>(q.x) + r0), 0,
        static_cast<int>(xBytes < 0x7FFFFFFFLL ? xBytes : 0x7FFFFFFFLL), 0x00020000);
    int64_t rowOff[kBtPreRows];
    float xRow[kBtPreRows];
#pragma unroll
    for (int u = 0; u < kBtPreRows; ++u) {
        const int i = tid + u * kTileThreads;
        if (u > 0 && R < u * kTileThreads) {  // past the tile's rows (uniform over the workgroup)
            rowOff[u] = 0;
            xRow[u] = 0.0f;
            continue;
        }
        if constexpr (sizeof(RowT) == 8) {
            rowOff[u] = static_cast<int64_t>(
                __builtin_bit_cast(uint64_t, __builtin_amdgcn_raw_buffer_load_b64(rn, i * 8, 0, 0)));
        } else {
            rowOff[u] = static_cast<int32_t>(__builtin_amdgcn_raw_buffer_load_b32(rn, i * 4, 0, 0));
        }
        xRow[u] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rx, i * 4, 0, 0));
    }
    const int64_t g0 = e0 >> 2;
    const int a0 = static_cast<int>(e0 - g0 * 4);  // entry e0's place in its group
    const int ng = (a0 + E + 3) >> 2;              // groups of 4 entries touching the tile
    const int64_t vBytes = (q.nnz - g0 * 4) * 4;
    const __amdgpu_buffer_rsrc_t rv = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<float*>(static_cast<const float*>(q.val) + g0 * 4), 0,
        static_cast<int>(vBytes < 0x7FFFFFFFLL ? vBytes : 0x7FFFFFFFLL), 0x00020000);
    const int64_t pBytes = (q.nnz + 8 - g0 * 4) * 2;
    const __amdgpu_buffer_rsrc_t rp = __builtin_amdgcn_make_buffer_rsrc(
        q.perm + g0 * 4, 0, static_cast<int>(pBytes < 0x7FFFFFFFLL ? pBytes : 0x7FFFFFFFLL), 0x00020000);
    uint4 gv[kGroupSlots];
#pragma unroll
    for (int u = 0; u < kGroupSlots; ++u) {
        const int gi = tid + u * kTileThreads;
        gv[u] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(rv, gi * 16, 0, 0));
    }
    asm volatile("" ::: "memory");

    // 3. the slot -> run map (as in the staged tile kernel): runDelta[r] =
    //    first destination slot of the run of rank r - its first tile slot
    for (int w = tid; w < 2 * kWindows; w += kTileThreads) {
        startBits[w] = 0U;
        if (w < kWindows) firstRank[w] = 0U;
    }
    uint32_t cnt[kBtScanIpt];
#pragma unroll
    for (int u = 0; u < kBtScanIpt; ++u) {
        const int s = tid * kBtScanIpt + u;
        const uint32_t c = s < nb ? runB[u] - runA[u] : 0U;
        cnt[u] = c | (c != 0U ? 0x10000U : 0U);
    }
    Scan(scanStorage).ExclusiveSum(cnt, cnt);  // its barriers also order the clearing above
#pragma unroll
    for (int u = 0; u < kBtScanIpt; ++u) {
        const int s = tid * kBtScanIpt + u;
        const uint32_t c = s < nb ? runB[u] - runA[u] : 0U;
        if (c != 0U) {
            const uint32_t o = cnt[u] & 0xFFFFU, r = cnt[u] >> 16;
            runDelta[r] = runA[u] - o;
            atomicOr(&startBits[o >> 5], 1U << (o & 31U));
            for (uint32_t w = (o + 63U) >> 6; w * 64U < o + c; ++w) firstRank[w] = r;
        }
    }
    // row ends relative to the first group (uint16: at most a0 + E < 2^16),
    // at the start of the area
    uint16_t* rel = reinterpret_cast<uint16_t*>(area);
    const int relWords = ((R + 2 + 1) / 2 + 3) & ~3;
    float* xs = area + relWords;  // x over the entries of the current half
    const float4* xs4 = reinterpret_cast<const float4*>(xs);
#pragma unroll
    for (int u = 0; u < kBtPreRows; ++u) {
        const int i = tid + u * kTileThreads;
        const int64_t d = rowOff[u] - e0;
        if (i <= R) rel[i] = static_cast<uint16_t>(a0 + static_cast<int32_t>(d < 0 ? 0 : d > E ? E : d));
    }
    for (int i = tid + kBtPreRows * kTileThreads; i <= R; i += kTileThreads) {  // tiles of many short rows
        const int64_t d = Norm<RowT>(q, r0 + i) - e0;
        rel[i] = static_cast<uint16_t>(a0 + static_cast<int32_t>(d < 0 ? 0 : d > E ? E : d));
    }
    if (tid == 0) {
        rel[R + 1] = static_cast<uint16_t>(a0 + E);
        longCount[0] = 0;
        longCount[1] = 0;
    }
    __syncthreads();

    // 4. products in two halves of the tile's groups: each row's x over its
    //    entries of the half (xs, by entry; long rows by a wave), then the
    //    half's products into registers.  The tile's two edge groups also
    //    hold entries of the neighbouring tiles, which are skipped below.
    const int gs = ng / 2, em = gs * 4;
    // each group's products replace its values in gv (the same registers)
#pragma unroll
    for (int ph = 0; ph < 2; ++ph) {
        const int lo = ph == 0 ? 0 : em, hi = ph == 0 ? em : ng * 4;
        for (int loc = tid, u = 0; loc < nLoc; loc += kTileThreads, ++u) {
            int a = rel[loc], b = rel[loc + 1];
            a = a > lo ? a : lo;
            b = b < hi ? b : hi;
            if (b <= a) continue;
            if (b - a > kLongRow) {
                longRows[atomicAdd(&longCount[ph], 1)] = static_cast<uint16_t>(loc);
                continue;
            }
            float xv = 0.0f;
#pragma unroll
            for (int h = 0; h < kBtPreRows; ++h) xv = u == h ? xRow[h] : xv;
            if (u >= kBtPreRows) xv = static_cast<const float*>(q.x)[r0 + loc];
            for (int k = a; k < b; ++k) xs[k - lo] = xv;
        }
        __syncthreads();
        const int nLong = longCount[ph];
        for (int li = wv; li < nLong; li += kTileWaves) {
            const int loc = longRows[li];
            int a = rel[loc], b = rel[loc + 1];
            a = a > lo ? a : lo;
            b = b < hi ? b : hi;
            const float xv = static_cast<const float*>(q.x)[r0 + loc];
            for (int k = a + lane; k < b; k += kWave) xs[k - lo] = xv;
        }
        __syncthreads();
        const int gb = ph == 0 ? 0 : gs, ge = ph == 0 ? gs : ng;
#pragma unroll
        for (int u = 0; u < kGroupSlots; ++u) {
            const int gi = tid + u * kTileThreads;
            if (gi >= gb && gi < ge) {
                const float4 xv4 = xs4[gi - gb];
                gv[u] = make_uint4(__float_as_uint(__uint_as_float(gv[u].x) * xv4.x),
                                   __float_as_uint(__uint_as_float(gv[u].y) * xv4.y),
                                   __float_as_uint(__uint_as_float(gv[u].z) * xv4.z),
                                   __float_as_uint(__uint_as_float(gv[u].w) * xv4.w));
            }
        }
        __syncthreads();  // xs is overwritten next
    }

    // 5. the slots (loaded only now: fewer registers live at once), then the
    //    products at their slots and the tile's runs, in two halves of the
    //    slots split at a 64-slot window: slot i of the 64-slot windows of
    //    wave w goes to prod[runDelta[run(i)] + i]
    uint2 gp[kGroupSlots];
#pragma unroll
    for (int u = 0; u < kGroupSlots; ++u) {
        const int gi = tid + u * kTileThreads;
        gp[u] = __builtin_bit_cast(uint2, __builtin_amdgcn_raw_buffer_load_b64(rp, gi * 8, 0, 0));
    }
    constexpr int kHalfLanes = CeilDiv(kTileItems / 2 + 64, kTileThreads);  // 64-slot windows per wave and half
    const int H = (E / 2 + 63) & ~63;
    const uint32_t maskLo = lane < 32 ? (2U << lane) - 2U : 0xFFFFFFFEU;
    const uint32_t maskHi = lane < 32 ? 0U : (2U << (lane - 32)) - 1U;
#pragma unroll
    for (int ph = 0; ph < 2; ++ph) {
        const int s0 = ph == 0 ? 0 : H;
        const int s1 = ph == 0 ? (H < E ? H : E) : E;
#pragma unroll
        for (int u = 0; u < kGroupSlots; ++u) {
            const int gi = tid + u * kTileThreads;
            const int lo = a0 - gi * 4, hi = a0 + E - gi * 4;  // entries [lo, hi) of the group are the tile's
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                const uint32_t pw = k < 2 ? gp[u].x : gp[u].y;
                const int slot = static_cast<int>((pw >> ((k & 1) * 16)) & 0xFFFFU);
                const uint32_t pv = k == 0 ? gv[u].x : k == 1 ? gv[u].y : k == 2 ? gv[u].z : gv[u].w;
                if (k >= lo && k < hi && slot >= s0 && slot < s1) area[slot - s0] = __uint_as_float(pv);
            }
        }
        __syncthreads();
        const int n = s1 - s0;
        const int span = (n + kTileWaves * kWave - 1) / (kTileWaves * kWave) * kWave;
        const int i0 = s0 + __builtin_amdgcn_readfirstlane(wv) * span;
        const int i1 = i0 + span < s1 ? i0 + span : s1;
#pragma unroll
        for (int m = 0; m < kHalfLanes; ++m) {
            const int w = (i0 >> 6) + m;
            const int i = (w << 6) + lane;
            const uint32_t fr = firstRank[w < kWindows ? w : 0];
            const uint32_t bLo = startBits[2 * (w < kWindows ? w : 0)], bHi = startBits[2 * (w < kWindows ? w : 0) + 1];
            const uint32_t r = fr + static_cast<uint32_t>(__builtin_popcount(bLo & maskLo)) +
                               static_cast<uint32_t>(__builtin_popcount(bHi & maskHi));
            const uint32_t d = runDelta[r];
            const float v = area[i < i1 ? i - s0 : 0];
            if (i < i1) q.prod[d + static_cast<uint32_t>(i)] = v;
        }
        if (ph == 0) __syncthreads();  // the first half's runs are read before the second half is placed
    }
}

// Pass 2: the buckets' columns (see above).  Persistent: kBtColGrid
// workgroups, one per CU (the bucket region takes most of a CU's LDS), each
// taking buckets w, w + grid, ...  While a bucket's columns are summed from
// LDS, the next bucket's loads are in flight: its products and places (by
// 16-byte loads from the 8-entry boundary at or before its first slot;
// entries outside the bucket are read and dropped) and the offsets, and with
// beta != 0 the old y, of each thread's first kBtColPre columns.
constexpr int kBtColPre = 2;  // columns per thread prefetched
constexpr int kBtColRounds = CeilDiv(static_cast<int>(kBtRegionCap) + 7, 8 * kBtColThreads);
constexpr int kBtColGrid = 256;

struct BtBucketLoads {
    int64_t rs;  // the bucket's first slot
    int n;       // its entries
    int skew;    // rs minus the 8-entry boundary the loads start at
    uint4 pv[kBtColRounds][2];
    uint4 lv[kBtColRounds];
    int64_t pa[kBtColPre], pe[kBtColPre];
    float py[kBtColPre];
};

template <typename RowT>
__device__ __forceinline__ void BtLoadBucket(const StageParams& q, int64_t b, bool betaNz, int tid, BtBucketLoads& L)
{
    const RowT* colptr = static_cast<const RowT*>(q.colptr);
    const float* y = static_cast<const float*>(q.y);
    const int64_t c0 = b << q.wshift;
    const int64_t c1 = c0 + (int64_t{1} << q.wshift) < q.cols ? c0 + (int64_t{1} << q.wshift) : q.cols;
#pragma unroll
    for (int u = 0; u < kBtColPre; ++u) {
        const int64_t c = c0 + tid + u * kBtColThreads;
        L.pa[u] = static_cast<int64_t>(colptr[c < c1 ? c : c1]);
        L.pe[u] = static_cast<int64_t>(colptr[c < c1 ? c + 1 : c1]);
        L.py[u] = betaNz && c < c1 ? y[c] : 0.0f;
    }
    L.rs = static_cast<int64_t>(colptr[c0]);
    L.n = static_cast<int>(static_cast<int64_t>(colptr[c1]) - L.rs);
    const int64_t j0 = L.rs & ~int64_t{7};
    L.skew = static_cast<int>(L.rs - j0);
    // the resources end with the bucket: loads past it read zero without
    // touching memory (place bytes rounded up to a dword, since the range
    // check drops a dword that crosses the limit; st_cl is padded by 8 places)
    const int64_t avail = L.skew + L.n;
    const int pBytes = static_cast<int>(avail * 4), lBytes = static_cast<int>((avail * 2 + 3) & ~int64_t{3});
    const __amdgpu_buffer_rsrc_t rp = __builtin_amdgcn_make_buffer_rsrc(q.prod + j0, 0, pBytes, 0x00020000);
    const __amdgpu_buffer_rsrc_t rl = __builtin_amdgcn_make_buffer_rsrc(q.cl + j0, 0, lBytes, 0x00020000);
#pragma unroll
    for (int r = 0; r < kBtColRounds; ++r) {
        if (r * 8 * kBtColThreads >= L.skew + L.n) break;  // uniform over the workgroup
        const int i = r * 8 * kBtColThreads + tid * 8;
        L.pv[r][0] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(rp, i * 4, 0, 0));
        L.pv[r][1] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(rp, i * 4 + 16, 0, 0));
        L.lv[r] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(rl, i * 2, 0, 0));
    }
}

template <typename RowT>
__global__ __launch_bounds__(kBtColThreads) void BtColumnKernel(StageParams q)
{
    __shared__ float buf[kBtRegionCap];
    __shared__ int32_t longCols[kBtMaxLongCols];
    __shared__ int longCount;
    if (FlagSet(q.flag) != 1U) return;
    int64_t b = blockIdx.x;
    if (b >= q.buckets) return;
    const int tid = threadIdx.x;
    const int lane = tid & (kWave - 1);
    const int wv = tid / kWave;
    const RowT* colptr = static_cast<const RowT*>(q.colptr);
    float alpha, beta;
    LoadScalars<AccKind::F32>(q.s, alpha, beta);
    const bool betaNz = beta != 0.0f;  // y is not read when beta == 0, wherever beta lives
    float* y = static_cast<float*>(q.y);
    BtBucketLoads cur;
    BtLoadBucket<RowT>(q, b, betaNz, tid, cur);
    for (; b < q.buckets; b += gridDim.x) {
        const int64_t c0 = b << q.wshift;
        const int64_t c1 = c0 + (int64_t{1} << q.wshift) < q.cols ? c0 + (int64_t{1} << q.wshift) : q.cols;
        const int64_t rs = cur.rs;
        const int n = cur.n;
        // products to their column-order places
#pragma unroll
        for (int r = 0; r < kBtColRounds; ++r) {
            if (r * 8 * kBtColThreads >= cur.skew + n) break;
            const int i = r * 8 * kBtColThreads + tid * 8 - cur.skew;  // the bucket's entry of the first lane slot
#pragma unroll
            for (int k = 0; k < 8; ++k) {
                const uint32_t w = WordOf(cur.lv[r], k >> 1);
                const uint32_t place = (k & 1) ? w >> 16 : w & 0xFFFFU;
                if (i + k >= 0 && i + k < n) buf[place] = __uint_as_float(WordOf(cur.pv[r][k >> 2], k & 3));
            }
        }
        if (tid == 0) longCount = 0;
        __syncthreads();
        int64_t pa[kBtColPre], pe[kBtColPre];
        float py[kBtColPre];
#pragma unroll
        for (int u = 0; u < kBtColPre; ++u) {
            pa[u] = cur.pa[u];
            pe[u] = cur.pe[u];
            py[u] = cur.py[u];
        }
        if (b + gridDim.x < q.buckets) BtLoadBucket<RowT>(q, b + gridDim.x, betaNz, tid, cur);  // uniform
        asm volatile("" ::: "memory");
        auto column = [&](int64_t c, int64_t ca, int64_t ce, float old) {
            const int a = static_cast<int>(ca - rs);
            const int e = static_cast<int>(ce - rs);
            if (e - a > kBtLongCol) {
                longCols[atomicAdd(&longCount, 1)] = static_cast<int32_t>(c - c0);
                return;
            }
            float sum = 0.0f;
            for (int k = a; k < e; ++k) sum += buf[k];
            StoreRowOld<OutKind::F32, AccKind::F32>(y, c, sum, alpha, beta, betaNz, old);
        };
#pragma unroll
        for (int u = 0; u < kBtColPre; ++u) {
            const int64_t c = c0 + tid + u * kBtColThreads;
            if (c < c1) column(c, pa[u], pe[u], py[u]);
        }
        for (int64_t c = c0 + tid + kBtColPre * kBtColThreads; c < c1; c += kBtColThreads) {
            column(c, static_cast<int64_t>(colptr[c]), static_cast<int64_t>(colptr[c + 1]), betaNz ? y[c] : 0.0f);
        }
        __syncthreads();
        const int nLong = longCount;
        for (int li = wv; li < nLong; li += kBtColThreads / kWave) {
            const int64_t c = c0 + longCols[li];
            const int a = static_cast<int>(static_cast<int64_t>(colptr[c]) - rs);
            const int e = static_cast<int>(static_cast<int64_t>(colptr[c + 1]) - rs);
            float part = 0.0f;
            for (int k = a + lane; k < e; k += kWave) part += buf[k];
            const float sum = WaveSum(part);
            if (lane == 0) StoreRow<OutKind::F32, AccKind::F32>(y, c, sum, alpha, beta, betaNz);
        }
        __syncthreads();  // the region is free for the next bucket
    }
}

// ------------------------------- launchers ----------------------------------

template <typename T>
T* At(void* ws, size_t off) { return reinterpret_cast<T*>(static_cast<uint8_t*>(ws) + off); }

StageParams MakeStageParams(const SpmvLaunch& l)
{
    const SpmvLayout& L = l.layout;
    StageParams q{};
    q.norm = At<void>(l.ws, L.rowptr_offset);
    q.col = l.col;
    q.base = l.base;
    q.buckets = L.st_buckets;
    q.wshift = L.st_wshift;
    q.line_shift = L.st_value_bytes == 4 ? 5 : 6;  // 32 or 64 values per 128-byte line
    q.val = l.val;
    q.x = l.x;
    q.y = l.y;
    q.rows = l.rows;
    q.cols = l.cols;
    q.nnz = l.nnz;
    q.tiles = L.st_tiles;
    q.tile_row = At<int32_t>(l.ws, L.st_tile_row_offset);
    q.tile_nnz = At<int64_t>(l.ws, L.st_tile_nnz_offset);
    q.counts = At<uint32_t>(l.ws, L.st_counts_offset);
    q.start_bm = At<uint32_t>(l.ws, L.st_start_bm_offset);
    q.start = At<uint32_t>(l.ws, L.st_start_offset);
    q.perm = At<uint16_t>(l.ws, L.st_perm_offset);
    q.cl = At<uint16_t>(l.ws, L.st_cl_offset);
    q.xg = At<void>(l.ws, L.st_xg_offset);
    q.head = At<float>(l.ws, L.st_head_offset);
    q.tail = At<float>(l.ws, L.st_tail_offset);
    q.metric = At<unsigned long long>(l.ws, L.st_metric_offset);
    q.flag = &At<SpmvWsHeader>(l.ws, 0)->staged_flag;
    q.part = L.st_part_size;
    q.rp16 = l.narrow && L.narrow ? At<uint16_t>(l.ws, L.nr_offset) : nullptr;
    q.tile_items = L.st_tile_items;
    // the one-pass banded transpose: 32-bit row offsets and positions whose
    // byte offsets fit a buffer resource (LaunchBandedTranspose)
    q.banded_ok = !l.rowptr64 && l.nnz <= 0x1FFFFFFFLL ? 1 : 0;
    q.chunk = L.st_value_bytes > 0 ? static_cast<int32_t>(StageChunkSlots(static_cast<uint32_t>(L.st_value_bytes))) : 1;
    q.colptr = At<void>(l.ws, L.colptr_offset);
    q.csc_pos = At<void>(l.ws, L.csc_pos_offset);
    q.inv = At<int32_t>(l.ws, L.key_b_offset);  // free once the CSC build is done
    q.entry_row = At<const int32_t>(l.ws, L.entry_row_offset);
    q.prod = At<float>(l.ws, L.prod_offset);
    q.s.device = l.device_scalars;
    q.s.alpha_re = l.alpha_re;
    q.s.beta_re = l.beta_re;
    q.s.alpha_ptr = l.alpha_ptr;
    q.s.beta_ptr = l.beta_ptr;
    return q;
}

unsigned XcdGrid(int64_t n) { return static_cast<unsigned>((n + kXcds - 1) / kXcds * kXcds); }

template <typename RowT>
int StagedPreprocessTyped(const SpmvLaunch& l, hipStream_t s)
{
    const SpmvLayout& L = l.layout;
    StageParams q = MakeStageParams(l);
    const int64_t T = L.st_tiles;
    hipLaunchKernelGGL((StageTileSplitKernel<RowT>), dim3(static_cast<unsigned>((T + 1 + 255) / 256)), dim3(256), 0,
                       s, q);
    hipLaunchKernelGGL(StageCountKernel, dim3(static_cast<unsigned>(T + 1)), dim3(kSortThreads), 0, s, q);
    hipLaunchKernelGGL(StageDecideKernel, dim3(1), dim3(1), 0, s, q);  // the rank kernel runs only when staged
    const int64_t cells = static_cast<int64_t>(L.st_buckets + 1) * (T + 1);
    void* temp = reinterpret_cast<void*>(
        (reinterpret_cast<uintptr_t>(At<uint8_t>(l.ws, L.st_scan_offset)) + 255) & ~uintptr_t{255});
    size_t tempBytes = L.st_scan_bytes;
    if (hipcub::DeviceScan::ExclusiveSum(temp, tempBytes, q.counts, q.start_bm, static_cast<int>(cells), s) !=
        hipSuccess) {
        return 1;
    }
    hipLaunchKernelGGL(StageTransposeKernel,
                       dim3(static_cast<unsigned>((T + 1 + 31) / 32), static_cast<unsigned>((L.st_buckets + 1 + 31) / 32)),
                       dim3(32, 8), 0, s, q);
    if (q.tile_items == kWide) {
        hipLaunchKernelGGL((StageRankKernel<kWide, kSortThreads>), dim3(static_cast<unsigned>(T)),
                           dim3(kSortThreads), 0, s, q);
    } else {
        hipLaunchKernelGGL((StageRankKernel<kNarrow, kSortThreads>), dim3(static_cast<unsigned>(T)),
                           dim3(kSortThreads), 0, s, q);
    }
    return 0;
}

template <typename RowT>
int BtPreprocessTyped(const SpmvLaunch& l, hipStream_t s)
{
    const SpmvLayout& L = l.layout;
    StageParams q = MakeStageParams(l);
    const int64_t T = L.st_tiles;
    hipLaunchKernelGGL((StageTileSplitKernel<RowT>), dim3(static_cast<unsigned>((T + 1 + 255) / 256)), dim3(256), 0,
                       s, q);
    hipLaunchKernelGGL((BtInvertKernel<RowT>), dim3(static_cast<unsigned>((l.nnz + 255) / 256)), dim3(256), 0, s, q);
    hipLaunchKernelGGL((BtCountKernel<RowT>), dim3(static_cast<unsigned>(T + 1)), dim3(kSortThreads), 0, s, q);
    const int64_t cells = static_cast<int64_t>(L.st_buckets + 1) * (T + 1);
    void* temp = reinterpret_cast<void*>(
        (reinterpret_cast<uintptr_t>(At<uint8_t>(l.ws, L.st_scan_offset)) + 255) & ~uintptr_t{255});
    size_t tempBytes = L.st_scan_bytes;
    if (hipcub::DeviceScan::ExclusiveSum(temp, tempBytes, q.counts, q.start_bm, static_cast<int>(cells), s) !=
        hipSuccess) {
        return 1;
    }
    hipLaunchKernelGGL(StageTransposeKernel,
                       dim3(static_cast<unsigned>((T + 1 + 31) / 32), static_cast<unsigned>((L.st_buckets + 1 + 31) / 32)),
                       dim3(32, 8), 0, s, q);
    hipLaunchKernelGGL((BtRankKernel<kWide, RowT>), dim3(static_cast<unsigned>(T)), dim3(kSortThreads), 0, s, q);
    hipLaunchKernelGGL((BtDecideKernel<RowT>), dim3(1), dim3(256), 0, s, q);
    hipLaunchKernelGGL((BtCscRowKernel<RowT>), dim3(static_cast<unsigned>((l.nnz + 255) / 256)), dim3(256), 0, s, q);
    return 0;
}

template <typename RowT>
void BtComputeTyped(const SpmvLaunch& l, hipStream_t s)
{
    const StageParams q = MakeStageParams(l);
    hipLaunchKernelGGL((BtScatterKernel<kWide, RowT>), dim3(XcdGrid(l.layout.st_tiles)), dim3(kTileThreads),
                       BtScatterLdsBytes(l.layout.st_buckets + 1), s, q);
    const int64_t colGrid = l.layout.st_buckets < kBtColGrid ? l.layout.st_buckets : kBtColGrid;
    hipLaunchKernelGGL((BtColumnKernel<RowT>), dim3(static_cast<unsigned>(colGrid)), dim3(kBtColThreads), 0, s, q);
}

template <typename RowT, ValKind V, OutKind O>
void LaunchStagedTyped(const SpmvLaunch& l, const StageParams& q, hipStream_t s)
{
    using Raw = typename StageVal<V>::Raw;
    const SpmvLayout& L = l.layout;
    hipLaunchKernelGGL((StageGatherKernel<Raw>), dim3(XcdGrid(L.st_parts)), dim3(kGatherThreads),
                       static_cast<unsigned>(kStageSegmentBytes), s, q);
    // fp32 values: the narrow tiles; fp16 / bf16: the wide ones (StageTileItems)
    constexpr int kItems = V == ValKind::F32 ? kNarrow : kWide;
    const unsigned lds = static_cast<unsigned>(TileLds<kItems, Raw>::DynBytes(L.st_buckets + 1));
    if (q.rp16 != nullptr) {
        hipLaunchKernelGGL((StageTileKernel<kItems, RowT, V, O, true>), dim3(XcdGrid(L.st_tiles)), dim3(kTileThreads),
                           lds, s, q);
    } else {
        hipLaunchKernelGGL((StageTileKernel<kItems, RowT, V, O, false>), dim3(XcdGrid(L.st_tiles)), dim3(kTileThreads),
                           lds, s, q);
    }
    hipLaunchKernelGGL((StageFixupKernel<RowT, O>), dim3(static_cast<unsigned>((L.st_tiles + 255) / 256)), dim3(256),
                       0, s, q);
}

template <typename RowT>
int LaunchStagedRowT(const SpmvLaunch& l, hipStream_t s)
{
    const StageParams q = MakeStageParams(l);
    switch (l.val_kind) {
        case ValKind::F32: LaunchStagedTyped<RowT, ValKind::F32, OutKind::F32>(l, q, s); return 0;
        case ValKind::F16:
            if (l.out_kind == OutKind::F16) LaunchStagedTyped<RowT, ValKind::F16, OutKind::F16>(l, q, s);
            else LaunchStagedTyped<RowT, ValKind::F16, OutKind::F32>(l, q, s);
            return 0;
        case ValKind::BF16:
            if (l.out_kind == OutKind::BF16) LaunchStagedTyped<RowT, ValKind::BF16, OutKind::BF16>(l, q, s);
            else LaunchStagedTyped<RowT, ValKind::BF16, OutKind::F32>(l, q, s);
            return 0;
        default: return 1;
    }
}

// Pass A's dynamic LDS (128 KiB) is beyond the 64 KiB that older parts
// allow; gfx950 has 160 KiB per workgroup.  The attribute is set once, and a
// runtime that does not need it may decline it (the launch reports real
// failures).
template <typename XT>
void AllowGatherLds()
{
    static const bool once = [] {
        (void)hipFuncSetAttribute(reinterpret_cast<const void*>(&StageGatherKernel<XT>),
                                  hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(kStageSegmentBytes));
        (void)hipGetLastError();
        return true;
    }();
    (void)once;
}

}  // namespace

size_t StageScanTempBytes(int64_t n)
{
    size_t bytes = 0;
    if (hipcub::DeviceScan::ExclusiveSum(nullptr, bytes, static_cast<uint32_t*>(nullptr),
                                         static_cast<uint32_t*>(nullptr), static_cast<int>(n)) != hipSuccess) {
        bytes = static_cast<size_t>(n) * 8 + (1 << 20);
    }
    return bytes;
}

int LaunchStagedPreprocess(const SpmvLaunch& l, void* stream)
{
    hipStream_t s = static_cast<hipStream_t>(stream);
    if (!l.layout.staged) return 1;
    if (l.op != ACL_SPARSE_OP_NON_TRANSPOSE) {
        return l.rowptr64 ? BtPreprocessTyped<int64_t>(l, s) : BtPreprocessTyped<int32_t>(l, s);
    }
    return l.rowptr64 ? StagedPreprocessTyped<int64_t>(l, s) : StagedPreprocessTyped<int32_t>(l, s);
}

int LaunchStagedCompute(const SpmvLaunch& l, void* stream)
{
    hipStream_t s = static_cast<hipStream_t>(stream);
    if (!l.layout.staged) return 1;
    if (l.op != ACL_SPARSE_OP_NON_TRANSPOSE) {
        if (l.val_kind != ValKind::F32 || l.out_kind != OutKind::F32) return 1;
        if (l.rowptr64) BtComputeTyped<int64_t>(l, s);
        else BtComputeTyped<int32_t>(l, s);
        return 0;
    }
    if (l.layout.st_value_bytes == 4) AllowGatherLds<uint32_t>();
    else AllowGatherLds<uint16_t>();
    return l.rowptr64 ? LaunchStagedRowT<int64_t>(l, s) : LaunchStagedRowT<int32_t>(l, s);
}

}  // namespace aclsp
