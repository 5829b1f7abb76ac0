// gfx950 kernels of the CSR SpMV path: y = alpha*op(A)*x + beta*y.
//
// Design (one GPU, HBM-bound, no MFMA):
//  * Preprocess: one launch normalises the row offsets (rowPtr[i*stride]-base,
//    clamped to [0, nnz]) into the workspace and computes the row-block
//    partition: block b owns the rows whose weighted merge-path coordinate
//    (16*row + rowOffset[row]) lies in [b*T, (b+1)*T), T <= 2032.  A block
//    has at most 127 rows (two per lane of a wave64) and about 500
//    non-zeros; only a row longer than that makes its block longer.  Blocks
//    of more than kLongChunks chunks are split into one task per 512-entry
//    chunk (task table: count, hipCUB scan, fill).  Reference counterpart:
//    the normalising kernel sparse/spmv/arch35/spmv_kernel.cpp:1144-1163
//    (one block, scalar loop).
//  * Non-transpose, real x/y (SpmvStreamFlatKernel): one wave64 per row
//    block, 4 waves per workgroup.  col_ind/values stream through 16-byte
//    buffer loads in 512-slot chunks, x is gathered, the products go to LDS
//    and rows are reduced by lane groups (short rows) or by the whole wave
//    (long rows, with a carried partial sum).  The first workgroups serve the
//    long-block tasks; the last task of a block combines the partial sums of
//    the rows that cross its chunks.  Replaces the warp-per-row kernel
//    sparse/spmv/arch35/spmv_kernel.cpp:501-577.  int8 and complex operands
//    (and real A with complex y) run on the same row blocks and chunk loads
//    with an int64 / complex accumulator (SpmvStreamGenKernel); strided or
//    unaligned operands use the general LDS-scan kernel (SpmvRowBlockKernel).
//  * Transpose: Preprocess builds a CSC pattern (radix sort of (column,
//    position) pairs); each SpMV streams the products a_k*x_row(k) in CSR
//    order and then sums every column's products in a fixed order
//    (deterministic, the reference's CSR_ALG2 semantics,
//    sparse/spmv/arch35/spmv_kernel.cpp:861-879).  Transposes beyond the
//    sort's int range (nnz > INT32_MAX) are rejected by the host.
//  * Block ids are remapped so that each of the 8 XCDs processes one
//    contiguous eighth of the matrix (x neighbourhoods stay in one L2).
#include <hip/hip_runtime.h>
#include <hipcub/hipcub.hpp>

#include <cstdint>
#include <cstdlib>
#include <type_traits>

#include "aclsparse_internal.h"
#include "compensated.h"
#include "spmv_device.h"

namespace aclsp {
namespace {

using namespace dev;

constexpr int kThreads = 256;
constexpr int kWave = 64;
constexpr int kWaves = kThreads / kWave;
constexpr int kChunk = 2048;                          // LDS product slots of the block kernel
constexpr int kIpt = kChunk / kThreads;               // 8 items per lane in the scan
constexpr int kMaxRows = static_cast<int>(kMaxRowsPerBlock);
constexpr int kXcds = 8;
constexpr int kPadded = kChunk + kChunk / kIpt;

static_assert(kChunk % (4 * kThreads) == 0, "chunk must be a multiple of one 16-byte load per lane");

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v2i __attribute__((ext_vector_type(2)));
typedef float v4f __attribute__((ext_vector_type(4)));
typedef float v2f __attribute__((ext_vector_type(2)));
typedef unsigned short v4u16 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ int Pad(int q) { return q + (q >> 3); }

// ------------------------------ shuffles ------------------------------------

__device__ __forceinline__ float ShflUp(float v, int d) { return __shfl_up(v, d, kWave); }
__device__ __forceinline__ long long ShflUp(long long v, int d) { return __shfl_up(v, d, kWave); }
__device__ __forceinline__ C64 ShflUp(C64 v, int d) { return C64{__shfl_up(v.re, d, kWave), __shfl_up(v.im, d, kWave)}; }

// ------------------------------ block mapping -------------------------------

// Hardware hands consecutive workgroup ids to the 8 XCDs round-robin.  Remap
// so that XCD k processes the contiguous block range [k*per, (k+1)*per).
__device__ __forceinline__ int64_t XcdBlock()
{
    const int64_t per = gridDim.x / kXcds;
    return static_cast<int64_t>(blockIdx.x % kXcds) * per + blockIdx.x / kXcds;
}

// ------------------------------ kernel params -------------------------------

struct RowBlockParams {
    const void* rp;          // normalised row offsets (RowT), rows+1
    const int32_t* blocks;   // num_blocks+1 block start rows
    const void* block_nnz;   // num_blocks+1 block start offsets (RowT)
    const int32_t* col;
    int64_t col_stride;
    const void* val;
    int64_t val_stride;
    const void* x;
    int64_t x_stride;
    void* y;                 // N: y; T: y (float/complex) or accumulator
    int64_t y_stride;
    int64_t rows, cols, nnz;
    int64_t num_blocks;
    int32_t base;
    int32_t conj;
    Scalars s;
    void* sink;  // per-lane dummy outputs
    // long-block tasks (see SpmvLayout): tables built by Preprocess
    const int32_t* task_start;
    const int32_t* task_block;
    float* task_head;
    float* task_tail;
    uint32_t* task_cnt;
    int32_t task_waves;  // waves serving tasks (0: tasks off)
    int32_t task_wgs;    // workgroups serving tasks (the first ones of the grid)
    int64_t max_tasks;   // capacity of the task arrays
    float* z;            // SpMVOp: output (y is then only read)
    int64_t rp_base;     // subtracted from p.rp entries (0 for the normalised copy)
    int32_t fixed_rows;  // SpMVOp ALG1: rows per block, blocks taken straight from p.rp
    // When set, the stream kernel exits at once unless bit (word) of run_mask
    // is set: Preprocess chose another path for this matrix (the staged
    // gather, the column-bucketed or the one-pass banded transpose, the
    // narrow columns), whose kernels are launched beside this one.
    const uint32_t* skip_flag;
    uint32_t run_mask;
    // narrow columns: column - base - (first row of the entry's block), int16[nnz]
    const int16_t* ncol;
    // with ncol: the low 16 bits of the normalised row offsets, uint16[rows+2]
    // (a row block of at most kLongChunks chunks spans fewer than 65536
    // entries, so its rows' offsets from its first entry follow from them)
    const uint16_t* rp16;
    // GATH with ncol: each streamed position as an offset from the entry's own
    // index in the streamed arrays, int16[nnz]
    const int16_t* npos;
    // ValKind::GATH: the fp32 values the streamed positions index
    const float* gval;
    int64_t gval_n;
    // Stream kernel: when > 0, the grid is capped and each wave loops over
    // the blocks tile, tile + block_stride, ... (block_stride = all block waves)
    int64_t block_stride;
};

// Loads the block's row offsets relative to its first non-zero into LDS.
template <typename RowT>
__device__ __forceinline__ int LoadBlockRows(const RowBlockParams& p, int64_t b, int32_t* sRp, int64_t& r0,
                                             int64_t& k0)
{
    const RowT* rp = static_cast<const RowT*>(p.rp);
    r0 = p.blocks[b];
    int64_t n = static_cast<int64_t>(p.blocks[b + 1]) - r0;
    n = n < 0 ? 0 : n > kMaxRows ? kMaxRows : n;
    const int nr = static_cast<int>(n);
    k0 = static_cast<int64_t>(rp[r0]);
    for (int i = threadIdx.x; i <= nr; i += kThreads) {
        int64_t v = static_cast<int64_t>(rp[r0 + i]) - k0;
        v = v < 0 ? 0 : v > 0x7FFFFFFFLL ? 0x7FFFFFFFLL : v;
        sRp[i] = static_cast<int32_t>(v);
    }
    return nr;
}

// First index i in [lo, hi) with key(i) >= target (keys non-decreasing).
__device__ __forceinline__ int LowerBound(const int32_t* a, int lo, int hi, int32_t target)
{
    while (lo < hi) {
        const int mid = (lo + hi) >> 1;
        if (a[mid] < target) lo = mid + 1;
        else hi = mid;
    }
    return lo;
}

// Product a_p * x[col_p] (zero when p is outside [lo, hi) or col is out of range).
template <ValKind V, AccKind A>
__device__ __forceinline__ typename AccOf<A>::T Product(typename ValOf<V>::T a, int32_t rawCol,
                                                        const typename ValOf<V>::T* x, int64_t xStride,
                                                        int32_t base, int64_t cols, bool valid)
{
    using Acc = typename AccOf<A>::T;
    const int64_t c = static_cast<int64_t>(rawCol) - base;
    if (!valid || c < 0 || c >= cols) return Zero<Acc>();
    return ToAcc<V, A>(a) * ToAcc<V, A>(x[c * xStride]);
}

// ------------------------- non-transpose row blocks -------------------------

template <typename RowT, ValKind V, OutKind O, AccKind A>
__global__ __launch_bounds__(kThreads) void SpmvRowBlockKernel(RowBlockParams p)
{
    using Acc = typename AccOf<A>::T;
    using ValT = typename ValOf<V>::T;
    using OutT = typename OutOf<O>::T;

    __shared__ int32_t sRp[kMaxRows + 1];
    __shared__ Acc sVal[kPadded];
    __shared__ uint32_t sFlagWords[kChunk / 4];
    __shared__ Acc sCarry[kThreads];
    __shared__ int32_t sFirst[kThreads];
    __shared__ Acc sWaveV[kWaves];
    __shared__ int32_t sWaveF[kWaves];
    __shared__ Acc sChunkCarry;
    uint8_t* sFlag = reinterpret_cast<uint8_t*>(sFlagWords);

    const int64_t b = XcdBlock();
    if (b >= p.num_blocks) return;
    const int tid = threadIdx.x;
    const int lane = tid & (kWave - 1);
    const int wave = tid / kWave;

    int64_t r0, k0;
    const int nr = LoadBlockRows<RowT>(p, b, sRp, r0, k0);
    Acc alpha, beta;
    LoadScalars<A>(p.s, alpha, beta);
    const bool betaNz = !IsZero(beta);
    const ValT* val = static_cast<const ValT*>(p.val);
    const ValT* x = static_cast<const ValT*>(p.x);
    OutT* y = static_cast<OutT*>(p.y);
    if (tid == 0) sChunkCarry = Zero<Acc>();
    __syncthreads();

    const int32_t kspan = sRp[nr];
    int32_t c0 = 0;
    for (;;) {
        const int64_t gStart = k0 + c0;
        const int64_t a0 = gStart;
        const int32_t d = static_cast<int32_t>(k0 - a0);  // LDS slot of relative offset r is r + d
        const int32_t lim = static_cast<int32_t>(a0 - k0) + kChunk;
        const int32_t c1 = kspan < lim ? kspan : lim;
        const bool last = c1 >= kspan;
        const int64_t gEnd = k0 + c1;

        for (int w = tid; w < kChunk / 4; w += kThreads) sFlagWords[w] = 0U;

        // Read col_ind / values of [gStart, gEnd) (any strides) and form the products.
        for (int q = tid; q < kChunk; q += kThreads) {
            const int64_t g = a0 + q;
            Acc prod = Zero<Acc>();
            if (g < gEnd) {
                prod = Product<V, A>(val[g * p.val_stride], p.col[g * p.col_stride], x, p.x_stride, p.base,
                                     p.cols, true);
            }
            sVal[Pad(q)] = prod;
        }

        __syncthreads();  // flag words are cleared before any lane sets a head

        // Rows that can touch this chunk.
        int lo = 0, hi = nr;
        if (!(c0 == 0 && last)) {
            lo = LowerBound(sRp + 1, 0, nr, c0);
            if (!last) hi = LowerBound(sRp, lo, nr, c1);
        }
        // Segment heads: the first non-zero of every non-empty row in the chunk.
        for (int i = lo + tid; i < hi; i += kThreads) {
            const int32_t s = sRp[i], e = sRp[i + 1];
            if (e > s && s >= c0 && s < c1) sFlag[s + d] = 1;
        }
        __syncthreads();

        // Per-lane segmented inclusive scan of 8 consecutive products.
        Acc run = Zero<Acc>();
        int first = kIpt;
#pragma unroll
        for (int j = 0; j < kIpt; ++j) {
            const int q = tid * kIpt + j;
            if (sFlag[q]) {
                if (first == kIpt) first = j;
                run = Zero<Acc>();
            }
            run = run + sVal[Pad(q)];
            sVal[Pad(q)] = run;
        }
        const int has = first < kIpt ? 1 : 0;

        // Block-wide exclusive segmented scan of the lane tails.
        Acc v = run;
        int f = has;
#pragma unroll
        for (int off = 1; off < kWave; off <<= 1) {
            const Acc vo = ShflUp(v, off);
            const int fo = __shfl_up(f, off, kWave);
            if (lane >= off) {
                if (!f) v = vo + v;
                f |= fo;
            }
        }
        Acc ve = ShflUp(v, 1);
        int fe = __shfl_up(f, 1, kWave);
        if (lane == 0) {
            ve = Zero<Acc>();
            fe = 0;
        }
        if (lane == kWave - 1) {
            sWaveV[wave] = v;
            sWaveF[wave] = f;
        }
        __syncthreads();
        Acc pv = sChunkCarry;
        for (int u = 0; u < wave; ++u) {
            if (sWaveF[u]) pv = sWaveV[u];
            else pv = pv + sWaveV[u];
        }
        const Acc excl = fe ? ve : pv + ve;
        sCarry[tid] = excl;
        sFirst[tid] = first;
        const Acc chunkTotal = has ? run : excl + run;  // meaningful on the last lane
        __syncthreads();

        // Finish the rows that end inside this chunk.
        for (int i = lo + tid; i < hi; i += kThreads) {
            const int32_t s = sRp[i], e = sRp[i + 1];
            if (e <= s) {
                if ((s >= c0 && s < c1) || (last && s >= c1)) {
                    StoreRow<O, A>(y, (r0 + i) * p.y_stride, Zero<Acc>(), alpha, beta, betaNz);
                }
            } else if (e > c0 && e <= c1) {
                const int q = e - 1 + d;
                const int t = q / kIpt;
                Acc sum = sVal[Pad(q)];
                if ((q % kIpt) < sFirst[t]) sum = sum + sCarry[t];
                StoreRow<O, A>(y, (r0 + i) * p.y_stride, sum, alpha, beta, betaNz);
            }
        }
        if (last) break;
        __syncthreads();
        if (tid == kThreads - 1) sChunkCarry = chunkTotal;
        c0 = c1;
        __syncthreads();
    }
}


// ------------------------ wave-per-block stream kernels ---------------------
//
// One wave64 owns one row block (<= 127 rows, ~500 non-zeros) at a time and
// reads it in chunks of 512 slots, 8 per lane.

constexpr int kWaveChunk = static_cast<int>(kChunkNnz);  // 512 slots, 8 per lane
constexpr int kLaneItems = kWaveChunk / kWave;           // 8
constexpr int kWaveRows = static_cast<int>(kMaxRowsPerBlock);
// Waves per workgroup of the stream kernels: one.  On the Laplacian after
// Preprocess (narrow columns, entry-aligned blocks, banded transposes) one
// wave per workgroup measured 0.3-2.5 µs faster than four (and than two);
// eight were slower.  Without Preprocess the power-law c3 takes 2.08 ms
// against 2.04 ms with four.
constexpr int kFlatWaves = 1;
// Block workgroups of the stream kernel when the staged path may take the
// matrix instead (multiple of the XCD count).
constexpr int64_t kStagedFallbackWgs = 2048;

static_assert(kLaneItems == 8, "the reductions are written for 8 slots per lane");
static_assert(kWaveRows <= 2 * kWave - 1, "two rows per lane");

struct Stage {
    int64_t tile;   // ordinal of the block among this worker's blocks
    int64_t r0;     // first row
    int64_t k0;     // first non-zero (normalised offset of r0)
    int64_t a0;     // 16-byte aligned global start of this chunk
    int32_t nr;     // rows in the block
    int32_t kspan;  // non-zeros in the block
    int32_t c0, c1; // chunk range, relative to k0
    bool first, last, valid;
};

__device__ __forceinline__ void ChunkBounds(Stage& s)
{
    const int64_t gStart = s.k0 + s.c0;
    s.a0 = gStart & ~static_cast<int64_t>(3);
    const int32_t lim = static_cast<int32_t>(s.a0 - s.k0) + kWaveChunk;
    s.c1 = s.kspan < lim ? s.kspan : lim;
    s.last = s.c1 >= s.kspan;
}

// The partition arrays do not change while a kernel runs: read them through
// the constant address space so that the (wave-uniform) reads become scalar
// loads, which never wait on the vector-memory counter of the prefetches.
template <typename T>
__device__ __forceinline__ T ConstLoad(const void* base, int64_t i)
{
    typedef const __attribute__((address_space(4))) T* CPtr;
    return reinterpret_cast<CPtr>(reinterpret_cast<uintptr_t>(base))[i];
}

// LDS byte address of a pointer into __shared__ memory (for inline asm).
__device__ __forceinline__ uint32_t LdsAddr(const float* p)
{
    typedef const __attribute__((address_space(3))) float* LdsPtr;
    return static_cast<uint32_t>(reinterpret_cast<uintptr_t>((LdsPtr)(p)));
}

__device__ __forceinline__ void WaveLdsSync() { asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory"); }

__device__ __forceinline__ float ReadLane(float v, int l) { return __shfl(v, l, kWave); }
__device__ __forceinline__ long long ReadLane(long long v, int l) { return __shfl(v, l, kWave); }
__device__ __forceinline__ C64 ReadLane(C64 v, int l) { return C64{__shfl(v.re, l, kWave), __shfl(v.im, l, kWave)}; }
__device__ __forceinline__ float ShflXorAcc(float v, int m) { return __shfl_xor(v, m, kWave); }
__device__ __forceinline__ int32_t ShflXorAcc(int32_t v, int m) { return __shfl_xor(v, m, kWave); }
__device__ __forceinline__ int32_t ReadLane(int32_t v, int l) { return __shfl(v, l, kWave); }
__device__ __forceinline__ long long ShflXorAcc(long long v, int m) { return __shfl_xor(v, m, kWave); }
__device__ __forceinline__ C64 ShflXorAcc(C64 v, int m)
{
    return C64{__shfl_xor(v.re, m, kWave), __shfl_xor(v.im, m, kWave)};
}


// ------------------------- stream row kernel (fp32 sums) ---------------------
//
// The same row blocks and 512-slot chunks as the kernel above, one block per
// wave (no persistence), with a cheaper reduction for the common case of
// short rows:
//  * col_ind / values are read with 16-byte buffer loads whose resource
//    starts at the chunk (a scalar base, a constant per-lane offset) and
//    ends at the chunk's last non-zero (rounded up to a 16-byte group), so
//    loads past it return zero without a memory request; x is gathered
//    through a resource bounded by the vector's length (32-bit offsets), and
//    slots past the chunk gather nothing;
//  * the products of a chunk go to the wave's LDS slice in slot order;
//  * phase 1: rows that lie inside the chunk and are short (SerialCap) are
//    summed from LDS by groups of G lanes (G = 1 for blocks of many short
//    rows, up to 64 for a block of one row), then reduced across the group;
//  * phase 2: the remaining rows (longer ones, and the rows that continue
//    from the previous chunk or into the next) are summed by the whole wave,
//    one after another; a row that crosses a chunk boundary carries its
//    partial sum in a scalar register.
// Rows 2l and 2l+1 of a block are owned by lane l, which writes y or, when a
// row does not finish in this chunk, the sink, so every lane issues the same
// stores in every chunk.

// Phase-1 row length limit: 8 entries for one lane per row, 16 per lane for
// groups (rows of medium length, few rows per block).
constexpr int kSerialCapOne = 8;
__device__ __forceinline__ int SerialCap(int lg) { return lg == 0 ? kSerialCapOne : (16 << lg); }

__device__ __forceinline__ __amdgpu_buffer_rsrc_t Rsrc(const void* base, int64_t bytes)
{
    const int64_t b = bytes < 0 ? 0 : bytes > 0x7FFFFFFFLL ? 0x7FFFFFFFLL : bytes;
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, static_cast<int>(b), 0x00020000);
}

constexpr int kBufNonTemporal = 2;  // cache policy bit of buffer loads: streaming data
constexpr int kGatherPolicy = 0;  // x gathers: default cache policy (the cached lines are reused)
constexpr int kRowPolicy = 0;  // row offsets / old y: default cache policy

template <ValKind V>
struct StreamVals;
template <>
struct StreamVals<ValKind::F32> {
    v4f v[2];
};
template <>
struct StreamVals<ValKind::F16> {
    v4i v;  // 8 halves
};
template <>
struct StreamVals<ValKind::BF16> {
    v4i v;
};
template <>
struct StreamVals<ValKind::I8> {
    uint32_t v[2];  // 4 bytes per group of 4 slots
};
template <>
struct StreamVals<ValKind::UNIT> {
};

// int8 operands on the stream kernel: products (|a*x| <= 16384) and their
// sums within one 512-slot chunk (below 2^23) are integers that fp32 holds
// exactly, whatever the order; a row's chunks are combined in double (exact
// up to 2^53) and the epilogue is the int64 one with saturation to int32.
template <ValKind V>
using StreamScal = typename std::conditional<V == ValKind::I8, long long, float>::type;  // alpha, beta
template <ValKind V>
using StreamSum = typename std::conditional<V == ValKind::I8, double, float>::type;  // row sums across chunks
template <>
struct StreamVals<ValKind::GATH> {
    v4i v[2];                 // positions of the 8 slots in the values array
    uint32_t g[kLaneItems];   // the gathered values
};

template <ValKind V>
__device__ __forceinline__ uint32_t RawVal(const StreamVals<V>& s, int j)
{
    if constexpr (V == ValKind::F32) {
        return __float_as_uint(s.v[j >> 2][j & 3]);
    } else if constexpr (V == ValKind::I8) {
        return (s.v[j >> 2] >> (8 * (j & 3))) & 0xFFU;
    } else {
        const uint32_t w = static_cast<uint32_t>(s.v[j >> 1]);
        return (j & 1) ? (w >> 16) : (w & 0xFFFFU);
    }
}

template <ValKind V>
__device__ __forceinline__ float ValToFloat(uint32_t raw)
{
    if constexpr (V == ValKind::F32) return __uint_as_float(raw);
    else if constexpr (V == ValKind::I8) return static_cast<float>(static_cast<int8_t>(static_cast<uint8_t>(raw)));
    else if constexpr (V == ValKind::F16) return HalfToFloat(static_cast<uint16_t>(raw));
    else return Bf16ToFloat(static_cast<uint16_t>(raw));
}

// Chunk slot held in register j (0..7) of a lane.
__device__ __forceinline__ int StreamSlot(int lane, int j) { return (j >> 2) * 256 + 4 * lane + (j & 3); }

// The same in either layout: lane-contiguous groups of 4 (StreamSlot), or,
// with kS, slot 64j + lane (the one-pass banded transpose, after its loads:
// each of its value and x gathers then covers 64 consecutive slots, a few
// columns, whose values and rows lie in a few cache lines instead of
// spreading over 256 slots).
template <bool kS>
__device__ __forceinline__ int SlotOf(int lane, int j)
{
    return kS ? kWave * j + lane : StreamSlot(lane, j);
}

template <typename RowT, ValKind V, OutKind O>
struct StreamLoad {
    v4i col[2];
    StreamVals<V> val;
    RowT rp[2];
    uint32_t rp16;  // kRows16: low halves of the two row offsets
    typename OutOf<O>::T yold[2];
    uint32_t xg[kLaneItems];  // gathered x of the 8 slots
};

// Half h of a and half h of b as the low and high halves of one word.
__device__ __forceinline__ int32_t Pack16(int32_t a, int32_t b, int h)
{
    const uint32_t ua = static_cast<uint32_t>(a), ub = static_cast<uint32_t>(b);
    return static_cast<int32_t>(h == 0 ? (ua & 0xFFFFU) | (ub << 16) : (ua >> 16) | (ub & 0xFFFF0000U));
}

// rb plus the signed 16-bit low / high half of w (wrapping 32-bit sums).
__device__ __forceinline__ int32_t Lo16(int32_t w, uint32_t rb)
{
    return static_cast<int32_t>(rb + static_cast<uint32_t>(static_cast<int32_t>(static_cast<int16_t>(w & 0xFFFF))));
}
__device__ __forceinline__ int32_t Hi16(int32_t w, uint32_t rb)
{
    return static_cast<int32_t>(rb + static_cast<uint32_t>(w >> 16));
}

template <typename RowT, ValKind V, OutKind O, bool kBeta, bool kNarrow = false, bool kRows16 = false,
          bool kEntry = false>
__device__ __forceinline__ void StreamLoadStage(const RowBlockParams& p, const Stage& s, int64_t tailStart, int lane,
                                                StreamLoad<RowT, V, O>& b)
{
    using ValT = typename ValOf<V>::T;
    using OutT = typename OutOf<O>::T;
    // An invalid stage loads from an empty resource: every load returns 0.
    // The resource ends at the chunk's last non-zero (rounded up to a whole
    // 16-byte group, never past the last whole group of the arrays): slots
    // past the chunk read 0 without touching memory, so a short block does
    // not stream (and gather for) the next block's entries.
    const int64_t a0 = s.valid ? s.a0 : 0;
    // entry-aligned blocks: the whole window from a0 (known from the block's
    // number alone), so these loads do not wait for the block's metadata
    int64_t end = kEntry ? a0 + kWaveChunk : (s.k0 + s.c1 + 3) & ~static_cast<int64_t>(3);
    end = end < tailStart ? end : tailStart;
    const int64_t avail = s.valid ? end - a0 : 0;
    const __amdgpu_buffer_rsrc_t rv = Rsrc(static_cast<const ValT*>(p.val) + a0, avail * sizeof(ValT));
    // Lane-contiguous groups of 4 slots: load h of lane l holds slots
    // 256h + 4l .. 256h + 4l + 3, so each load instruction reads 1 KiB of
    // col_ind (narrow columns 512 B; values: 1 KiB fp32, 512 B fp16) without
    // gaps.
    if constexpr (kNarrow && V == ValKind::GATH) {
        // the one-pass banded transpose on 16-bit copies: each slot's row
        // offset (low half) and position offset (high half) packed in one
        // word of b.col, decoded by StreamGather after the move to slot
        // 64j + lane
        const __amdgpu_buffer_rsrc_t rn = Rsrc(p.ncol + a0, avail * 2);
        const __amdgpu_buffer_rsrc_t rq = Rsrc(p.npos + a0, avail * 2);
        const v2i lo = __builtin_bit_cast(v2i, __builtin_amdgcn_raw_buffer_load_b64(rn, lane * 8, 0, kBufNonTemporal));
        const v2i hi =
            __builtin_bit_cast(v2i, __builtin_amdgcn_raw_buffer_load_b64(rn, 512 + lane * 8, 0, kBufNonTemporal));
        const v2i plo = __builtin_bit_cast(v2i, __builtin_amdgcn_raw_buffer_load_b64(rq, lane * 8, 0, kBufNonTemporal));
        const v2i phi =
            __builtin_bit_cast(v2i, __builtin_amdgcn_raw_buffer_load_b64(rq, 512 + lane * 8, 0, kBufNonTemporal));
        b.col[0] = v4i{Pack16(lo.x, plo.x, 0), Pack16(lo.x, plo.x, 1), Pack16(lo.y, plo.y, 0), Pack16(lo.y, plo.y, 1)};
        b.col[1] = v4i{Pack16(hi.x, phi.x, 0), Pack16(hi.x, phi.x, 1), Pack16(hi.y, phi.y, 0), Pack16(hi.y, phi.y, 1)};
    } else if constexpr (kNarrow) {
        // 16-bit offsets from the block's first row; decoded to col_ind's
        // values (the block is the one the chunk belongs to, so entries of
        // the previous block read before the chunk decode to other columns,
        // whose products are never summed)
        const __amdgpu_buffer_rsrc_t rn = Rsrc(p.ncol + a0, avail * 2);
        const uint32_t rb = static_cast<uint32_t>(s.r0) + static_cast<uint32_t>(p.base);
        const v2i lo = __builtin_bit_cast(v2i, __builtin_amdgcn_raw_buffer_load_b64(rn, lane * 8, 0, kBufNonTemporal));
        const v2i hi =
            __builtin_bit_cast(v2i, __builtin_amdgcn_raw_buffer_load_b64(rn, 512 + lane * 8, 0, kBufNonTemporal));
        b.col[0] = v4i{Lo16(lo.x, rb), Hi16(lo.x, rb), Lo16(lo.y, rb), Hi16(lo.y, rb)};
        b.col[1] = v4i{Lo16(hi.x, rb), Hi16(hi.x, rb), Lo16(hi.y, rb), Hi16(hi.y, rb)};
    } else {
        const __amdgpu_buffer_rsrc_t rc = Rsrc(p.col + a0, avail * 4);
        b.col[0] = __builtin_bit_cast(v4i, __builtin_amdgcn_raw_buffer_load_b128(rc, lane * 16, 0, kBufNonTemporal));
        b.col[1] =
            __builtin_bit_cast(v4i, __builtin_amdgcn_raw_buffer_load_b128(rc, 1024 + lane * 16, 0, kBufNonTemporal));
    }
    if constexpr (V == ValKind::UNIT) {
        (void)rv;  // no values
    } else if constexpr (V == ValKind::GATH && kNarrow) {
        (void)rv;  // positions: packed with the rows above
    } else if constexpr (V == ValKind::GATH) {
        b.val.v[0] = __builtin_bit_cast(v4i, __builtin_amdgcn_raw_buffer_load_b128(rv, lane * 16, 0, kBufNonTemporal));
        b.val.v[1] =
            __builtin_bit_cast(v4i, __builtin_amdgcn_raw_buffer_load_b128(rv, 1024 + lane * 16, 0, kBufNonTemporal));
    } else if constexpr (V == ValKind::F32) {
        b.val.v[0] = __builtin_bit_cast(v4f, __builtin_amdgcn_raw_buffer_load_b128(rv, lane * 16, 0, kBufNonTemporal));
        b.val.v[1] =
            __builtin_bit_cast(v4f, __builtin_amdgcn_raw_buffer_load_b128(rv, 1024 + lane * 16, 0, kBufNonTemporal));
    } else if constexpr (V == ValKind::I8) {
        b.val.v[0] = __builtin_amdgcn_raw_buffer_load_b32(rv, lane * 4, 0, kBufNonTemporal);
        b.val.v[1] = __builtin_amdgcn_raw_buffer_load_b32(rv, 256 + lane * 4, 0, kBufNonTemporal);
    } else {
        const v2i lo = __builtin_bit_cast(v2i, __builtin_amdgcn_raw_buffer_load_b64(rv, lane * 8, 0, kBufNonTemporal));
        const v2i hi = __builtin_bit_cast(v2i, __builtin_amdgcn_raw_buffer_load_b64(rv, 512 + lane * 8, 0, kBufNonTemporal));
        b.val.v = v4i{lo.x, lo.y, hi.x, hi.y};
    }
    // Rows 2l and 2l+1 of the block belong to lane l: their row offsets come
    // in one 8-byte (int32) or 16-byte (int64) load.  The resource covers
    // nr+1 offsets rounded up to an even count (the workspace array has a pad
    // entry), so a pair is either wholly inside or wholly past it (past: 0,
    // never used).  Old y values are loaded one per row.
    const int64_t r0 = s.valid ? s.r0 : 0;
    int64_t nrp = s.valid ? ((s.nr + 2) & ~1) : 0;
    // never past the offsets array (rows + 1 entries; the pad entry of the
    // workspace copy is not needed: a pair past it is never used)
    if (nrp > p.rows + 1 - r0) nrp = p.rows + 1 - r0;
    if constexpr (kRows16) {
        // The lane's two low halves, entries r0 + 2l and r0 + 2l + 1, from
        // an 8-byte load at the even entry below (4-byte aligned; the copy
        // has rows + 2 entries, so the rounded range stays inside it).
        const int64_t odd = r0 & 1;
        const __amdgpu_buffer_rsrc_t r16 = Rsrc(p.rp16 + (r0 - odd), ((odd + nrp + 1) & ~int64_t{1}) * 2);
        const v2i w = __builtin_bit_cast(v2i, __builtin_amdgcn_raw_buffer_load_b64(r16, lane * 4, 0, kRowPolicy));
        b.rp16 = __builtin_amdgcn_alignbit(static_cast<uint32_t>(w.y), static_cast<uint32_t>(w.x),
                                           static_cast<uint32_t>(odd) * 16U);
    } else if constexpr (sizeof(RowT) == 8) {
        const __amdgpu_buffer_rsrc_t rr = Rsrc(static_cast<const RowT*>(p.rp) + r0, nrp * sizeof(RowT));
        const v4i w = __builtin_bit_cast(v4i, __builtin_amdgcn_raw_buffer_load_b128(rr, lane * 16, 0, kRowPolicy));
        b.rp[0] = static_cast<RowT>((static_cast<uint64_t>(static_cast<uint32_t>(w.y)) << 32) |
                                    static_cast<uint32_t>(w.x)) - static_cast<RowT>(p.rp_base);
        b.rp[1] = static_cast<RowT>((static_cast<uint64_t>(static_cast<uint32_t>(w.w)) << 32) |
                                    static_cast<uint32_t>(w.z)) - static_cast<RowT>(p.rp_base);
    } else {
        const __amdgpu_buffer_rsrc_t rr = Rsrc(static_cast<const RowT*>(p.rp) + r0, nrp * sizeof(RowT));
        const v2i w = __builtin_bit_cast(v2i, __builtin_amdgcn_raw_buffer_load_b64(rr, lane * 8, 0, kRowPolicy));
        b.rp[0] = static_cast<RowT>(w.x) - static_cast<RowT>(p.rp_base);
        b.rp[1] = static_cast<RowT>(w.y) - static_cast<RowT>(p.rp_base);
    }
    int64_t ny = s.valid ? s.nr : 0;
    if (ny > p.rows - r0) ny = p.rows - r0;
    const __amdgpu_buffer_rsrc_t ry = Rsrc(static_cast<const OutT*>(p.y) + r0, ny * sizeof(OutT));
    if constexpr (kBeta && sizeof(OutT) == 4) {
        // both rows of the lane in one 8-byte load; buffer range checks are
        // per dword, so a row past the block reads 0 (and is never used)
        // (loaded as a float2: taking __builtin_bit_cast(float, ...) of the
        // elements of an int2 load makes this hipcc emit a one-dword load)
        if constexpr (O == OutKind::I32) {
            const v2i w = __builtin_bit_cast(v2i, __builtin_amdgcn_raw_buffer_load_b64(ry, lane * 8, 0, kRowPolicy));
            b.yold[0] = w.x;
            b.yold[1] = w.y;
        } else {
            const v2f w = __builtin_bit_cast(v2f, __builtin_amdgcn_raw_buffer_load_b64(ry, lane * 8, 0, kRowPolicy));
            b.yold[0] = w.x;
            b.yold[1] = w.y;
        }
    } else {
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const int i = 2 * lane + h;
            if constexpr (kBeta) {
                b.yold[h] = __builtin_bit_cast(OutT, __builtin_amdgcn_raw_buffer_load_b16(ry, i * 2, 0, kRowPolicy));
            } else {
                b.yold[h] = OutT{};
            }
        }
    }
}

// Gathers x for the 8 slots of this lane.  The last nnz % 4 entries of the
// arrays (not covered by any 16-byte group) are read here, in the one chunk
// that reaches them.
template <typename RowT, ValKind V, OutKind O, bool kS = false, bool kPacked = false>
__device__ __forceinline__ void StreamGather(const RowBlockParams& p, const Stage& s, int64_t tailStart,
                                             __amdgpu_buffer_rsrc_t rx, int lane, StreamLoad<RowT, V, O>& b,
                                             uint32_t xg[kLaneItems], float* sVal = nullptr)
{
    using ValT = typename ValOf<V>::T;
    if constexpr (kPacked) {
        // packed 16-bit row / position offsets (StreamLoadStage): moved to
        // slot 64j + lane through the wave's LDS slice, then decoded there
        static_assert(kS && V == ValKind::GATH, "packed offsets: the banded transpose on 16-bit copies");
        int32_t* t = reinterpret_cast<int32_t*>(sVal);
        *reinterpret_cast<v4i*>(&t[4 * lane]) = b.col[0];
        *reinterpret_cast<v4i*>(&t[256 + 4 * lane]) = b.col[1];
        const uint32_t rb = static_cast<uint32_t>(s.r0) + static_cast<uint32_t>(p.base);
        const uint32_t k0 = static_cast<uint32_t>(s.valid ? s.a0 : 0) + static_cast<uint32_t>(lane);
#pragma unroll
        for (int j = 0; j < kLaneItems; ++j) {
            const int32_t w = t[kWave * j + lane];
            b.col[j >> 2][j & 3] = Lo16(w, rb);
            b.val.v[j >> 2][j & 3] = Hi16(w, k0 + static_cast<uint32_t>(kWave * j));
        }
    }
    if (s.valid && s.a0 + kWaveChunk > tailStart && tailStart < p.nnz) {
        // Uniform branch: only the chunk that reaches the end of the arrays.
        int32_t tc[3];
        ValT tv3[3] = {};
#pragma unroll
        for (int e = 0; e < 3; ++e) {
            const int64_t k = tailStart + e < p.nnz ? tailStart + e : p.nnz - 1;
            tc[e] = ConstLoad<int32_t>(p.col, k);
            if constexpr (V != ValKind::UNIT) tv3[e] = ConstLoad<ValT>(p.val, k);
        }
#pragma unroll
        for (int j = 0; j < kLaneItems; ++j) {
            const int64_t k = s.a0 + SlotOf<kPacked>(lane, j) - tailStart;
            if (k >= 0 && k < 3) {
                const int kk = static_cast<int>(k);
                b.col[j >> 2][j & 3] = kk == 0 ? tc[0] : kk == 1 ? tc[1] : tc[2];
                const ValT tv = kk == 0 ? tv3[0] : kk == 1 ? tv3[1] : tv3[2];
                if constexpr (V == ValKind::UNIT) {
                    (void)tv;
                } else if constexpr (V == ValKind::GATH) {
                    b.val.v[j >> 2][j & 3] = __float_as_int(tv);
                } else if constexpr (V == ValKind::F32) {
                    b.val.v[j >> 2][j & 3] = tv;
                } else if constexpr (V == ValKind::I8) {
                    const uint32_t sh = 8U * static_cast<uint32_t>(j & 3);
                    b.val.v[j >> 2] =
                        (b.val.v[j >> 2] & ~(0xFFU << sh)) | (static_cast<uint32_t>(static_cast<uint8_t>(tv)) << sh);
                } else {
                    const uint32_t raw = static_cast<uint32_t>(tv);
                    uint32_t w = static_cast<uint32_t>(b.val.v[j >> 1]);
                    w = (j & 1) ? ((w & 0xFFFFU) | (raw << 16)) : ((w & 0xFFFF0000U) | raw);
                    b.val.v[j >> 1] = static_cast<int>(w);
                }
            }
        }
    }
    if constexpr (kS && !kPacked) {
        static_assert(V == ValKind::GATH, "slot layout 64j + lane: gathered values only");
        int32_t* t = reinterpret_cast<int32_t*>(sVal);
        // The loads hold lane-contiguous groups (StreamSlot); register j of
        // lane l moves to slot 64j + l (SlotOf<true>) through the wave's own
        // LDS slice: the columns, and the positions of a gathered value.
        *reinterpret_cast<v4i*>(&t[4 * lane]) = b.col[0];
        *reinterpret_cast<v4i*>(&t[256 + 4 * lane]) = b.col[1];
        int32_t c[kLaneItems];
#pragma unroll
        for (int j = 0; j < kLaneItems; ++j) c[j] = t[kWave * j + lane];
        *reinterpret_cast<v4i*>(&t[4 * lane]) = b.val.v[0];
        *reinterpret_cast<v4i*>(&t[256 + 4 * lane]) = b.val.v[1];
#pragma unroll
        for (int j = 0; j < kLaneItems; ++j) {
            b.col[j >> 2][j & 3] = c[j];
            b.val.v[j >> 2][j & 3] = t[kWave * j + lane];
        }
    }
    // Slots past the chunk's last non-zero gather nothing (an offset past the
    // resource reads 0 without a memory request).
    const int32_t hiSlot = s.valid ? static_cast<int32_t>(s.k0 + s.c1 - s.a0) : 0;
    // (entry-aligned blocks: slots before the block's first entry gather nothing either)
    const int32_t loSlot = s.valid ? static_cast<int32_t>(s.k0 + s.c0 - s.a0) : 0;
#pragma unroll
    for (int j = 0; j < kLaneItems; ++j) {
        uint32_t off = static_cast<uint32_t>(b.col[j >> 2][j & 3] - p.base) * static_cast<uint32_t>(sizeof(ValT));
        off = SlotOf<kS>(lane, j) < hiSlot && SlotOf<kS>(lane, j) >= loSlot ? off : 0xFFFFFFF0U;
        if constexpr (sizeof(ValT) == 4) {
            xg[j] = __builtin_amdgcn_raw_buffer_load_b32(rx, static_cast<int>(off), 0, kGatherPolicy);
        } else if constexpr (sizeof(ValT) == 2) {
            xg[j] = __builtin_amdgcn_raw_buffer_load_b16(rx, static_cast<int>(off), 0, kGatherPolicy);
        } else {
            xg[j] = __builtin_amdgcn_raw_buffer_load_b8(rx, static_cast<int>(off), 0, kGatherPolicy);
        }
    }
    if constexpr (V == ValKind::GATH) {
        // the slots' values, by position (positions past the chunk read 0)
        const __amdgpu_buffer_rsrc_t rg = Rsrc(p.gval, p.gval_n * 4);
#pragma unroll
        for (int j = 0; j < kLaneItems; ++j) {
            uint32_t off = static_cast<uint32_t>(b.val.v[j >> 2][j & 3]) * 4U;
            off = SlotOf<kS>(lane, j) < hiSlot ? off : 0xFFFFFFF0U;
            b.val.g[j] = __builtin_amdgcn_raw_buffer_load_b32(rg, static_cast<int>(off), 0, kGatherPolicy);
        }
    }
}

// Butterfly step across lanes l and l^m (m < 32) without address setup.
template <int M>
__device__ __forceinline__ float SwizzleXor(float v)
{
    static_assert(M > 0 && M < 32, "swizzle reaches within 32 lanes");
    constexpr int kPattern = 0x1F | (M << 10);  // and 0x1F, or 0, xor M
    return __int_as_float(__builtin_amdgcn_ds_swizzle(__float_as_int(v), kPattern));
}

// Sum over the lanes of groups of 2^lg consecutive lanes (lg <= 5), on every lane.
__device__ __forceinline__ float GroupSum(float v, int lg)
{
    if (lg >= 1) v += SwizzleXor<1>(v);
    if (lg >= 2) v += SwizzleXor<2>(v);
    if (lg >= 3) v += SwizzleXor<4>(v);
    if (lg >= 4) v += SwizzleXor<8>(v);
    if (lg >= 5) v += SwizzleXor<16>(v);
    return v;
}

// Sum over the wave (wave-uniform result).
__device__ __forceinline__ float WaveSum(float v)
{
    v = GroupSum(v, 5);
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 0)) +
           __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 32));
}

// Value of lane l+1 (lane 63 receives `last`).
__device__ __forceinline__ int32_t FromNextLane(int32_t v, int32_t last)
{
    constexpr int kWaveShl1 = 0x130;
    return __builtin_amdgcn_update_dpp(last, v, kWaveShl1, 0xF, 0xF, false);
}

// LDS product slots per wave: one chunk plus 8 so that a predicated read of
// 8 entries from any slot stays inside the wave's slice.
constexpr int kStreamLds = kWaveChunk + 8;

// Reduces one loaded and gathered chunk: products to LDS, phase 1 (short
// rows, lane groups), phase 2 (long or chunk-crossing rows, whole wave), y.
// Row i = 2*lane + h of the block has its offsets in registers: its start
// in this lane's rp[h], its end in the next row's.
// Task mode (kTask): the chunk is one task of a long block; rows that cross
// the chunk's first slot leave their partial sum in `head` (also when they
// cross both ends), the row that crosses its last slot in `tail`, and neither
// is written to y here.
template <typename RowT, ValKind V, OutKind O, bool kBeta, bool kTask = false, bool kRows16 = false, bool kS = false>
__device__ __forceinline__ void StreamChunk(const Stage& cur, const StreamLoad<RowT, V, O>& lc, float* sVal, int lane,
                                            StreamScal<V> alpha, StreamScal<V> beta, StreamSum<V>& carry, int& lg,
                                            typename OutOf<O>::T* y,
                                            typename OutOf<O>::T* sink, float* head = nullptr,
                                            float* tail = nullptr)
{
    using OutT = typename OutOf<O>::T;
    float prod[kLaneItems];
#pragma unroll
    for (int j = 0; j < kLaneItems; ++j) {
        if constexpr (V == ValKind::UNIT) prod[j] = __uint_as_float(lc.xg[j]);
        else if constexpr (V == ValKind::GATH) prod[j] = __uint_as_float(lc.val.g[j]) * __uint_as_float(lc.xg[j]);
        else prod[j] = ValToFloat<V>(RawVal<V>(lc.val, j)) * ValToFloat<V>(lc.xg[j]);
    }

    const int32_t c0 = cur.c0, c1 = cur.c1;
    const int32_t shift = static_cast<int32_t>(cur.a0 - cur.k0);  // LDS slot of relative offset r: r - shift
    const int nr = cur.nr;
    if constexpr (kTask) {
        lg = 0;
        *head = 0.0f;
        *tail = 0.0f;
    } else if (cur.first) {
        carry = 0;
        // Lanes per row: as many as keep every row of the block on its own
        // lane group, 1 when the block spans several chunks.
        lg = 0;
        if (cur.last) {
            while (lg < 6 && (nr << (lg + 1)) <= kWave) ++lg;
        }
    }
    if constexpr (kS) {
#pragma unroll
        for (int j = 0; j < kLaneItems; ++j) sVal[SlotOf<true>(lane, j)] = prod[j];
    } else {
        *reinterpret_cast<v4f*>(&sVal[4 * lane]) = v4f{prod[0], prod[1], prod[2], prod[3]};
        *reinterpret_cast<v4f*>(&sVal[256 + 4 * lane]) = v4f{prod[4], prod[5], prod[6], prod[7]};
    }

    // Row offsets relative to the block's first non-zero.  Lane l holds rows
    // 2l and 2l+1: row 2l ends where row 2l+1 starts, row 2l+1 where lane
    // l+1's first row starts (row 127 never exists: blocks have <= 127 rows).
    const int32_t k0lo = static_cast<int32_t>(cur.k0);
    int32_t rs[2], re[2];
    if constexpr (kRows16) {
        // offsets from the block's first entry, below 65536 in such a block
        const uint32_t k0l16 = static_cast<uint32_t>(cur.k0) & 0xFFFFU;
        rs[0] = static_cast<int32_t>(((lc.rp16 & 0xFFFFU) - k0l16) & 0xFFFFU);
        rs[1] = static_cast<int32_t>(((lc.rp16 >> 16) - k0l16) & 0xFFFFU);
    } else {
        rs[0] = static_cast<int32_t>(lc.rp[0]) - k0lo;
        rs[1] = static_cast<int32_t>(lc.rp[1]) - k0lo;
    }
    re[0] = rs[1];
    re[1] = FromNextLane(rs[0], rs[1]);

    const int gsz = 1 << lg;
    bool fin[2], defer[2], active[2], crosses[2];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
        const int i = 2 * lane + h;
        const bool in = i < nr;
        const bool empty = re[h] <= rs[h];
        active[h] = in && (empty ? ((rs[h] >= c0 && rs[h] < c1) || (cur.last && rs[h] >= c1))
                                 : (rs[h] < c1 && re[h] > c0));
        crosses[h] = !empty && (rs[h] < c0 || re[h] > c1);
    }
    // One lane per row reads 8 entries per row; when a row of 9-16 entries
    // lies inside the chunk, 16 (rows of 9-16 entries would otherwise be
    // summed one at a time by the whole wave).
    bool wide = false;
    if (lg == 0) {
        const bool mid0 = active[0] && !crosses[0] && re[0] - rs[0] > kSerialCapOne && re[0] - rs[0] <= 16;
        const bool mid1 = active[1] && !crosses[1] && re[1] - rs[1] > kSerialCapOne && re[1] - rs[1] <= 16;
        wide = __ballot(mid0 || mid1) != 0;
    }
    const int cap = wide ? 16 : SerialCap(lg);
#pragma unroll
    for (int h = 0; h < 2; ++h) {
        defer[h] = active[h] && (crosses[h] || re[h] - rs[h] > cap);
        fin[h] = active[h] && !defer[h];
    }
    WaveLdsSync();

    // Phase 1.
    StreamSum<V> sum[2] = {0, 0};
    if (lg == 0) {
        // One lane per row: 8 predicated LDS reads per row, all issued
        // before one wait (the compiler's own schedule waits after each read
        // pair); a second round of 8 when some row has 9-16 entries.
        int32_t len[2];
        uint32_t addr[2];
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            len[h] = fin[h] ? re[h] - rs[h] : 0;
            addr[h] = LdsAddr(sVal + (fin[h] ? rs[h] - shift : 0));
        }
        for (int round = 0; round < 2; ++round) {
            if (round == 1 && !wide) break;
            v2f e[2][4];
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                asm volatile("ds_read2_b32 %0, %4 offset1:1\n\t"
                             "ds_read2_b32 %1, %4 offset0:2 offset1:3\n\t"
                             "ds_read2_b32 %2, %4 offset0:4 offset1:5\n\t"
                             "ds_read2_b32 %3, %4 offset0:6 offset1:7"
                             : "=&v"(e[h][0]), "=&v"(e[h][1]), "=&v"(e[h][2]), "=&v"(e[h][3])
                             : "v"(addr[h] + 32U * round));
            }
            asm volatile("s_waitcnt lgkmcnt(0)"
                         : "+v"(e[0][0]), "+v"(e[0][1]), "+v"(e[0][2]), "+v"(e[0][3]), "+v"(e[1][0]), "+v"(e[1][1]),
                           "+v"(e[1][2]), "+v"(e[1][3]));
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                float acc = sum[h];
#pragma unroll
                for (int t = 0; t < kSerialCapOne; ++t) acc += t + 8 * round < len[h] ? e[h][t >> 1][t & 1] : 0.0f;
                sum[h] = acc;
            }
        }
    } else {
        // Group g = lane >> lg reduces row g (nr <= 32 here); lane g/2 holds
        // its offsets in half g&1.
        const int g = lane >> lg;
        const int sub = lane & (gsz - 1);
        const bool in = g < nr;
        const int src = (g >> 1) & (kWave - 1);
        const int32_t a0s = __shfl(rs[0], src, kWave), a1s = __shfl(rs[1], src, kWave);
        const int32_t a1e = __shfl(re[1], src, kWave);
        const int32_t gs = (g & 1) ? a1s : a0s;
        const int32_t ge = (g & 1) ? a1e : a1s;
        // cap = 16 * gsz, so a lane reads at most 16 entries: 16 predicated
        // reads issued back to back (two asm groups walking one address
        // register), one wait.
        const bool ok = in && ge - gs <= cap;
        const int32_t n = ok ? ge - gs - sub : 0;  // this lane's entries: t * gsz < n
        uint32_t addr = LdsAddr(sVal + (ok ? gs + sub - shift : 0));
        const uint32_t step = static_cast<uint32_t>(gsz) * 4U;
        float e[16];
        asm volatile("ds_read_b32 %0, %8\n\tv_add_u32 %8, %8, %9\n\t"
                     "ds_read_b32 %1, %8\n\tv_add_u32 %8, %8, %9\n\t"
                     "ds_read_b32 %2, %8\n\tv_add_u32 %8, %8, %9\n\t"
                     "ds_read_b32 %3, %8\n\tv_add_u32 %8, %8, %9\n\t"
                     "ds_read_b32 %4, %8\n\tv_add_u32 %8, %8, %9\n\t"
                     "ds_read_b32 %5, %8\n\tv_add_u32 %8, %8, %9\n\t"
                     "ds_read_b32 %6, %8\n\tv_add_u32 %8, %8, %9\n\t"
                     "ds_read_b32 %7, %8\n\tv_add_u32 %8, %8, %9"
                     : "=&v"(e[0]), "=&v"(e[1]), "=&v"(e[2]), "=&v"(e[3]), "=&v"(e[4]), "=&v"(e[5]), "=&v"(e[6]),
                       "=&v"(e[7]), "+&v"(addr)
                     : "v"(step));
        asm volatile("ds_read_b32 %0, %8\n\tv_add_u32 %8, %8, %9\n\t"
                     "ds_read_b32 %1, %8\n\tv_add_u32 %8, %8, %9\n\t"
                     "ds_read_b32 %2, %8\n\tv_add_u32 %8, %8, %9\n\t"
                     "ds_read_b32 %3, %8\n\tv_add_u32 %8, %8, %9\n\t"
                     "ds_read_b32 %4, %8\n\tv_add_u32 %8, %8, %9\n\t"
                     "ds_read_b32 %5, %8\n\tv_add_u32 %8, %8, %9\n\t"
                     "ds_read_b32 %6, %8\n\tv_add_u32 %8, %8, %9\n\t"
                     "ds_read_b32 %7, %8"
                     : "=&v"(e[8]), "=&v"(e[9]), "=&v"(e[10]), "=&v"(e[11]), "=&v"(e[12]), "=&v"(e[13]),
                       "=&v"(e[14]), "=&v"(e[15]), "+&v"(addr)
                     : "v"(step));
        asm volatile("s_waitcnt lgkmcnt(0)"
                     : "+v"(e[0]), "+v"(e[1]), "+v"(e[2]), "+v"(e[3]), "+v"(e[4]), "+v"(e[5]), "+v"(e[6]), "+v"(e[7]),
                       "+v"(e[8]), "+v"(e[9]), "+v"(e[10]), "+v"(e[11]), "+v"(e[12]), "+v"(e[13]), "+v"(e[14]),
                       "+v"(e[15]));
        float part = 0.0f;
#pragma unroll
        for (int t = 0; t < 16; ++t) part += t * gsz < n ? e[t] : 0.0f;
        if (lg <= 5) {
            part = GroupSum(part, lg);
        } else {
            part = WaveSum(part);
        }
        // the group of row 2l+h starts at lane (2l+h) << lg
        sum[0] = __shfl(part, ((2 * lane) << lg) & (kWave - 1), kWave);
        sum[1] = __shfl(part, ((2 * lane + 1) << lg) & (kWave - 1), kWave);
    }

    // Phase 2: deferred rows, whole wave per row, in row order (rows 2l+h).
    uint64_t pending0 = __ballot(defer[0]), pending1 = __ballot(defer[1]);
    while (pending0 | pending1) {
        const int l0 = pending0 ? __builtin_ctzll(pending0) : kWave;
        const int l1 = pending1 ? __builtin_ctzll(pending1) : kWave;
        const int h = (2 * l1 + 1 < 2 * l0) ? 1 : 0;
        const int l = h ? l1 : l0;
        if (h) {
            pending1 &= pending1 - 1;
        } else {
            pending0 &= pending0 - 1;
        }
        const int32_t s0 = __builtin_amdgcn_readlane(h ? rs[1] : rs[0], l);
        const int32_t e0 = __builtin_amdgcn_readlane(h ? re[1] : re[0], l);
        const int32_t lo = s0 > c0 ? s0 : c0;
        const int32_t hi = e0 < c1 ? e0 : c1;
        float part = 0.0f;
        for (int32_t q = lo + lane; q < hi; q += kWave) part += sVal[q - shift];
        StreamSum<V> total = WaveSum(part);
        bool finish = false;
        if constexpr (kTask) {
            if (s0 < c0) {
                *head = total;
            } else if (e0 > c1) {
                *tail = total;
            } else {
                finish = true;
            }
        } else {
            if (s0 < c0) total += carry;
            if (e0 > c1) {
                carry = total;
            } else {
                finish = true;
            }
        }
        if (finish && lane == l) {
            if (h) {
                sum[1] = total;
                fin[1] = true;
            } else {
                sum[0] = total;
                fin[0] = true;
            }
        }
    }

    OutT out[2];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
        // beta == 0 (possible at run time with device scalars) never reads y
        if constexpr (V == ValKind::I8) {
            const long long old = kBeta && beta != 0 ? static_cast<long long>(lc.yold[h]) : 0LL;
            out[h] = FromAcc<O, AccKind::I64>(ScaledI64(static_cast<long long>(sum[h]), alpha, beta, old));
        } else {
            float r = alpha * sum[h];
            if constexpr (kBeta) {
                if (beta != 0.0f) r += beta * OutToAcc<O, AccKind::F32>(lc.yold[h]);
            }
            out[h] = FromAcc<O, AccKind::F32>(r);
        }
    }
    // When every row of the block that this chunk touches finishes here (one-
    // chunk blocks), each lane stores its two rows with one 8-byte buffer
    // store; the range check (per dword) drops rows past the block.
    bool pair = false;
    if constexpr (sizeof(OutT) == 4) {
        const bool ok = (fin[0] || 2 * lane >= nr) && (fin[1] || 2 * lane + 1 >= nr);
        pair = __ballot(!ok) == 0;
    }
    if (pair) {
        const __amdgpu_buffer_rsrc_t rys = Rsrc(y + cur.r0, static_cast<int64_t>(nr) * 4);
        if constexpr (sizeof(OutT) == 4) {  // pair is false otherwise
            const v2i w = {__builtin_bit_cast(int32_t, out[0]), __builtin_bit_cast(int32_t, out[1])};
            __builtin_amdgcn_raw_buffer_store_b64(w, rys, lane * 8, 0, 0);
        }
    } else {
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const int i = 2 * lane + h;
            OutT* dst = fin[h] ? y + (cur.r0 + i) : sink + h * kWave;
            *dst = out[h];
        }
    }
    WaveLdsSync();  // this chunk's LDS reads complete before the next chunk overwrites
}

// Opens block `tile` with both metadata pairs loaded at once (no dependent
// scalar loads).
template <typename RowT>
__device__ __forceinline__ Stage OpenTileFlat(const RowBlockParams& p, int64_t tile)
{
    typedef int v2s __attribute__((ext_vector_type(2)));
    Stage s{};
    s.tile = 0;
    s.valid = true;
    const v2s rr = ConstLoad<v2s>(p.blocks + tile, 0);
    int64_t k0, k1;
    if constexpr (sizeof(RowT) == 8) {
        typedef long long v2l __attribute__((ext_vector_type(2)));
        const v2l kk = ConstLoad<v2l>(static_cast<const int64_t*>(p.block_nnz) + tile, 0);
        k0 = kk.x;
        k1 = kk.y;
    } else {
        const v2s kk = ConstLoad<v2s>(static_cast<const int32_t*>(p.block_nnz) + tile, 0);
        k0 = kk.x;
        k1 = kk.y;
    }
    s.r0 = rr.x;
    const int32_t n = rr.y - rr.x;
    s.nr = n < 0 ? 0 : n > kWaveRows ? kWaveRows : n;
    s.k0 = k0;
    const int64_t span = k1 - k0;
    s.kspan = static_cast<int32_t>(span < 0 ? 0 : span > 0x7FFFFFFFLL ? 0x7FFFFFFFLL : span);
    s.c0 = 0;
    s.first = true;
    ChunkBounds(s);
    return s;
}

// Number of chunks of a block (the first chunk starts at the block's
// 16-byte-aligned first non-zero).
__device__ __forceinline__ int64_t BlockChunks(int64_t k0, int64_t kspan)
{
    return (kspan + (k0 & 3) + kWaveChunk - 1) / kWaveChunk;
}

// Combines the partial sums of the rows of long block b that cross chunk
// boundaries, in chunk order: tail of the chunk where the row starts, then the
// heads of the following chunks up to the one where it ends.  Run by the last
// task of the block to arrive.
template <typename RowT, OutKind O>
__device__ __forceinline__ void FixupLongBlock(const RowBlockParams& p, const Stage& blk, int32_t ts, int32_t nT,
                                               int lane, float alpha, float beta)
{
    using OutT = typename OutOf<O>::T;
    const int64_t r0 = blk.r0;
    const int nr = blk.nr;
    const RowT* rp = static_cast<const RowT*>(p.rp);
    const int32_t k0lo = static_cast<int32_t>(blk.k0);
    int32_t rs[2], re[2];
    bool in[2];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
        const int i = lane + h * kWave;
        in[h] = i < nr;
        rs[h] = in[h] ? static_cast<int32_t>(rp[r0 + i]) - k0lo : 0;
        re[h] = in[h] ? static_cast<int32_t>(rp[r0 + i + 1]) - k0lo : 0;
    }
    const int32_t sh = static_cast<int32_t>(blk.k0 & 3);
    OutT* y = static_cast<OutT*>(p.y);
    for (int32_t j = 1; j < nT;) {
        const int32_t cj = j * kWaveChunk - sh;
        const uint64_t m0 = __ballot(in[0] && rs[0] < cj && re[0] > cj);
        const uint64_t m1 = __ballot(in[1] && rs[1] < cj && re[1] > cj);
        if (m0 == 0 && m1 == 0) {
            ++j;
            continue;
        }
        const int h = m0 != 0 ? 0 : 1;
        const int l = __builtin_ctzll(m0 != 0 ? m0 : m1);
        const int32_t e0 = __builtin_amdgcn_readlane(h == 0 ? re[0] : re[1], l);
        const int32_t jend = (e0 - 1 + sh) / kWaveChunk;  // chunk of the row's last entry
        float part = 0.0f;
        for (int32_t u = j + lane; u <= jend; u += kWave) {
            part += __hip_atomic_load(p.task_head + ts + u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
        const float total =
            WaveSum(part) + __hip_atomic_load(p.task_tail + ts + j - 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (lane == 0) StoreRow<O, AccKind::F32>(y, r0 + l + h * kWave, total, alpha, beta, beta != 0.0f);
        j = jend + 1;
    }
}

// One block per wave, no persistence: the hardware keeps as many waves
// resident as registers allow (the kernel is built for 7-8 waves per SIMD) and
// their independent loads keep HBM busy.  Chunks of a block of up to
// kLongChunks chunks are processed one after another; longer blocks (rows of
// thousands of entries) are split by Preprocess into one task per chunk,
// served round-robin by the first task_waves waves of the grid, so a long row
// is reduced by many waves at once.  Each task stores the partial sums of its
// chunk-crossing rows; the block's last task to arrive combines them.
//
// kGated: the launch made when another path may have taken the matrix (the
// decision is on the device only): the kernel exits unless p.skip_flag reads
// a value whose bit is set in p.run_mask, and a capped grid loops over the
// blocks (block_stride).  Ungated launches carry neither (one block per wave,
// no flag load).  kNarrow: column indices from the narrow copy p.ncol.
template <typename RowT, ValKind V, OutKind O, bool kBeta, bool kGated = false, bool kNarrow = false,
          bool kEntry = false>
__global__ __launch_bounds__(kWave* kFlatWaves) __attribute__((amdgpu_waves_per_eu(6)))
void SpmvStreamFlatKernel(RowBlockParams p)
{
    using ValT = typename ValOf<V>::T;
    using OutT = typename OutOf<O>::T;
    using L = StreamLoad<RowT, V, O>;
    constexpr bool kStrided = V == ValKind::GATH;  // slot layout SlotOf<true> (gathered values)

    __shared__ float sValAll[kFlatWaves][kStreamLds];

    if constexpr (kGated) {
        const uint32_t flag = ConstLoad<uint32_t>(p.skip_flag, 0);
        if (flag >= 32U || ((p.run_mask >> flag) & 1U) == 0U) return;
    }
    const int lane = threadIdx.x & (kWave - 1);
    const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
    float* sVal = sValAll[wv];

    StreamScal<V> alpha, beta;
    LoadScalars<V == ValKind::I8 ? AccKind::I64 : AccKind::F32>(p.s, alpha, beta);
    OutT* y = static_cast<OutT*>(p.y);
    OutT* sink = static_cast<OutT*>(p.sink) + lane;
    const __amdgpu_buffer_rsrc_t rx = Rsrc(p.x, p.cols * static_cast<int64_t>(sizeof(ValT)));
    const int64_t tailStart = p.nnz & ~static_cast<int64_t>(3);
    StreamSum<V> carry = 0;
    int lg = 0;

    // (int8 launches have no tasks: a long block is summed chunk by chunk by its own wave)
    if (V != ValKind::I8 && static_cast<int32_t>(blockIdx.x) < p.task_wgs) {
        // Task worker.
        const int64_t e = static_cast<int64_t>(blockIdx.x) * kFlatWaves + wv;
        int64_t total = ConstLoad<int32_t>(p.task_start, p.num_blocks);
        total = total < p.max_tasks ? total : p.max_tasks;
        for (int64_t t = e; t < total; t += p.task_waves) {
            const int32_t b = ConstLoad<int32_t>(p.task_block, t);
            if (b < 0 || b >= p.num_blocks) continue;
            const int32_t ts = ConstLoad<int32_t>(p.task_start, b);
            const int32_t nT = ConstLoad<int32_t>(p.task_start, b + 1) - ts;
            const int32_t j = static_cast<int32_t>(t) - ts;
            const Stage blk = OpenTileFlat<RowT>(p, b);
            Stage cur = blk;
            cur.c0 = j == 0 ? 0 : j * kWaveChunk - static_cast<int32_t>(blk.k0 & 3);
            cur.first = j == 0;
            ChunkBounds(cur);
            L bl;
            StreamLoadStage<RowT, V, O, kBeta, kNarrow>(p, cur, tailStart, lane, bl);
            StreamGather<RowT, V, O, kStrided, kStrided && kNarrow>(p, cur, tailStart, rx, lane, bl, bl.xg, sVal);
            float head = 0.0f, tail = 0.0f;
            StreamChunk<RowT, V, O, kBeta, true, false, kStrided>(cur, bl, sVal, lane, alpha, beta, carry, lg, y, sink,
                                                                 &head, &tail);
            // The partial sums go to memory with device-scope stores (they
            // bypass this XCD's L2), complete before the arrival is counted,
            // and the last task reads them with device-scope loads: no
            // whole-cache write-back or invalidate per task.
            uint32_t prev = 0;
            if (lane == 0) {
                __hip_atomic_store(p.task_head + t, head, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                __hip_atomic_store(p.task_tail + t, tail, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
                prev = __hip_atomic_fetch_add(p.task_cnt + b, 1U, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            }
            prev = __builtin_amdgcn_readfirstlane(prev);
            if (prev == static_cast<uint32_t>(nT - 1)) {
                if (lane == 0) p.task_cnt[b] = 0U;  // ready for the next call
                FixupLongBlock<RowT, O>(p, blk, ts, nT, lane, alpha, beta);
            }
        }
        return;
    }

    // Block worker: one block per wave, or (block_stride > 0, capped grid)
    // blocks tile, tile + block_stride, ...
    const int64_t wg = static_cast<int64_t>(blockIdx.x) - p.task_wgs;
    const int64_t per = (static_cast<int64_t>(gridDim.x) - p.task_wgs) / kXcds;
    auto block = [&](int64_t tile) {
        Stage cur = OpenTileFlat<RowT>(p, tile);
        if constexpr (kEntry) {
            // one chunk: the window [kEntryChunk*tile, +kWaveChunk) holds the block
            cur.a0 = tile * kEntryChunk;
            cur.c1 = cur.kspan;
            cur.last = true;
        }
        const bool shortBlock = kEntry || BlockChunks(cur.k0, cur.kspan) <= kLongChunks;
        if (p.task_waves > 0 && !shortBlock) return;  // served by tasks
        carry = 0;
        auto chunks = [&](auto rows16) {
            constexpr bool k16 = decltype(rows16)::value;
            while (cur.valid) {
                L b;
                StreamLoadStage<RowT, V, O, kBeta, kNarrow, k16, kEntry>(p, cur, tailStart, lane, b);
                StreamGather<RowT, V, O, kStrided, kStrided && kNarrow>(p, cur, tailStart, rx, lane, b, b.xg, sVal);
                StreamChunk<RowT, V, O, kBeta, false, k16, kStrided>(cur, b, sVal, lane, alpha, beta, carry, lg, y,
                                                                      sink);
                if (cur.last) break;
                cur.c0 = cur.c1;
                cur.first = false;
                ChunkBounds(cur);
            }
        };
        // the narrow kernel reads the 16-bit row offsets of short blocks
        if (kNarrow && shortBlock && p.rp16 != nullptr) chunks(std::true_type{});
        else chunks(std::false_type{});
    };
    const int64_t first = ((wg % kXcds) * per + wg / kXcds) * kFlatWaves + wv;
    if constexpr (kGated) {
        const int64_t stride = p.block_stride > 0 ? p.block_stride : p.num_blocks;
        for (int64_t tile = first; tile < p.num_blocks; tile += stride) block(tile);
    } else {
        if (first < p.num_blocks) block(first);
    }
}

// --------------- stream kernel for int8 and complex64 operands ---------------
//
// The stream kernel's row blocks, chunk loads (16-byte col_ind groups, value
// loads clipped to the chunk) and gathers, for operands whose accumulator is
// not fp32: int8 values and x summed exactly in int64 (int32 output, with the
// reference's saturating epilogue), and complex64.  Products go to LDS in the
// accumulator type; rows are reduced by one lane, a lane group or the whole
// wave as in the fp32 kernel, without the fp32 kernel's tasks (a long block is
// processed chunk by chunk by its own wave).

template <ValKind V>
struct GenVals;
template <>
struct GenVals<ValKind::I8> {
    uint32_t v[2];  // 4 bytes per 16-byte group of slots
};
template <>
struct GenVals<ValKind::F32> {
    v4f v[2];
};
template <>
struct GenVals<ValKind::C64> {
    v4f v[4];  // two complex values per 16 bytes
};
template <>
struct GenVals<ValKind::UNIT> {
};

// Bytes of one gathered x element: the accumulator type for UNIT (the
// transpose's column pass gathers its products), else the value type.
template <ValKind V, AccKind A>
constexpr int64_t GenXBytes()
{
    return V == ValKind::UNIT ? static_cast<int64_t>(sizeof(typename AccOf<A>::T))
                              : static_cast<int64_t>(sizeof(typename ValOf<V>::T));
}

// In-chunk type of products and partial sums: int8 products (|a*x| <=
// 16384) summed over one 512-slot chunk stay below 2^23, so they are added
// exactly in int32; a row's chunks are combined, and the epilogue computed,
// in the int64 accumulator.  Other kinds use the accumulator throughout.
template <ValKind V, AccKind A>
using GenPart = typename std::conditional<V == ValKind::I8 && A == AccKind::I64, int32_t, typename AccOf<A>::T>::type;

template <ValKind V, AccKind A>
struct GenLoad {
    v4i col[2];
    GenVals<V> val;  // values of the lane's 8 slots
    int64_t rp[2];
    GenPart<V, A> xg[kLaneItems];
};

// kGath (complex64, fp32 values with complex compute, int8): the one-pass
// banded transpose on the CSC pattern:
// p.col holds each entry's row (x is gathered by it), p.val its CSR position
// (int32), and the value is gathered from p.gval by that position, conjugated
// when p.conj is set.  With kPack, p.col holds one word per entry instead:
// the row as an offset from the block's first column (low half) and the
// position as an offset from the entry's own CSC index (high half).
template <typename RowT, ValKind V, AccKind A, bool kGath = false, bool kPack = false, bool kNc = false>
__device__ __forceinline__ void GenLoadStage(const RowBlockParams& p, const Stage& s, int64_t tailStart, int lane,
                                             __amdgpu_buffer_rsrc_t rx, GenLoad<V, A>& b, int32_t* t = nullptr)
{
    static_assert(!kGath || V == ValKind::C64 || V == ValKind::F32 || V == ValKind::I8,
                  "gathered values: complex64, fp32 (complex compute) or int8");
    static_assert(!kPack || kGath, "packed offsets: the gathered-value transpose");
    v4i pos[2] = {};  // kGath: the slots' positions
    using ValT = typename ValOf<V>::T;
    const int64_t a0 = s.valid ? s.a0 : 0;
    int64_t end = (s.k0 + s.c1 + 3) & ~static_cast<int64_t>(3);
    end = end < tailStart ? end : tailStart;
    const int64_t avail = s.valid ? end - a0 : 0;
    const __amdgpu_buffer_rsrc_t rv = Rsrc(static_cast<const ValT*>(p.val) + a0, avail * sizeof(ValT));
    if constexpr (kNc) {
        // the narrow column copy (16-bit offsets from the block's first row),
        // as the row kernel of fp32 values reads it
        const __amdgpu_buffer_rsrc_t rn = Rsrc(p.ncol + a0, avail * 2);
        const uint32_t rb = static_cast<uint32_t>(s.valid ? s.r0 : 0) + static_cast<uint32_t>(p.base);
        const v2i lo = __builtin_bit_cast(v2i, __builtin_amdgcn_raw_buffer_load_b64(rn, lane * 8, 0, kBufNonTemporal));
        const v2i hi =
            __builtin_bit_cast(v2i, __builtin_amdgcn_raw_buffer_load_b64(rn, 512 + lane * 8, 0, kBufNonTemporal));
        b.col[0] = v4i{Lo16(lo.x, rb), Hi16(lo.x, rb), Lo16(lo.y, rb), Hi16(lo.y, rb)};
        b.col[1] = v4i{Lo16(hi.x, rb), Hi16(hi.x, rb), Lo16(hi.y, rb), Hi16(hi.y, rb)};
    } else {
        const __amdgpu_buffer_rsrc_t rc = Rsrc(p.col + a0, avail * 4);
        b.col[0] = __builtin_bit_cast(v4i, __builtin_amdgcn_raw_buffer_load_b128(rc, lane * 16, 0, kBufNonTemporal));
        b.col[1] =
            __builtin_bit_cast(v4i, __builtin_amdgcn_raw_buffer_load_b128(rc, 1024 + lane * 16, 0, kBufNonTemporal));
    }
    if constexpr (kPack) {
        (void)rv;  // positions: packed with the rows
    } else if constexpr (kGath) {
        const __amdgpu_buffer_rsrc_t rq = Rsrc(static_cast<const int32_t*>(p.val) + a0, avail * 4);
        pos[0] = __builtin_bit_cast(v4i, __builtin_amdgcn_raw_buffer_load_b128(rq, lane * 16, 0, kBufNonTemporal));
        pos[1] = __builtin_bit_cast(v4i, __builtin_amdgcn_raw_buffer_load_b128(rq, 1024 + lane * 16, 0, kBufNonTemporal));
        (void)rv;
    } else if constexpr (V == ValKind::UNIT) {
        (void)rv;
    } else if constexpr (V == ValKind::I8) {
        b.val.v[0] = __builtin_amdgcn_raw_buffer_load_b32(rv, lane * 4, 0, kBufNonTemporal);
        b.val.v[1] = __builtin_amdgcn_raw_buffer_load_b32(rv, 256 + lane * 4, 0, kBufNonTemporal);
    } else if constexpr (V == ValKind::F32) {
        b.val.v[0] = __builtin_bit_cast(v4f, __builtin_amdgcn_raw_buffer_load_b128(rv, lane * 16, 0, kBufNonTemporal));
        b.val.v[1] =
            __builtin_bit_cast(v4f, __builtin_amdgcn_raw_buffer_load_b128(rv, 1024 + lane * 16, 0, kBufNonTemporal));
    } else {
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const int off = (q >> 1) * 2048 + lane * 32 + (q & 1) * 16;
            b.val.v[q] = __builtin_bit_cast(v4f, __builtin_amdgcn_raw_buffer_load_b128(rv, off, 0, kBufNonTemporal));
        }
    }
    const int64_t r0 = s.valid ? s.r0 : 0;
    const int64_t nrp = s.valid ? ((s.nr + 2) & ~1) : 0;
    const __amdgpu_buffer_rsrc_t rr = Rsrc(static_cast<const RowT*>(p.rp) + r0, nrp * sizeof(RowT));
    if constexpr (sizeof(RowT) == 8) {
        const v4i w = __builtin_bit_cast(v4i, __builtin_amdgcn_raw_buffer_load_b128(rr, lane * 16, 0, kRowPolicy));
        b.rp[0] = static_cast<int64_t>((static_cast<uint64_t>(static_cast<uint32_t>(w.y)) << 32) |
                                       static_cast<uint32_t>(w.x));
        b.rp[1] = static_cast<int64_t>((static_cast<uint64_t>(static_cast<uint32_t>(w.w)) << 32) |
                                       static_cast<uint32_t>(w.z));
    } else {
        const v2i w = __builtin_bit_cast(v2i, __builtin_amdgcn_raw_buffer_load_b64(rr, lane * 8, 0, kRowPolicy));
        b.rp[0] = w.x;
        b.rp[1] = w.y;
    }
    // the last nnz % 4 entries (no whole 16-byte group): scalar loads, only
    // in the chunk that reaches them
    if (s.valid && s.a0 + kWaveChunk > tailStart && tailStart < p.nnz) {
#pragma unroll
        for (int j = 0; j < kLaneItems; ++j) {
            const int64_t k = s.a0 + StreamSlot(lane, j);
            if (k >= tailStart && k < p.nnz) {
                b.col[j >> 2][j & 3] = p.col[k];
                if constexpr (kPack) {
                } else if constexpr (kGath) {
                    pos[j >> 2][j & 3] = static_cast<const int32_t*>(p.val)[k];
                } else if constexpr (V == ValKind::UNIT) {
                } else if constexpr (V == ValKind::I8) {
                    const ValT v = static_cast<const ValT*>(p.val)[k];
                    const uint32_t sh = 8U * static_cast<uint32_t>(j & 3);
                    b.val.v[j >> 2] =
                        (b.val.v[j >> 2] & ~(0xFFU << sh)) | (static_cast<uint32_t>(static_cast<uint8_t>(v)) << sh);
                } else if constexpr (V == ValKind::F32) {
                    const ValT v = static_cast<const ValT*>(p.val)[k];
                    b.val.v[j >> 2][j & 3] = v;
                } else {
                    const ValT v = static_cast<const ValT*>(p.val)[k];
                    b.val.v[j >> 1][(j & 1) * 2] = v.re;
                    b.val.v[j >> 1][(j & 1) * 2 + 1] = v.im;
                }
            }
        }
    }
    if constexpr (kPack) {
        // the packed words move to slot 64j + lane (SlotOf<true>) through
        // the wave's LDS slice, then are decoded there
        *reinterpret_cast<v4i*>(&t[4 * lane]) = b.col[0];
        *reinterpret_cast<v4i*>(&t[256 + 4 * lane]) = b.col[1];
        const uint32_t rb = static_cast<uint32_t>(s.valid ? s.r0 : 0) + static_cast<uint32_t>(p.base);
        const uint32_t k0 = static_cast<uint32_t>(a0) + static_cast<uint32_t>(lane);
#pragma unroll
        for (int j = 0; j < kLaneItems; ++j) {
            const int32_t w = t[kWave * j + lane];
            b.col[j >> 2][j & 3] = Lo16(w, rb);
            pos[j >> 2][j & 3] = Hi16(w, k0 + static_cast<uint32_t>(kWave * j));
        }
    } else if constexpr (kGath) {
        // rows and positions move to slot 64j + lane (SlotOf<true>) through
        // the wave's LDS slice: each gather instruction then covers 64
        // consecutive slots
        *reinterpret_cast<v4i*>(&t[4 * lane]) = b.col[0];
        *reinterpret_cast<v4i*>(&t[256 + 4 * lane]) = b.col[1];
        int32_t c[kLaneItems];
#pragma unroll
        for (int j = 0; j < kLaneItems; ++j) c[j] = t[kWave * j + lane];
        *reinterpret_cast<v4i*>(&t[4 * lane]) = pos[0];
        *reinterpret_cast<v4i*>(&t[256 + 4 * lane]) = pos[1];
#pragma unroll
        for (int j = 0; j < kLaneItems; ++j) {
            b.col[j >> 2][j & 3] = c[j];
            pos[j >> 2][j & 3] = t[kWave * j + lane];
        }
    }
    const int32_t hiSlot = s.valid ? static_cast<int32_t>(s.k0 + s.c1 - s.a0) : 0;
#pragma unroll
    for (int j = 0; j < kLaneItems; ++j) {
        uint32_t off = static_cast<uint32_t>(b.col[j >> 2][j & 3] - p.base) *
                       static_cast<uint32_t>(GenXBytes<V, A>());
        off = SlotOf<kGath>(lane, j) < hiSlot ? off : 0xFFFFFFF0U;
        if constexpr (V == ValKind::UNIT) {
            const v2i w = __builtin_bit_cast(v2i, __builtin_amdgcn_raw_buffer_load_b64(rx, static_cast<int>(off), 0,
                                                                                     kGatherPolicy));
            if constexpr (A == AccKind::C64) {
                b.xg[j] = C64{__int_as_float(w.x), __int_as_float(w.y)};
            } else {
                b.xg[j] = static_cast<long long>((static_cast<uint64_t>(static_cast<uint32_t>(w.y)) << 32) |
                                                 static_cast<uint32_t>(w.x));
            }
        } else if constexpr (V == ValKind::I8) {
            const uint32_t raw = __builtin_amdgcn_raw_buffer_load_b8(rx, static_cast<int>(off), 0, kGatherPolicy);
            if constexpr (A == AccKind::I64) b.xg[j] = static_cast<int8_t>(static_cast<uint8_t>(raw));
            else b.xg[j] = ToAcc<V, A>(static_cast<int8_t>(static_cast<uint8_t>(raw)));
        } else if constexpr (V == ValKind::F32) {
            b.xg[j] = ToAcc<V, A>(
                __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rx, static_cast<int>(off), 0, kGatherPolicy)));
        } else {
            const v2f w = __builtin_bit_cast(v2f, __builtin_amdgcn_raw_buffer_load_b64(rx, static_cast<int>(off), 0,
                                                                                     kGatherPolicy));
            b.xg[j] = C64{w.x, w.y};
        }
    }
    if constexpr (kGath) {
        const __amdgpu_buffer_rsrc_t rg = Rsrc(p.gval, p.gval_n * static_cast<int64_t>(sizeof(ValT)));
        const bool conj = p.conj != 0;
        if constexpr (V == ValKind::I8) {
            b.val.v[0] = 0U;
            b.val.v[1] = 0U;
        }
#pragma unroll
        for (int j = 0; j < kLaneItems; ++j) {
            uint32_t off = static_cast<uint32_t>(pos[j >> 2][j & 3]) * static_cast<uint32_t>(sizeof(ValT));
            off = SlotOf<true>(lane, j) < hiSlot ? off : 0xFFFFFFF0U;
            if constexpr (V == ValKind::C64) {
                const v2f w = __builtin_bit_cast(
                    v2f, __builtin_amdgcn_raw_buffer_load_b64(rg, static_cast<int>(off), 0, kGatherPolicy));
                b.val.v[j >> 1][(j & 1) * 2] = w.x;
                b.val.v[j >> 1][(j & 1) * 2 + 1] = conj ? -w.y : w.y;  // as MaybeConj
            } else if constexpr (V == ValKind::F32) {  // (no conjugate: launched for opA = T only)
                b.val.v[j >> 2][j & 3] = __builtin_bit_cast(
                    float, __builtin_amdgcn_raw_buffer_load_b32(rg, static_cast<int>(off), 0, kGatherPolicy));
            } else {
                const uint32_t raw = __builtin_amdgcn_raw_buffer_load_b8(rg, static_cast<int>(off), 0, kGatherPolicy);
                b.val.v[j >> 2] |= (raw & 0xFFU) << (8U * static_cast<uint32_t>(j & 3));
            }
        }
    }
}

template <ValKind V, AccKind A>
__device__ __forceinline__ GenPart<V, A> GenVal(const GenLoad<V, A>& b, int j)
{
    if constexpr (V == ValKind::I8 && A == AccKind::I64) {
        return static_cast<int8_t>((b.val.v[j >> 2] >> (8 * (j & 3))) & 0xFFU);
    } else if constexpr (V == ValKind::I8) {
        return ToAcc<V, A>(static_cast<int8_t>((b.val.v[j >> 2] >> (8 * (j & 3))) & 0xFFU));
    } else if constexpr (V == ValKind::F32) {
        return ToAcc<V, A>(b.val.v[j >> 2][j & 3]);
    } else {
        return C64{b.val.v[j >> 1][(j & 1) * 2], b.val.v[j >> 1][(j & 1) * 2 + 1]};
    }
}

template <typename T>
__device__ __forceinline__ T WaveAllSum(T v)
{
    for (int m = 1; m < kWave; m <<= 1) v = v + ShflXorAcc(v, m);
    return v;
}

template <typename RowT, ValKind V, OutKind O, AccKind A, bool kS = false>
__device__ __forceinline__ void GenChunk(const RowBlockParams& p, const Stage& cur, const GenLoad<V, A>& lc,
                                         GenPart<V, A>* sVal, int lane, typename AccOf<A>::T alpha,
                                         typename AccOf<A>::T beta, bool betaNz, typename AccOf<A>::T& carry, int& lg)
{
    using Acc = typename AccOf<A>::T;
    using Part = GenPart<V, A>;
    using OutT = typename OutOf<O>::T;
    Part prod[kLaneItems];
#pragma unroll
    for (int j = 0; j < kLaneItems; ++j) {
        if constexpr (V == ValKind::UNIT) prod[j] = lc.xg[j];
        else prod[j] = GenVal<V, A>(lc, j) * lc.xg[j];
    }
    const int32_t c0 = cur.c0, c1 = cur.c1;
    const int32_t shift = static_cast<int32_t>(cur.a0 - cur.k0);
    const int nr = cur.nr;
    if (cur.first) {
        carry = Zero<Acc>();
        lg = 0;
        if (cur.last) {
            while (lg < 6 && (nr << (lg + 1)) <= kWave) ++lg;
        }
    }
#pragma unroll
    for (int j = 0; j < kLaneItems; ++j) sVal[SlotOf<kS>(lane, j)] = prod[j];

    const int32_t k0lo = static_cast<int32_t>(cur.k0);
    int32_t rs[2], re[2];
    rs[0] = static_cast<int32_t>(lc.rp[0]) - k0lo;
    rs[1] = static_cast<int32_t>(lc.rp[1]) - k0lo;
    re[0] = rs[1];
    re[1] = FromNextLane(rs[0], rs[1]);
    const int gsz = 1 << lg;
    bool fin[2], defer[2], active[2], crosses[2];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
        const int i = 2 * lane + h;
        const bool in = i < nr;
        const bool empty = re[h] <= rs[h];
        active[h] = in && (empty ? ((rs[h] >= c0 && rs[h] < c1) || (cur.last && rs[h] >= c1))
                                 : (rs[h] < c1 && re[h] > c0));
        crosses[h] = !empty && (rs[h] < c0 || re[h] > c1);
    }
    // one lane per row: 16 entries when a row of 9-16 lies inside the chunk
    bool wide = false;
    if (lg == 0) {
        const bool mid0 = active[0] && !crosses[0] && re[0] - rs[0] > kSerialCapOne && re[0] - rs[0] <= 16;
        const bool mid1 = active[1] && !crosses[1] && re[1] - rs[1] > kSerialCapOne && re[1] - rs[1] <= 16;
        wide = __ballot(mid0 || mid1) != 0;
    }
    const int cap = wide ? 16 : SerialCap(lg);
#pragma unroll
    for (int h = 0; h < 2; ++h) {
        defer[h] = active[h] && (crosses[h] || re[h] - rs[h] > cap);
        fin[h] = active[h] && !defer[h];
    }
    WaveLdsSync();

    Acc sum[2] = {Zero<Acc>(), Zero<Acc>()};
    if (lg == 0) {
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const int32_t len = fin[h] ? re[h] - rs[h] : 0;
            const int32_t base = fin[h] ? rs[h] - shift : 0;
            Part acc = Zero<Part>();
#pragma unroll
            for (int t = 0; t < 16; ++t) {
                if (t < kSerialCapOne || wide) {
                    const Part v = sVal[base + t];
                    acc = acc + (t < len ? v : Zero<Part>());
                }
            }
            sum[h] = static_cast<Acc>(acc);
        }
    } else {
        const int g = lane >> lg;
        const int sub = lane & (gsz - 1);
        const bool in = g < nr;
        const int src = (g >> 1) & (kWave - 1);
        const int32_t a0s = __shfl(rs[0], src, kWave), a1s = __shfl(rs[1], src, kWave);
        const int32_t a1e = __shfl(re[1], src, kWave);
        const int32_t gs = (g & 1) ? a1s : a0s;
        const int32_t ge = (g & 1) ? a1e : a1s;
        Part part = Zero<Part>();
        if (in && ge - gs <= cap) {
            for (int32_t q = gs + sub; q < ge; q += gsz) part = part + sVal[q - shift];
        }
        for (int m = 1; m < gsz; m <<= 1) part = part + ShflXorAcc(part, m);
        sum[0] = static_cast<Acc>(ReadLane(part, ((2 * lane) << lg) & (kWave - 1)));
        sum[1] = static_cast<Acc>(ReadLane(part, ((2 * lane + 1) << lg) & (kWave - 1)));
    }

    uint64_t pending0 = __ballot(defer[0]), pending1 = __ballot(defer[1]);
    while (pending0 | pending1) {
        const int l0 = pending0 ? __builtin_ctzll(pending0) : kWave;
        const int l1 = pending1 ? __builtin_ctzll(pending1) : kWave;
        const int h = (2 * l1 + 1 < 2 * l0) ? 1 : 0;
        const int l = h ? l1 : l0;
        if (h) {
            pending1 &= pending1 - 1;
        } else {
            pending0 &= pending0 - 1;
        }
        const int32_t s0 = __builtin_amdgcn_readlane(h ? rs[1] : rs[0], l);
        const int32_t e0 = __builtin_amdgcn_readlane(h ? re[1] : re[0], l);
        const int32_t lo = s0 > c0 ? s0 : c0;
        const int32_t hi = e0 < c1 ? e0 : c1;
        Part part = Zero<Part>();
        for (int32_t q = lo + lane; q < hi; q += kWave) part = part + sVal[q - shift];
        Acc total = static_cast<Acc>(WaveAllSum(part));
        if (s0 < c0) total = carry + total;
        if (e0 > c1) {
            carry = total;
        } else if (lane == l) {
            sum[h] = total;
            fin[h] = true;
        }
    }
    OutT* y = static_cast<OutT*>(p.y);
#pragma unroll
    for (int h = 0; h < 2; ++h) {
        if (fin[h]) StoreRow<O, A>(y, cur.r0 + 2 * lane + h, sum[h], alpha, beta, betaNz);
    }
    WaveLdsSync();  // this chunk's LDS reads complete before the next chunk overwrites
}

template <typename RowT, ValKind V, OutKind O, AccKind A, bool kGath = false, bool kPack = false, bool kNc = false>
__global__ __launch_bounds__(kWave* kFlatWaves) void SpmvStreamGenKernel(RowBlockParams p)
{
    using Acc = typename AccOf<A>::T;
    __shared__ GenPart<V, A> sValAll[kFlatWaves][kStreamLds];
    const int lane = threadIdx.x & (kWave - 1);
    const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
    Acc alpha, beta;
    LoadScalars<A>(p.s, alpha, beta);
    const bool betaNz = !IsZero(beta);
    const __amdgpu_buffer_rsrc_t rx = Rsrc(p.x, p.cols * GenXBytes<V, A>());
    const int64_t tailStart = p.nnz & ~static_cast<int64_t>(3);
    const int64_t wg = static_cast<int64_t>(blockIdx.x);
    const int64_t per = static_cast<int64_t>(gridDim.x) / kXcds;
    const int64_t tile = ((wg % kXcds) * per + wg / kXcds) * kFlatWaves + wv;
    if (tile >= p.num_blocks) return;
    Stage cur = OpenTileFlat<RowT>(p, tile);
    Acc carry = Zero<Acc>();
    int lg = 0;
    while (cur.valid) {
        GenLoad<V, A> b;
        GenLoadStage<RowT, V, A, kGath, kPack, kNc>(p, cur, tailStart, lane, rx, b, reinterpret_cast<int32_t*>(sValAll[wv]));
        GenChunk<RowT, V, O, A, kGath>(p, cur, b, sValAll[wv], lane, alpha, beta, betaNz, carry, lg);
        if (cur.last) break;
        cur.c0 = cur.c1;
        cur.first = false;
        ChunkBounds(cur);
    }
}

// ------------------------ SpMVOp on the row blocks ---------------------------
//
// z = alpha*(A*x) + beta*y with Priest's doubly compensated dot product, on
// the same row blocks, chunk loads and gathers as the stream kernel above.
// Each product is split exactly (prod, err) and both halves go to LDS; a row
// is accumulated in a triple by one lane (short rows), a lane group (medium
// rows; group triples merged by TwoSum butterflies) or the whole wave (long
// or chunk-crossing rows, with a triple carried from chunk to chunk).  The
// summation order depends only on the matrix, so results are reproducible.
// Long blocks are processed chunk by chunk by their own wave (no tasks).

template <typename RowT, bool kBeta>
__device__ __forceinline__ void StreamChunkOp(const Stage& cur, const StreamLoad<RowT, ValKind::F32, OutKind::F32>& lc,
                                              float* sP, float* sE, int lane, float alpha, float beta, Triple& carry,
                                              int& lg, float* z)
{
#pragma clang fp contract(off)
    float pr[kLaneItems], er[kLaneItems];
#pragma unroll
    for (int j = 0; j < kLaneItems; ++j) {
        const float a = lc.val.v[j >> 2][j & 3];
        const float xv = __uint_as_float(lc.xg[j]);
        pr[j] = a * xv;
        er[j] = __fmaf_rn(a, xv, -pr[j]);
    }
    const int32_t c0 = cur.c0, c1 = cur.c1;
    const int32_t shift = static_cast<int32_t>(cur.a0 - cur.k0);
    const int nr = cur.nr;
    if (cur.first) {
        carry = Triple{0.0f, 0.0f, 0.0f};
        lg = 0;
        if (cur.last) {
            while (lg < 6 && (nr << (lg + 1)) <= kWave) ++lg;
        }
    }
    *reinterpret_cast<v4f*>(&sP[4 * lane]) = v4f{pr[0], pr[1], pr[2], pr[3]};
    *reinterpret_cast<v4f*>(&sP[256 + 4 * lane]) = v4f{pr[4], pr[5], pr[6], pr[7]};
    *reinterpret_cast<v4f*>(&sE[4 * lane]) = v4f{er[0], er[1], er[2], er[3]};
    *reinterpret_cast<v4f*>(&sE[256 + 4 * lane]) = v4f{er[4], er[5], er[6], er[7]};

    const int32_t k0lo = static_cast<int32_t>(cur.k0);
    int32_t rs[2], re[2];
    rs[0] = static_cast<int32_t>(lc.rp[0]) - k0lo;
    rs[1] = static_cast<int32_t>(lc.rp[1]) - k0lo;
    re[0] = rs[1];
    re[1] = FromNextLane(rs[0], rs[1]);

    const int gsz = 1 << lg;
    bool fin[2], defer[2], active[2], crosses[2];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
        const int i = 2 * lane + h;
        const bool in = i < nr;
        const bool empty = re[h] <= rs[h];
        active[h] = in && (empty ? ((rs[h] >= c0 && rs[h] < c1) || (cur.last && rs[h] >= c1))
                                 : (rs[h] < c1 && re[h] > c0));
        crosses[h] = !empty && (rs[h] < c0 || re[h] > c1);
    }
    // one lane per row: 16 entries when a row of 9-16 lies inside the chunk
    bool wide = false;
    if (lg == 0) {
        const bool mid0 = active[0] && !crosses[0] && re[0] - rs[0] > kSerialCapOne && re[0] - rs[0] <= 16;
        const bool mid1 = active[1] && !crosses[1] && re[1] - rs[1] > kSerialCapOne && re[1] - rs[1] <= 16;
        wide = __ballot(mid0 || mid1) != 0;
    }
    const int cap = wide ? 16 : SerialCap(lg);
#pragma unroll
    for (int h = 0; h < 2; ++h) {
        defer[h] = active[h] && (crosses[h] || re[h] - rs[h] > cap);
        fin[h] = active[h] && !defer[h];
    }
    WaveLdsSync();

    // Phase 1.  Adding (0, 0) to a triple is exact, so masked entries add zeros.
    Triple sum[2] = {Triple{0.0f, 0.0f, 0.0f}, Triple{0.0f, 0.0f, 0.0f}};
    if (lg == 0) {
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const int32_t len = fin[h] ? re[h] - rs[h] : 0;
            const int32_t base = fin[h] ? rs[h] - shift : 0;
#pragma unroll
            for (int t = 0; t < 16; ++t) {
                if (t < kSerialCapOne || wide) {
                    const bool on = t < len;
                    PriestAddSplit(sum[h], on ? sP[base + t] : 0.0f, on ? sE[base + t] : 0.0f);
                }
            }
        }
    } else {
        const int g = lane >> lg;
        const int sub = lane & (gsz - 1);
        const bool in = g < nr;
        const int src = (g >> 1) & (kWave - 1);
        const int32_t a0s = __shfl(rs[0], src, kWave), a1s = __shfl(rs[1], src, kWave);
        const int32_t a1e = __shfl(re[1], src, kWave);
        const int32_t gs = (g & 1) ? a1s : a0s;
        const int32_t ge = (g & 1) ? a1e : a1s;
        Triple part{0.0f, 0.0f, 0.0f};
        if (in && ge - gs <= cap) {
            for (int32_t q = gs + sub; q < ge; q += gsz) PriestAddSplit(part, sP[q - shift], sE[q - shift]);
        }
        for (int m = 1; m < gsz; m <<= 1) part = Merge(part, ShflXor(part, m));
        sum[0] = Shfl(part, ((2 * lane) << lg) & (kWave - 1));
        sum[1] = Shfl(part, ((2 * lane + 1) << lg) & (kWave - 1));
    }

    // Phase 2: deferred rows, whole wave per row, in row order.
    uint64_t pending0 = __ballot(defer[0]), pending1 = __ballot(defer[1]);
    while (pending0 | pending1) {
        const int l0 = pending0 ? __builtin_ctzll(pending0) : kWave;
        const int l1 = pending1 ? __builtin_ctzll(pending1) : kWave;
        const int h = (2 * l1 + 1 < 2 * l0) ? 1 : 0;
        const int l = h ? l1 : l0;
        if (h) {
            pending1 &= pending1 - 1;
        } else {
            pending0 &= pending0 - 1;
        }
        const int32_t s0 = __builtin_amdgcn_readlane(h ? rs[1] : rs[0], l);
        const int32_t e0 = __builtin_amdgcn_readlane(h ? re[1] : re[0], l);
        const int32_t lo = s0 > c0 ? s0 : c0;
        const int32_t hi = e0 < c1 ? e0 : c1;
        Triple part{0.0f, 0.0f, 0.0f};
        for (int32_t q = lo + lane; q < hi; q += kWave) PriestAddSplit(part, sP[q - shift], sE[q - shift]);
        for (int m = 1; m < kWave; m <<= 1) part = Merge(part, ShflXor(part, m));
        if (s0 < c0) part = Merge(carry, part);
        if (e0 > c1) {
            carry = part;
        } else if (lane == l) {
            sum[h] = part;
            fin[h] = true;
        }
    }

#pragma unroll
    for (int h = 0; h < 2; ++h) {
        const int i = 2 * lane + h;
        float yv = 0.0f;
        if constexpr (kBeta) {
            if (beta != 0.0f) yv = lc.yold[h];
        }
        if (fin[h]) z[cur.r0 + i] = CombineZ(sum[h], alpha, beta, yv);
    }
    WaveLdsSync();
}

// ALG1 (no buffer, kFixed): block b is rows [b*R, (b+1)*R) of the caller's
// row offsets, R from the mean row length.
template <typename RowT>
__device__ __forceinline__ Stage OpenFixedTile(const RowBlockParams& p, int64_t tile)
{
    Stage s{};
    s.valid = true;
    const int64_t r0 = tile * p.fixed_rows;
    int64_t n = p.rows - r0;
    n = n > p.fixed_rows ? p.fixed_rows : n;
    s.r0 = r0;
    s.nr = static_cast<int32_t>(n);
    const int64_t k0 = static_cast<int64_t>(ConstLoad<RowT>(p.rp, r0)) - p.rp_base;
    const int64_t k1 = static_cast<int64_t>(ConstLoad<RowT>(p.rp, r0 + n)) - p.rp_base;
    s.k0 = k0;
    const int64_t span = k1 - k0;
    s.kspan = static_cast<int32_t>(span < 0 ? 0 : span > 0x7FFFFFFFLL ? 0x7FFFFFFFLL : span);
    s.c0 = 0;
    s.first = true;
    ChunkBounds(s);
    return s;
}

// kGated / kNarrow / kEntry: as in SpmvStreamFlatKernel (the ALG2 buffer
// holds the same narrow column copy and entry-aligned blocks).
template <typename RowT, bool kBeta, bool kFixed = false, bool kGated = false, bool kNarrow = false,
          bool kEntry = false>
__global__ __launch_bounds__(kWave* kFlatWaves) void SpmvOpStreamKernel(RowBlockParams p)
{
    using L = StreamLoad<RowT, ValKind::F32, OutKind::F32>;
    __shared__ float sPAll[kFlatWaves][kStreamLds];
    __shared__ float sEAll[kFlatWaves][kStreamLds];
    if constexpr (kGated) {
        const uint32_t flag = ConstLoad<uint32_t>(p.skip_flag, 0);
        if (flag >= 32U || ((p.run_mask >> flag) & 1U) == 0U) return;
    }
    const int lane = threadIdx.x & (kWave - 1);
    const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
    float alpha, beta;
    LoadScalars<AccKind::F32>(p.s, alpha, beta);
    const __amdgpu_buffer_rsrc_t rx = Rsrc(p.x, p.cols * static_cast<int64_t>(sizeof(float)));
    const int64_t tailStart = p.nnz & ~static_cast<int64_t>(3);
    const int64_t wg = static_cast<int64_t>(blockIdx.x);
    const int64_t per = static_cast<int64_t>(gridDim.x) / kXcds;
    const int64_t tile = ((wg % kXcds) * per + wg / kXcds) * kFlatWaves + wv;
    if (tile >= p.num_blocks) return;
    Stage cur = kFixed ? OpenFixedTile<RowT>(p, tile) : OpenTileFlat<RowT>(p, tile);
    if constexpr (kEntry) {
        cur.a0 = tile * kEntryChunk;  // the window holds the whole block
        cur.c1 = cur.kspan;
        cur.last = true;
    }
    Triple carry{0.0f, 0.0f, 0.0f};
    int lg = 0;
    while (cur.valid) {
        L b;
        StreamLoadStage<RowT, ValKind::F32, OutKind::F32, kBeta, kNarrow, false, kEntry>(p, cur, tailStart, lane, b);
        StreamGather<RowT, ValKind::F32, OutKind::F32>(p, cur, tailStart, rx, lane, b, b.xg);
        StreamChunkOp<RowT, kBeta>(cur, b, sPAll[wv], sEAll[wv], lane, alpha, beta, carry, lg, p.z);
        if (cur.last) break;
        cur.c0 = cur.c1;
        cur.first = false;
        ChunkBounds(cur);
    }
}

// ------------------------------- transpose ----------------------------------

// Transpose of a matrix without non-zeros: y = beta*y in place (y is not
// read when beta == 0).  Used when y's type is the accumulator type.
template <OutKind O, AccKind A>
__global__ __launch_bounds__(kThreads) void ScaleKernel(typename OutOf<O>::T* y, int64_t n, int64_t stride,
                                                         Scalars s)
{
    using Acc = typename AccOf<A>::T;
    Acc alpha, beta;
    LoadScalars<A>(s, alpha, beta);
    const bool betaNz = !IsZero(beta);
    for (int64_t j = blockIdx.x * static_cast<int64_t>(kThreads) + threadIdx.x; j < n;
         j += static_cast<int64_t>(gridDim.x) * kThreads) {
        y[j * stride] = betaNz ? beta * y[j * stride] : Zero<Acc>();
    }
}

template <AccKind A>
__global__ __launch_bounds__(kThreads) void ClearKernel(typename AccOf<A>::T* acc, int64_t n)
{
    for (int64_t j = blockIdx.x * static_cast<int64_t>(kThreads) + threadIdx.x; j < n;
         j += static_cast<int64_t>(gridDim.x) * kThreads) {
        acc[j] = Zero<typename AccOf<A>::T>();
    }
}

// y = finalize(acc) with acc cleared (transpose without non-zeros, y not of
// the accumulator type): the reference's epilogue of a zero sum
// (sparse/spmv/arch35/spmv_kernel.cpp:626-668).
template <OutKind O, AccKind A>
__global__ __launch_bounds__(kThreads) void FinalizeKernel(const typename AccOf<A>::T* acc,
                                                            typename OutOf<O>::T* y, int64_t n, int64_t stride,
                                                            Scalars s)
{
    using Acc = typename AccOf<A>::T;
    Acc alpha, beta;
    LoadScalars<A>(s, alpha, beta);
    const bool betaNz = !IsZero(beta);
    for (int64_t j = blockIdx.x * static_cast<int64_t>(kThreads) + threadIdx.x; j < n;
         j += static_cast<int64_t>(gridDim.x) * kThreads) {
        const Acc oldY = betaNz ? OutToAcc<O, A>(y[j * stride]) : Zero<Acc>();
        Acc r;
        if constexpr (A == AccKind::I64) r = ScaledI64(acc[j], alpha, beta, oldY);
        else r = betaNz ? acc[j] + beta * oldY : acc[j];
        y[j * stride] = FromAcc<O, A>(r);
    }
}

template <ValKind V, AccKind A>
__device__ __forceinline__ typename AccOf<A>::T MaybeConj(typename AccOf<A>::T v, int conj)
{
    if constexpr (A == AccKind::C64) return conj ? C64{v.re, -v.im} : v;
    else return v;
}

// ------------------------- transpose by columns ------------------------------
//
// Preprocess sorts the entries by column (stable radix sort of (column,
// position) pairs), so y_j = alpha * sum_{i} conj?(a_ij) * x_i + beta * y_j is
// a gather over column j's entries: no atomics, a fixed summation order
// (deterministic results, the reference's CSR_ALG2 transpose semantics,
// sparse/spmv/arch35/spmv_kernel.cpp:861-879), and the values are read from
// the caller's array at execution time.

struct CscBuildParams {
    const int32_t* col;
    int64_t col_stride;
    int32_t base;
    int64_t rows, cols, nnz;
    const void* norm;  // normalised row offsets (RowT)
    int32_t* key;      // sort keys: column, or cols for entries outside the matrix
    void* pos;         // sort values: position in the CSR arrays
};

template <typename RowT>
__global__ __launch_bounds__(kThreads) void CscInitKernel(CscBuildParams q)
{
    const RowT* norm = static_cast<const RowT*>(q.norm);
    const int64_t first = static_cast<int64_t>(norm[0]);
    const int64_t last = static_cast<int64_t>(norm[q.rows]);
    RowT* pos = static_cast<RowT*>(q.pos);
    for (int64_t k = blockIdx.x * static_cast<int64_t>(kThreads) + threadIdx.x; k < q.nnz;
         k += static_cast<int64_t>(gridDim.x) * kThreads) {
        const int64_t c = static_cast<int64_t>(q.col[k * q.col_stride]) - q.base;
        const bool ok = k >= first && k < last && c >= 0 && c < q.cols;
        q.key[k] = static_cast<int32_t>(ok ? c : q.cols);
        pos[k] = static_cast<RowT>(k);
    }
}

// colptr[c] = first sorted entry with column >= c, for c in [0, cols].
template <typename RowT>
__global__ __launch_bounds__(kThreads) void CscColPtrKernel(const int32_t* keys, int64_t nnz, int64_t cols,
                                                            RowT* colptr)
{
    for (int64_t k = blockIdx.x * static_cast<int64_t>(kThreads) + threadIdx.x; k <= nnz;
         k += static_cast<int64_t>(gridDim.x) * kThreads) {
        const int64_t prev = k == 0 ? -1 : static_cast<int64_t>(keys[k - 1]);
        const int64_t cur = k == nnz ? cols : static_cast<int64_t>(keys[k]);
        for (int64_t c = prev + 1; c <= cur; ++c) colptr[c] = static_cast<RowT>(k);
    }
}

// Row of every entry in CSR order (the last row whose normalised offset is
// <= k; entries outside [norm[0], norm[rows]) get row 0 and are never used);
// the sorted positions move to their final array if the sort left them in
// the other buffer.  One wave per workgroup; a wave takes kFinishSpan
// consecutive entries: it finds the rows ra and rb of its first and last
// in-range entry (wave-uniform searches), marks in LDS the first entry of
// every row after ra that starts in its span (the largest row where several
// empty rows share a start), and a running maximum over the marks gives each
// entry its row: 16 consecutive entries per lane, then a prefix maximum over
// the lanes.  The rows go out through LDS again, so that the stores are
// coalesced.
constexpr int kFinishPer = 16;
constexpr int kFinishSpan = kFinishPer * kWave;
template <typename RowT>
__device__ __forceinline__ int64_t LastRowAtOrBefore(const RowT* norm, int64_t lo, int64_t hi, int64_t k)
{
    while (lo < hi) {
        const int64_t mid = (lo + hi + 1) >> 1;
        if (static_cast<int64_t>(norm[mid]) <= k) lo = mid;
        else hi = mid - 1;
    }
    return lo;
}

template <typename RowT>
__global__ __launch_bounds__(kWave) void CscFinishKernel(const RowT* sortedPos, RowT* pos, int32_t* entryRow,
                                                         const RowT* norm, int64_t rows, int64_t n)
{
    __shared__ int32_t mark[kFinishSpan];
    const int64_t first = static_cast<int64_t>(norm[0]);
    const int64_t last = static_cast<int64_t>(norm[rows]);
    const int lane = threadIdx.x;
    for (int64_t w = blockIdx.x; w * kFinishSpan < n; w += gridDim.x) {
        const int64_t base = w * kFinishSpan;
        const int64_t end = base + kFinishSpan < n ? base + kFinishSpan : n;
        if (sortedPos != pos) {
            for (int64_t k = base + lane; k < end; k += kWave) pos[k] = sortedPos[k];
        }
        const int64_t a = base > first ? base : first;
        const int64_t b = (end < last ? end : last) - 1;
        if (a > b) {  // no entry of the span lies in a row (uniform)
            for (int64_t k = base + lane; k < end; k += kWave) entryRow[k] = 0;
            continue;
        }
        const int64_t ra = LastRowAtOrBefore(norm, 0, rows - 1, a);
        const int64_t rb = LastRowAtOrBefore(norm, ra, rows - 1, b);
        for (int i = lane; i < kFinishSpan; i += kWave) mark[i] = -1;
        __syncthreads();
        for (int64_t r = ra + 1 + lane; r <= rb; r += kWave) {
            const int64_t st = static_cast<int64_t>(norm[r]) - base;
            if (st >= 0 && st < kFinishSpan) atomicMax(&mark[st], static_cast<int32_t>(r));
        }
        __syncthreads();
        // running maximum over the lane's 16 entries, then over the lanes before it
        int32_t v[kFinishPer];
        int32_t run = -1;
#pragma unroll
        for (int j = 0; j < kFinishPer; ++j) {
            const int32_t m = mark[lane * kFinishPer + j];
            run = m > run ? m : run;
            v[j] = run;
        }
        int32_t carry = run;  // inclusive prefix maximum of the lanes' maxima
#pragma unroll
        for (int d = 1; d < kWave; d <<= 1) {
            const int32_t o = __shfl_up(carry, d, kWave);
            if (lane >= d) carry = o > carry ? o : carry;
        }
        int32_t before = __shfl_up(carry, 1, kWave);
        before = lane == 0 ? -1 : before;
        const int32_t start = before > static_cast<int32_t>(ra) ? before : static_cast<int32_t>(ra);
        __syncthreads();
#pragma unroll
        for (int j = 0; j < kFinishPer; ++j) {
            const int64_t k = base + lane * kFinishPer + j;
            const int32_t r = v[j] > start ? v[j] : start;
            mark[lane * kFinishPer + j] = k >= first && k < last ? r : 0;
        }
        __syncthreads();
        for (int64_t k = base + lane; k < end; k += kWave) entryRow[k] = mark[k - base];
        __syncthreads();
    }
}

// Compact row table: one workgroup per group of kRowGroup entries.  Rows are
// non-decreasing over [norm[0], norm[rows]), so the span of a group is its
// last in-range row minus its first; entries outside that range get delta 0.
template <typename RowT>
__global__ __launch_bounds__(kThreads) void CscRowDeltaKernel(const int32_t* entryRow, const RowT* norm, int64_t rows,
                                                              int32_t* groupRow, uint8_t* delta)
{
    static_assert(kRowGroup == kThreads, "one thread per entry of a group");
    const int64_t g = blockIdx.x;
    const int64_t first = static_cast<int64_t>(norm[0]);
    const int64_t last = static_cast<int64_t>(norm[rows]);
    int64_t kf = g * kRowGroup, kl = kf + kRowGroup - 1;
    kf = kf > first ? kf : first;
    kl = kl < last - 1 ? kl : last - 1;
    int32_t base = 0;
    bool narrow = true;
    if (kf <= kl) {
        base = entryRow[kf];
        narrow = entryRow[kl] - base <= 255;
    }
    const int64_t k = g * kRowGroup + threadIdx.x;
    const int32_t r = k >= kf && k <= kl ? entryRow[k] : base;
    delta[k] = narrow ? static_cast<uint8_t>(r - base) : uint8_t{0};
    // a group with no entry inside the matrix takes the per-entry path (it reads nothing)
    if (threadIdx.x == 0) groupRow[g] = narrow && kf <= kl ? base : -1;
}

struct CscParams {
    const void* colptr;  // RowT[cols+1]
    const int32_t* entry_row;
    const int32_t* group_row;   // compact row table (see the workspace layout)
    const uint32_t* row_delta;  // four 8-bit deltas per dword
    int64_t row_groups;
    const void* pos;     // RowT[nnz]
    void* prod;          // Acc[nnz]
    const void* val;
    int64_t val_stride;
    const void* x;
    int64_t x_stride;
    void* y;
    int64_t y_stride;
    const void* norm;     // RowT[rows+1]: entries [norm[0], norm[rows]) belong to rows
    int64_t rows;
    int64_t cols;
    int32_t lg;  // log2 lanes per column
    int32_t conj;
    const uint32_t* skip_flag;  // non-null: exit when it reads 1 (the column-bucketed kernels run instead)
    Scalars s;
};

#ifndef PROD_MAX_BLOCKS
#define PROD_MAX_BLOCKS 2048
#endif
// Product pass grid: 2048 workgroups (8 per CU), waves looping over the
// groups (1024 and 4096 measured slower; one workgroup per 4 groups slower still).
constexpr int64_t kProdMaxBlocks = PROD_MAX_BLOCKS;

// Four consecutive elements, moved by one vector access.
template <typename T>
struct alignas(4 * sizeof(T)) Quad {
    T v[4];
};

// Pass 1, in CSR order: prod[k] = conj?(a_k) * x[row(k)].  One wave per
// group of kRowGroup entries, four consecutive entries per lane.  The rows
// come from the compact table: one dword of 8-bit deltas per lane over the
// group's first row, so the group's x values are the contiguous run
// x[row0 .. row0 + span], which the wave reads once, coalesced, into LDS and
// then indexes by delta.  A group spanning more than 255 rows reads its rows
// from the int32 table and gathers x per entry (so does a strided x).
// Values and products move as whole 4-entry vectors when the values are
// contiguous and aligned (kVec; the products always are).
template <typename RowT, ValKind V, AccKind A, bool kVec>
__global__ __launch_bounds__(kThreads) void CscProductKernel(CscParams q)
{
    using Acc = typename AccOf<A>::T;
    using ValT = typename ValOf<V>::T;
    static_assert(kRowGroup == 4 * kWave, "a group is one wave of 4 entries per lane");
    if (q.skip_flag != nullptr && ConstLoad<uint32_t>(q.skip_flag, 0) != 0U) return;
    __shared__ ValT sx[kThreads / kWave][kRowGroup];
    const ValT* val = static_cast<const ValT*>(q.val);
    const ValT* x = static_cast<const ValT*>(q.x);
    Acc* prod = static_cast<Acc*>(q.prod);
    const RowT* norm = static_cast<const RowT*>(q.norm);
    const int wv = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x) / kWave);
    const int lane = static_cast<int>(threadIdx.x) & (kWave - 1);
    const int64_t first = static_cast<int64_t>(norm[0]);
    const int64_t last = static_cast<int64_t>(norm[q.rows]);
    for (int64_t g = static_cast<int64_t>(blockIdx.x) * (kThreads / kWave) + wv; g < q.row_groups;
         g += static_cast<int64_t>(gridDim.x) * (kThreads / kWave)) {
        const int64_t k0 = g * kRowGroup + 4 * lane;
        const bool full = k0 >= first && k0 + 4 <= last;
        const int32_t gr = ConstLoad<int32_t>(q.group_row, g);
        const bool run = gr >= 0 && q.x_stride == 1;  // wave-uniform
        int32_t row[4];
        if (gr >= 0) {
            const uint32_t d = q.row_delta[g * (kRowGroup / 4) + lane];
#pragma unroll
            for (int u = 0; u < 4; ++u) row[u] = static_cast<int32_t>((d >> (8 * u)) & 0xFFU);
        } else if (full) {
            const v4i r = *reinterpret_cast<const v4i*>(q.entry_row + k0);
            row[0] = r.x;
            row[1] = r.y;
            row[2] = r.z;
            row[3] = r.w;
        } else {
#pragma unroll
            for (int u = 0; u < 4; ++u) row[u] = k0 + u >= first && k0 + u < last ? q.entry_row[k0 + u] : 0;
        }
        ValT v[4];
        if (kVec && full) {
            const Quad<ValT> w = *reinterpret_cast<const Quad<ValT>*>(val + k0);
#pragma unroll
            for (int u = 0; u < 4; ++u) v[u] = w.v[u];
        } else {
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                const int64_t k = k0 + u;
                v[u] = k >= first && k < last ? val[k * q.val_stride] : ValT{};
            }
        }
        ValT xv[4];
        if (run) {
            // span = largest delta of the group (entries outside the matrix have delta 0)
            int span = row[0] > row[1] ? row[0] : row[1];
            span = span > row[2] ? span : row[2];
            span = span > row[3] ? span : row[3];
#pragma unroll
            for (int m = 1; m < kWave; m <<= 1) {
                const int o = __shfl_xor(span, m, kWave);
                span = span > o ? span : o;
            }
#pragma unroll
            for (int j = 0; j < kRowGroup / kWave; ++j) {
                const int i = lane + j * kWave;
                if (j * kWave <= span && i <= span) sx[wv][i] = x[static_cast<int64_t>(gr) + i];
            }
            WaveLdsSync();
#pragma unroll
            for (int u = 0; u < 4; ++u) xv[u] = sx[wv][row[u]];
        } else {
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                const int64_t r = static_cast<int64_t>(gr >= 0 ? gr + row[u] : row[u]);
                xv[u] = k0 + u >= first && k0 + u < last ? x[r * q.x_stride] : ValT{};
            }
        }
        Quad<Acc> out;
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const int64_t k = k0 + u;
            const Acc xr = k >= first && k < last ? ToAcc<V, A>(xv[u]) : Zero<Acc>();
            out.v[u] = MaybeConj<V, A>(ToAcc<V, A>(v[u]), q.conj) * xr;
        }
        if (full) {
            *reinterpret_cast<Quad<Acc>*>(prod + k0) = out;
        } else {
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                const int64_t k = k0 + u;
                if (k >= first && k < last) prod[k] = out.v[u];
            }
        }
        WaveLdsSync();  // this group's LDS reads complete before the next group's writes
    }
}

// Pass 2, by columns: 2^lg lanes per column, each summing the products of a
// strided subset of the column's entries (one random read per entry), merged
// by a fixed butterfly; the first lane applies the epilogue.
template <typename RowT, ValKind V, OutKind O, AccKind A>
__global__ __launch_bounds__(kThreads) void SpmvCscGatherKernel(CscParams q)
{
    using Acc = typename AccOf<A>::T;
    if (q.skip_flag != nullptr && ConstLoad<uint32_t>(q.skip_flag, 0) != 0U) return;
    const int lg = q.lg;
    const int g = 1 << lg;
    const int64_t c = (static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x) >> lg;
    const int sub = threadIdx.x & (g - 1);
    Acc alpha, beta;
    LoadScalars<A>(q.s, alpha, beta);
    const RowT* colptr = static_cast<const RowT*>(q.colptr);
    const RowT* pos = static_cast<const RowT*>(q.pos);
    const Acc* prod = static_cast<const Acc*>(q.prod);
    Acc sum = Zero<Acc>();
    if (c < q.cols) {
        const int64_t k1 = static_cast<int64_t>(colptr[c + 1]);
        // batches of 4 entries per lane: the 4 position loads, then the 4
        // product reads, are in flight together; the sum keeps entry order
        constexpr int kB = 4;
        for (int64_t k0 = static_cast<int64_t>(colptr[c]) + sub; k0 < k1; k0 += kB * g) {
            int64_t pk[kB];
#pragma unroll
            for (int u = 0; u < kB; ++u) pk[u] = k0 + u * g < k1 ? static_cast<int64_t>(pos[k0 + u * g]) : -1;
            Acc v[kB];
#pragma unroll
            for (int u = 0; u < kB; ++u) v[u] = pk[u] >= 0 ? prod[pk[u]] : Zero<Acc>();
#pragma unroll
            for (int u = 0; u < kB; ++u) {
                if (pk[u] >= 0) sum = sum + v[u];
            }
        }
    }
    for (int m = 1; m < g; m <<= 1) sum = sum + ShflXorAcc(sum, m);
    if (c < q.cols && sub == 0) {
        StoreRow<O, A>(static_cast<typename OutOf<O>::T*>(q.y), c * q.y_stride, sum, alpha, beta, !IsZero(beta));
    }
}

// ------------------------------- preprocess ---------------------------------

struct PrepParams {
    const void* rp;        // original row offsets
    int64_t stride;
    int64_t base;
    int64_t rows, cols, nnz;
    void* norm;            // normalised row offsets (RowT)
    int32_t* blocks;
    void* block_nnz;
    int64_t num_blocks;
    int64_t items;         // T
    SpmvWsHeader* header;
    SpmvWsHeader header_value;
};

template <typename SrcT>
__device__ __forceinline__ int64_t NormRow(const PrepParams& p, int64_t i)
{
    int64_t v = static_cast<int64_t>(static_cast<const SrcT*>(p.rp)[i * p.stride]) - p.base;
    return v < 0 ? 0 : v > p.nnz ? p.nnz : v;
}

template <typename SrcT>
__global__ __launch_bounds__(kThreads) void SpmvPreprocessKernel(PrepParams p)
{
    const int64_t i = blockIdx.x * static_cast<int64_t>(kThreads) + threadIdx.x;
    if (i <= p.rows) {
        const SrcT v = static_cast<SrcT>(NormRow<SrcT>(p, i));
        static_cast<SrcT*>(p.norm)[i] = v;
        if (i == p.rows) static_cast<SrcT*>(p.norm)[i + 1] = v;  // pad entry (offsets are read in pairs)
    }
    if (i <= p.num_blocks) {
        int32_t start;
        if (i == p.num_blocks) {
            start = static_cast<int32_t>(p.rows);
        } else {
            // First row r in [0, rows] whose coordinate 16*r + offset(r) >= i*T.
            const int64_t diag = i * p.items;
            int64_t lo = 0, hi = p.rows;
            while (lo < hi) {
                const int64_t mid = (lo + hi) >> 1;
                if (kRowWeight * mid + NormRow<SrcT>(p, mid) >= diag) hi = mid;
                else lo = mid + 1;
            }
            start = static_cast<int32_t>(lo);
        }
        p.blocks[i] = start;
        static_cast<SrcT*>(p.block_nnz)[i] = static_cast<SrcT>(NormRow<SrcT>(p, start));
    }
    if (i == 0 && p.header != nullptr) *p.header = p.header_value;
}

int GridFor(int64_t n)
{
    int64_t g = (n + kThreads - 1) / kThreads;
    if (g < 1) g = 1;
    if (g > 65536) g = 65536;
    return static_cast<int>(g);
}

template <typename T>
T* At(void* ws, size_t off) { return reinterpret_cast<T*>(static_cast<uint8_t*>(ws) + off); }

RowBlockParams MakeRowBlockParams(const SpmvLaunch& l)
{
    RowBlockParams p{};
    p.run_mask = 1U;  // gated launches: the row / CSC kernels' flag value 0
    p.ncol = l.layout.narrow ? At<const int16_t>(l.ws, l.layout.nc_offset) : nullptr;
    p.rp16 = l.layout.narrow ? At<const uint16_t>(l.ws, l.layout.nr_offset) : nullptr;
    p.rp = At<void>(l.ws, l.layout.rowptr_offset);
    p.blocks = At<int32_t>(l.ws, l.layout.blocks_offset);
    p.block_nnz = At<void>(l.ws, l.layout.block_nnz_offset);
    p.sink = At<void>(l.ws, l.layout.sink_offset);
    if (l.layout.tasks) {
        p.task_start = At<int32_t>(l.ws, l.layout.task_start_offset);
        p.task_block = At<int32_t>(l.ws, l.layout.task_block_offset);
        p.task_head = At<float>(l.ws, l.layout.task_head_offset);
        p.task_tail = At<float>(l.ws, l.layout.task_tail_offset);
        p.task_cnt = At<uint32_t>(l.ws, l.layout.task_cnt_offset);
        p.max_tasks = l.layout.max_tasks;
    }
    p.col = l.col;
    p.col_stride = l.col_stride;
    p.val = l.val;
    p.val_stride = l.val_stride;
    p.x = l.x;
    p.x_stride = l.x_stride;
    p.y = l.y;
    p.y_stride = l.y_stride;
    p.rows = l.rows;
    p.cols = l.cols;
    p.nnz = l.nnz;
    p.num_blocks = l.layout.num_blocks;
    p.base = l.base;
    p.conj = l.op == ACL_SPARSE_OP_CONJUGATE_TRANSPOSE ? 1 : 0;
    p.s.device = l.device_scalars;
    p.s.alpha_re = l.alpha_re;
    p.s.alpha_im = l.alpha_im;
    p.s.beta_re = l.beta_re;
    p.s.beta_im = l.beta_im;
    p.s.alpha_i = l.alpha_i;
    p.s.beta_i = l.beta_i;
    p.s.alpha_ptr = l.alpha_ptr;
    p.s.beta_ptr = l.beta_ptr;
    return p;
}

unsigned RowBlockGrid(int64_t numBlocks)
{
    const int64_t per = (numBlocks + kXcds - 1) / kXcds;
    return static_cast<unsigned>(per * kXcds);
}

bool Aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15U) == 0U; }

// Waves serving long-block tasks (ACLSPARSE_HIP_TASK_WAVES overrides, for tuning).
int64_t TaskWaves()
{
    static const int64_t waves = [] {
        const char* e = std::getenv("ACLSPARSE_HIP_TASK_WAVES");
        const long long v = e != nullptr ? std::atoll(e) : 0;
        return v > 0 ? static_cast<int64_t>(v) : int64_t{2048};
    }();
    return waves;
}

template <typename RowT, ValKind V, OutKind O, AccKind A>
int LaunchRowBlock(const SpmvLaunch& l, hipStream_t stream)
{
    hipStream_t stream_ = stream;
    if (l.staged && l.staged_choice == 1) return 0;  // Preprocess chose the staged kernels
    RowBlockParams p = MakeRowBlockParams(l);
    const bool chosen = l.staged || l.narrow;  // Preprocess left a path choice in the header
    const unsigned grid = RowBlockGrid(p.num_blocks);
    constexpr bool kCanVec = V == ValKind::F32 || V == ValKind::F16 || V == ValKind::BF16;
    // int8 values and x, int32 y, exact int64 semantics (see StreamSum)
    constexpr bool kInt8 = V == ValKind::I8 && A == AccKind::I64 && O == OutKind::I32;
    // The stream kernels read col_ind / values as 16-byte groups of arrays
    // that start 16-byte aligned, with unit strides.
    const bool vec = (kCanVec || kInt8) && l.nnz >= 4 && l.col_stride == 1 && l.val_stride == 1 &&
                     l.x_stride == 1 && l.y_stride == 1 && Aligned16(l.col) && Aligned16(l.val);
    if constexpr ((kCanVec && A == AccKind::F32) || kInt8) {
        // Stream kernel: 32-bit buffer offsets into x, contiguous y.
        const bool stream = vec && static_cast<int64_t>(l.cols) * static_cast<int64_t>(sizeof(typename ValOf<V>::T)) <=
                                       0x7FFFFFFFLL;
        if (stream) {
            const bool betaNz = l.device_scalars || (kInt8 ? l.beta_i != 0 : l.beta_re != 0.0f);
            const int64_t wgs = (p.num_blocks + kFlatWaves - 1) / kFlatWaves;
            int64_t taskWgs = 0;
            if (l.layout.tasks && !kInt8) {
                // task waves: a multiple of 8 workgroups (even over the XCDs)
                const int64_t waves = l.layout.max_tasks < TaskWaves() ? l.layout.max_tasks : TaskWaves();
                taskWgs = (waves + kFlatWaves * kXcds - 1) / (kFlatWaves * kXcds) * kXcds;
            }
            p.task_wgs = static_cast<int32_t>(taskWgs);
            p.task_waves = static_cast<int32_t>(taskWgs * kFlatWaves);
            int64_t blockWgs = (wgs + kXcds - 1) / kXcds * kXcds;
            const dim3 wg(kWave * kFlatWaves);
            const bool narrow = l.narrow && p.ncol != nullptr;
            // the entry-aligned blocks (no tasks: every block is one window)
            RowBlockParams pe = p;
            pe.blocks = At<const int32_t>(l.ws, l.layout.eb_offset);
            pe.block_nnz = At<const void>(l.ws, l.layout.en_offset);
            pe.num_blocks = l.layout.entry_blocks;
            pe.task_wgs = 0;
            pe.task_waves = 0;
            const int64_t eWgs = ((pe.num_blocks + kFlatWaves - 1) / kFlatWaves + kXcds - 1) / kXcds * kXcds;
            if (narrow && l.staged_choice == kEntryFlag) {
                if (betaNz) {
                    hipLaunchKernelGGL((SpmvStreamFlatKernel<RowT, V, O, true, false, true, true>),
                                       dim3(static_cast<unsigned>(eWgs)), wg, 0, stream_, pe);
                } else {
                    hipLaunchKernelGGL((SpmvStreamFlatKernel<RowT, V, O, false, false, true, true>),
                                       dim3(static_cast<unsigned>(eWgs)), wg, 0, stream_, pe);
                }
                return 0;
            }
            if (narrow && l.staged_choice == kNarrowFlag) {
                const unsigned g = static_cast<unsigned>(taskWgs + blockWgs);
                if (betaNz) {
                    hipLaunchKernelGGL((SpmvStreamFlatKernel<RowT, V, O, true, false, true>), dim3(g), wg, 0, stream_,
                                       p);
                } else {
                    hipLaunchKernelGGL((SpmvStreamFlatKernel<RowT, V, O, false, false, true>), dim3(g), wg, 0,
                                       stream_, p);
                }
                return 0;
            }
            if (chosen && l.staged_choice < 0) {
                // Another path may take this matrix (decided on the device,
                // not yet known here): capped grids keep the launches that
                // exit cheap.  The plain row kernel runs on flag 0, and on
                // the flags of paths whose kernels are not launched here.
                p.skip_flag = &At<SpmvWsHeader>(l.ws, 0)->staged_flag;
                p.run_mask = 1U | (l.staged ? 0U : 2U) | (narrow ? 0U : (1U << kNarrowFlag) | (1U << kEntryFlag));
                if (blockWgs > kStagedFallbackWgs) {
                    blockWgs = kStagedFallbackWgs;
                    p.block_stride = blockWgs * kFlatWaves;
                }
            }
            const unsigned g = static_cast<unsigned>(taskWgs + blockWgs);
            if (p.skip_flag != nullptr) {
                if (betaNz) hipLaunchKernelGGL((SpmvStreamFlatKernel<RowT, V, O, true, true>), dim3(g), wg, 0, stream_, p);
                else hipLaunchKernelGGL((SpmvStreamFlatKernel<RowT, V, O, false, true>), dim3(g), wg, 0, stream_, p);
                if (narrow) {
                    RowBlockParams e = pe;
                    e.skip_flag = p.skip_flag;
                    e.run_mask = 1U << kEntryFlag;
                    int64_t ew = eWgs;
                    if (ew > kStagedFallbackWgs) {
                        ew = kStagedFallbackWgs;
                        e.block_stride = ew * kFlatWaves;
                    }
                    if (betaNz) {
                        hipLaunchKernelGGL((SpmvStreamFlatKernel<RowT, V, O, true, true, true, true>),
                                           dim3(static_cast<unsigned>(ew)), wg, 0, stream_, e);
                    } else {
                        hipLaunchKernelGGL((SpmvStreamFlatKernel<RowT, V, O, false, true, true, true>),
                                           dim3(static_cast<unsigned>(ew)), wg, 0, stream_, e);
                    }
                    RowBlockParams q = p;
                    q.run_mask = 1U << kNarrowFlag;
                    if (betaNz) {
                        hipLaunchKernelGGL((SpmvStreamFlatKernel<RowT, V, O, true, true, true>), dim3(g), wg, 0,
                                           stream_, q);
                    } else {
                        hipLaunchKernelGGL((SpmvStreamFlatKernel<RowT, V, O, false, true, true>), dim3(g), wg, 0,
                                           stream_, q);
                    }
                }
            } else if (betaNz) {
                hipLaunchKernelGGL((SpmvStreamFlatKernel<RowT, V, O, true>), dim3(g), wg, 0, stream_, p);
            } else {
                hipLaunchKernelGGL((SpmvStreamFlatKernel<RowT, V, O, false>), dim3(g), wg, 0, stream_, p);
            }
            return 0;
        }
    }
    if constexpr ((V == ValKind::I8 && A == AccKind::I64) || (V == ValKind::I8 && A == AccKind::F32) ||
                  (V == ValKind::C64 && A == AccKind::C64) || (V == ValKind::F32 && A == AccKind::C64)) {
        // int8 -> int32 / fp32, complex64, and real fp32 A with complex y on
        // the stream kernel's row blocks
        const bool gen = l.nnz > 0 && l.col_stride == 1 && l.val_stride == 1 && l.x_stride == 1 && l.y_stride == 1 &&
                         Aligned16(l.col) && Aligned16(l.val) &&
                         static_cast<int64_t>(l.cols) * static_cast<int64_t>(sizeof(typename ValOf<V>::T)) <=
                             0x7FFFFFFFLL;
        if (gen) {
            const int64_t wgs = (p.num_blocks + kFlatWaves - 1) / kFlatWaves;
            const unsigned g = static_cast<unsigned>((wgs + kXcds - 1) / kXcds * kXcds);
            {
                // the narrow column copy, once Preprocess's choice of it is on the host
                if (l.narrow && p.ncol != nullptr && l.staged_choice == kNarrowFlag) {
                    hipLaunchKernelGGL((SpmvStreamGenKernel<RowT, V, O, A, false, false, true>), dim3(g),
                                       dim3(kWave * kFlatWaves), 0, stream_, p);
                    return 0;
                }
            }
            hipLaunchKernelGGL((SpmvStreamGenKernel<RowT, V, O, A>), dim3(g), dim3(kWave * kFlatWaves), 0, stream_,
                               p);
            return 0;
        }
    }
    if (l.staged) return 1;  // the staged path needs the stream kernel's operands (unit strides, aligned)
    hipLaunchKernelGGL((SpmvRowBlockKernel<RowT, V, O, A>), dim3(grid), dim3(kThreads), 0, stream, p);
    return 0;
}

// One-pass column kernel of banded fp32 transposes: the stream kernel on the
// CSC pattern with each entry's row as its "column" (x gathered by row) and
// its CSR position as its value (the value gathered by position).
uint16_t* BandedCols16(const SpmvLaunch& l);

template <bool kGated, bool kNarrowB = false>
void LaunchBandedTranspose(const SpmvLaunch& l, const RowBlockParams& p, hipStream_t stream)
{
    RowBlockParams c = p;
    c.rp16 = kNarrowB ? BandedCols16(l) : nullptr;
    c.ncol = kNarrowB ? At<const int16_t>(l.ws, l.layout.key_a_offset) : nullptr;
    c.npos = kNarrowB ? At<const int16_t>(l.ws, l.layout.val_b_offset) : nullptr;
    c.rp = At<void>(l.ws, l.layout.colptr_offset);
    c.blocks = At<int32_t>(l.ws, l.layout.csc_blocks_offset);
    c.block_nnz = At<void>(l.ws, l.layout.csc_block_nnz_offset);
    c.num_blocks = l.layout.csc_num_blocks;
    c.col = At<const int32_t>(l.ws, l.layout.key_b_offset);  // csc_row, built by the bucketed Preprocess
    c.col_stride = 1;
    c.val = At<const void>(l.ws, l.layout.csc_pos_offset);
    c.val_stride = 1;
    c.x = l.x;
    c.x_stride = 1;
    c.rows = l.cols;
    c.cols = l.rows;  // length of x
    c.base = 0;
    c.task_wgs = 0;
    c.task_waves = 0;
    c.gval = static_cast<const float*>(l.val);
    c.gval_n = l.nnz;
    c.skip_flag = kGated ? &At<SpmvWsHeader>(l.ws, 0)->staged_flag : nullptr;
    c.run_mask = 1U << (kNarrowB ? kBandedNarrowFlag : 2);
    const int64_t wgs = (c.num_blocks + kFlatWaves - 1) / kFlatWaves;
    const unsigned g = static_cast<unsigned>((wgs + kXcds - 1) / kXcds * kXcds);
    const dim3 wg(kWave * kFlatWaves);
    const bool betaNz = l.device_scalars || l.beta_re != 0.0f;
    if (betaNz) {
        hipLaunchKernelGGL((SpmvStreamFlatKernel<int32_t, ValKind::GATH, OutKind::F32, true, kGated, kNarrowB>), dim3(g),
                           wg, 0, stream, c);
    } else {
        hipLaunchKernelGGL((SpmvStreamFlatKernel<int32_t, ValKind::GATH, OutKind::F32, false, kGated, kNarrowB>),
                           dim3(g), wg, 0, stream, c);
    }
}

// ------------------- transpose by atomic scatter (CSR_ALG1) ------------------
//
// The reference's non-deterministic transpose (sparse/spmv/arch35/
// spmv_kernel.cpp:579-668): acc is cleared, every entry adds
// conj?(a_k) * x[row(k)] to acc[col(k)] atomically, then y = alpha*acc +
// beta*y with the output's epilogue.  It needs only the normalised row
// offsets and the row-block partition beside the cols-long accumulator, so it
// is the route of the reference-sized workspace (CSR_ALG1); the order in which
// a column's products arrive is not fixed, so fp32 results can differ in the
// last bits from run to run (int64 accumulation is exact in any order).

struct AtomicParams {
    const void* norm;        // RowT[rows+2], normalised row offsets
    const int32_t* blocks;   // int32[B+1], first row of each row block
    const void* block_nnz;   // RowT[B+1]
    int64_t num_blocks;
    const int32_t* col;
    int64_t col_stride;
    const void* val;
    int64_t val_stride;
    const void* x;
    int64_t x_stride;
    void* acc;
    int64_t cols;
    int32_t base;
    int32_t conj;
};

template <AccKind A>
__device__ __forceinline__ void AtomicAcc(typename AccOf<A>::T* acc, int64_t c, typename AccOf<A>::T v)
{
    if constexpr (A == AccKind::F32) {
        unsafeAtomicAdd(acc + c, v);  // the hardware float atomic (coarse-grained device memory)
    } else if constexpr (A == AccKind::C64) {
        float* f = reinterpret_cast<float*>(acc + c);
        unsafeAtomicAdd(f, v.re);
        unsafeAtomicAdd(f + 1, v.im);
    } else {
        atomicAdd(reinterpret_cast<unsigned long long*>(acc + c), static_cast<unsigned long long>(v));
    }
}

// One row block (at most kWaveRows rows) per wave, 4 waves per workgroup; the
// block's row offsets go to the wave's LDS slice and each lane finds the row
// of its entry by binary search there.
template <typename RowT, ValKind V, AccKind A>
__global__ __launch_bounds__(kThreads) void AtomicTransposeKernel(AtomicParams p)
{
    using Acc = typename AccOf<A>::T;
    using ValT = typename ValOf<V>::T;
    constexpr int kW = kThreads / kWave;
    __shared__ int64_t sOff[kW][kWaveRows + 2];
    const int wv = threadIdx.x / kWave;
    const int lane = threadIdx.x & (kWave - 1);
    const int64_t b = static_cast<int64_t>(blockIdx.x) * kW + wv;
    if (b >= p.num_blocks) return;
    const RowT* norm = static_cast<const RowT*>(p.norm);
    const int64_t r0 = p.blocks[b];
    const int nr = static_cast<int>(p.blocks[b + 1] - r0);
    const int64_t e0 = static_cast<int64_t>(static_cast<const RowT*>(p.block_nnz)[b]);
    const int64_t e1 = static_cast<int64_t>(static_cast<const RowT*>(p.block_nnz)[b + 1]);
    for (int i = lane; i <= nr; i += kWave) sOff[wv][i] = static_cast<int64_t>(norm[r0 + i]);
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    const ValT* val = static_cast<const ValT*>(p.val);
    const ValT* x = static_cast<const ValT*>(p.x);
    Acc* acc = static_cast<Acc*>(p.acc);
    for (int64_t k = e0 + lane; k < e1; k += kWave) {
        // the row of entry k: the last i with sOff[i] <= k (rows may be empty)
        int lo = 0, hi = nr;  // sOff[0] <= k < sOff[nr]
        while (hi - lo > 1) {
            const int mid = (lo + hi) >> 1;
            if (sOff[wv][mid] <= k) lo = mid;
            else hi = mid;
        }
        const int64_t c = static_cast<int64_t>(p.col[k * p.col_stride]) - p.base;
        if (c < 0 || c >= p.cols) continue;
        const Acc a = MaybeConj<V, A>(ToAcc<V, A>(val[k * p.val_stride]), p.conj);
        AtomicAcc<A>(acc, c, a * ToAcc<V, A>(x[(r0 + lo) * p.x_stride]));
    }
}

// y = alpha*acc + beta*y (y not read when beta == 0), the row kernels' epilogue.
template <OutKind O, AccKind A>
__global__ __launch_bounds__(kThreads) void AtomicFinalizeKernel(const typename AccOf<A>::T* acc,
                                                                  typename OutOf<O>::T* y, int64_t n, int64_t stride,
                                                                  Scalars s)
{
    using Acc = typename AccOf<A>::T;
    Acc alpha, beta;
    LoadScalars<A>(s, alpha, beta);
    const bool betaNz = !IsZero(beta);
    for (int64_t j = blockIdx.x * static_cast<int64_t>(kThreads) + threadIdx.x; j < n;
         j += static_cast<int64_t>(gridDim.x) * kThreads) {
        StoreRow<O, A>(y, j * stride, acc[j], alpha, beta, betaNz);
    }
}

template <typename RowT, ValKind V, OutKind O, AccKind A>
void LaunchAtomicTranspose(const SpmvLaunch& l, const RowBlockParams& rb, hipStream_t stream)
{
    using Acc = typename AccOf<A>::T;
    Acc* acc = At<Acc>(l.ws, l.layout.acc_offset);
    const int64_t n = l.cols;
    hipLaunchKernelGGL((ClearKernel<A>), dim3(GridFor(n)), dim3(kThreads), 0, stream, acc, n);
    AtomicParams p{};
    p.norm = rb.rp;
    p.blocks = rb.blocks;
    p.block_nnz = rb.block_nnz;
    p.num_blocks = l.layout.num_blocks;
    p.col = l.col;
    p.col_stride = l.col_stride;
    p.val = l.val;
    p.val_stride = l.val_stride;
    p.x = l.x;
    p.x_stride = l.x_stride;
    p.acc = acc;
    p.cols = n;
    p.base = l.base;
    p.conj = l.op == ACL_SPARSE_OP_CONJUGATE_TRANSPOSE ? 1 : 0;
    constexpr int kW = kThreads / kWave;
    const unsigned g = static_cast<unsigned>((p.num_blocks + kW - 1) / kW);
    hipLaunchKernelGGL((AtomicTransposeKernel<RowT, V, A>), dim3(g), dim3(kThreads), 0, stream, p);
    hipLaunchKernelGGL((AtomicFinalizeKernel<O, A>), dim3(GridFor(n)), dim3(kThreads), 0, stream, acc,
                       static_cast<typename OutOf<O>::T*>(l.y), n, l.y_stride, rb.s);
}

template <typename RowT, ValKind V, OutKind O, AccKind A>
int LaunchTranspose(const SpmvLaunch& l, hipStream_t stream)
{
    using Acc = typename AccOf<A>::T;
    RowBlockParams p = MakeRowBlockParams(l);
    const int64_t n = l.cols;
    if (l.layout.csc) {
        if (n <= 0) return 0;
        if (l.staged && l.staged_choice == 1) return 0;  // Preprocess chose the column-bucketed kernels
        if constexpr (std::is_same<RowT, int32_t>::value && V == ValKind::F32 && A == AccKind::F32 &&
                      O == OutKind::F32) {
            // Banded fp32 transposes (Preprocess's choice 2): one pass over
            // the CSC pattern gathering each entry's value and x, both local
            const bool banded = l.staged && l.y_stride == 1 && l.x_stride == 1 && l.val_stride == 1 &&
                                l.nnz <= 0x1FFFFFFFLL;
            if (banded && l.staged_choice == kBandedNarrowFlag) {
                LaunchBandedTranspose<false, true>(l, p, stream);
                return 0;
            }
            if (banded && l.staged_choice == 2) {
                LaunchBandedTranspose<false>(l, p, stream);
                return 0;
            }
            if (banded && l.staged_choice < 0) {  // each runs on its own choice only
                LaunchBandedTranspose<true>(l, p, stream);
                LaunchBandedTranspose<true, true>(l, p, stream);
            }
        }
        if constexpr (std::is_same<RowT, int32_t>::value &&
                      ((V == ValKind::C64 && A == AccKind::C64) || (V == ValKind::F32 && A == AccKind::C64) ||
                       (V == ValKind::I8 && A == AccKind::I64))) {
            // Banded complex64, real-to-complex and int8 transposes
            // (Preprocess's choice kCbandFlag or kCbandNarrowFlag, known on
            // the host): one pass over the CSC pattern gathering each entry's
            // value (by its CSR position) and x (by its row)
            const bool packed = l.staged_choice == kCbandNarrowFlag;
            // (real values under opA = H keep the product pass, which conjugates
            // them to a -0 imaginary part)
            const bool opOk = V != ValKind::F32 || l.op == ACL_SPARSE_OP_TRANSPOSE;
            if (opOk && l.cband && l.layout.cband && (l.staged_choice == kCbandFlag || packed) && l.y_stride == 1 &&
                l.x_stride == 1 && l.val_stride == 1) {
                RowBlockParams c = p;
                c.rp = At<void>(l.ws, l.layout.colptr_offset);
                c.blocks = At<int32_t>(l.ws, l.layout.csc_blocks_offset);
                c.block_nnz = At<void>(l.ws, l.layout.csc_block_nnz_offset);
                c.num_blocks = l.layout.csc_num_blocks;
                c.col = At<const int32_t>(l.ws, l.layout.val_b_offset);  // each CSC entry's row (packed: with its position)
                c.col_stride = 1;
                c.val = At<const int32_t>(l.ws, l.layout.csc_pos_offset);
                c.val_stride = 1;
                c.gval = static_cast<const float*>(l.val);
                c.gval_n = l.nnz;
                c.conj = l.op == ACL_SPARSE_OP_CONJUGATE_TRANSPOSE ? 1 : 0;
                c.x = l.x;
                c.x_stride = 1;
                c.rows = n;
                c.cols = l.rows;  // length of x
                c.base = 0;
                c.task_wgs = 0;
                c.task_waves = 0;
                const int64_t wgs = (c.num_blocks + kFlatWaves - 1) / kFlatWaves;
                const unsigned g = static_cast<unsigned>((wgs + kXcds - 1) / kXcds * kXcds);
                if (packed) {
                    hipLaunchKernelGGL((SpmvStreamGenKernel<int32_t, V, O, A, true, true>), dim3(g),
                                       dim3(kWave * kFlatWaves), 0, stream, c);
                } else {
                    hipLaunchKernelGGL((SpmvStreamGenKernel<int32_t, V, O, A, true>), dim3(g),
                                       dim3(kWave * kFlatWaves), 0, stream, c);
                }
                return 0;
            }
        }
        CscParams q{};
        q.colptr = At<void>(l.ws, l.layout.colptr_offset);
        q.entry_row = At<int32_t>(l.ws, l.layout.entry_row_offset);
        q.pos = At<void>(l.ws, l.layout.csc_pos_offset);
        q.prod = At<void>(l.ws, l.layout.prod_offset);
        q.norm = At<const void>(l.ws, l.layout.rowptr_offset);
        q.rows = l.rows;
        q.val = l.val;
        q.val_stride = l.val_stride;
        q.x = l.x;
        q.x_stride = l.x_stride;
        q.y = l.y;
        q.y_stride = l.y_stride;
        q.cols = n;
        q.conj = l.op == ACL_SPARSE_OP_CONJUGATE_TRANSPOSE ? 1 : 0;
        q.s = p.s;
        // the column-bucketed kernels (launched after these) run instead when Preprocess chose them
        q.skip_flag = l.staged && l.staged_choice < 0 ? &At<SpmvWsHeader>(l.ws, 0)->staged_flag : nullptr;
        // lanes per column: the power of two nearest below the mean column length, <= 64
        const int64_t mean = l.nnz / n;
        int lg = 0;
        while (lg < 6 && (int64_t{2} << lg) <= mean) ++lg;
        q.lg = lg;
        const int64_t threads = n << lg;
        const unsigned grid = static_cast<unsigned>((threads + kThreads - 1) / kThreads);
        q.group_row = At<const int32_t>(l.ws, l.layout.group_row_offset);
        q.row_delta = At<const uint32_t>(l.ws, l.layout.row_delta_offset);
        q.row_groups = l.layout.row_groups;
        int64_t pgb = (l.layout.row_groups + kThreads / kWave - 1) / (kThreads / kWave);
        pgb = pgb > kProdMaxBlocks ? kProdMaxBlocks : pgb;
        const dim3 pg(static_cast<unsigned>(pgb));
        using ValT = typename ValOf<V>::T;
        if (l.val_stride == 1 && reinterpret_cast<uintptr_t>(l.val) % (4 * sizeof(ValT)) == 0) {
            hipLaunchKernelGGL((CscProductKernel<RowT, V, A, true>), pg, dim3(kThreads), 0, stream, q);
        } else {
            hipLaunchKernelGGL((CscProductKernel<RowT, V, A, false>), pg, dim3(kThreads), 0, stream, q);
        }
        if constexpr (std::is_same<RowT, int32_t>::value && A == AccKind::F32 && O != OutKind::I32) {
            // fp32 products and 32-bit positions: the column pass is an SpMV
            // of the CSC pattern (unit values) with the products as x, on the
            // stream kernel and the columns' row-block partition.
            if (l.y_stride == 1 && l.nnz <= 0x1FFFFFFFLL) {
                RowBlockParams c = p;
                c.rp = At<void>(l.ws, l.layout.colptr_offset);
                c.blocks = At<int32_t>(l.ws, l.layout.csc_blocks_offset);
                c.block_nnz = At<void>(l.ws, l.layout.csc_block_nnz_offset);
                c.num_blocks = l.layout.csc_num_blocks;
                c.col = At<const int32_t>(l.ws, l.layout.csc_pos_offset);
                c.col_stride = 1;
                c.val = nullptr;
                c.val_stride = 1;
                c.x = q.prod;
                c.x_stride = 1;
                c.rows = n;
                c.cols = l.nnz;  // length of the gathered array
                c.base = 0;
                c.task_wgs = 0;
                c.task_waves = 0;
                c.skip_flag = q.skip_flag;
                const int64_t wgs = (c.num_blocks + kFlatWaves - 1) / kFlatWaves;
                const unsigned g = static_cast<unsigned>((wgs + kXcds - 1) / kXcds * kXcds);
                const bool betaNz = l.device_scalars || l.beta_re != 0.0f;
                const dim3 wg(kWave * kFlatWaves);
                if (c.skip_flag != nullptr) {
                    if (betaNz) {
                        hipLaunchKernelGGL((SpmvStreamFlatKernel<int32_t, ValKind::UNIT, O, true, true>), dim3(g), wg,
                                           0, stream, c);
                    } else {
                        hipLaunchKernelGGL((SpmvStreamFlatKernel<int32_t, ValKind::UNIT, O, false, true>), dim3(g), wg,
                                           0, stream, c);
                    }
                } else if (betaNz) {
                    hipLaunchKernelGGL((SpmvStreamFlatKernel<int32_t, ValKind::UNIT, O, true>), dim3(g), wg, 0, stream,
                                       c);
                } else {
                    hipLaunchKernelGGL((SpmvStreamFlatKernel<int32_t, ValKind::UNIT, O, false>), dim3(g), wg, 0,
                                       stream, c);
                }
                return 0;
            }
        }
        if constexpr (std::is_same<RowT, int32_t>::value && (A == AccKind::C64 || A == AccKind::I64)) {
            // complex / int64 products: the same column pass on the stream
            // loads of the int8/complex kernel (8-byte products as x)
            if (l.y_stride == 1 && l.nnz <= 0x0FFFFFFFLL) {
                RowBlockParams c = p;
                c.rp = At<void>(l.ws, l.layout.colptr_offset);
                c.blocks = At<int32_t>(l.ws, l.layout.csc_blocks_offset);
                c.block_nnz = At<void>(l.ws, l.layout.csc_block_nnz_offset);
                c.num_blocks = l.layout.csc_num_blocks;
                c.col = At<const int32_t>(l.ws, l.layout.csc_pos_offset);
                c.col_stride = 1;
                c.val = nullptr;
                c.val_stride = 1;
                c.x = q.prod;
                c.x_stride = 1;
                c.rows = n;
                c.cols = l.nnz;
                c.base = 0;
                const int64_t wgs = (c.num_blocks + kFlatWaves - 1) / kFlatWaves;
                const unsigned g = static_cast<unsigned>((wgs + kXcds - 1) / kXcds * kXcds);
                hipLaunchKernelGGL((SpmvStreamGenKernel<int32_t, ValKind::UNIT, O, A>), dim3(g),
                                   dim3(kWave * kFlatWaves), 0, stream, c);
                return 0;
            }
        }
        hipLaunchKernelGGL((SpmvCscGatherKernel<RowT, V, O, A>), dim3(grid), dim3(kThreads), 0, stream, q);
        return 0;
    }
    if (l.layout.lean && l.nnz > 0 && n > 0) {  // CSR_ALG1: the reference-sized workspace
        LaunchAtomicTranspose<RowT, V, O, A>(l, p, stream);
        return 0;
    }
    // No non-zeros (the CSC path covers 0 < nnz <= INT32_MAX; larger
    // transposes are rejected by the host): y = beta*y.
    constexpr bool kDirect = (O == OutKind::F32 && A == AccKind::F32) || (O == OutKind::C64 && A == AccKind::C64);
    if constexpr (kDirect) {
        hipLaunchKernelGGL((ScaleKernel<O, A>), dim3(GridFor(n)), dim3(kThreads), 0, stream,
                           static_cast<typename OutOf<O>::T*>(l.y), n, l.y_stride, p.s);
    } else {
        Acc* acc = At<Acc>(l.ws, l.layout.acc_offset);
        hipLaunchKernelGGL((ClearKernel<A>), dim3(GridFor(n)), dim3(kThreads), 0, stream, acc, n);
        hipLaunchKernelGGL((FinalizeKernel<O, A>), dim3(GridFor(n)), dim3(kThreads), 0, stream, acc,
                           static_cast<typename OutOf<O>::T*>(l.y), n, l.y_stride, p.s);
    }
    return 0;
}

// fp32 matrices of at most kSmallFloatRows rows (fp32 values, x, y and
// compute, opA = N): one thread per row sums its entries in CSR order with
// Kahan compensation and keeps the rounding error of every product (FMA
// residual), then applies both corrections in the epilogue; when a product or
// the plain running sum is not finite the plain sum is used instead.  This is
// the reference's small-matrix path (sparse/spmv/arch35/spmv_kernel.cpp:448-499,
// taken for rows <= 64 at :569-572), so {2^24, 1, -2^24} . {1, 1, 1} gives
// exactly 1 as it does there.  Reads the caller's arrays (strides, index
// base); entries outside [0, nnz) or columns outside [0, cols) are skipped.
constexpr int64_t kSmallFloatRows = 64;

template <typename RowT>
__global__ __launch_bounds__(kWave) void SpmvSmallFloatKernel(const RowT* rp, int64_t rpStride, const int32_t* col,
                                                             int64_t colStride, const float* val, int64_t valStride,
                                                             const float* x, int64_t xStride, float* y,
                                                             int64_t yStride, int64_t rows, int64_t cols,
                                                             int64_t nnz, int32_t base, Scalars sc)
{
#pragma clang fp contract(off)
    const int64_t row = threadIdx.x;
    if (row >= rows) return;
    float alpha, beta;
    LoadScalars<AccKind::F32>(sc, alpha, beta);
    const int64_t begin = static_cast<int64_t>(rp[row * rpStride]) - base;
    const int64_t end = static_cast<int64_t>(rp[(row + 1) * rpStride]) - base;
    float sum = 0.0f, plain = 0.0f, comp = 0.0f, resid = 0.0f;
    bool special = false;
    if (begin >= 0 && end >= begin) {
        for (int64_t p = begin; p < end && p < nnz; ++p) {
            const int64_t c = static_cast<int64_t>(col[p * colStride]) - base;
            if (c < 0 || c >= cols) continue;
            const float a = val[p * valStride];
            const float b = x[c * xStride];
            const float prod = a * b;
            plain = plain + prod;
            special = special || !__builtin_isfinite(prod) || !__builtin_isfinite(plain);
            resid = resid + __builtin_fmaf(a, b, -prod);
            const float adj = prod - comp;
            const float next = sum + adj;
            comp = (next - sum) - adj;
            sum = next;
        }
    }
    const bool betaNz = beta != 0.0f;  // y is not read when beta == 0
    float out;
    if (special) {
        out = betaNz ? alpha * plain + beta * y[row * yStride] : alpha * plain;
    } else {
        const float corr = alpha * (resid - comp);
        out = betaNz ? __builtin_fmaf(alpha, sum, beta * y[row * yStride]) + corr : __builtin_fmaf(alpha, sum, corr);
    }
    y[row * yStride] = out;
}

template <typename RowT, ValKind V, OutKind O, AccKind A>
int LaunchTyped(const SpmvLaunch& l, hipStream_t stream)
{
    if (l.op == ACL_SPARSE_OP_NON_TRANSPOSE) return LaunchRowBlock<RowT, V, O, A>(l, stream);
    return LaunchTranspose<RowT, V, O, A>(l, stream);
}

template <typename RowT>
int DispatchTypes(const SpmvLaunch& l, hipStream_t s)
{
    using VK = ValKind;
    using OK = OutKind;
    using AK = AccKind;
    if (l.acc_kind == AK::I64) return LaunchTyped<RowT, VK::I8, OK::I32, AK::I64>(l, s);
    if (l.acc_kind == AK::C64) {
        if (l.val_kind == VK::F32) return LaunchTyped<RowT, VK::F32, OK::C64, AK::C64>(l, s);
        return LaunchTyped<RowT, VK::C64, OK::C64, AK::C64>(l, s);
    }
    switch (l.val_kind) {
        case VK::I8: return LaunchTyped<RowT, VK::I8, OK::F32, AK::F32>(l, s);
        case VK::F16:
            return l.out_kind == OK::F16 ? LaunchTyped<RowT, VK::F16, OK::F16, AK::F32>(l, s)
                                         : LaunchTyped<RowT, VK::F16, OK::F32, AK::F32>(l, s);
        case VK::BF16:
            return l.out_kind == OK::BF16 ? LaunchTyped<RowT, VK::BF16, OK::BF16, AK::F32>(l, s)
                                          : LaunchTyped<RowT, VK::BF16, OK::F32, AK::F32>(l, s);
        case VK::F32: return LaunchTyped<RowT, VK::F32, OK::F32, AK::F32>(l, s);
        default: return 1;
    }
}

// Task table of the long blocks: counts[b] = chunks of block b when it has
// more than kLongChunks, else 0 (counts[B] = 0); arrival counters cleared.
template <typename RowT>
__global__ __launch_bounds__(kThreads) void TaskCountKernel(const RowT* blockNnz, int64_t numBlocks, int32_t* counts,
                                                            uint32_t* cnt)
{
    for (int64_t b = blockIdx.x * static_cast<int64_t>(kThreads) + threadIdx.x; b <= numBlocks;
         b += static_cast<int64_t>(gridDim.x) * kThreads) {
        int32_t n = 0;
        if (b < numBlocks) {
            const int64_t k0 = static_cast<int64_t>(blockNnz[b]);
            const int64_t kspan = static_cast<int64_t>(blockNnz[b + 1]) - k0;
            const int64_t chunks = (kspan + (k0 & 3) + kChunkNnz - 1) / kChunkNnz;
            n = chunks > kLongChunks ? static_cast<int32_t>(chunks) : 0;
        }
        counts[b] = n;
        cnt[b] = 0U;
    }
}

__global__ __launch_bounds__(kThreads) void TaskFillKernel(const int32_t* taskStart, int64_t numBlocks,
                                                           int32_t* taskBlock)
{
    for (int64_t b = blockIdx.x * static_cast<int64_t>(kThreads) + threadIdx.x; b < numBlocks;
         b += static_cast<int64_t>(gridDim.x) * kThreads) {
        const int32_t t0 = taskStart[b], t1 = taskStart[b + 1];
        for (int32_t t = t0; t < t1; ++t) taskBlock[t] = static_cast<int32_t>(b);
    }
}

template <typename RowT>
int BuildTasks(const SpmvLaunch& l, hipStream_t s)
{
    const int64_t nb = l.layout.num_blocks;
    int32_t* counts = At<int32_t>(l.ws, l.layout.task_head_offset);  // temporary: max_tasks >= nb + 1
    int32_t* start = At<int32_t>(l.ws, l.layout.task_start_offset);
    hipLaunchKernelGGL((TaskCountKernel<RowT>), dim3(GridFor(nb + 1)), dim3(kThreads), 0, s,
                       At<const RowT>(l.ws, l.layout.block_nnz_offset), nb, counts,
                       At<uint32_t>(l.ws, l.layout.task_cnt_offset));
    void* temp = reinterpret_cast<void*>(
        (reinterpret_cast<uintptr_t>(At<uint8_t>(l.ws, l.layout.task_scan_offset)) + 255) & ~uintptr_t{255});
    size_t tempBytes = l.layout.task_scan_bytes;
    if (hipcub::DeviceScan::ExclusiveSum(temp, tempBytes, counts, start, static_cast<int>(nb + 1), s) != hipSuccess) {
        return 1;
    }
    hipLaunchKernelGGL(TaskFillKernel, dim3(GridFor(nb)), dim3(kThreads), 0, s, start, nb,
                       At<int32_t>(l.ws, l.layout.task_block_offset));
    return 0;
}

// Narrow columns: one wave per row block writes each entry's column as a
// signed 16-bit offset from the block's first row (nc[k] = col[k] - base -
// r0); a wave that finds an entry out of that range sets narrow_bad.  Entries
// outside every block (before the first row's offset or after the last) are
// never summed and are not written.  Nothing is written when the staged
// gather was chosen: its tables share the storage.
struct NarrowParams {
    const int32_t* blocks;
    const void* block_nnz;
    const int32_t* col;
    int16_t* nc;
    int64_t num_blocks;
    int32_t base;
    const uint32_t* flag;  // staged_flag
    uint32_t* bad;         // narrow_bad
    // the entry-aligned blocks, used instead when they fit (entry_bad == 0)
    const int32_t* eblocks;
    const void* eblock_nnz;
    int64_t num_eblocks;
    const uint32_t* entry_bad;
};

// Entry-aligned row blocks: block t starts at the first row whose offset is
// at least kEntryChunk*t (lower bound over the normalised offsets; t = E gives
// rows).  One thread per block boundary.
template <typename RowT>
__global__ __launch_bounds__(kThreads) void EntryBlocksKernel(const RowT* norm, int64_t rows, int64_t numE,
                                                             int32_t* eb, RowT* en)
{
    const int64_t t = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x;
    if (t > numE) return;
    int64_t lo = rows;
    if (t < numE) {
        const int64_t target = t * kEntryChunk;
        int64_t hi = rows;
        lo = 0;
        while (lo < hi) {
            const int64_t mid = (lo + hi) >> 1;
            if (static_cast<int64_t>(norm[mid]) >= target) hi = mid;
            else lo = mid + 1;
        }
    }
    eb[t] = static_cast<int32_t>(lo);
    en[t] = norm[lo];
}

// Every entry-aligned block must have at most kWaveRows rows and end within
// kWaveChunk entries of its window's start; otherwise entry_bad is set.
template <typename RowT>
__global__ __launch_bounds__(kThreads) void EntryCheckKernel(const int32_t* eb, const RowT* en, int64_t numE,
                                                            uint32_t* bad)
{
    const int64_t t = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x;
    bool out = false;
    if (t < numE) {
        out = eb[t + 1] - eb[t] > kWaveRows ||
              static_cast<int64_t>(en[t + 1]) > t * kEntryChunk + kWaveChunk;
    }
    if (__ballot(out) != 0 && (threadIdx.x & (kWave - 1)) == 0) {
        __hip_atomic_fetch_or(bad, 1U, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
}

template <typename RowT>
__global__ __launch_bounds__(kThreads) void NarrowColKernel(NarrowParams q)
{
    const int64_t b = static_cast<int64_t>(blockIdx.x) * kWaves + threadIdx.x / kWave;
    const int lane = threadIdx.x & (kWave - 1);
    if (*q.flag == 1U) return;
    const bool entry = q.eblocks != nullptr && *q.entry_bad == 0U;  // the partition the kernel will use
    if (b >= (entry ? q.num_eblocks : q.num_blocks)) return;
    const int64_t rb = static_cast<int64_t>(entry ? q.eblocks[b] : q.blocks[b]) + q.base;
    const RowT* bn = static_cast<const RowT*>(entry ? q.eblock_nnz : q.block_nnz);
    const int64_t k1 = static_cast<int64_t>(bn[b + 1]);
    bool bad = false;
    for (int64_t k = static_cast<int64_t>(bn[b]) + lane; k < k1; k += kWave) {
        const int64_t d = static_cast<int64_t>(q.col[k]) - rb;
        bad |= d < -32768 || d > 32767;
        q.nc[k] = static_cast<int16_t>(d);
    }
    if (__ballot(bad) != 0 && lane == 0) __hip_atomic_fetch_or(q.bad, 1U, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Low 16 bits of the normalised row offsets (the pad entry reads 0).
template <typename RowT>
__global__ __launch_bounds__(kThreads) void NarrowRowsKernel(const RowT* norm, int64_t rows, uint16_t* rp16)
{
    const int64_t i = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x;
    if (i <= rows) rp16[i] = static_cast<uint16_t>(static_cast<uint64_t>(norm[i]) & 0xFFFFU);
    if (i == rows + 1) rp16[i] = 0;
}

// Flag 3 (the narrow-column row kernel) unless the staged gather was chosen
// or some entry did not fit.
__global__ void NarrowDecideKernel(uint32_t* flag, const uint32_t* bad, const uint32_t* entryBad)
{
    if (*flag != 1U && *bad == 0U) *flag = static_cast<uint32_t>(*entryBad == 0U ? kEntryFlag : kNarrowFlag);
}

// *flag = v (one thread).
__global__ void SetFlagKernel(uint32_t* flag, uint32_t v)
{
    if (threadIdx.x == 0) *flag = v;
}

template <typename RowT>
void BuildNarrow(const SpmvLaunch& l, hipStream_t s)
{
    SpmvWsHeader* h = At<SpmvWsHeader>(l.ws, 0);
    NarrowParams q{};
    q.blocks = At<const int32_t>(l.ws, l.layout.blocks_offset);
    q.block_nnz = At<const void>(l.ws, l.layout.block_nnz_offset);
    q.col = l.col;
    q.nc = At<int16_t>(l.ws, l.layout.nc_offset);
    q.num_blocks = l.layout.num_blocks;
    q.base = l.base;
    q.flag = &h->staged_flag;
    q.bad = &h->narrow_bad;
    // complex64, int8 -> fp32 and real-to-complex values run on the stream
    // kernel of non-fp32 accumulators, which has no entry-aligned variant:
    // the merge-path blocks only
    const bool entry = l.val_kind != ValKind::C64 && l.acc_kind != AccKind::C64 &&
                       !(l.val_kind == ValKind::I8 && l.acc_kind == AccKind::F32);
    const int64_t ne = entry ? l.layout.entry_blocks : 0;
    q.eblocks = entry ? At<const int32_t>(l.ws, l.layout.eb_offset) : nullptr;
    q.eblock_nnz = At<const void>(l.ws, l.layout.en_offset);
    q.num_eblocks = ne;
    q.entry_bad = &h->entry_bad;
    if (entry) {
        const unsigned eg = static_cast<unsigned>((ne + 1 + kThreads - 1) / kThreads);
        hipLaunchKernelGGL((EntryBlocksKernel<RowT>), dim3(eg), dim3(kThreads), 0, s,
                           At<const RowT>(l.ws, l.layout.rowptr_offset), l.rows, ne,
                           At<int32_t>(l.ws, l.layout.eb_offset), At<RowT>(l.ws, l.layout.en_offset));
        hipLaunchKernelGGL((EntryCheckKernel<RowT>), dim3(eg), dim3(kThreads), 0, s, q.eblocks,
                           static_cast<const RowT*>(q.eblock_nnz), ne, &h->entry_bad);
    } else {
        hipLaunchKernelGGL(SetFlagKernel, dim3(1), dim3(1), 0, s, &h->entry_bad, 1U);
    }
    const int64_t waves = q.num_blocks > ne ? q.num_blocks : ne;
    const unsigned grid = static_cast<unsigned>((waves + kWaves - 1) / kWaves);
    hipLaunchKernelGGL((NarrowColKernel<RowT>), dim3(grid), dim3(kThreads), 0, s, q);
    hipLaunchKernelGGL((NarrowRowsKernel<RowT>), dim3(static_cast<unsigned>((l.rows + 2 + kThreads - 1) / kThreads)),
                       dim3(kThreads), 0, s, At<const RowT>(l.ws, l.layout.rowptr_offset), l.rows,
                       At<uint16_t>(l.ws, l.layout.nr_offset));
    hipLaunchKernelGGL(NarrowDecideKernel, dim3(1), dim3(1), 0, s, &h->staged_flag,
                       static_cast<const uint32_t*>(&h->narrow_bad), static_cast<const uint32_t*>(&h->entry_bad));
}

// Banded transpose on 16-bit copies: one wave per CSC row block (columns as
// rows) writes each entry's row as an offset from the block's first column
// (into key_a) and its CSR position as an offset from its own CSC index (into
// val_b); any entry out of range sets narrow_bad.  Runs only when the
// bucketed Preprocess chose the banded kernel (flag 2), whose copies these
// are; both regions are sort storage that only the CSC build uses.
__global__ __launch_bounds__(kThreads) void BandedNarrowKernel(const int32_t* cblocks, const int32_t* cblockNnz,
                                                               const int32_t* cscRow, const int32_t* cscPos,
                                                               int64_t numBlocks, int16_t* nrow, int16_t* npos,
                                                               const uint32_t* flag, uint32_t* bad)
{
    const int64_t b = static_cast<int64_t>(blockIdx.x) * kWaves + threadIdx.x / kWave;
    const int lane = threadIdx.x & (kWave - 1);
    if (b >= numBlocks || *flag != 2U) return;
    const int64_t c0 = cblocks[b];
    const int64_t k1 = cblockNnz[b + 1];
    bool out = false;
    for (int64_t k = static_cast<int64_t>(cblockNnz[b]) + lane; k < k1; k += kWave) {
        const int64_t d1 = static_cast<int64_t>(cscRow[k]) - c0;
        const int64_t d2 = static_cast<int64_t>(cscPos[k]) - k;
        out |= d1 < -32768 || d1 > 32767 || d2 < -32768 || d2 > 32767;
        nrow[k] = static_cast<int16_t>(d1);
        npos[k] = static_cast<int16_t>(d2);
    }
    if (__ballot(out) != 0 && lane == 0) __hip_atomic_fetch_or(bad, 1U, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// The low 16 bits of the column offsets, for the banded kernel's short blocks
// (only when the banded kernel was chosen: the region is key_a's second half).
__global__ __launch_bounds__(kThreads) void BandedNarrowColsKernel(const int32_t* colptr, int64_t cols, uint16_t* cp16,
                                                                   const uint32_t* flag)
{
    const int64_t i = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x;
    if (i > cols + 1 || *flag != 2U) return;
    cp16[i] = i <= cols ? static_cast<uint16_t>(static_cast<uint32_t>(colptr[i]) & 0xFFFFU) : uint16_t{0};
}

// Where the banded kernel's 16-bit column offsets go: after the row offsets
// in key_a (4 bytes per entry, half used), when cols + 2 of them fit.
uint16_t* BandedCols16(const SpmvLaunch& l)
{
    const size_t n = static_cast<size_t>(l.nnz);
    const size_t used = AlignUp(n * sizeof(int16_t));
    if (used + (static_cast<size_t>(l.cols) + 2) * sizeof(uint16_t) > n * sizeof(int32_t)) return nullptr;
    return reinterpret_cast<uint16_t*>(At<uint8_t>(l.ws, l.layout.key_a_offset) + used);
}

__global__ void BandedNarrowDecideKernel(uint32_t* flag, const uint32_t* bad)
{
    if (*flag == 2U && *bad == 0U) *flag = static_cast<uint32_t>(kBandedNarrowFlag);
}

void BuildBandedNarrow(const SpmvLaunch& l, hipStream_t s)
{
    SpmvWsHeader* h = At<SpmvWsHeader>(l.ws, 0);
    const int64_t nb = l.layout.csc_num_blocks;
    hipLaunchKernelGGL(BandedNarrowKernel, dim3(static_cast<unsigned>((nb + kWaves - 1) / kWaves)), dim3(kThreads), 0,
                       s, At<const int32_t>(l.ws, l.layout.csc_blocks_offset),
                       At<const int32_t>(l.ws, l.layout.csc_block_nnz_offset),
                       At<const int32_t>(l.ws, l.layout.key_b_offset), At<const int32_t>(l.ws, l.layout.csc_pos_offset),
                       nb, At<int16_t>(l.ws, l.layout.key_a_offset), At<int16_t>(l.ws, l.layout.val_b_offset),
                       static_cast<const uint32_t*>(&h->staged_flag), &h->narrow_bad);
    if (uint16_t* cp16 = BandedCols16(l)) {
        hipLaunchKernelGGL(BandedNarrowColsKernel, dim3(static_cast<unsigned>((l.cols + 2 + kThreads - 1) / kThreads)),
                           dim3(kThreads), 0, s, At<const int32_t>(l.ws, l.layout.colptr_offset), l.cols, cp16,
                           static_cast<const uint32_t*>(&h->staged_flag));
    }
    hipLaunchKernelGGL(BandedNarrowDecideKernel, dim3(1), dim3(1), 0, s, &h->staged_flag,
                       static_cast<const uint32_t*>(&h->narrow_bad));
}

// Complex banded transpose (kCbandFlag): each CSC entry's row, csc_row[j] =
// entry_row[csc_pos[j]] (into val_b), and the count of entries far from the
// band: a CSC entry more than 2^16 positions from its CSR position (its
// value gather), or a CSR entry whose row is more than 2^16 from its column
// (its x gather).
__global__ __launch_bounds__(kThreads) void CbandRowKernel(const int32_t* pos, const int32_t* entryRow,
                                                          const int32_t* col, int32_t base, int32_t* cscRow,
                                                          int64_t nnz, uint32_t* far)
{
    // grid-stride: the grid is capped (GridFor)
    const int64_t stride = static_cast<int64_t>(gridDim.x) * kThreads;
    const int64_t first = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x;
    for (int64_t i0 = static_cast<int64_t>(blockIdx.x) * kThreads; i0 < nnz; i0 += stride) {  // wave-uniform
        const int64_t i = i0 + (first - static_cast<int64_t>(blockIdx.x) * kThreads);
        uint32_t n = 0;
        if (i < nnz) {
            const int32_t q = pos[i];
            cscRow[i] = entryRow[q];
            const int64_t dv = static_cast<int64_t>(q) - i;
            const int64_t dx = static_cast<int64_t>(entryRow[i]) - (static_cast<int64_t>(col[i]) - base);
            n = (dv >= 65536 || dv <= -65536 ? 1U : 0U) + (dx >= 65536 || dx <= -65536 ? 1U : 0U);
        }
        const uint64_t b = __ballot(n != 0U);
        if (b != 0U) {
            // the wave's count, by its lanes' counts of 0..2
            const uint32_t c =
                static_cast<uint32_t>(__popcll(b)) + static_cast<uint32_t>(__popcll(__ballot(n == 2U)));
            if ((threadIdx.x & (kWave - 1)) == 0) {
                __hip_atomic_fetch_add(far, c, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            }
        }
    }
}

// One wave per CSC block (first column cb, entries [k0, k1)): every entry's
// row minus cb and CSR position minus its CSC index within int16, else bad.
__global__ __launch_bounds__(kThreads) void CbandNarrowCheckKernel(const int32_t* cscRow, const int32_t* pos,
                                                                  const int32_t* blocks, const int32_t* blockNnz,
                                                                  int64_t numBlocks, uint32_t* bad)
{
    const int64_t b = static_cast<int64_t>(blockIdx.x) * kWaves + threadIdx.x / kWave;
    const int lane = threadIdx.x & (kWave - 1);
    if (b >= numBlocks) return;
    const int64_t cb = blocks[b], k0 = blockNnz[b], k1 = blockNnz[b + 1];
    bool out = false;
    for (int64_t j = k0 + lane; j < k1; j += kWave) {
        const int64_t dr = static_cast<int64_t>(cscRow[j]) - cb, dp = static_cast<int64_t>(pos[j]) - j;
        out = out || dr < -32768 || dr > 32767 || dp < -32768 || dp > 32767;
    }
    if (__ballot(out) != 0 && lane == 0) __hip_atomic_fetch_or(bad, 1U, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// With flag kCbandNarrowFlag: the rows and positions packed in place of the
// rows (cscRow[j] becomes (row - cb) | (pos - j) << 16).
__global__ __launch_bounds__(kThreads) void CbandNarrowPackKernel(int32_t* cscRow, const int32_t* pos,
                                                                 const int32_t* blocks, const int32_t* blockNnz,
                                                                 int64_t numBlocks, const uint32_t* flag)
{
    const int64_t b = static_cast<int64_t>(blockIdx.x) * kWaves + threadIdx.x / kWave;
    const int lane = threadIdx.x & (kWave - 1);
    if (*flag != static_cast<uint32_t>(kCbandNarrowFlag) || b >= numBlocks) return;
    const int64_t cb = blocks[b], k0 = blockNnz[b], k1 = blockNnz[b + 1];
    for (int64_t j = k0 + lane; j < k1; j += kWave) {
        const uint32_t dr = static_cast<uint32_t>(cscRow[j] - static_cast<int32_t>(cb));
        const uint32_t dp = static_cast<uint32_t>(pos[j] - static_cast<int32_t>(j));
        cscRow[j] = static_cast<int32_t>((dr & 0xFFFFU) | (dp << 16));
    }
}

// The complex banded decision: when at most 1/16 of the 2*nnz checks of
// CbandRowKernel failed, kCbandNarrowFlag if every entry fits 16 bits
// (CbandNarrowCheckKernel), else kCbandFlag; otherwise 0 (the CSC product and
// column passes).
__global__ void CbandDecideKernel(const uint32_t* far, const uint32_t* narrowBad, int64_t nnz, uint32_t* flag)
{
    if (threadIdx.x == 0) {
        const bool banded = static_cast<int64_t>(*far) * 16 <= 2 * nnz;
        *flag = !banded ? 0U : *narrowBad == 0U ? static_cast<uint32_t>(kCbandNarrowFlag)
                                                : static_cast<uint32_t>(kCbandFlag);
    }
}

template <typename RowT>
int BuildCsc(const SpmvLaunch& l, hipStream_t s)
{
    const int64_t nnz = l.nnz;
    CscBuildParams q{};
    q.col = l.col;
    q.col_stride = l.col_stride;
    q.base = l.base;
    q.rows = l.rows;
    q.cols = l.cols;
    q.nnz = nnz;
    q.norm = At<void>(l.ws, l.layout.rowptr_offset);
    q.key = At<int32_t>(l.ws, l.layout.key_a_offset);
    q.pos = At<void>(l.ws, l.layout.csc_pos_offset);
    hipLaunchKernelGGL((CscInitKernel<RowT>), dim3(GridFor(nnz)), dim3(kThreads), 0, s, q);
    hipcub::DoubleBuffer<int32_t> keys(At<int32_t>(l.ws, l.layout.key_a_offset),
                                       At<int32_t>(l.ws, l.layout.key_b_offset));
    hipcub::DoubleBuffer<RowT> vals(At<RowT>(l.ws, l.layout.csc_pos_offset), At<RowT>(l.ws, l.layout.val_b_offset));
    int endBit = 1;
    while (endBit < 31 && (int64_t{1} << endBit) <= l.cols) ++endBit;
    void* temp = reinterpret_cast<void*>(
        (reinterpret_cast<uintptr_t>(At<uint8_t>(l.ws, l.layout.sort_offset)) + 255) & ~uintptr_t{255});
    size_t tempBytes = l.layout.sort_bytes;
    if (hipcub::DeviceRadixSort::SortPairs(temp, tempBytes, keys, vals, static_cast<int>(nnz), 0, endBit, s) !=
        hipSuccess) {
        return 1;
    }
    hipLaunchKernelGGL((CscColPtrKernel<RowT>), dim3(GridFor(nnz + 1)), dim3(kThreads), 0, s, keys.Current(), nnz,
                       l.cols, At<RowT>(l.ws, l.layout.colptr_offset));
    const int64_t finishWaves = (nnz + kFinishSpan - 1) / kFinishSpan;
    hipLaunchKernelGGL((CscFinishKernel<RowT>),
                       dim3(static_cast<unsigned>(finishWaves < 65536 ? (finishWaves > 0 ? finishWaves : 1) : 65536)),
                       dim3(kWave), 0, s, vals.Current(),
                       At<RowT>(l.ws, l.layout.csc_pos_offset), At<int32_t>(l.ws, l.layout.entry_row_offset),
                       At<const RowT>(l.ws, l.layout.rowptr_offset), l.rows, nnz);
    hipLaunchKernelGGL((CscRowDeltaKernel<RowT>), dim3(static_cast<unsigned>(l.layout.row_groups)), dim3(kThreads),
                       0, s, At<const int32_t>(l.ws, l.layout.entry_row_offset),
                       At<const RowT>(l.ws, l.layout.rowptr_offset), l.rows,
                       At<int32_t>(l.ws, l.layout.group_row_offset), At<uint8_t>(l.ws, l.layout.row_delta_offset));
    // Row-block partition of the columns (the column pass runs the stream
    // kernel on the CSC pattern); colptr is already normalised, so the
    // partition kernel rewrites it in place with the same values.
    PrepParams pp{};
    pp.rp = At<void>(l.ws, l.layout.colptr_offset);
    pp.stride = 1;
    pp.base = 0;
    pp.rows = l.cols;
    pp.cols = l.rows;
    pp.nnz = nnz;
    pp.norm = At<void>(l.ws, l.layout.colptr_offset);
    pp.blocks = At<int32_t>(l.ws, l.layout.csc_blocks_offset);
    pp.block_nnz = At<void>(l.ws, l.layout.csc_block_nnz_offset);
    pp.num_blocks = l.layout.csc_num_blocks;
    pp.items = l.layout.csc_items_per_block;
    pp.header = nullptr;
    const int64_t n = (l.cols > pp.num_blocks ? l.cols : pp.num_blocks) + 1;
    hipLaunchKernelGGL((SpmvPreprocessKernel<RowT>), dim3(static_cast<unsigned>((n + kThreads - 1) / kThreads)),
                       dim3(kThreads), 0, s, pp);
    return 0;
}

}  // namespace

size_t TaskScanTempBytes(int64_t n)
{
    size_t bytes = 0;
    if (hipcub::DeviceScan::ExclusiveSum(nullptr, bytes, static_cast<int32_t*>(nullptr),
                                         static_cast<int32_t*>(nullptr), static_cast<int>(n)) != hipSuccess) {
        bytes = static_cast<size_t>(n) * 16 + (64 << 10);  // no device to ask: a generous bound
    }
    return bytes;
}

size_t CscSortTempBytes(int64_t nnz, uint32_t posBytes)
{
    size_t bytes = 0;
    hipcub::DoubleBuffer<int32_t> k(nullptr, nullptr);
    hipError_t e;
    if (posBytes == 8) {
        hipcub::DoubleBuffer<int64_t> v(nullptr, nullptr);
        e = hipcub::DeviceRadixSort::SortPairs(nullptr, bytes, k, v, static_cast<int>(nnz), 0, 31);
    } else {
        hipcub::DoubleBuffer<int32_t> v(nullptr, nullptr);
        e = hipcub::DeviceRadixSort::SortPairs(nullptr, bytes, k, v, static_cast<int>(nnz), 0, 31);
    }
    if (e != hipSuccess) bytes = static_cast<size_t>(nnz) * 16 + (1 << 20);
    return bytes;
}

int LaunchSpmvOpStreamFixed(const SpmvLaunch& l, float* z, void* stream)
{
    if (l.rows <= 0) return 0;
    RowBlockParams p{};
    p.rp = l.row_ptr;
    p.rp_base = l.base;
    p.col = l.col;
    p.col_stride = 1;
    p.val = l.val;
    p.val_stride = 1;
    p.x = l.x;
    p.x_stride = 1;
    p.y = l.y;
    p.y_stride = 1;
    p.z = z;
    p.rows = l.rows;
    p.cols = l.cols;
    p.nnz = l.nnz;
    p.base = l.base;
    p.s.device = l.device_scalars;
    p.s.alpha_re = l.alpha_re;
    p.s.beta_re = l.beta_re;
    p.s.alpha_ptr = l.alpha_ptr;
    p.s.beta_ptr = l.beta_ptr;
    // about one 512-slot chunk of non-zeros per block, at most 127 rows
    int64_t r = l.nnz > 0 ? static_cast<int64_t>((496.0 * static_cast<double>(l.rows)) / static_cast<double>(l.nnz))
                          : kWaveRows;
    r = r < 1 ? 1 : r > kWaveRows ? kWaveRows : r;
    p.fixed_rows = static_cast<int32_t>(r);
    p.num_blocks = (l.rows + r - 1) / r;
    hipStream_t s = static_cast<hipStream_t>(stream);
    const int64_t wgs = (p.num_blocks + kFlatWaves - 1) / kFlatWaves;
    const unsigned g = static_cast<unsigned>((wgs + kXcds - 1) / kXcds * kXcds);
    const bool betaNz = l.device_scalars || l.beta_re != 0.0f;
    if (l.rowptr64) {
        if (betaNz) hipLaunchKernelGGL((SpmvOpStreamKernel<int64_t, true, true>), dim3(g), dim3(kWave * kFlatWaves), 0, s, p);
        else hipLaunchKernelGGL((SpmvOpStreamKernel<int64_t, false, true>), dim3(g), dim3(kWave * kFlatWaves), 0, s, p);
    } else {
        if (betaNz) hipLaunchKernelGGL((SpmvOpStreamKernel<int32_t, true, true>), dim3(g), dim3(kWave * kFlatWaves), 0, s, p);
        else hipLaunchKernelGGL((SpmvOpStreamKernel<int32_t, false, true>), dim3(g), dim3(kWave * kFlatWaves), 0, s, p);
    }
    return 0;
}

template <typename RowT, bool kGated, bool kNarrow, bool kEntry>
void LaunchOpStreamVariant(const RowBlockParams& p, bool betaNz, hipStream_t s)
{
    const int64_t wgs = (p.num_blocks + kFlatWaves - 1) / kFlatWaves;
    const unsigned g = static_cast<unsigned>((wgs + kXcds - 1) / kXcds * kXcds);
    if (betaNz) {
        hipLaunchKernelGGL((SpmvOpStreamKernel<RowT, true, false, kGated, kNarrow, kEntry>), dim3(g),
                           dim3(kWave * kFlatWaves), 0, s, p);
    } else {
        hipLaunchKernelGGL((SpmvOpStreamKernel<RowT, false, false, kGated, kNarrow, kEntry>), dim3(g),
                           dim3(kWave * kFlatWaves), 0, s, p);
    }
}

template <typename RowT>
void LaunchOpStreamTyped(const SpmvLaunch& l, RowBlockParams p, bool betaNz, hipStream_t s)
{
    const bool narrow = l.narrow && p.ncol != nullptr;
    RowBlockParams pe = p;  // the entry-aligned blocks
    pe.blocks = At<const int32_t>(l.ws, l.layout.eb_offset);
    pe.block_nnz = At<const void>(l.ws, l.layout.en_offset);
    pe.num_blocks = l.layout.entry_blocks;
    if (narrow && l.staged_choice == kEntryFlag) {
        LaunchOpStreamVariant<RowT, false, true, true>(pe, betaNz, s);
    } else if (narrow && l.staged_choice == kNarrowFlag) {
        LaunchOpStreamVariant<RowT, false, true, false>(p, betaNz, s);
    } else if (narrow && l.staged_choice < 0) {
        // choice not on the host yet: every variant, each runs on its own flag
        const uint32_t* flag = &At<SpmvWsHeader>(l.ws, 0)->staged_flag;
        p.skip_flag = flag;
        pe.skip_flag = flag;
        RowBlockParams pn = p;
        p.run_mask = 1U;
        pn.run_mask = 1U << kNarrowFlag;
        pe.run_mask = 1U << kEntryFlag;
        LaunchOpStreamVariant<RowT, true, false, false>(p, betaNz, s);
        LaunchOpStreamVariant<RowT, true, true, false>(pn, betaNz, s);
        LaunchOpStreamVariant<RowT, true, true, true>(pe, betaNz, s);
    } else {
        LaunchOpStreamVariant<RowT, false, false, false>(p, betaNz, s);
    }
}

int LaunchSpmvOpStream(const SpmvLaunch& l, float* z, void* stream)
{
    if (l.rows <= 0) return 0;
    RowBlockParams p = MakeRowBlockParams(l);
    p.z = z;
    hipStream_t s = static_cast<hipStream_t>(stream);
    const bool betaNz = l.device_scalars || l.beta_re != 0.0f;
    if (l.rowptr64) LaunchOpStreamTyped<int64_t>(l, p, betaNz, s);
    else LaunchOpStreamTyped<int32_t>(l, p, betaNz, s);
    return 0;
}

int LaunchSpmvPreprocess(const SpmvLaunch& l, void* stream)
{
    if (l.rows <= 0) return 0;
    PrepParams p{};
    p.rp = l.row_ptr;
    p.stride = l.row_stride;
    p.base = l.base;
    p.rows = l.rows;
    p.cols = l.cols;
    p.nnz = l.nnz;
    p.norm = At<void>(l.ws, l.layout.rowptr_offset);
    p.blocks = At<int32_t>(l.ws, l.layout.blocks_offset);
    p.block_nnz = At<void>(l.ws, l.layout.block_nnz_offset);
    p.num_blocks = l.layout.num_blocks;
    p.items = l.layout.items_per_block;
    p.header = At<SpmvWsHeader>(l.ws, 0);
    SpmvWsHeader& h = p.header_value;
    h.magic = kWsMagic;
    h.version = 1;
    h.rows = static_cast<uint64_t>(l.rows);
    h.cols = static_cast<uint64_t>(l.cols);
    h.nnz = static_cast<uint64_t>(l.nnz);
    h.items_per_block = static_cast<uint64_t>(l.layout.items_per_block);
    h.num_blocks = static_cast<uint64_t>(l.layout.num_blocks);
    h.rowptr_offset = l.layout.rowptr_offset;
    h.blocks_offset = l.layout.blocks_offset;
    h.block_nnz_offset = l.layout.block_nnz_offset;
    h.sink_offset = l.layout.sink_offset;
    h.acc_offset = l.layout.acc_offset;
    h.rowptr_bytes = l.layout.rowptr_bytes;
    h.index_base = static_cast<uint32_t>(l.base);
    h.op = static_cast<uint32_t>(l.op);
    h.long_chunks = static_cast<uint32_t>(kLongChunks);
    h.task_start_offset = l.layout.tasks ? l.layout.task_start_offset : 0;
    h.task_block_offset = l.layout.tasks ? l.layout.task_block_offset : 0;
    h.max_tasks = l.layout.tasks ? static_cast<uint64_t>(l.layout.max_tasks) : 0;
    if (l.staged) {  // staged_flag stays 0 until the staged or narrow preprocess decides
        h.staged_buckets = static_cast<uint32_t>(l.layout.st_buckets);
        h.staged_tiles = static_cast<uint64_t>(l.layout.st_tiles);
        h.staged_tile_row_offset = l.layout.st_tile_row_offset;
        h.staged_tile_nnz_offset = l.layout.st_tile_nnz_offset;
    }
    const int64_t n = (l.rows > p.num_blocks ? l.rows : p.num_blocks) + 1;
    const unsigned grid = static_cast<unsigned>((n + kThreads - 1) / kThreads);
    hipStream_t s = static_cast<hipStream_t>(stream);
    if (l.rowptr64) {
        hipLaunchKernelGGL((SpmvPreprocessKernel<int64_t>), dim3(grid), dim3(kThreads), 0, s, p);
        if (l.layout.csc) {
            if (BuildCsc<int64_t>(l, s) != 0) return 1;
            return l.staged ? LaunchStagedPreprocess(l, stream) : 0;
        }
        if (l.layout.tasks && BuildTasks<int64_t>(l, s) != 0) return 1;
        if (l.staged && LaunchStagedPreprocess(l, stream) != 0) return 1;
        if (l.narrow && l.layout.narrow) BuildNarrow<int64_t>(l, s);
        return 0;
    } else {
        hipLaunchKernelGGL((SpmvPreprocessKernel<int32_t>), dim3(grid), dim3(kThreads), 0, s, p);
        if (l.layout.csc) {
            if (BuildCsc<int32_t>(l, s) != 0) return 1;
            if (l.cband && l.layout.cband) {
                SpmvWsHeader* h = At<SpmvWsHeader>(l.ws, 0);
                hipLaunchKernelGGL(CbandRowKernel, dim3(GridFor(l.nnz)), dim3(kThreads), 0, s,
                                   At<const int32_t>(l.ws, l.layout.csc_pos_offset),
                                   At<const int32_t>(l.ws, l.layout.entry_row_offset), l.col,
                                   static_cast<int32_t>(l.base), At<int32_t>(l.ws, l.layout.val_b_offset), l.nnz,
                                   &h->narrow_bad);
                const int64_t nb = l.layout.csc_num_blocks;
                const unsigned bg = static_cast<unsigned>((nb + kWaves - 1) / kWaves);
                hipLaunchKernelGGL(CbandNarrowCheckKernel, dim3(bg), dim3(kThreads), 0, s,
                                   At<const int32_t>(l.ws, l.layout.val_b_offset),
                                   At<const int32_t>(l.ws, l.layout.csc_pos_offset),
                                   At<const int32_t>(l.ws, l.layout.csc_blocks_offset),
                                   At<const int32_t>(l.ws, l.layout.csc_block_nnz_offset), nb, &h->entry_bad);
                hipLaunchKernelGGL(CbandDecideKernel, dim3(1), dim3(kWave), 0, s,
                                   static_cast<const uint32_t*>(&h->narrow_bad),
                                   static_cast<const uint32_t*>(&h->entry_bad), l.nnz, &h->staged_flag);
                hipLaunchKernelGGL(CbandNarrowPackKernel, dim3(bg), dim3(kThreads), 0, s,
                                   At<int32_t>(l.ws, l.layout.val_b_offset),
                                   At<const int32_t>(l.ws, l.layout.csc_pos_offset),
                                   At<const int32_t>(l.ws, l.layout.csc_blocks_offset),
                                   At<const int32_t>(l.ws, l.layout.csc_block_nnz_offset), nb,
                                   static_cast<const uint32_t*>(&h->staged_flag));
            }
            if (!l.staged) return 0;
            if (LaunchStagedPreprocess(l, stream) != 0) return 1;
            // the banded kernel's 16-bit copies (32-bit offsets and positions only)
            if (l.nnz <= 0x1FFFFFFFLL && l.val_kind == ValKind::F32) BuildBandedNarrow(l, s);
            return 0;
        }
        if (l.layout.tasks && BuildTasks<int32_t>(l, s) != 0) return 1;
        if (l.staged && LaunchStagedPreprocess(l, stream) != 0) return 1;
        if (l.narrow && l.layout.narrow) BuildNarrow<int32_t>(l, s);
        return 0;
    }
}

int LaunchSpmvCompute(const SpmvLaunch& l, void* stream)
{
    hipStream_t s = static_cast<hipStream_t>(stream);
    if (l.op == ACL_SPARSE_OP_NON_TRANSPOSE && l.rows <= 0) return 0;
    if (l.op == ACL_SPARSE_OP_NON_TRANSPOSE && l.rows <= kSmallFloatRows && l.val_kind == ValKind::F32 &&
        l.out_kind == OutKind::F32 && l.acc_kind == AccKind::F32) {
        // the reference's compensated small-matrix path (no staged or narrow kernels)
        const Scalars sc = MakeRowBlockParams(l).s;
        if (l.rowptr64) {
            hipLaunchKernelGGL((SpmvSmallFloatKernel<int64_t>), dim3(1), dim3(kWave), 0, s,
                               static_cast<const int64_t*>(l.row_ptr), l.row_stride, l.col, l.col_stride,
                               static_cast<const float*>(l.val), l.val_stride, static_cast<const float*>(l.x),
                               l.x_stride, static_cast<float*>(l.y), l.y_stride, l.rows, l.cols, l.nnz, l.base, sc);
        } else {
            hipLaunchKernelGGL((SpmvSmallFloatKernel<int32_t>), dim3(1), dim3(kWave), 0, s,
                               static_cast<const int32_t*>(l.row_ptr), l.row_stride, l.col, l.col_stride,
                               static_cast<const float*>(l.val), l.val_stride, static_cast<const float*>(l.x),
                               l.x_stride, static_cast<float*>(l.y), l.y_stride, l.rows, l.cols, l.nnz, l.base, sc);
        }
        return 0;
    }
    const int rc = l.rowptr64 ? DispatchTypes<int64_t>(l, s) : DispatchTypes<int32_t>(l, s);
    // staged gather: the row kernel above exits when Preprocess chose this path
    if (rc == 0 && l.staged && (l.staged_choice == 1 || l.staged_choice < 0)) return LaunchStagedCompute(l, stream);
    return rc;
}

}  // namespace aclsp
