// SpMMOp kernels for gfx950: C = alpha * A * op(B) + beta * C with A in CSR
// (fp32 or fp16 values, I32/I64 row offsets, index base 0/1) and B, C dense
// in row or column order.
//
// Arithmetic restates sparse/spmm_op/arch35/spmm_op_kernel.cpp:
//  * per output element, the products v_p * op(B)(c_p, j) of the row's
//    entries are added in CSR order into an fp32 sum, each product and each
//    sum rounded separately (:386-424, Muls then Add); entries whose column
//    lies outside [0, k) are skipped there;
//  * ALG1_HIGH_PRECISION (fp32 only) adds with Kahan compensation
//    (:529-547: y = p - comp, t = acc + y, comp = (t - acc) - y, acc = t);
//  * out = alpha * sum, then, when beta != 0, out = out + beta * C_old, each
//    step rounded (:549-596, :598-640); beta == 0 never reads C;
//  * fp16 output: clamped to +-65504, then rounded to nearest with ties away
//    from zero (:89-127, RoundMode::CAST_ROUND);
//  * nnz == 0: C = beta * C_old, or 0 when beta == 0 (:687-880).
// The whole kernel is compiled without floating-point contraction so that
// every step rounds as above: results are bit-identical run to run and to a
// sequential fp32 restatement of the same steps.
//
// Mapping (MI355X-first): one wave covers RPW = 64/G rows and a tile of G*J
// output columns; the G lanes of a row each own J adjacent columns, so a row
// of op(B) (row-major B with opB = N, column-major B with opB = T) is read by
// 16-byte (fp32, J = 4) or 8-byte (fp16) vector loads, fully coalesced.  The
// row's column indices and values are read G at a time (one per lane) and
// handed to the group by cross-lane reads; eight entries' B rows are in
// flight at a time.  Short outputs (n < 64) pack several rows
// into one wave instead of idling lanes; outputs of 8 to 32 columns (a
// multiple of 4) give each row 2, 4 or 8 lanes of 4 columns (32, 16 or 8 rows
// per wave), each lane reading 4, 2 or 1 of a window's 8 entries, so that a
// wave keeps 8 entries' B rows in flight for many rows at once.  Wider
// outputs whose width is a multiple of 4 give each row 16, 32 or 64 lanes of 4
// columns (4, 2 or 1 rows per wave).
#include <hip/hip_runtime.h>

#include <cstdint>
#include <utility>

#include "aclsparse_internal.h"

namespace aclsp {
namespace {

#pragma clang fp contract(off)

constexpr int kMmThreads = 256;
constexpr int kMmWave = 64;
constexpr float kFp16Max = 65504.0f;
constexpr int kU = 8;  // entries whose B rows are in flight together
typedef float v4f __attribute__((ext_vector_type(4)));
typedef int v4i __attribute__((ext_vector_type(4)));
#ifndef SPMM_MAX_BLOCKS
#define SPMM_MAX_BLOCKS 8192
#endif
constexpr int64_t kMmMaxBlocks = SPMM_MAX_BLOCKS;  // grid cap (32 per CU); waves loop over the rest

__device__ __forceinline__ float Half2Float(uint16_t h) { return static_cast<float>(__builtin_bit_cast(_Float16, h)); }

// fp32 -> fp16, round to nearest, ties away from zero (|f| <= 65504 or NaN).
__device__ __forceinline__ uint16_t FloatToHalfAway(float f)
{
    const uint32_t x = __float_as_uint(f);
    const uint32_t sign = (x >> 16) & 0x8000U;
    const uint32_t ax = x & 0x7FFFFFFFU;
    if (ax > 0x7F800000U) return static_cast<uint16_t>(sign | 0x7E00U);  // NaN
    if (ax >= 0x38800000U) {                                             // |f| >= 2^-14: normal
        const uint32_t e = (ax >> 23) - 112U;                            // rebias 127 -> 15
        const uint32_t h = (e << 10) | ((ax >> 13) & 0x3FFU);
        return static_cast<uint16_t>(sign | (h + ((ax >> 12) & 1U)));   // carry may bump the exponent
    }
    if (ax < 0x33000000U) return static_cast<uint16_t>(sign);           // below 2^-25: zero
    // subnormal: value = mant * 2^(e-150), fp16 unit 2^-24
    const uint32_t mant = (ax & 0x7FFFFFU) | 0x800000U;
    const uint32_t shift = 126U - (ax >> 23);                            // 14..25
    const uint32_t q = mant >> shift;
    const uint32_t half = 1U << (shift - 1U);
    return static_cast<uint16_t>(sign | (q + ((mant & ((1U << shift) - 1U)) >= half ? 1U : 0U)));
}

// Wave-uniform reads of arrays the kernel never writes: through the constant
// address space, so they become scalar loads.
template <typename T>
__device__ __forceinline__ T ConstLoad(const void* base, int64_t i)
{
    typedef const __attribute__((address_space(4))) T* CPtr;
    return reinterpret_cast<CPtr>(reinterpret_cast<uintptr_t>(base))[i];
}

// Value i of A (fp32 or fp16) by a scalar load (fp16: the aligned dword that holds it).
template <bool kHalf>
__device__ __forceinline__ float ScalarVal(const void* val, int64_t i)
{
    if constexpr (kHalf) {
        const uintptr_t a = reinterpret_cast<uintptr_t>(val) + static_cast<uintptr_t>(i) * 2;
        const uint32_t w = ConstLoad<uint32_t>(reinterpret_cast<const void*>(a & ~uintptr_t{3}), 0);
        return Half2Float(static_cast<uint16_t>(w >> ((a & 2) * 8)));
    } else {
        return ConstLoad<float>(val, i);
    }
}

template <bool kHalf>
struct Elem;
template <>
struct Elem<false> {
    using T = float;
    __device__ static float Load(const T* p, int64_t i) { return p[i]; }
    __device__ static void Store(T* p, int64_t i, float v) { p[i] = v; }
};
template <>
struct Elem<true> {
    using T = uint16_t;
    __device__ static float Load(const T* p, int64_t i) { return Half2Float(p[i]); }
    __device__ static void Store(T* p, int64_t i, float v)
    {
        v = v > kFp16Max ? kFp16Max : v;
        v = v < -kFp16Max ? -kFp16Max : v;
        p[i] = FloatToHalfAway(v);
    }
};

template <typename T, int J>
struct alignas(J * sizeof(T)) Vec {
    T v[J];
};

struct MmParams {
    const void* rp;
    const int32_t* col;
    const void* val;
    const void* b;
    void* c;
    int64_t m, k, n, ldb, ldc, nnz;
    int32_t base;
    int32_t b_contig;    // op(B)(c, j) = b[c*ldb + j]; else b[j*ldb + c]
    int32_t b_vec;       // rows of op(B) can be read J elements at a time
    int32_t c_row;       // C(i, j) = c[i*ldc + j]; else c[j*ldc + i]
    int32_t c_vec;
    int32_t has_b;       // k > 0: op(B) has rows to read
    int32_t b_ubuf;      // fp32 rows of op(B) read as 16-byte buffer loads from any 4-byte
                         // boundary (widths not a multiple of 4, or rows not 16-byte aligned);
                         // loads past B's last element read 0
    int32_t b_bytes;     // B's extent in bytes when b_ubuf
    int32_t c_ubuf;      // fp32 row-major C whose rows are not 16-byte aligned: J = 4 columns
                         // read and (when wholly inside the row) written by 16-byte buffer
                         // accesses from any 4-byte boundary
    int32_t c_bytes;     // C's extent in bytes when c_ubuf
    int32_t lg;          // log2 of lanes per row
    int64_t tiles;       // column tiles per row group
    int64_t waves;       // row groups * tiles
    float alpha, beta;
    const float* alpha_ptr;
    const float* beta_ptr;
};

template <bool kHalf, int J>
__device__ __forceinline__ void LoadRowJ(const typename Elem<kHalf>::T* base, int64_t j0, int64_t n, int64_t stride,
                                         bool vec, float out[J])
{
    using T = typename Elem<kHalf>::T;
    if (vec && j0 + J <= n) {
        const Vec<T, J> w = *reinterpret_cast<const Vec<T, J>*>(base + j0);
#pragma unroll
        for (int q = 0; q < J; ++q) {
            if constexpr (kHalf) out[q] = Half2Float(w.v[q]);
            else out[q] = w.v[q];
        }
    } else {
#pragma unroll
        for (int q = 0; q < J; ++q) out[q] = j0 + q < n ? Elem<kHalf>::Load(base, (j0 + q) * stride) : 0.0f;
    }
}

// Loads the op(B) rows of a batch of kU entries (cc < 0: skipped entry).
template <bool kHalf, int J>
__device__ __forceinline__ void SpmmLoad(const MmParams& p, const typename Elem<kHalf>::T* b, int64_t j0, bool fast,
                                         bool strided, const int32_t cc[kU], float bv[kU][J])
{
    using T = typename Elem<kHalf>::T;
    if (fast && !kHalf && J == 4 && p.b_ubuf) {
        // one 16-byte buffer load per entry at any 4-byte boundary; columns
        // past n read the next row (never stored), past B's end read 0
        const __amdgpu_buffer_rsrc_t rb =
            __builtin_amdgcn_make_buffer_rsrc(const_cast<T*>(b), 0, p.b_bytes, 0x00020000);
#pragma unroll
        for (int q = 0; q < kU; ++q) {
            const int64_t r = cc[q] >= 0 ? cc[q] : 0;
            const int off = static_cast<int>((r * p.ldb + j0) * 4);
            const v4f w = __builtin_bit_cast(v4f, __builtin_amdgcn_raw_buffer_load_b128(rb, off, 0, 0));
#pragma unroll
            for (int t = 0; t < J; ++t) bv[q][t] = w[t];
        }
    } else if (fast) {
        // one unconditional vector load per entry (a skipped entry reads row 0)
#pragma unroll
        for (int q = 0; q < kU; ++q) {
            const int64_t r = cc[q] >= 0 ? cc[q] : 0;
            const Vec<T, J> w = *reinterpret_cast<const Vec<T, J>*>(b + r * p.ldb + j0);
#pragma unroll
            for (int t = 0; t < J; ++t) {
                if constexpr (kHalf) bv[q][t] = Half2Float(w.v[t]);
                else bv[q][t] = w.v[t];
            }
        }
    } else if (strided) {
        // B(c, j) = b[j*ldb + c]: unconditional element loads at clamped positions
#pragma unroll
        for (int q = 0; q < kU; ++q) {
            const int64_t r = cc[q] >= 0 ? cc[q] : 0;
#pragma unroll
            for (int t = 0; t < J; ++t) {
                const int64_t j = j0 + t < p.n ? j0 + t : p.n - 1;
                bv[q][t] = Elem<kHalf>::Load(b, j * p.ldb + r);
            }
        }
    } else {
#pragma unroll
        for (int q = 0; q < kU; ++q) {
            if (cc[q] >= 0) {
                LoadRowJ<kHalf, J>(b + static_cast<int64_t>(cc[q]) * p.ldb, j0, p.n, 1, false, bv[q]);
            } else {
#pragma unroll
                for (int t = 0; t < J; ++t) bv[q][t] = 0.0f;
            }
        }
    }
}

// Adds a batch's products into the sums, in entry order.
template <bool kKahan, int J>
__device__ __forceinline__ void SpmmAccum(const int32_t cc[kU], const float vv[kU], const float bv[kU][J],
                                          float acc[J], float comp[J])
{
#pragma unroll
    for (int q = 0; q < kU; ++q) {
        const bool take = cc[q] >= 0;  // skipped entries leave the sums untouched
#pragma unroll
        for (int t = 0; t < J; ++t) {
            const float prod = vv[q] * bv[q][t];
            if constexpr (kKahan) {
                const float y = prod - comp[t];
                const float s2 = acc[t] + y;
                const float c2 = (s2 - acc[t]) - y;
                acc[t] = take ? s2 : acc[t];
                comp[t] = take ? c2 : comp[t];
            } else {
                const float s2 = acc[t] + prod;
                acc[t] = take ? s2 : acc[t];
            }
        }
    }
}

// C_old of one lane's J columns of one row (read before the row's products,
// so that the read is not a step of the dependent chain); 0 past n.
template <bool kHalf, int J>
__device__ __forceinline__ void SpmmLoadC(const MmParams& p, const typename Elem<kHalf>::T* c, int64_t row, int64_t j0,
                                          float old[J])
{
    if (!kHalf && J == 4 && p.c_ubuf) {
        // columns past n read the next row (never stored), past C's end read 0
        const __amdgpu_buffer_rsrc_t rc =
            __builtin_amdgcn_make_buffer_rsrc(const_cast<typename Elem<kHalf>::T*>(c), 0, p.c_bytes, 0x00020000);
        const v4f w = __builtin_bit_cast(
            v4f, __builtin_amdgcn_raw_buffer_load_b128(rc, static_cast<int>((row * p.ldc + j0) * 4), 0, 0));
#pragma unroll
        for (int q = 0; q < J; ++q) old[q] = j0 + q < p.n ? w[q] : 0.0f;
    } else if (p.c_row) {
        LoadRowJ<kHalf, J>(c + row * p.ldc, j0, p.n, 1, p.c_vec != 0, old);
    } else {
#pragma unroll
        for (int q = 0; q < J; ++q) old[q] = j0 + q < p.n ? Elem<kHalf>::Load(c, (j0 + q) * p.ldc + row) : 0.0f;
    }
}

// out = alpha * sum, then + beta * C_old when beta != 0 (each step rounded),
// stored with the element type's rounding; one lane's J columns of one row.
template <bool kHalf, int J>
__device__ __forceinline__ void SpmmStore(const MmParams& p, typename Elem<kHalf>::T* c, int64_t row, int64_t j0,
                                          const float acc[J], float alpha, float beta, bool betaZero,
                                          const float old[J])
{
    using T = typename Elem<kHalf>::T;
    float out[J];
#pragma unroll
    for (int q = 0; q < J; ++q) out[q] = alpha * acc[q];
    if (!betaZero) {
#pragma unroll
        for (int q = 0; q < J; ++q) out[q] = out[q] + beta * old[q];
    }
    if (!kHalf && J == 4 && p.c_ubuf && j0 + J <= p.n) {
        const __amdgpu_buffer_rsrc_t rc = __builtin_amdgcn_make_buffer_rsrc(c, 0, p.c_bytes, 0x00020000);
        const v4f w = {out[0], out[1], J > 2 ? out[2 % J] : 0.0f, J > 3 ? out[3 % J] : 0.0f};
        __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(v4i, w), rc,
                                               static_cast<int>((row * p.ldc + j0) * 4), 0, 0);
    } else if (p.c_row) {
        T* crow = c + row * p.ldc;
        if (p.c_vec && j0 + J <= p.n && !kHalf) {
            Vec<T, J> wv;
#pragma unroll
            for (int q = 0; q < J; ++q) wv.v[q] = out[q];
            *reinterpret_cast<Vec<T, J>*>(crow + j0) = wv;
        } else {
#pragma unroll
            for (int q = 0; q < J; ++q) {
                if (j0 + q < p.n) Elem<kHalf>::Store(crow, j0 + q, out[q]);
            }
        }
    } else {
#pragma unroll
        for (int q = 0; q < J; ++q) {
            if (j0 + q < p.n) Elem<kHalf>::Store(c, (j0 + q) * p.ldc + row, out[q]);
        }
    }
}

// One row per wave: entries u0 .. u0+kU-1 of the window, read from the lanes
// that loaded them into scalar registers (no LDS traffic; -1 past the row).
__device__ __forceinline__ void SpmmFetchWave(int myc, float myv, int u0, int cnt, int32_t cc[kU], float vv[kU])
{
#pragma unroll
    for (int q = 0; q < kU; ++q) {
        const int u = u0 + q < kMmWave ? u0 + q : kMmWave - 1;
        const int32_t cq = __builtin_amdgcn_readlane(myc, u);
        vv[q] = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(myv), u));
        cc[q] = u0 + q < cnt ? cq : -1;
    }
}

// Entries u0 .. u0+kU-1 of the group's current window, read from the lanes
// that loaded them (-1 past the row).
__device__ __forceinline__ void SpmmFetch(int myc, float myv, int gbase, int g, int u0, int cnt, int32_t cc[kU],
                                          float vv[kU])
{
#pragma unroll
    for (int q = 0; q < kU; ++q) {
        const int u = u0 + q < g ? u0 + q : g - 1;
        const int32_t cq = __shfl(myc, gbase + u, kMmWave);
        vv[q] = __shfl(myv, gbase + u, kMmWave);
        cc[q] = u0 + q < cnt ? cq : -1;
    }
}

// kNG > 0: groups of kNG < kU lanes (g == kNG), each lane reading kU / kNG
// entries per window, so that a window fills one batch of kU entries.
// Narrow groups: at least 5 waves per SIMD (at most 102 VGPRs; 4 waves at the
// 124 the compiler picks otherwise: 264 -> 251 us on the Laplacian x 16; 6
// waves spill).
#ifndef SPMM_NARROW_WPE
#define SPMM_NARROW_WPE 5
#endif
template <typename RowT, bool kHalf, bool kKahan, int J, bool kWave, int kNG = 0>
__global__ __launch_bounds__(kMmThreads) __attribute__((amdgpu_waves_per_eu(kNG > 0 ? SPMM_NARROW_WPE : 1)))
void SpmmOpKernel(MmParams p)
{
    using T = typename Elem<kHalf>::T;
    const RowT* rp = static_cast<const RowT*>(p.rp);
    const T* val = static_cast<const T*>(p.val);
    const T* b = static_cast<const T*>(p.b);
    T* c = static_cast<T*>(p.c);
    const float alpha = p.alpha_ptr != nullptr ? *p.alpha_ptr : p.alpha;
    const float beta = p.beta_ptr != nullptr ? *p.beta_ptr : p.beta;
    const bool betaZero = beta == 0.0f;
    const int lane = static_cast<int>(threadIdx.x) & (kMmWave - 1);
    const int g = 1 << p.lg;
    const int rpw = kMmWave >> p.lg;
    const int64_t waveStep = static_cast<int64_t>(gridDim.x) * (kMmThreads / kMmWave);
    const int wv = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x) / kMmWave);
    for (int64_t w = static_cast<int64_t>(blockIdx.x) * (kMmThreads / kMmWave) + wv; w < p.waves; w += waveStep) {
        // (one column tile, the common case, needs no division; 32-bit division otherwise)
        int64_t tile = 0, rg = w;
        if (p.tiles != 1) {
            if (p.waves <= 0x7FFFFFFF) {
                const uint32_t wq = static_cast<uint32_t>(w) / static_cast<uint32_t>(p.tiles);
                tile = static_cast<int64_t>(static_cast<uint32_t>(w) - wq * static_cast<uint32_t>(p.tiles));
                rg = wq;
            } else {
                tile = w % p.tiles;
                rg = w / p.tiles;
            }
        }
        const int64_t row = rg * rpw + (lane >> p.lg);
        const int64_t j0 = (tile * g + (lane & (g - 1))) * J;
        // every lane of a row's group walks the row (its entries are shared
        // across the group); only lanes inside [0, n) store
        const bool live = row < p.m && j0 < p.n;
        // wave-uniform load paths: whole tiles of contiguous, aligned rows of op(B); or B
        // stored the other way (element loads); else the guarded general path
        const bool fullTile = (tile + 1) * g * J <= p.n;
        // (n a multiple of J: a lane's J columns lie wholly inside or wholly
        // past n, and lanes past n read column 0 of the same rows)
        const bool fast = p.has_b && p.b_contig && ((p.b_vec && (fullTile || p.n % J == 0)) || p.b_ubuf);
        const int64_t jf = j0 < p.n ? j0 : 0;
        const bool strided = p.has_b && !p.b_contig;
        int64_t rs = 0, re = 0;
        if (row < p.m) {
            rs = static_cast<int64_t>(rp[row]) - p.base;
            re = static_cast<int64_t>(rp[row + 1]) - p.base;
        }
        float acc[J], comp[J], old[J];
#pragma unroll
        for (int q = 0; q < J; ++q) {
            acc[q] = 0.0f;
            comp[q] = 0.0f;
            old[q] = 0.0f;
        }
        if (live && !betaZero) SpmmLoadC<kHalf, J>(p, c, row, j0, old);
        // Each group reads its row's entries G at a time, one per lane, and
        // hands them to the group by cross-lane reads, kU at a time.
        const int gl = lane & (g - 1);
        const int gbase = lane & ~(g - 1);
        if constexpr (kNG > 0) {
            constexpr int kE = kU / kNG;
            for (int64_t e0 = rs; e0 < re; e0 += kU) {
                int32_t myc[kE];
                float myv[kE];
#pragma unroll
                for (int s = 0; s < kE; ++s) {
                    const int64_t e = e0 + s * kNG + gl;
                    myc[s] = -1;
                    myv[s] = 0.0f;
                    if (e < re) {
                        const int32_t ci = p.col[e] - p.base;
                        myc[s] = ci >= 0 && ci < p.k ? ci : -1;
                        myv[s] = Elem<kHalf>::Load(val, e);
                    }
                }
                const int cnt = re - e0 < kU ? static_cast<int>(re - e0) : kU;
                int32_t cc[kU];
                float vv[kU];
                float bv[kU][J];
#pragma unroll
                for (int q = 0; q < kU; ++q) {
                    const int32_t cq = __shfl(myc[q / kNG], gbase + q % kNG, kMmWave);
                    vv[q] = __shfl(myv[q / kNG], gbase + q % kNG, kMmWave);
                    cc[q] = q < cnt ? cq : -1;
                }
                SpmmLoad<kHalf, J>(p, b, fast ? jf : j0, fast, strided, cc, bv);
                SpmmAccum<kKahan, J>(cc, vv, bv, acc, comp);
            }
        } else
        for (int64_t e0 = rs; e0 < re; e0 += g) {
            int32_t myc = -1;
            float myv = 0.0f;
            if (e0 + gl < re) {
                const int32_t ci = p.col[e0 + gl] - p.base;
                myc = ci >= 0 && ci < p.k ? ci : -1;
                myv = Elem<kHalf>::Load(val, e0 + gl);
            }
            const int cnt = re - e0 < g ? static_cast<int>(re - e0) : g;
            for (int u0 = 0; u0 < cnt; u0 += kU) {
                int32_t cc[kU];
                float vv[kU];
                float bv[kU][J];
                if constexpr (kWave) SpmmFetchWave(myc, myv, u0, cnt, cc, vv);
                else SpmmFetch(myc, myv, gbase, g, u0, cnt, cc, vv);
                SpmmLoad<kHalf, J>(p, b, fast ? jf : j0, fast, strided, cc, bv);
                SpmmAccum<kKahan, J>(cc, vv, bv, acc, comp);
            }
        }
        if (live) SpmmStore<kHalf, J>(p, c, row, j0, acc, alpha, beta, betaZero, old);
    }
}

// Small k (k * 64 * J fp32 values fit the workgroup's 64 KiB of LDS): the
// workgroup stages the column tile op(B)[0:k, tile] in LDS once (fp16 widened
// to fp32, exactly) and its four waves then take their rows' products from
// LDS; op(B) is read from L2 once per workgroup instead of once per entry.
// One row per wave at a time, its entries shared by cross-lane reads.
constexpr int kLdsBytes = 64 * 1024;
constexpr int kLdsWideBytes = 128 * 1024;  // J = 4 tiles without compensation
constexpr int kLdsThreads = 1024;  // 16 waves share one staged tile
constexpr int kLdsRowsPerWave = 4;

template <typename RowT, bool kHalf, bool kKahan, int J>
__global__ __launch_bounds__(kLdsThreads) __attribute__((amdgpu_waves_per_eu(8))) void SpmmOpLdsKernel(MmParams p)
{
    using T = typename Elem<kHalf>::T;
    extern __shared__ float sB[];
    constexpr int TW = kMmWave * J;
    const RowT* rp = static_cast<const RowT*>(p.rp);
    const T* val = static_cast<const T*>(p.val);
    const T* b = static_cast<const T*>(p.b);
    T* c = static_cast<T*>(p.c);
    const float alpha = p.alpha_ptr != nullptr ? *p.alpha_ptr : p.alpha;
    const float beta = p.beta_ptr != nullptr ? *p.beta_ptr : p.beta;
    const bool betaZero = beta == 0.0f;
    const int lane = static_cast<int>(threadIdx.x) & (kMmWave - 1);
    const int wv = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x) / kMmWave);
    const int64_t tile = static_cast<int64_t>(blockIdx.x) % p.tiles;
    const int64_t chunk = static_cast<int64_t>(blockIdx.x) / p.tiles;
    const int64_t jt = tile * TW;
    const int k = static_cast<int>(p.k);
    if (p.b_contig) {
        for (int idx = static_cast<int>(threadIdx.x); idx < k * TW; idx += kLdsThreads) {
            const int r = idx / TW, cj = idx - r * TW;
            const int64_t j = jt + cj;
            sB[idx] = j < p.n ? Elem<kHalf>::Load(b, static_cast<int64_t>(r) * p.ldb + j) : 0.0f;
        }
    } else {
        for (int idx = static_cast<int>(threadIdx.x); idx < k * TW; idx += kLdsThreads) {
            const int cj = idx / k, r = idx - cj * k;
            const int64_t j = jt + cj;
            sB[r * TW + cj] = j < p.n ? Elem<kHalf>::Load(b, j * p.ldb + r) : 0.0f;
        }
    }
    __syncthreads();
    const int64_t j0 = jt + lane * J;
    const int64_t row0 = (chunk * (kLdsThreads / kMmWave) + wv) * kLdsRowsPerWave;
    for (int rr = 0; rr < kLdsRowsPerWave; ++rr) {
        const int64_t row = row0 + rr;
        if (row >= p.m) break;
        // the row's entries are read 64 at a time, one per lane, and handed out
        // through scalar registers; their tiles of op(B) come from LDS
        const int64_t rs = static_cast<int64_t>(rp[row]) - p.base;
        const int64_t re = static_cast<int64_t>(rp[row + 1]) - p.base;
        float acc[J], comp[J], old[J];
#pragma unroll
        for (int q = 0; q < J; ++q) {
            acc[q] = 0.0f;
            comp[q] = 0.0f;
            old[q] = 0.0f;
        }
        if (j0 < p.n && !betaZero) SpmmLoadC<kHalf, J>(p, c, row, j0, old);
        for (int64_t e0 = rs; e0 < re; e0 += kMmWave) {
            int32_t myc = -1;
            float myv = 0.0f;
            if (e0 + lane < re) {
                const int32_t ci = p.col[e0 + lane] - p.base;
                myc = ci >= 0 && ci < p.k ? ci : -1;
                myv = Elem<kHalf>::Load(val, e0 + lane);
            }
            const int cnt = re - e0 < kMmWave ? static_cast<int>(re - e0) : kMmWave;
            for (int u0 = 0; u0 < cnt; u0 += kU) {
                int32_t cc[kU];
                float vv[kU];
                float bv[kU][J];
                SpmmFetchWave(myc, myv, u0, cnt, cc, vv);
                bool all = true;
#pragma unroll
                for (int q = 0; q < kU; ++q) {
                    const int r = cc[q] >= 0 ? cc[q] : 0;
                    all = all && cc[q] >= 0;
                    const Vec<float, J> w = *reinterpret_cast<const Vec<float, J>*>(&sB[r * TW + lane * J]);
#pragma unroll
                    for (int t = 0; t < J; ++t) bv[q][t] = w.v[t];
                }
                if (all) {  // wave-uniform: every entry of the batch counts, no selects
#pragma unroll
                    for (int q = 0; q < kU; ++q) {
#pragma unroll
                        for (int t = 0; t < J; ++t) {
                            const float prod = vv[q] * bv[q][t];
                            if constexpr (kKahan) {
                                const float y = prod - comp[t];
                                const float s2 = acc[t] + y;
                                comp[t] = (s2 - acc[t]) - y;
                                acc[t] = s2;
                            } else {
                                acc[t] = acc[t] + prod;
                            }
                        }
                    }
                } else {
                    SpmmAccum<kKahan, J>(cc, vv, bv, acc, comp);
                }
            }
        }
        if (j0 < p.n) SpmmStore<kHalf, J>(p, c, row, j0, acc, alpha, beta, betaZero, old);
    }
}

// Stages op(B)[0:k, jt:jt+TW] in LDS as fp32 (row r at sB[r*TW]; columns past
// n read as 0).  Full tiles of a row-major op(B) whose rows start on a
// 4-element boundary move 4 elements per load, four loads in flight per
// thread; other tiles element by element.
template <bool kHalf, int TW>
__device__ __forceinline__ void StageBTile(const MmParams& p, const typename Elem<kHalf>::T* b, float* sB, int64_t jt,
                                          int k)
{
    using T = typename Elem<kHalf>::T;
    if (p.b_contig && p.b_vec && jt + TW <= p.n) {
        constexpr int kQ = TW / 4;  // 4-element groups per staged row
        const int total = k * kQ;
        for (int i0 = static_cast<int>(threadIdx.x); i0 < total; i0 += 4 * kLdsThreads) {
            Vec<T, 4> w[4];
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                const int idx = i0 + u * kLdsThreads;
                const int r = idx < total ? idx / kQ : 0, q = idx < total ? idx % kQ : 0;
                w[u] = *reinterpret_cast<const Vec<T, 4>*>(b + static_cast<int64_t>(r) * p.ldb + jt + 4 * q);
            }
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                const int idx = i0 + u * kLdsThreads;
                if (idx < total) {
                    float4 f;
                    if constexpr (kHalf) {
                        f = make_float4(Half2Float(w[u].v[0]), Half2Float(w[u].v[1]), Half2Float(w[u].v[2]),
                                        Half2Float(w[u].v[3]));
                    } else {
                        f = make_float4(w[u].v[0], w[u].v[1], w[u].v[2], w[u].v[3]);
                    }
                    *reinterpret_cast<float4*>(&sB[(idx / kQ) * TW + 4 * (idx % kQ)]) = f;
                }
            }
        }
    } else if (p.b_contig) {
        for (int idx = static_cast<int>(threadIdx.x); idx < k * TW; idx += kLdsThreads) {
            const int r = idx / TW, cj = idx - r * TW;
            const int64_t j = jt + cj;
            sB[idx] = j < p.n ? Elem<kHalf>::Load(b, static_cast<int64_t>(r) * p.ldb + j) : 0.0f;
        }
    } else {
        for (int idx = static_cast<int>(threadIdx.x); idx < k * TW; idx += kLdsThreads) {
            const int cj = idx / k, r = idx - cj * k;
            const int64_t j = jt + cj;
            sB[r * TW + cj] = j < p.n ? Elem<kHalf>::Load(b, j * p.ldb + r) : 0.0f;
        }
    }
}

// Lane Q of the lane's 16-lane row (DPP row_newbcast: the compiler folds it
// into the instruction that uses the value).
template <int Q>
__device__ __forceinline__ int RowBcast(int v)
{
    return __builtin_amdgcn_mov_dpp(v, 0x150 + Q, 0xF, 0xF, true);
}

// Entry Q of a batch of 16 held by lanes 0..15 of every 16-lane row (byte
// offset of its op(B) row in LDS, with the sign bit set for a skipped entry,
// and its value): its products with the lane's J columns added in order.
template <int J, bool kAll, int Q>
__device__ __forceinline__ void BcastEntry(const char* sB, uint32_t laneOff, int off, float v, float acc[J])
{
    bool take = true;
    int o;
    if constexpr (kAll) {
        o = RowBcast<Q>(off);
    } else {
        o = RowBcast<Q>(off);
        take = o >= 0;
        o &= 0x7FFFFFFF;  // a skipped entry reads row 0
    }
    const Vec<float, J> w = *reinterpret_cast<const Vec<float, J>*>(sB + (o + laneOff));
    const float vq = __int_as_float(RowBcast<Q>(__float_as_int(v)));
#pragma unroll
    for (int t = 0; t < J; ++t) {
        const float s2 = acc[t] + vq * w.v[t];
        acc[t] = take ? s2 : acc[t];
    }
}

template <int J, bool kAll, int... Q>
__device__ __forceinline__ void BcastBatch(std::integer_sequence<int, Q...>, const char* sB, uint32_t laneOff, int off,
                                           float v, float acc[J])
{
    (BcastEntry<J, kAll, Q>(sB, laneOff, off, v, acc), ...);
}

// Entries first..15 of a batch whose columns are all in range (a row's last
// batch holds its entries in the top slots): wave-uniform branches, no selects.
template <int J, int Q>
__device__ __forceinline__ void BcastFrom(int first, const char* sB, uint32_t laneOff, int off, float v, float acc[J])
{
    if (first <= Q) BcastEntry<J, true, Q>(sB, laneOff, off, v, acc);
    if constexpr (Q < 15) BcastFrom<J, Q + 1>(first, sB, laneOff, off, v, acc);
}

// The small-k LDS kernel without compensation, entries handed out by DPP
// broadcasts instead of readlane: each 16-lane row of the wave loads the same
// 16 entries (column as an LDS byte offset, value), and entry q reaches every
// lane as the broadcast operand of the address add and of the multiplies.
// Per entry and lane: one address add, one LDS read of J columns, J
// multiplies and J adds.  Same tiles, rows and sums as SpmmOpLdsKernel.
template <typename RowT, bool kHalf, int J>
__global__ __launch_bounds__(kLdsThreads) __attribute__((amdgpu_waves_per_eu(J >= 4 ? 4 : 8))) void SpmmOpLdsBcastKernel(MmParams p)
{
    using T = typename Elem<kHalf>::T;
    extern __shared__ float sB[];
    constexpr int TW = kMmWave * J;
    constexpr int kBatch = 16;
    constexpr int kWindow = J >= 4 ? 5 : 4;  // batches loaded together (J = 4: rows of up to 80 entries in one)
    const T* val = static_cast<const T*>(p.val);
    const T* b = static_cast<const T*>(p.b);
    T* c = static_cast<T*>(p.c);
    const float alpha = p.alpha_ptr != nullptr ? *p.alpha_ptr : p.alpha;
    const float beta = p.beta_ptr != nullptr ? *p.beta_ptr : p.beta;
    const bool betaZero = beta == 0.0f;
    const int lane = static_cast<int>(threadIdx.x) & (kMmWave - 1);
    const int sub = lane & (kBatch - 1);
    const int wv = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x) / kMmWave);
    const int64_t tile = static_cast<int64_t>(blockIdx.x) % p.tiles;
    const int64_t chunk = static_cast<int64_t>(blockIdx.x) / p.tiles;
    const int64_t jt = tile * TW;
    const int k = static_cast<int>(p.k);
    const int64_t row0 = (chunk * (kLdsThreads / kMmWave) + wv) * kLdsRowsPerWave;
    const int nRows = static_cast<int>(p.m - row0 < kLdsRowsPerWave ? (p.m - row0 > 0 ? p.m - row0 : 0)
                                                                     : kLdsRowsPerWave);
    // A window of kWindow batches: lane sub of every 16-lane row holds slot
    // sub of each batch; a batch's entries fill its slots first..15.
    struct Window {
        int off[kWindow];
        float v[kWindow];
        int first[kWindow];
    };
    auto load = [&](int64_t e0, int64_t re, Window& w) {
#pragma unroll
        for (int q = 0; q < kWindow; ++q) {
            const int64_t left = re - (e0 + q * kBatch);
            w.first[q] = left >= kBatch ? 0 : left > 0 ? kBatch - static_cast<int>(left) : kBatch;
            const int64_t e = e0 + q * kBatch + sub - w.first[q];
            int32_t ci = -1;
            float x = 0.0f;
            if (sub >= w.first[q]) {
                ci = p.col[e] - p.base;
                x = Elem<kHalf>::Load(val, e);
            }
            w.off[q] = ci >= 0 && ci < k ? ci * (TW * 4) : static_cast<int>(0x80000000U);
            w.v[q] = x;
        }
    };
    StageBTile<kHalf, TW>(p, b, sB, jt, k);
    __syncthreads();
    const char* sBytes = reinterpret_cast<const char*>(sB);
    const uint32_t laneOff = static_cast<uint32_t>(lane * J * 4);
    const int64_t j0 = jt + lane * J;
    for (int rr = 0; rr < nRows; ++rr) {
        const int64_t row = row0 + rr;
        const int64_t rs = static_cast<int64_t>(ConstLoad<RowT>(p.rp, row)) - p.base;
        const int64_t re = static_cast<int64_t>(ConstLoad<RowT>(p.rp, row + 1)) - p.base;
        float acc[J], old[J];
#pragma unroll
        for (int q = 0; q < J; ++q) {
            acc[q] = 0.0f;
            old[q] = 0.0f;
        }
        if (j0 < p.n && !betaZero) SpmmLoadC<kHalf, J>(p, c, row, j0, old);
        for (int64_t e0 = rs; e0 < re; e0 += kBatch * kWindow) {
            Window cur;
            load(e0, re, cur);
#pragma unroll
            for (int q = 0; q < kWindow; ++q) {
                if (cur.first[q] == kBatch) break;  // wave-uniform: no entries left
                if (__ballot(cur.off[q] < 0 && sub >= cur.first[q]) == 0) {  // every entry of the batch taken
                    if (cur.first[q] == 0) {
                        BcastBatch<J, true>(std::make_integer_sequence<int, kBatch>{}, sBytes, laneOff, cur.off[q],
                                            cur.v[q], acc);
                    } else {
                        BcastFrom<J, 0>(cur.first[q], sBytes, laneOff, cur.off[q], cur.v[q], acc);
                    }
                } else {
                    BcastBatch<J, false>(std::make_integer_sequence<int, kBatch>{}, sBytes, laneOff, cur.off[q],
                                         cur.v[q], acc);
                }
            }
        }
        if (j0 < p.n) SpmmStore<kHalf, J>(p, c, row, j0, acc, alpha, beta, betaZero, old);
    }
}

// nnz == 0: C = beta * C_old (0 when beta == 0), every element of the m x n view.
template <bool kHalf>
__global__ __launch_bounds__(kMmThreads) void SpmmOpBetaCKernel(MmParams p)
{
    using T = typename Elem<kHalf>::T;
    T* c = static_cast<T*>(p.c);
    const float beta = p.beta_ptr != nullptr ? *p.beta_ptr : p.beta;
    const bool betaZero = beta == 0.0f;
    const int64_t total = p.m * p.n;
    for (int64_t t = static_cast<int64_t>(blockIdx.x) * kMmThreads + threadIdx.x; t < total;
         t += static_cast<int64_t>(gridDim.x) * kMmThreads) {
        int64_t idx;
        if (p.c_row) {
            idx = (t / p.n) * p.ldc + t % p.n;
        } else {
            idx = (t / p.m) * p.ldc + t % p.m;
        }
        const float o = betaZero ? 0.0f : beta * Elem<kHalf>::Load(c, idx);
        Elem<kHalf>::Store(c, idx, o);
    }
}

template <typename RowT, bool kHalf>
void Dispatch(const MmParams& p, int J, bool kahan, unsigned grid, hipStream_t s)
{
#define SPMM_LAUNCH(JJ, KK, WW) \
    hipLaunchKernelGGL((SpmmOpKernel<RowT, kHalf, KK, JJ, WW>), dim3(grid), dim3(kMmThreads), 0, s, p)
#define SPMM_NARROW(KK, NG) \
    hipLaunchKernelGGL((SpmmOpKernel<RowT, kHalf, KK, 4, false, NG>), dim3(grid), dim3(kMmThreads), 0, s, p)
    const bool wave = p.lg == 6;  // one row per wave
    if (J == 4 && (p.lg == 4 || p.lg == 5)) {  // 16 or 32 lanes of 4 columns per row
        if (kahan && !kHalf) SPMM_LAUNCH(4, true, false);
        else SPMM_LAUNCH(4, false, false);
    } else if (J == 4 && p.lg < 6) {  // narrow groups: 2, 4 or 8 lanes of 4 columns per row
        const bool k2 = kahan && !kHalf;
        if (p.lg == 1) { if (k2) SPMM_NARROW(true, 2); else SPMM_NARROW(false, 2); }
        else if (p.lg == 2) { if (k2) SPMM_NARROW(true, 4); else SPMM_NARROW(false, 4); }
        else { if (k2) SPMM_NARROW(true, 8); else SPMM_NARROW(false, 8); }
    } else if (kahan && !kHalf) {
        if (J == 4) SPMM_LAUNCH(4, true, true);
        else if (J == 2) SPMM_LAUNCH(2, true, true);
        else if (wave) SPMM_LAUNCH(1, true, true);
        else SPMM_LAUNCH(1, true, false);
    } else {
        if (J == 4) SPMM_LAUNCH(4, false, true);
        else if (J == 2) SPMM_LAUNCH(2, false, true);
        else if (wave) SPMM_LAUNCH(1, false, true);
        else SPMM_LAUNCH(1, false, false);
    }
#undef SPMM_LAUNCH
#undef SPMM_NARROW
}

template <typename RowT, bool kHalf>
void DispatchLds(const MmParams& p, int J, bool kahan, unsigned grid, unsigned lds, hipStream_t s)
{
#define SPMM_LDS(JJ, KK) \
    hipLaunchKernelGGL((SpmmOpLdsKernel<RowT, kHalf, KK, JJ>), dim3(grid), dim3(kLdsThreads), lds, s, p)
#define SPMM_BCAST(JJ) \
    hipLaunchKernelGGL((SpmmOpLdsBcastKernel<RowT, kHalf, JJ>), dim3(grid), dim3(kLdsThreads), lds, s, p)
    if (kahan && !kHalf) {
        if (J == 4) SPMM_LDS(4, true);
        else if (J == 2) SPMM_LDS(2, true);
        else SPMM_LDS(1, true);
    } else if (lds > static_cast<unsigned>(kLdsBytes)) {  // J = 4 over up to 128 KiB: one workgroup per CU
        // gfx950 allows 160 KiB per workgroup; the attribute is set once, and
        // a runtime that does not need it may decline it (the launch reports
        // real failures)
        static const bool once = [] {
            (void)hipFuncSetAttribute(reinterpret_cast<const void*>(&SpmmOpLdsBcastKernel<RowT, kHalf, 4>),
                                      hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(kLdsWideBytes));
            (void)hipGetLastError();
            return true;
        }();
        (void)once;
        SPMM_BCAST(4);
    } else {
        if (J == 4) SPMM_LDS(4, false);  // (the broadcast kernel spills at J = 4 and eight waves per SIMD)
        else if (J == 2) SPMM_BCAST(2);
        else SPMM_BCAST(1);
    }
#undef SPMM_LDS
#undef SPMM_BCAST
}

bool AlignedTo(const void* p, size_t a) { return reinterpret_cast<uintptr_t>(p) % a == 0; }

}  // namespace

int LaunchSpmmOp(const SpmmLaunch& l, void* stream)
{
    hipStream_t s = static_cast<hipStream_t>(stream);
    if (l.m <= 0 || l.n <= 0) return 0;
    MmParams p{};
    p.rp = l.row_offsets;
    p.col = l.col_ind;
    p.val = l.values;
    p.b = l.b;
    p.c = l.c;
    p.m = l.m;
    p.k = l.k;
    p.n = l.n;
    p.ldb = l.ldb;
    p.ldc = l.ldc;
    p.nnz = l.nnz;
    p.base = l.base;
    p.b_contig = (l.b_row_major != 0) != (l.b_trans != 0) ? 1 : 0;
    p.c_row = l.c_row_major;
    p.has_b = l.k > 0 ? 1 : 0;
    p.alpha = l.alpha;
    p.beta = l.beta;
    p.alpha_ptr = l.alpha_ptr;
    p.beta_ptr = l.beta_ptr;
    const size_t esz = l.fp16 ? 2 : 4;
    if (l.nnz == 0) {
        const int64_t total = l.m * l.n;
        int64_t g = (total + kMmThreads - 1) / kMmThreads;
        g = g > 65536 ? 65536 : g;
        if (l.fp16) hipLaunchKernelGGL(SpmmOpBetaCKernel<true>, dim3(static_cast<unsigned>(g)), dim3(kMmThreads), 0, s, p);
        else hipLaunchKernelGGL(SpmmOpBetaCKernel<false>, dim3(static_cast<unsigned>(g)), dim3(kMmThreads), 0, s, p);
        return 0;
    }
    const bool kahan = l.high_precision != 0;
    // small k: op(B) column tiles staged in LDS (n of at least one wave's width)
    if (l.k > 0 && l.n >= kMmWave && l.k * kMmWave * 4 <= kLdsBytes) {
        const int J = l.k * kMmWave * 4 * 4 <= (kahan ? kLdsBytes : kLdsWideBytes) ? 4
                      : l.k * kMmWave * 4 * 2 <= kLdsBytes                      ? 2
                                                                                : 1;
        const int64_t tw = int64_t{kMmWave} * J;
        p.tiles = (l.n + tw - 1) / tw;
        p.c_vec = l.c_row_major && l.ldc % J == 0 && AlignedTo(l.c, J * esz) ? 1 : 0;
        p.b_vec = l.ldb % 4 == 0 && AlignedTo(l.b, 4 * esz) ? 1 : 0;  // staging 4 elements per load
        const int64_t rowsPerBlock = int64_t{kLdsThreads / kMmWave} * kLdsRowsPerWave;
        const int64_t blocks = (l.m + rowsPerBlock - 1) / rowsPerBlock * p.tiles;
        if (blocks <= 0x7FFFFFFF) {
            const unsigned lds = static_cast<unsigned>(l.k * tw * 4);
            if (l.rowptr64) {
                if (l.fp16) DispatchLds<int64_t, true>(p, J, false, static_cast<unsigned>(blocks), lds, s);
                else DispatchLds<int64_t, false>(p, J, kahan, static_cast<unsigned>(blocks), lds, s);
            } else {
                if (l.fp16) DispatchLds<int32_t, true>(p, J, false, static_cast<unsigned>(blocks), lds, s);
                else DispatchLds<int32_t, false>(p, J, kahan, static_cast<unsigned>(blocks), lds, s);
            }
            return 0;
        }
    }
    // lanes per row (power of two) and columns per lane
    int J = 1, lg = 6;
    const int64_t bElems = p.b_contig ? (l.k - 1) * l.ldb + l.n : 0;
    const bool aligned4 = l.n % 4 == 0 && l.ldb % 4 == 0 && AlignedTo(l.b, 4 * esz);
    if (!l.fp16 && p.b_contig && p.has_b && l.n >= 8 && !aligned4 && bElems * 4 + 16 <= 0x7FFFFFFF &&
        AlignedTo(l.b, 4)) {
        // fp32 rows of op(B) that 16-byte loads cannot take aligned (a width
        // or leading dimension not a multiple of 4): 4 columns per lane by
        // buffer loads from 4-byte boundaries, 2 ... 64 lanes per row
        J = 4;
        lg = 1;
        while (lg < 6 && (int64_t{4} << lg) < l.n) ++lg;
        p.b_ubuf = 1;
        p.b_bytes = static_cast<int32_t>(bElems * 4);
        const int64_t cElems = (l.m - 1) * l.ldc + l.n;
        if (l.c_row_major && (l.ldc % 4 != 0 || !AlignedTo(l.c, 16)) && cElems * 4 + 16 <= 0x7FFFFFFF &&
            AlignedTo(l.c, 4)) {
            p.c_ubuf = 1;
            p.c_bytes = static_cast<int32_t>(cElems * 4);
        }
    } else if (l.n >= 8 && l.n % 4 == 0) {
        J = 4;  // 2, 4, ... 64 lanes of 4 columns per row
        lg = 1;
        while (lg < 6 && (int64_t{4} << lg) < l.n) ++lg;
    } else if (l.n > 2 * kMmWave) {
        J = 4;
    } else if (l.n > kMmWave) {
        J = 2;
    } else {
        while (lg > 0 && (int64_t{1} << (lg - 1)) >= l.n) --lg;
    }
    p.lg = lg;
    const int64_t tileCols = (int64_t{1} << lg) * J;
    const int64_t rpw = kMmWave >> lg;
    p.tiles = (l.n + tileCols - 1) / tileCols;
    p.waves = ((l.m + rpw - 1) / rpw) * p.tiles;
    p.b_vec = p.b_contig && l.ldb % J == 0 && AlignedTo(l.b, J * esz) ? 1 : 0;
    p.c_vec = l.c_row_major && l.ldc % J == 0 && AlignedTo(l.c, J * esz) ? 1 : 0;
    int64_t grid = (p.waves + kMmThreads / kMmWave - 1) / (kMmThreads / kMmWave);
    grid = grid > kMmMaxBlocks ? kMmMaxBlocks : grid;
    const unsigned g = static_cast<unsigned>(grid);
    if (l.rowptr64) {
        if (l.fp16) Dispatch<int64_t, true>(p, J, kahan, g, s);
        else Dispatch<int64_t, false>(p, J, kahan, g, s);
    } else {
        if (l.fp16) Dispatch<int32_t, true>(p, J, kahan, g, s);
        else Dispatch<int32_t, false>(p, J, kahan, g, s);
    }
    return 0;
}

}  // namespace aclsp
