// Device-side numeric helpers shared by the SpMV kernels (spmv_kernels.hip,
// spmv_staged_kernels.hip): value / accumulator / output types, the 16-bit
// conversions, the int8 saturating epilogue, alpha/beta loading and the
// row store y = alpha*sum + beta*y.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

#include "aclsparse_internal.h"

namespace aclsp {
namespace dev {

// ------------------------------ numeric types -------------------------------

struct C64 {
    float re, im;
};

__device__ __forceinline__ C64 operator+(C64 a, C64 b) { return {a.re + b.re, a.im + b.im}; }
// Each product and sum rounded as written (no fused multiply-add), so that
// every kernel that multiplies the same operands gets the same bits.
__device__ __forceinline__ C64 operator*(C64 a, C64 b)
{
#pragma clang fp contract(off)
    return {a.re * b.re - a.im * b.im, a.re * b.im + a.im * b.re};
}

template <AccKind A> struct AccOf;
template <> struct AccOf<AccKind::F32> { using T = float; };
template <> struct AccOf<AccKind::I64> { using T = long long; };
template <> struct AccOf<AccKind::C64> { using T = C64; };

template <ValKind V> struct ValOf;
template <> struct ValOf<ValKind::F32> { using T = float; };
template <> struct ValOf<ValKind::F16> { using T = uint16_t; };
template <> struct ValOf<ValKind::BF16> { using T = uint16_t; };
template <> struct ValOf<ValKind::I8> { using T = int8_t; };
template <> struct ValOf<ValKind::C64> { using T = C64; };
template <> struct ValOf<ValKind::UNIT> { using T = float; };  // the gathered "x" holds the products
template <> struct ValOf<ValKind::GATH> { using T = float; };  // int32 positions stream; fp32 values gathered

template <OutKind O> struct OutOf;
template <> struct OutOf<OutKind::F32> { using T = float; };
template <> struct OutOf<OutKind::F16> { using T = uint16_t; };
template <> struct OutOf<OutKind::BF16> { using T = uint16_t; };
template <> struct OutOf<OutKind::I32> { using T = int32_t; };
template <> struct OutOf<OutKind::C64> { using T = C64; };

template <typename T> __device__ __forceinline__ T Zero() { return T{}; }
__device__ __forceinline__ bool IsZero(float v) { return v == 0.0f; }
__device__ __forceinline__ bool IsZero(long long v) { return v == 0; }
__device__ __forceinline__ bool IsZero(C64 v) { return v.re == 0.0f && v.im == 0.0f; }

__device__ __forceinline__ float HalfToFloat(uint16_t h) { return static_cast<float>(__builtin_bit_cast(_Float16, h)); }
__device__ __forceinline__ float Bf16ToFloat(uint16_t b) { return __uint_as_float(static_cast<uint32_t>(b) << 16); }

// IEEE binary32 -> binary16, round to nearest, ties to even: the hardware
// conversion (overflow goes to inf, NaN stays NaN, results below the
// smallest normal half are rounded to subnormal halves: these kernels keep
// fp16 denormals).
__device__ __forceinline__ uint16_t FloatToHalfRne(float f)
{
    return __builtin_bit_cast(uint16_t, static_cast<_Float16>(f));
}

// binary32 -> bfloat16, round to nearest even; NaN stays NaN.
__device__ __forceinline__ uint16_t FloatToBf16Rne(float f)
{
    const uint32_t u = __float_as_uint(f);
    if ((u & 0x7F800000U) == 0x7F800000U && (u & 0x7FFFFFU) != 0U) {
        return static_cast<uint16_t>((u >> 16) | 0x0040U);
    }
    return static_cast<uint16_t>((u + 0x7FFFU + ((u >> 16) & 1U)) >> 16);
}

template <ValKind V, AccKind A>
__device__ __forceinline__ typename AccOf<A>::T ToAcc(typename ValOf<V>::T v)
{
    if constexpr (V == ValKind::F32) {
        if constexpr (A == AccKind::C64) return C64{v, 0.0f};
        else return v;
    } else if constexpr (V == ValKind::F16) {
        return HalfToFloat(v);
    } else if constexpr (V == ValKind::BF16) {
        return Bf16ToFloat(v);
    } else if constexpr (V == ValKind::I8) {
        if constexpr (A == AccKind::I64) return static_cast<long long>(v);
        else return static_cast<float>(v);
    } else {
        return v;
    }
}

template <OutKind O, AccKind A>
__device__ __forceinline__ typename AccOf<A>::T OutToAcc(typename OutOf<O>::T v)
{
    if constexpr (O == OutKind::F16) return HalfToFloat(v);
    else if constexpr (O == OutKind::BF16) return Bf16ToFloat(v);
    else if constexpr (O == OutKind::I32) return static_cast<long long>(v);
    else return v;
}

// INT8 products accumulate exactly in int64; the output saturates to int32
// while keeping cancellation between alpha*sum and beta*y
// (sparse/spmv/arch35/spmv_kernel.cpp:341-376).
__device__ __forceinline__ long long SaturateI32(long long v)
{
    return v > 2147483647LL ? 2147483647LL : v < -2147483648LL ? -2147483648LL : v;
}

__device__ __forceinline__ long long ScaledI64(long long sum, long long alpha, long long beta, long long oldY)
{
    const long long betaTerm = beta * oldY;
    if (alpha == 0) return SaturateI32(betaTerm);
    const long long mag = sum < 0 ? -sum : sum;
    const long long scale = alpha < 0 ? -alpha : alpha;
    const bool negative = (sum < 0) != (alpha < 0);
    // |alpha| <= 2^31, so mag * scale can only overflow int64 when mag >= 2^32;
    // the (slow, software) 64-bit division is taken only then
    if (mag >= (1LL << 32) && mag > 9223372036854775807LL / scale) return negative ? -2147483648LL : 2147483647LL;
    const long long prod = negative ? -(mag * scale) : mag * scale;
    if (prod > 2147483647LL - betaTerm) return 2147483647LL;
    if (prod < -2147483648LL - betaTerm) return -2147483648LL;
    return prod + betaTerm;
}

template <OutKind O, AccKind A>
__device__ __forceinline__ typename OutOf<O>::T FromAcc(typename AccOf<A>::T v)
{
    if constexpr (O == OutKind::F16) return FloatToHalfRne(v);
    else if constexpr (O == OutKind::BF16) return FloatToBf16Rne(v);
    else if constexpr (O == OutKind::I32) return static_cast<int32_t>(SaturateI32(v));
    else return v;
}

// ------------------------------- scalars ------------------------------------

struct Scalars {
    int32_t device;
    float alpha_re, alpha_im, beta_re, beta_im;
    int32_t alpha_i, beta_i;
    const void* alpha_ptr;
    const void* beta_ptr;
};

template <AccKind A>
__device__ __forceinline__ void LoadScalars(const Scalars& s, typename AccOf<A>::T& alpha,
                                            typename AccOf<A>::T& beta)
{
    if constexpr (A == AccKind::I64) {
        alpha = s.device ? *static_cast<const int32_t*>(s.alpha_ptr) : s.alpha_i;
        beta = s.device ? *static_cast<const int32_t*>(s.beta_ptr) : s.beta_i;
    } else if constexpr (A == AccKind::C64) {
        if (s.device) {
            const float* a = static_cast<const float*>(s.alpha_ptr);
            const float* b = static_cast<const float*>(s.beta_ptr);
            alpha = C64{a[0], a[1]};
            beta = C64{b[0], b[1]};
        } else {
            alpha = C64{s.alpha_re, s.alpha_im};
            beta = C64{s.beta_re, s.beta_im};
        }
    } else {
        alpha = s.device ? *static_cast<const float*>(s.alpha_ptr) : s.alpha_re;
        beta = s.device ? *static_cast<const float*>(s.beta_ptr) : s.beta_re;
    }
}

// y[idx] = alpha*sum + beta*oldY, oldY being y[idx] as the caller read it
// (unused when beta == 0).
template <OutKind O, AccKind A>
__device__ __forceinline__ void StoreRowOld(typename OutOf<O>::T* y, int64_t idx, typename AccOf<A>::T sum,
                                            typename AccOf<A>::T alpha, typename AccOf<A>::T beta, bool betaNz,
                                            typename AccOf<A>::T oldY)
{
    using Acc = typename AccOf<A>::T;
    Acc r;
    if constexpr (A == AccKind::I64) {
        r = ScaledI64(sum, alpha, beta, oldY);
    } else {
        r = betaNz ? alpha * sum + beta * oldY : alpha * sum;
    }
    y[idx] = FromAcc<O, A>(r);
}

// y = alpha*sum + beta*y; y is not read when beta == 0
// (sparse/spmv/arch35/spmv_kernel.cpp:341-345,544-552).
template <OutKind O, AccKind A>
__device__ __forceinline__ void StoreRow(typename OutOf<O>::T* y, int64_t idx, typename AccOf<A>::T sum,
                                         typename AccOf<A>::T alpha, typename AccOf<A>::T beta, bool betaNz)
{
    using Acc = typename AccOf<A>::T;
    StoreRowOld<O, A>(y, idx, sum, alpha, beta, betaNz, betaNz ? OutToAcc<O, A>(y[idx]) : Zero<Acc>());
}

}  // namespace dev
}  // namespace aclsp
