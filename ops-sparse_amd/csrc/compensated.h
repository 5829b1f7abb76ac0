// Doubly compensated fp32 accumulation shared by the SpMVOp kernels.
//
// Priest's triple (hi, md, lo): each product is split exactly by an FMA
// (TwoProduct), the high part is added to hi by TwoSum, the rounding error
// of that sum plus the product's error is added to md by a second TwoSum,
// and the last error collects in lo (the recurrence of
// sparse/spmv_op/arch35/spmv_op_kernel.cpp:100-124).  Every function turns
// off FP contraction in its own body: fusing a*b + c into an FMA breaks the
// error-free transformations, whatever the including file's setting.
#pragma once

#include <hip/hip_runtime.h>

namespace aclsp {

struct Triple {
    float hi, md, lo;
};

__device__ __forceinline__ void TwoSum(float a, float b, float& s, float& e)
{
#pragma clang fp contract(off)
    s = a + b;
    const float v = s - a;
    e = (a - (s - v)) + (b - v);
}

// Adds the exact product prod + err (err = a*b - prod) to the triple.
__device__ __forceinline__ void PriestAddSplit(Triple& t, float prod, float err)
{
#pragma clang fp contract(off)
    float s1, e1;
    TwoSum(t.hi, prod, s1, e1);
    t.hi = s1;
    const float ee = e1 + err;
    float s2, e2;
    TwoSum(t.md, ee, s2, e2);
    t.md = s2;
    t.lo = t.lo + e2;
}

// Adds a*b to the triple.
__device__ __forceinline__ void PriestAdd(Triple& t, float a, float b)
{
#pragma clang fp contract(off)
    const float prod = a * b;
    PriestAddSplit(t, prod, __fmaf_rn(a, b, -prod));
}

// Merges two triples keeping the rounding error of both leading sums.
__device__ __forceinline__ Triple Merge(const Triple& a, const Triple& b)
{
#pragma clang fp contract(off)
    Triple r;
    float e1, e2;
    TwoSum(a.hi, b.hi, r.hi, e1);
    float m;
    TwoSum(a.md, b.md, m, e2);
    float e3;
    TwoSum(m, e1, r.md, e3);
    r.lo = a.lo + b.lo + e2 + e3;
    return r;
}

__device__ __forceinline__ Triple ShflXor(const Triple& t, int m)
{
    return Triple{__shfl_xor(t.hi, m, 64), __shfl_xor(t.md, m, 64), __shfl_xor(t.lo, m, 64)};
}

__device__ __forceinline__ Triple Shfl(const Triple& t, int src)
{
    return Triple{__shfl(t.hi, src, 64), __shfl(t.md, src, 64), __shfl(t.lo, src, 64)};
}

// z = a*(hi + md + lo) + b*y.  The reference folds this as
// fma(a, hi, fma(a, md + lo, b*y)) (spmv_op_kernel.cpp:177-181), whose inner
// rounding happens at the magnitude of b*y: when A*x nearly cancels y the
// relative error of z grows without bound.  Here both leading products are
// split exactly (TwoProduct by FMA) and added by TwoSum, so z is rounded
// once at its own magnitude, up to the small tail terms.  Non-finite terms
// keep the reference's fold so Inf/NaN propagate alike.  yv must be 0 when
// b == 0 (y is then not read).
__device__ __forceinline__ float CombineZ(const Triple& t, float a, float b, float yv)
{
#pragma clang fp contract(off)
    const float p1 = a * t.hi;
    const float e1 = __fmaf_rn(a, t.hi, -p1);
    const float p2 = b * yv;
    const float e2 = __fmaf_rn(b, yv, -p2);
    float s, es;
    TwoSum(p1, p2, s, es);
    const float tail = __fmaf_rn(a, t.md + t.lo, es + (e1 + e2));
    return __builtin_isfinite(s) ? s + tail : __fmaf_rn(a, t.hi, __fmaf_rn(a, t.md + t.lo, p2));
}

}  // namespace aclsp
