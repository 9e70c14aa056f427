// fastdiv.hpp -- exact division shortcuts for divisors shared by many
// quotients (host and device).
#pragma once

#include <hip/hip_runtime.h>
#include <math.h>
#include <stdint.h>

namespace coset {

// a / b rounded to nearest even, from y = RN(1/b) (one correctly rounded
// reciprocal shared by many quotients): q = RN(a y), then STEPS times
// q <- RN(q + RN(a - b q) y), each a single fused operation.
// Domain: b, y, a / b and every residual in the normal range -- the callers
// take 2^-64 <= |b| <= 2^64 and a = 0 or 1/2 <= |a| <= 2^46.  Scaling a and
// b by powers of two changes nothing there, so take b in [1, 2):
//  - q0 = RN(a y) is within 1.5 ulp of a / b (|y - 1/b| <= 2^-25), so after
//    the first step, whose residual is a - b q0 to 2^-24 relative, q1 is
//    within 1/2 ulp + 2^-22 ulp of a / b: a faithful rounding;
//  - for a faithful q1 the residual a - b q1 is exact (a multiple of
//    ulp(q1) 2^-23 below 2 ulp(q1)), and RN(q1 + r y) = RN(a / b)
//    (Markstein's theorem: q1 + r y is within |r| 2^-25 of a / b, less than
//    the distance from a / b to the nearest midpoint, which a quotient of
//    two 24-bit significands never equals).
// So STEPS = 2 is exact on the whole domain.  STEPS = 1 is exact where q0 is
// already faithful; the CPU checker (tests/fastpath, divq) finds it exact for
// every b significand and every half-integer |a| <= 16384, which bounds the
// decoded sums of q = 8 with M <= 4 and q = 16 with M <= 3 (a level's
// residual coordinates are at most 3q/2 in magnitude: 12 (1 + 8 + 64 + 512)
// and 24 (1 + 16 + 256) are below 7100).
// a = -0 with b > 0 gives +0 (the callers' a is never -0: sums that start at
// +0 and add with round-to-nearest).
template <int STEPS>
__host__ __device__ inline float div_by_recip(float a, float b, float y)
{
    float q = a * y;
#pragma unroll
    for (int s = 0; s < STEPS; ++s) q = fmaf(fmaf(-q, b, a), y, q);
    return q;
}

// floor(n / d) for 32-bit n and a divisor d >= 1 fixed per launch, from a
// multiplier and shift computed once on the host (Granlund and Montgomery,
// "Division by invariant integers using multiplication", 1994, Thm. 4.2):
// with l = ceil(log2 d) and m = floor(2^(32 + l) / d) + 1, 2^(32+l) < m d <=
// 2^(32+l) + 2^l, so floor(n / d) = floor(m n / 2^(32+l)) for every n < 2^32;
// m = 2^32 + magic, and floor(m n / 2^(32+l)) = (umulhi(magic, n) + n) >> l
// in 64-bit arithmetic.
struct U32Div {
    uint32_t magic;
    uint32_t shift;
};

__host__ __device__ inline U32Div u32div_of(uint32_t d)
{
    uint32_t l = 0;
    while (l < 32 && (1ull << l) < d) ++l;
    U32Div r;
    r.magic = (uint32_t)((((1ull << l) - d) << 32) / d + 1);
    r.shift = l;
    return r;
}

__host__ __device__ inline uint32_t u32div(uint32_t n, U32Div dv)
{
    const uint32_t hi = (uint32_t)(((uint64_t)dv.magic * n) >> 32);
    return (uint32_t)(((uint64_t)hi + n) >> dv.shift);
}

}  // namespace coset
