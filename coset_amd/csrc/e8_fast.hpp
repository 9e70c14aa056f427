// e8_fast.hpp -- fast path of the core E8 projection used by the encoders.
//
// project<false, false> (e8_core.hpp) restates the reference fp32 sequence
// (coset/core/e8/lattice.py:67-169): custom_round, the core g_x parity fix,
// and the comparison of two correctly rounded norms.  Away from ties the same
// result follows from cheaper operations; project_fast computes it that way
// and reports whether every condition below held.  When it returns false the
// caller runs the exact sequence, so results are bit-identical either way.
//
// Conditions and why they suffice (t - rint t is exact in fp32 for |t| < 2^22):
//   (1) max |x_i| < 2^21.
//   (2) |x_i - rint x_i| < 1/2 - 2^-20 for all i.  Then custom_round(x_i) =
//       rint(x_i) (checked for every float |t| < 2^22 by the CPU test), so the
//       D8 candidate rounds to f0 = rint(x) and d0 = x - f0 is the reference's
//       exact |t - f| used by argmax.
//   (3) |fl(x_i - 1/2) - floor x_i| < 1/2 - 2^-20.  Then floor(x_i) is the
//       integer nearest to t = fl(x_i - 1/2), so custom_round(t) = rint(t) =
//       floor(x_i): the D8 + 1/2 candidate rounds to f1 = floor(x), and
//       d1 = t - f1 is again exact.
//   (4) The two squared distances, evaluated as sum d^2 (+ 1 - 2 adj d_k for
//       the flipped coordinate) with fused multiply-adds, differ by more than
//       2^-14.  For the D8 + 1/2 candidate the terms use |x - f1 - 1/2| =
//       1/2 - |d0| (equal as reals under (2)).  Both evaluations and the
//       reference's rounded sums of rounded squares stay within 140 ulp(1)
//       of the exact sums (all terms are below 5), and a gap of 2^-14 also
//       keeps the correctly rounded square roots apart, so the reference's
//       strict comparison has the same outcome.
// NaN or infinite inputs fail (1) or (4).
#pragma once

#include <hip/hip_runtime.h>
#include <math.h>

namespace coset {

constexpr float kFastMaxAbs = 2097152.0f;              // 2^21
constexpr float kFastTieLimit = 0.5f - 9.5367431640625e-07f;  // 1/2 - 2^-20
constexpr float kFastDistGap = 6.103515625e-05f;        // 2^-14

// Core-rule E8 closest point of x (contiguous distance rule).  Returns false
// when a condition above fails; y is then unspecified.
__host__ __device__ inline bool project_fast(const float x[8], float y[8])
{
    float f0[8], d0[8], f1[8], d1[8];
    float m = 0.f, best0 = 0.f, best1 = 0.f, s0 = 0.f, s1 = 0.f, a = 0.f, b = 0.f;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        f0[i] = rintf(x[i]);
        d0[i] = x[i] - f0[i];
        f1[i] = floorf(x[i]);
        d1[i] = (x[i] - 0.5f) - f1[i];
        m = fmaxf(m, fabsf(x[i]));
        best0 = fmaxf(best0, fabsf(d0[i]));
        best1 = fmaxf(best1, fabsf(d1[i]));
        s0 += f0[i];
        s1 += f1[i];
        a = fmaf(d0[i], d0[i], a);
        // x - floor(x) - 1/2 = d0 - 1/2 (d0 > 0) or d0 + 1/2 (d0 < 0) under
        // (2): its magnitude is 1/2 - |d0|, exact up to one rounding
        const float e = 0.5f - fabsf(d0[i]);
        b = fmaf(e, e, b);
    }
    bool ok = m < kFastMaxAbs && best0 < kFastTieLimit && best1 < kFastTieLimit;

    // first index of the largest |d| (torch.argmax): scan from the back
    bool first0[8], first1[8];
    float xk0 = x[0], xk1 = x[0];
    bool seen0 = false, seen1 = false;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        bool h0 = fabsf(d0[i]) == best0, h1 = fabsf(d1[i]) == best1;
        first0[i] = h0 && !seen0;
        first1[i] = h1 && !seen1;
        seen0 = seen0 || h0;
        seen1 = seen1 || h1;
        xk0 = first0[i] ? x[i] : xk0;
        xk1 = first1[i] ? x[i] : xk1;
    }
    // the worst coordinates' differences, recomputed from x_k
    const float dk0 = xk0 - rintf(xk0);
    const float fk1 = floorf(xk1);
    const float tk1 = xk1 - 0.5f;
    const float dk1 = tk1 - fk1;
    const float ek1 = (xk1 - fk1) - 0.5f;  // within 2^-25 of x_k - (f_k + 1/2)
    // core g_x: an odd coordinate sum moves the worst coordinate by +1 when
    // t_k >= 0 and f_k < t_k (d_k > 0), by -1 otherwise
    const bool odd0 = ((int)s0 & 1) != 0, odd1 = ((int)s1 & 1) != 0;
    const float adj0 = odd0 ? ((xk0 >= 0.f && dk0 > 0.f) ? 1.f : -1.f) : 0.f;
    const float adj1 = odd1 ? ((tk1 >= 0.f && dk1 > 0.f) ? 1.f : -1.f) : 0.f;

    // (d - adj)^2 = d^2 - 2 adj d + adj^2, adj^2 = |adj|
    a += fmaf(-2.f * adj0, dk0, fabsf(adj0));
    b += fmaf(-2.f * adj1, ek1, fabsf(adj1));
    const bool pick0 = b - a > kFastDistGap;
    ok = ok && (pick0 || a - b > kFastDistGap);

    const float adj = pick0 ? adj0 : adj1;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const bool at_k = pick0 ? first0[i] : first1[i];
        const float base = pick0 ? f0[i] : f1[i] + 0.5f;
        // adding the (possibly zero) adjustment also turns rint's -0 into +0
        y[i] = base + (at_k ? adj : 0.f);
    }
    return ok;
}

// custom_round (coset/core/base.py:179-202): floor((x - sign(x) eps) + 1/2)
// in fp32, for host and device.
__host__ __device__ inline float custom_round_hd(float x)
{
    const float y = x - copysignf(1.1920928955078125e-07f, x);
    return floorf(y + 0.5f);
}

// Exact core-rule E8 projection of a block whose coordinates are multiples
// of 2^-6 with |x| < 8 -- the decoders' input G b / q for q = 2^k <= 32.
// For such blocks every difference, square and sum of the reference's
// projection is exact in fp32, so the reference's comparison of correctly
// rounded norms is the exact comparison a < b of the squared distances
// (distinct sums differ by >= 2^-12, far above the roots' rounding), and the
// contiguous and batched distance rules coincide.  custom_round, the
// first-index argmax and the core g_x step are the reference's.
__host__ __device__ inline void project_dyadic(const float x[8], float y[8])
{
    float f0[8], d0[8], t1[8], f1[8], d1[8];
    float best0 = 0.f, best1 = 0.f, s0 = 0.f, s1 = 0.f, a = 0.f, b = 0.f;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        f0[i] = custom_round_hd(x[i]);
        d0[i] = x[i] - f0[i];
        t1[i] = x[i] - 0.5f;
        f1[i] = custom_round_hd(t1[i]);
        d1[i] = t1[i] - f1[i];
        best0 = fmaxf(best0, fabsf(d0[i]));
        best1 = fmaxf(best1, fabsf(d1[i]));
        s0 += f0[i];
        s1 += f1[i];
        a = fmaf(d0[i], d0[i], a);
        b = fmaf(d1[i], d1[i], b);
    }
    bool first0[8], first1[8];
    float xk0 = x[0], dk0 = d0[0], tk1 = t1[0], dk1 = d1[0];
    bool seen0 = false, seen1 = false;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const bool h0 = fabsf(d0[i]) == best0, h1 = fabsf(d1[i]) == best1;
        first0[i] = h0 && !seen0;
        first1[i] = h1 && !seen1;
        seen0 = seen0 || h0;
        seen1 = seen1 || h1;
        xk0 = first0[i] ? x[i] : xk0;
        dk0 = first0[i] ? d0[i] : dk0;
        tk1 = first1[i] ? t1[i] : tk1;
        dk1 = first1[i] ? d1[i] : dk1;
    }
    const bool odd0 = ((int)s0 & 1) != 0, odd1 = ((int)s1 & 1) != 0;
    const float adj0 = odd0 ? ((xk0 >= 0.f && dk0 > 0.f) ? 1.f : -1.f) : 0.f;
    const float adj1 = odd1 ? ((tk1 >= 0.f && dk1 > 0.f) ? 1.f : -1.f) : 0.f;
    // (d - adj)^2 = d^2 - 2 adj d + |adj|, all exact here
    a += fmaf(-2.f * adj0, dk0, fabsf(adj0));
    b += fmaf(-2.f * adj1, dk1, fabsf(adj1));
    const bool pick0 = a < b;  // ties go to D8 + 1/2, as the reference's strict <
    const float adj = pick0 ? adj0 : adj1;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const bool at_k = pick0 ? first0[i] : first1[i];
        const float base = pick0 ? f0[i] : f1[i] + 0.5f;
        y[i] = base + (at_k ? adj : 0.f);
    }
}

}  // namespace coset
