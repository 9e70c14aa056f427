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
//   (4) The two squared distances a (D8) and b (D8 + 1/2) differ by more
//       than 2^-14, with b - a evaluated as 2 - sum |d0| (+ |adj1| -
//       2 adj1 e_k1 - |adj0| + 2 adj0 d0_k for the flipped coordinates):
//       x_i - f1_i - 1/2 = d0_i -+ 1/2 as reals under (2) and (3), and
//       (1/2 - |d0_i|)^2 - d0_i^2 = 1/4 - |d0_i|.  This evaluation (within
//       12 ulp(1)) and the reference's rounded sums of rounded squares
//       (within 140 ulp(1) of the exact sums, all terms are below 5) keep
//       a gap of 2^-14 from reversing the reference's strict comparison, and
//       the gap also keeps the correctly rounded square roots apart.
// Under (2) and (3) floor x_i = rint x_i - [d0_i < 0] (d0_i = 0 fails (3)),
// so the parity of sum floor x is that of sum rint x plus the number of
// negative d0_i.
// NaN or infinite inputs fail (1) or (4).
//
// Where (3) fails (a coordinate within 2^-20 of an integer: exact zeros, and
// every coordinate of a block with max |x_i| < 2^-20) the D8 + 1/2 candidate's
// rounding is the reference's tie rule, which the fast path does not restate.
// The D8 candidate, which needs only (1) and (2), is still the answer when
//   (5) 2 - sum |d0_i| - (|adj0| - 2 adj0 d0_k) > 2^-14:
// every point of D8 + 1/2 -- the reference's candidate with or without its
// parity adjustment -- has half-integer coordinates, so its squared distance
// from x is at least sum (1/2 - |d0_i|)^2 = a + 2 - sum |d0_i| (as reals,
// |d0_i| <= 1/2 under (2)), which exceeds the adjusted D8 distance by the
// left side of (5); the evaluation and rounding bounds of (4) apply
// unchanged.  Callers that take (5) (CLEAR_D8) accept such blocks with the
// D8 rows; blocks with max |x_i| < 1/8, whose every level encodes to 0, are
// among them.
#pragma once

#include <hip/hip_runtime.h>
#include <math.h>
#include <stdint.h>

namespace coset {

constexpr float kFastMaxAbs = 2097152.0f;              // 2^21
constexpr float kFastTieLimit = 0.5f - 9.5367431640625e-07f;  // 1/2 - 2^-20
constexpr float kFastDistGap = 6.103515625e-05f;        // 2^-14

// Lane conditions as masks.  On the device a mask is the wave's 64-bit
// ballot: the first-index scan and the choice between the two candidates'
// masks are then scalar operations, and a mask is read back per lane for
// free (a per-lane select of two booleans costs five vector operations
// there).  On the host a mask is all ones or zero, with the same algebra.
typedef uint64_t lanes_t;

__host__ __device__ inline lanes_t lanes_of(bool c)
{
#if defined(__HIP_DEVICE_COMPILE__)
    return __builtin_amdgcn_ballot_w64(c);
#else
    return c ? ~0ull : 0ull;
#endif
}

__host__ __device__ inline bool lane_in(lanes_t m)
{
#if defined(__HIP_DEVICE_COMPILE__)
    return __builtin_amdgcn_inverse_ballot_w64(m);
#else
    return m != 0ull;
#endif
}

// The decision of the fast path: both candidates' integer parts, the first
// index of each one's worst coordinate, each one's parity adjustment and
// which candidate is closer.  Returns false when a condition above fails.
struct FastChoice {
    float f0[8];        // rint(x): the D8 candidate before its adjustment
    float f1[8];        // floor(x): the D8 + 1/2 candidate is f1 + 1/2
    lanes_t first0[8];  // worst coordinate of each candidate (first index)
    lanes_t first1[8];
    float adj0, adj1;   // -1, 0 or +1 added at that coordinate
    lanes_t pick0;      // the D8 candidate is the closer one
};

// Condition (1).  Callers that know a bound on |x| pass it to fast_choose.
__host__ __device__ inline bool fast_in_range(const float x[8])
{
    float m = fabsf(x[0]);
#pragma unroll
    for (int i = 1; i < 8; ++i) m = fmaxf(m, fabsf(x[i]));
    return m < kFastMaxAbs;
}

template <bool CLEAR_D8 = false>
__host__ __device__ inline bool fast_choose(const float x[8], FastChoice& c, bool in_range)
{
    float d0[8], d1[8];
    float best0 = 0.f, best1 = 0.f, s0, sa;
    uint32_t neg = 0u;  // sign bits of d0, xor-ed
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        c.f0[i] = rintf(x[i]);
        d0[i] = x[i] - c.f0[i];
        c.f1[i] = floorf(x[i]);
        d1[i] = (x[i] - 0.5f) - c.f1[i];
        best0 = fmaxf(best0, fabsf(d0[i]));
        best1 = fmaxf(best1, fabsf(d1[i]));
        neg ^= __builtin_bit_cast(uint32_t, d0[i]);
        if (i == 0) {
            s0 = c.f0[0];
            sa = fabsf(d0[0]);
        } else {
            s0 += c.f0[i];
            sa += fabsf(d0[i]);
        }
    }
    const bool tie0 = best0 < kFastTieLimit, tie1 = best1 < kFastTieLimit;  // (2), (3)

    // first index of the largest |d| (torch.argmax)
    float xk0 = x[0], xk1 = x[0];
    lanes_t seen0 = 0ull, seen1 = 0ull;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const lanes_t h0 = lanes_of(fabsf(d0[i]) == best0), h1 = lanes_of(fabsf(d1[i]) == best1);
        c.first0[i] = h0 & ~seen0;
        c.first1[i] = h1 & ~seen1;
        seen0 |= h0;
        seen1 |= h1;
        xk0 = lane_in(c.first0[i]) ? x[i] : xk0;
        xk1 = lane_in(c.first1[i]) ? x[i] : xk1;
    }
    // the worst coordinates' differences, recomputed from x_k
    const float dk0 = xk0 - rintf(xk0);
    const float fk1 = floorf(xk1);
    const float tk1 = xk1 - 0.5f;
    const float dk1 = tk1 - fk1;
    const float ek1 = (xk1 - fk1) - 0.5f;  // within 2^-25 of x_k - (f_k + 1/2)
    // core g_x: an odd coordinate sum moves the worst coordinate by +1 when
    // t_k >= 0 and f_k < t_k (d_k > 0), by -1 otherwise
    const bool odd0 = ((int)s0 & 1) != 0, odd1 = odd0 != ((neg >> 31) != 0u);
    c.adj0 = odd0 ? ((xk0 >= 0.f && dk0 > 0.f) ? 1.f : -1.f) : 0.f;
    c.adj1 = odd1 ? ((tk1 >= 0.f && dk1 > 0.f) ? 1.f : -1.f) : 0.f;

    // b - a, with (d - adj)^2 - d^2 = adj^2 - 2 adj d and adj^2 = |adj|
    const float base = 2.f - sa;
    const float t0 = fmaf(-2.f * c.adj0, dk0, fabsf(c.adj0));
    const float diff = base + (fmaf(-2.f * c.adj1, ek1, fabsf(c.adj1)) - t0);
    const bool pick0 = diff > kFastDistGap;
    c.pick0 = lanes_of(pick0);
    const bool decided = tie1 && (pick0 || diff < -kFastDistGap);
    if constexpr (CLEAR_D8) {
        // (5); it implies pick0: the adj1 term is >= 0 (ek1 in [-1/2, 1/2)),
        // so diff >= base - t0 in rounded arithmetic too
        return in_range && tie0 && (decided || base - t0 > kFastDistGap);
    }
    return in_range && tie0 && decided;
}

// The chosen candidate's worst coordinate, as a lane mask.
__host__ __device__ inline lanes_t fast_at(const FastChoice& c, int i)
{
    return (c.pick0 & c.first0[i]) | (~c.pick0 & c.first1[i]);
}

// Core-rule E8 closest point of x (contiguous distance rule).  Returns false
// when a condition above fails; y is then unspecified.
__host__ __device__ inline bool project_fast(const float x[8], float y[8])
{
    FastChoice c;
    const bool ok = fast_choose(x, c, fast_in_range(x));
    const bool pick0 = lane_in(c.pick0);
    const float adj = pick0 ? c.adj0 : c.adj1;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const float base = pick0 ? c.f0[i] : c.f1[i] + 0.5f;
        // adding the (possibly zero) adjustment also turns rint's -0 into +0
        y[i] = base + (lane_in(fast_at(c, i)) ? adj : 0.f);
    }
    return ok;
}

// The rows of G^-1 y (coset/core/base.py:134-155) for the point project_fast
// chooses, without forming y.  With Y the chosen candidate's integer part
// after the adjustment (y = Y, or Y + 1/2 on the D8 + 1/2 coset):
//   (G^-1 y)_r = sum_{j = r..6} (Y_j - Y_7)        r = 1..6
//   (G^-1 y)_0 = sum_{j = 0..6} (Y_j - Y_7) / 2    (an even sum for y in E8)
//   (G^-1 y)_7 = 2 Y_7 (+ 1 on the coset)
// all exact in int32 under condition (1).  The adjustment enters the sums
// through the single term j = k.  Returns false exactly when project_fast
// does (in_range = fast_in_range(x)), or with CLEAR_D8 when neither (3) nor
// (5) decides the block; rows are then unspecified.
template <bool CLEAR_D8 = false>
__host__ __device__ inline bool fast_rows(const float x[8], int rows[8], bool in_range)
{
    FastChoice c;
    const bool ok = fast_choose<CLEAR_D8>(x, c, in_range);
    const bool pick0 = lane_in(c.pick0);
    const uint32_t adj = (uint32_t)(int)(pick0 ? c.adj0 : c.adj1);
    uint32_t Y[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) Y[i] = (uint32_t)(int)(pick0 ? c.f0[i] : c.f1[i]);
    const uint32_t y7 = Y[7] + (lane_in(fast_at(c, 7)) ? adj : 0u);
    const uint32_t n7 = 0u - y7, n7a = n7 + adj;  // -Y_7, and -Y_7 + adj for j = k
    uint32_t w = 0u;                               // wrapping sums: no signed overflow on failed lanes
#pragma unroll
    for (int r = 6; r >= 1; --r) {
        w += Y[r] + (lane_in(fast_at(c, r)) ? n7a : n7);
        rows[r] = (int)w;
    }
    w += Y[0] + (lane_in(fast_at(c, 0)) ? n7a : n7);
    rows[0] = (int)w >> 1;
    rows[7] = (int)(2u * y7 + (pick0 ? 0u : 1u));
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
    float f0[8], d0[8], f1[8], d1[8];
    float best0 = 0.f, best1 = 0.f, s0, s1, a, b;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        f0[i] = custom_round_hd(x[i]);
        d0[i] = x[i] - f0[i];
        const float t1 = x[i] - 0.5f;
        f1[i] = custom_round_hd(t1);
        d1[i] = t1 - f1[i];
        best0 = fmaxf(best0, fabsf(d0[i]));
        best1 = fmaxf(best1, fabsf(d1[i]));
        s0 = i == 0 ? f0[0] : s0 + f0[i];
        s1 = i == 0 ? f1[0] : s1 + f1[i];
        a = i == 0 ? d0[0] * d0[0] : fmaf(d0[i], d0[i], a);
        b = i == 0 ? d1[0] * d1[0] : fmaf(d1[i], d1[i], b);
    }
    // first index of each candidate's largest |d| as lane masks, and x at it
    lanes_t first0[8], first1[8], seen0 = 0ull, seen1 = 0ull;
    float xk0 = x[0], xk1 = x[0];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const lanes_t h0 = lanes_of(fabsf(d0[i]) == best0), h1 = lanes_of(fabsf(d1[i]) == best1);
        first0[i] = h0 & ~seen0;
        first1[i] = h1 & ~seen1;
        seen0 |= h0;
        seen1 |= h1;
        xk0 = lane_in(first0[i]) ? x[i] : xk0;
        xk1 = lane_in(first1[i]) ? x[i] : xk1;
    }
    // the worst coordinates' differences, recomputed from x_k (same operations)
    const float dk0 = xk0 - custom_round_hd(xk0);
    const float tk1 = xk1 - 0.5f;
    const float dk1 = tk1 - custom_round_hd(tk1);
    const bool odd0 = ((int)s0 & 1) != 0, odd1 = ((int)s1 & 1) != 0;
    const float adj0 = odd0 ? ((xk0 >= 0.f && dk0 > 0.f) ? 1.f : -1.f) : 0.f;
    const float adj1 = odd1 ? ((tk1 >= 0.f && dk1 > 0.f) ? 1.f : -1.f) : 0.f;
    // (d - adj)^2 = d^2 - 2 adj d + |adj|, all exact here
    a += fmaf(-2.f * adj0, dk0, fabsf(adj0));
    b += fmaf(-2.f * adj1, dk1, fabsf(adj1));
    const bool pick0 = a < b;  // ties go to D8 + 1/2, as the reference's strict <
    const lanes_t p0 = lanes_of(pick0);
    const float adj = pick0 ? adj0 : adj1;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const lanes_t at = (p0 & first0[i]) | (~p0 & first1[i]);
        const float base = pick0 ? f0[i] : f1[i] + 0.5f;
        y[i] = base + (lane_in(at) ? adj : 0.f);
    }
}

// The decoders' residual of one level, r = G b - q P(G b / q)
// (coset/core/e8/codecs.py:164-166, core rule), for q = 8, 16, 32 straight
// from the digits b_j in [0, q), in fewer operations than project_dyadic.
//
// z = G b / q = Z / (2q) with Z = 2 G b an integer: Z_0 = 4 b_0 - 2 b_1 + b_7,
// Z_i = 2 (b_i - b_i+1) + b_7 (i = 1..5), Z_6 = 2 b_6 + b_7, Z_7 = b_7, so
// -2q < Z_i < 5q and -1 < z_i < 5/2.  On this grid (steps of 1/(2q)):
//  - custom_round's ties are z in {-1/2, 1/2, 3/2} for the D8 candidate and
//    z - 1/2 in {-1/2, 1/2, 3/2} for D8 + 1/2, all of magnitude below 2,
//    where it rounds toward zero (its 2^-23 nudge is exact there); so the D8
//    candidate is f0 = trunc(z + copysign(1/2 - 1/(4q), z)) and the D8 + 1/2
//    candidate's integer part is f1 = floor(z) but z - 1 for the integers
//    z >= 1, i.e. floor(z - 1/(4q)) for z > 0 and floor(z + 1/(4q)) for z <= 0;
//  - with d0 = z - f0 in [-1/2, 1/2] and d1 = z - 1/2 - f1, |d1_i| =
//    1/2 - |d0_i| exactly, so the first argmax of |d1| (torch.argmax) is the
//    first argmin of |d0|, and the squared distances of the two adjusted
//    candidates differ by b - a = 2 - sum |d0_i| + corr1 - corr0 with
//    corr = (d_k - adj)^2 - d_k^2 = |adj| - 2 adj d_k (d_k the worst
//    coordinate's difference, adj the core g_x step).
// Every value is a small multiple of 1/(2q): sums, products and the
// comparison are exact in fp32, which makes the reference's comparison of
// correctly rounded norms the exact test b - a > 0 (ties to D8 + 1/2), under
// both of its distance rules.  The argmax, the g_x step and the tie rules are
// the reference's, as in project_dyadic; the CPU checker compares r with the
// oracle's for every code at q = 8 and q = 16 (all 2^32) and a sample at 32.
template <int Q>
__host__ __device__ inline void residual_dyadic(const int b[8], float r[8])
{
    static_assert(Q == 8 || Q == 16 || Q == 32, "the grid bounds above are those of q = 8, 16, 32");
    constexpr float kInv = 1.f / (float)(2 * Q);          // z = Z kInv, exact
    constexpr float kRound = 0.5f - 1.f / (float)(4 * Q); // toward zero on ties, nearest elsewhere
    constexpr float kNudge = 1.f / (float)(4 * Q);        // below the grid step
    // nz = -Z in fp32: Z = 0 converts to +0, so copysignf(c, nz) takes the
    // sign of -Z and of z <= 0 for zero, as the rules above need
    float nz[8];
    int nb7 = -b[7];
#if defined(__HIP_DEVICE_COMPILE__)
    asm volatile("" : "+v"(nb7));  // each coordinate is then one shift-and-add after the difference
#endif
    nz[0] = (float)(((b[1] - 2 * b[0]) << 1) + nb7);
#pragma unroll
    for (int i = 1; i < 6; ++i) nz[i] = (float)(((b[i + 1] - b[i]) << 1) + nb7);
    nz[6] = (float)(b[6] * -2 + nb7);
    nz[7] = (float)nb7;

    // g0 = -f0 = trunc(-z + copysign(1/2 - 1/(4q), -z)) (trunc is odd), so
    // no negated copysign is needed; the parity of sum f0 is that of sum g0
    float g0[8], f1[8], d0[8];
    float s0, s1, sa, best, least;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        g0[i] = truncf(fmaf(nz[i], kInv, copysignf(kRound, nz[i])));
        d0[i] = fmaf(nz[i], -kInv, g0[i]);
        f1[i] = floorf(fmaf(nz[i], -kInv, copysignf(kNudge, nz[i])));
        const float ad = fabsf(d0[i]);
        s0 = i == 0 ? g0[0] : s0 + g0[i];
        s1 = i == 0 ? f1[0] : s1 + f1[i];
        sa = i == 0 ? ad : sa + ad;
        best = i == 0 ? ad : fmaxf(best, ad);
        least = i == 0 ? ad : fminf(least, ad);
    }
    // first index of the largest |d0| (D8) and of the smallest (D8 + 1/2),
    // and -Z at each
    lanes_t first0[8], first1[8], seen0 = 0ull, seen1 = 0ull;
    float nk0 = nz[0], nk1 = nz[0];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const float ad = fabsf(d0[i]);
        const lanes_t h0 = lanes_of(ad == best), h1 = lanes_of(ad == least);
        first0[i] = h0 & ~seen0;
        first1[i] = h1 & ~seen1;
        seen0 |= h0;
        seen1 |= h1;
        nk0 = lane_in(first0[i]) ? nz[i] : nk0;
        nk1 = lane_in(first1[i]) ? nz[i] : nk1;
    }
    // the worst coordinates' differences, recomputed from z_k (same operations)
    const float dk0 = fmaf(nk0, -kInv, truncf(fmaf(nk0, kInv, copysignf(kRound, nk0))));
    const float tk1 = fmaf(nk1, -kInv, -0.5f);
    const float dk1 = tk1 - floorf(fmaf(nk1, -kInv, copysignf(kNudge, nk1)));
    // core g_x: an odd sum moves the worst coordinate by +1 when t_k >= 0 and
    // d_k > 0 (t = z for D8, z - 1/2 for D8 + 1/2), by -1 otherwise
    const bool odd0 = ((int)s0 & 1) != 0, odd1 = ((int)s1 & 1) != 0;
    const float adj0 = odd0 ? ((nk0 <= 0.f && dk0 > 0.f) ? 1.f : -1.f) : 0.f;
    const float adj1 = odd1 ? ((tk1 >= 0.f && dk1 > 0.f) ? 1.f : -1.f) : 0.f;
    const float diff = (2.f - sa) + (fmaf(-2.f * adj1, dk1, fabsf(adj1)) - fmaf(-2.f * adj0, dk0, fabsf(adj0)));
    const bool pick0 = diff > 0.f;  // a < b; ties go to D8 + 1/2
    const lanes_t p0 = lanes_of(pick0);
    // r = G b - q y with y = f0 (+ adj0 at k0) or f1 + 1/2 (+ adj1 at k1):
    // r_i = (-nz_i / 2 + c_i) + q g0_i or (...) - q f1_i, c_i = -q (1/2 if
    // D8 + 1/2) - q adj at the moved coordinate; every term and partial sum
    // is exact, and -nz_i / 2 + c_i is +0 (not -0) where it is zero, as the
    // reference's G b - q c is
    const float c_off = pick0 ? 0.f : -0.5f * (float)Q;
    float c_at = c_off - (float)Q * (pick0 ? adj0 : adj1);
#if defined(__HIP_DEVICE_COMPILE__)
    // keep c_at a value of its own, so that each coordinate selects between
    // two registers (one operation) rather than subtracting a selected term
    asm volatile("" : "+v"(c_at));
#endif
    const float qs = pick0 ? (float)Q : -(float)Q;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const lanes_t at = (p0 & first0[i]) | (~p0 & first1[i]);
        const float g = fmaf(nz[i], -0.5f, lane_in(at) ? c_at : c_off);
        r[i] = fmaf(qs, pick0 ? g0[i] : f1[i], g);
    }
}

// The same residual in integers, from a table of per-coordinate quantities
// (the layer round-trip kernel at q = 8, 16, the QAT backward at q = 2, 4,
// 8, 16; the grid argument above holds for q = 2 and 4 as well, and the CPU
// checker compares every code of q = 2, 4, 8 and 16 with the oracle's
// residual).  Everything residual_dyadic derives for coordinate i is a
// function of Z_i alone, an integer in [-2(q-1), 5(q-1)], so a 7q-entry
// table indexed by Z + 2q holds it:
//   f0 = the nearest integer to z = Z / 2q, ties toward zero (g0 = -f0);
//   D0 = 2q d0 = Z - 2q f0, in [-q, q];
//   f1 = floor(z - 1/(4q)) for Z > 0, floor(z + 1/(4q)) for Z <= 0, i.e.
//        floor((Z - 1) / 2q) and floor(Z / 2q);
//   D1 = 2q d1 = Z - q - 2q f1, with |D1| = q - |D0|;
//   c0 = [Z >= 0 and D0 > 0], c1 = [Z >= q and D1 > 0]: the direction of
//        the g_x step at the worst coordinate (nk0 <= 0 and dk0 > 0, tk1 >= 0
//        and dk1 > 0 above).
// Entry words, laid out so that the maximum of word + (7 - i) << 24 over the
// eight coordinates is the first index of the largest |D| with that
// coordinate's own low fields, and the plain sum of the eight words holds the
// sums without carries between fields:
//   x = |D0| << 27 | (f0 & 1) << 21 | |D0| << 13 | c0 << 9 | (D0 + q)
//   y = |D1| << 27 | (f1 & 1) << 21 |              c1 << 9 | (D1 + q)
//   z = (D0 + q) | (D1 + q) << 16
// (sums over eight coordinates: D + q <= 2q each, at most 16q = 256 in bits
// 0-8; c counts <= 8 in bits 9-12; sum |D0| <= 8q = 128 in bits 13-20; the
// parity count's low bit at 21, its carries in bits 22 and up, unused).  The
// largest |D1| is the smallest |D0|, so y's maximum is the first argmin of
// |d0| as above, and in units of 1/(2q) the comparison is the integer
//   4q - sum |D0| + (2q |adj1| - 2 adj1 D1_k1) - (2q |adj0| - 2 adj0 D0_k0) > 0.
template <int Q>
__host__ __device__ inline uint4 dyadic_table_entry(int Z)
{
    const int f0 = Z >= 0 ? (Z + Q - 1) / (2 * Q) : -((Q - 1 - Z) / (2 * Q));
    const int d0 = Z - 2 * Q * f0;
    const int f1 = Z > 0 ? (Z - 1) / (2 * Q) : -((2 * Q - 1 - Z) / (2 * Q));
    const int d1 = Z - Q - 2 * Q * f1;
    const uint32_t a0 = (uint32_t)(d0 < 0 ? -d0 : d0), a1 = (uint32_t)(d1 < 0 ? -d1 : d1);
    const uint32_t c0 = Z >= 0 && d0 > 0, c1 = Z >= Q && d1 > 0;
    uint4 e;
    e.x = a0 << 27 | (uint32_t)(f0 & 1) << 21 | a0 << 13 | c0 << 9 | (uint32_t)(d0 + Q);
    e.y = a1 << 27 | (uint32_t)(f1 & 1) << 21 | c1 << 9 | (uint32_t)(d1 + Q);
    e.z = (uint32_t)(d0 + Q) | (uint32_t)(d1 + Q) << 16;
    e.w = 0u;
    return e;
}

__host__ __device__ inline int mad24(int a, int b, int c)
{
#if defined(__HIP_DEVICE_COMPILE__)
    return __mul24(a, b) + c;  // one v_mad_i32_i24
#else
    return a * b + c;
#endif
}

// One level of the sum 2 x_hat = sum_m q^m (2 r_m), in integers: adds
// (2 r_i + q) << shift to acc2[i] (FIRST: sets it), where 2 r is twice the
// residual residual_dyadic<Q>(b) returns and tab the 7q-entry table above
// (tab[Z + 2q] = dyadic_table_entry<Q>(Z)).  The caller subtracts
// q sum_m q^m once at the end.
template <int Q, bool FIRST>
__host__ __device__ inline void dyadic_level_acc(const int b[8], const uint4* tab, int shift, int acc2[8])
{
    static_assert(Q == 2 || Q == 4 || Q == 8 || Q == 16, "the table fields hold q <= 16");
    const uint4* t7 = tab + (b[7] + 2 * Q);  // Z_i = 2 (..) + b_7
    uint4 e[8];
    e[0] = t7[2 * (2 * b[0] - b[1])];
#pragma unroll
    for (int i = 1; i < 6; ++i) e[i] = t7[2 * (b[i] - b[i + 1])];
    e[6] = t7[2 * b[6]];
    e[7] = t7[0];
    uint32_t kx[8], ky[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        kx[i] = e[i].x + ((uint32_t)(7 - i) << 24);
        ky[i] = e[i].y + ((uint32_t)(7 - i) << 24);
    }
    uint32_t mx = kx[0], my = ky[0], sx = kx[0], sy = ky[0];
#pragma unroll
    for (int i = 1; i < 8; ++i) {
        mx = mx > kx[i] ? mx : kx[i];
        my = my > ky[i] ? my : ky[i];
        sx += kx[i];
        sy += ky[i];
    }
    const int sa = (int)((sx >> 13) & 0xffu);
    const int adj0 = (sx >> 21) & 1u ? (((mx >> 9) & 1u) ? 1 : -1) : 0;
    const int adj1 = (sy >> 21) & 1u ? (((my >> 9) & 1u) ? 1 : -1) : 0;
    const int dk0 = (int)(mx & 0x1ffu) - Q, dk1 = (int)(my & 0x1ffu) - Q;
    const int diff = 4 * Q - sa + (2 * Q * (adj1 != 0) - 2 * adj1 * dk1) - (2 * Q * (adj0 != 0) - 2 * adj0 * dk0);
    const bool pick0 = diff > 0;  // ties go to D8 + 1/2
    const uint32_t sel = pick0 ? 0u : 16u;
    const uint32_t mk = 1u << (7u - ((pick0 ? mx : my) >> 24 & 7u));  // the moved coordinate
    const int t = -2 * Q * (pick0 ? adj0 : adj1);
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const int v = mad24((int)((mk >> i) & 1u), t, (int)((e[i].z >> sel) & 0xffffu));
        acc2[i] = FIRST ? v << shift : (v << shift) + acc2[i];
    }
}

// residual_dyadic<Q>(b) through the table (the same values, +0 for zero): for
// the decoders whose levels accumulate in fp32.
template <int Q>
__host__ __device__ inline void residual_table(const int b[8], const uint4* tab, float r[8])
{
    int r2[8];
    dyadic_level_acc<Q, true>(b, tab, 0, r2);
#pragma unroll
    for (int i = 0; i < 8; ++i) r[i] = 0.5f * (float)(r2[i] - Q);
}

}  // namespace coset
