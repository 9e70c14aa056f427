// e8_core.hpp -- device functions for E8 closest point and HNLQ digits (gfx950).
//
// Bit-exact restatement of the reference fp32 arithmetic: one IEEE
// round-to-nearest-even operation per reference operation.  The __f*_rn
// helpers are plain operators in HIP, so the library is built with
// -ffp-contract=off to keep a*b+c from fusing:
//   custom_round   coset/core/base.py:179-202
//   g_x            coset/core/e8/lattice.py:67-112 (core: negative x_k -> -1)
//                  coset/legacy/lattices/e8.py:41-68 (legacy: flip toward x)
//   projection     coset/core/e8/lattice.py:114-169 / legacy e8.py:70-103
//   encode_coords  coset/core/base.py:134-154  (G^-1 y, exact, then mod q)
//   decode_coords  coset/core/base.py:156-176  (G b, exact)
//
// The distance comparison `norm(x-y0) < norm(x-y1)` compares correctly rounded
// square roots of fp32 sums of squares.  Contiguous rows sum the rounded
// squares in order; the batched decode (strided rows in the reference) sums
// with fused multiply-adds.  sqrt is monotone, so d0 >= d1 decides without a
// sqrt, and d0 < d1 needs the two roots only when d1/d0 < 1 + 2^-20 (where
// both roots could round to one float).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "e8_fast.hpp"

namespace coset {

constexpr float kEps32 = 1.1920928955078125e-07f;  // torch.finfo(float32).eps

__device__ __forceinline__ float custom_round(float x)
{
    // floor((x - sign(x)*eps) + 0.5).  copysign gives +-eps at x = +-0 where
    // the reference subtracts 0; both give floor(~0.5) = 0 there.
    float y = __fsub_rn(x, copysignf(kEps32, x));
    return floorf(__fadd_rn(y, 0.5f));
}

// Parity of an exact integer-valued fp32 sum: 1 when odd.  Exact for every
// finite value (fp32 values >= 2^24 are even, as fmod(s, 2) says).
__device__ __forceinline__ float odd_f(float s)
{
    return __fsub_rn(s, __fmul_rn(2.f, floorf(__fmul_rn(s, 0.5f))));
}

// One D_n candidate for input t (n = 8: the D8 cosets of E8; n = 4: the D4
// lattice, coset/core/d4/lattice.py:62-146): f = round(t) if sum(f) is even,
// else g(t) (f with the worst coordinate pushed by +-1).  ALWAYS_G returns
// g(t) whatever the parity (the reference g_x itself).
template <int D, bool LEGACY, bool ALWAYS_G = false>
__device__ __forceinline__ void dn_candidate(const float t[D], float y[D])
{
    float f[D];
    float s = 0.f;
#pragma unroll
    for (int i = 0; i < D; ++i) {
        f[i] = custom_round(t[i]);
        s = __fadd_rn(s, f[i]);
    }
    // first argmax of |t - f| (torch.argmax returns the first maximum)
    float best = fabsf(__fsub_rn(t[0], f[0]));
    int k = 0;
    float tk = t[0], fk = f[0];
#pragma unroll
    for (int i = 1; i < D; ++i) {
        float d = fabsf(__fsub_rn(t[i], f[i]));
        bool gt = d > best;
        best = gt ? d : best;
        k = gt ? i : k;
        tk = gt ? t[i] : tk;
        fk = gt ? f[i] : fk;
    }
    bool up;
    if (LEGACY)
        up = (tk >= 0.f) ? (fk < tk) : (fk <= tk);
    else
        up = (tk >= 0.f) && (fk < tk);
    float adj = (ALWAYS_G || odd_f(s) != 0.f) ? (up ? 1.f : -1.f) : 0.f;
#pragma unroll
    for (int i = 0; i < D; ++i) y[i] = (i == k) ? __fadd_rn(f[i], adj) : f[i];
}

template <bool LEGACY, bool ALWAYS_G = false>
__device__ __forceinline__ void d8_candidate(const float t[8], float y[8])
{
    dn_candidate<8, LEGACY, ALWAYS_G>(t, y);
}

template <bool STRIDED>
__device__ __forceinline__ float sumsq_diff(const float x[8], const float y[8])
{
    float acc = 0.f;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        float e = __fsub_rn(x[i], y[i]);
        if (STRIDED)
            acc = __fmaf_rn(e, e, acc);
        else
            acc = __fadd_rn(acc, __fmul_rn(e, e));
    }
    return acc;
}

// Correctly rounded fp32 square root.  HIP's __fsqrt_rn is the native
// v_sqrt_f32 (about 1 ulp), so go through double: the f64 sqrt is correctly
// rounded, and rounding a correctly rounded 53-bit root to 24 bits gives the
// correctly rounded 24-bit root (53 >= 2*24 + 2).
__device__ __forceinline__ float cr_sqrtf(float a)
{
    return (float)__builtin_sqrt((double)a);
}

// norm(x-y0) < norm(x-y1) with correctly rounded roots.
__device__ __forceinline__ bool nearer(float a, float b)
{
    if (!(a < b)) return false;
    // b >= a*(1+2^-20) cannot share a rounded root with a
    if (b > __fmul_rn(a, 1.00000095367431640625f)) return true;
    return cr_sqrtf(a) < cr_sqrtf(b);
}

// Per-element select written as a bit blend, so the compiler keeps both
// candidates in registers instead of selecting between two stack arrays.
__device__ __forceinline__ float blend(uint32_t mask, float a, float b)
{
    return __uint_as_float((__float_as_uint(a) & mask) | (__float_as_uint(b) & ~mask));
}

// E8 closest point, reference semantics (core or legacy g_x rule).
template <bool LEGACY, bool STRIDED>
__device__ __forceinline__ void project(const float x[8], float out[8])
{
    float y0[8], y1[8], xs[8];
    d8_candidate<LEGACY>(x, y0);
#pragma unroll
    for (int i = 0; i < 8; ++i) xs[i] = __fsub_rn(x[i], 0.5f);
    d8_candidate<LEGACY>(xs, y1);
#pragma unroll
    for (int i = 0; i < 8; ++i) y1[i] = __fadd_rn(y1[i], 0.5f);
    float a = sumsq_diff<STRIDED>(x, y0);
    float b = sumsq_diff<STRIDED>(x, y1);
    uint32_t pick0 = nearer(a, b) ? 0xffffffffu : 0u;
#pragma unroll
    for (int i = 0; i < 8; ++i) out[i] = blend(pick0, y0[i], y1[i]);
}

// encode_coords: b = (G^-1 y) mod q for y in E8 (exact integers).
//   (G^-1 y)_0 = (y0+..+y6)/2 - 3.5 y7
//   (G^-1 y)_r = (y_r+..+y6) - (7-r) y7     r = 1..6
//   (G^-1 y)_7 = 2 y7
// computed on u = 2y as int32: exact for |y| < 2^30 (for q = 2^k the digits
// only need the low bits, which wrap-around keeps).  y in E8 makes every row
// an integer; a row can be fractional only for |x| >= 2^23, where fp32 cannot
// hold the D8 + 1/2 coset and the projection leaves E8 -- such rows are
// rounded half to even, the reference's torch.round of the exact product.
template <int Q>
__device__ __forceinline__ void lattice_digits(const float y[8], int q, int b[8])
{
    int u[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) u[i] = (int)__fmul_rn(2.f, y[i]);  // 2y: exact integers
    int suf = 0;  // 2 * (y_r + .. + y6)
    int c[8];
#pragma unroll
    for (int r = 6; r >= 1; --r) {
        suf += u[r];
        const int v = suf - (7 - r) * u[7];  // 2 * row
        c[r] = (v + ((v >> 1) & 1)) >> 1;    // v / 2, ties to even
    }
    suf += u[0];
    const int v0 = suf - 7 * u[7];           // 4 * row 0
    c[0] = (v0 + 1 + ((v0 >> 2) & 1)) >> 2;  // v0 / 4, nearest, ties to even
    c[7] = u[7];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        if (Q > 0 && (Q & (Q - 1)) == 0) {
            b[i] = c[i] & (Q - 1);  // two's complement & == Python-style mod
        } else {
            int qq = Q > 0 ? Q : q;
            int m = c[i] % qq;
            b[i] = m < 0 ? m + qq : m;
        }
    }
}

// decode_coords: y = G b (exact).
__device__ __forceinline__ void lattice_point(const int b[8], float y[8])
{
    float h = 0.5f * (float)b[7];
    y[0] = __fadd_rn((float)(2 * b[0] - b[1]), h);
#pragma unroll
    for (int i = 1; i < 6; ++i) y[i] = __fadd_rn((float)(b[i] - b[i + 1]), h);
    y[6] = __fadd_rn((float)b[6], h);
    y[7] = h;
}

// Same from float digits (compat path: e8_decode accepts float code tensors).
__device__ __forceinline__ void lattice_point_f(const float b[8], float y[8])
{
    float h = __fmul_rn(0.5f, b[7]);
    y[0] = __fadd_rn(__fsub_rn(__fmul_rn(2.f, b[0]), b[1]), h);
#pragma unroll
    for (int i = 1; i < 6; ++i) y[i] = __fadd_rn(__fsub_rn(b[i], b[i + 1]), h);
    y[6] = __fadd_rn(b[6], h);
    y[7] = h;
}

// Level word idx(b) = sum_j b_j q^(7-j) (coset/legacy/quant/vlut.py:217-238).
template <int Q>
__device__ __forceinline__ uint32_t pack_word(const int b[8], int q)
{
    uint32_t w = 0;
    if (Q > 0 && (Q & (Q - 1)) == 0) {
        constexpr int L = Q == 2 ? 1 : Q == 4 ? 2 : Q == 8 ? 3 : 4;
#pragma unroll
        for (int j = 0; j < 8; ++j) w = (w << L) | (uint32_t)b[j];
    } else {
        uint32_t qq = Q > 0 ? Q : q;
#pragma unroll
        for (int j = 0; j < 8; ++j) w = w * qq + (uint32_t)b[j];
    }
    return w;
}

template <int Q>
__device__ __forceinline__ void unpack_word(uint32_t w, int q, int b[8])
{
    if (Q > 0 && (Q & (Q - 1)) == 0) {
        constexpr int L = Q == 2 ? 1 : Q == 4 ? 2 : Q == 8 ? 3 : 4;
#pragma unroll
        for (int j = 7; j >= 0; --j) {
            b[j] = (int)(w & (Q - 1));
            w >>= L;
        }
    } else {
        uint32_t qq = Q > 0 ? Q : q;
#pragma unroll
        for (int j = 7; j >= 0; --j) {
            b[j] = (int)(w % qq);
            w /= qq;
        }
    }
}

// x / q in fp32.  For q = 2^k the quotient is exactly x * 2^-k as a real
// number, so the multiply rounds to the same float as the correctly rounded
// divide; other q take the IEEE divide.
template <int Q>
__device__ __forceinline__ float div_q(float x, float qf)
{
    if (Q > 0 && (Q & (Q - 1)) == 0) return __fmul_rn(x, 1.0f / (float)Q);
    return __fdiv_rn(x, qf);
}

// One level's residual r = G b - q * P(G b / q) (coset/core/e8/codecs.py:164-166).
// For q = 2^k the core rule goes through project_dyadic (e8_fast.hpp): G b / q
// is dyadic and small, where it equals the reference sequence exactly.
template <bool LEGACY, bool STRIDED, int Q = 0>
__device__ __forceinline__ void residual_from_point(const float gb[8], float qf, float r[8])
{
    float z[8], c[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) z[i] = div_q<Q>(gb[i], qf);
    if constexpr (!LEGACY && Q > 0 && Q <= 32 && (Q & (Q - 1)) == 0) {
        project_dyadic(z, c);
        // q c and G b - q c are exact here (small dyadic values), so one
        // fused operation gives the reference's two
#pragma unroll
        for (int i = 0; i < 8; ++i) r[i] = __fmaf_rn(-qf, c[i], gb[i]);
        return;
    } else {
        project<LEGACY, STRIDED>(z, c);
    }
#pragma unroll
    for (int i = 0; i < 8; ++i) r[i] = __fsub_rn(gb[i], __fmul_rn(qf, c[i]));
}

// One level's core-rule residual from its digits: residual_dyadic for
// q = 8, 16, 32 (the same values in fewer operations), else the lattice
// point and residual_from_point.
template <bool STRIDED, int Q>
__device__ __forceinline__ void level_residual(const int b[8], float qf, float r[8])
{
    if constexpr (Q == 8 || Q == 16 || Q == 32) {
        residual_dyadic<Q>(b, r);
    } else {
        float gb[8];
        lattice_point(b, gb);
        residual_from_point<false, STRIDED, Q>(gb, qf, r);
    }
}

// acc += w r for one level.  With q = 2^k, w = q^m and r a half-integer of
// the residual's range, w r is exact, so one fused operation rounds the sum
// as the reference's multiply and add do; other q keep the two operations.
template <int Q>
__device__ __forceinline__ void add_level(float acc[8], float w, const float r[8])
{
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        if constexpr (Q > 0 && (Q & (Q - 1)) == 0)
            acc[j] = __fmaf_rn(w, r[j], acc[j]);
        else
            acc[j] = __fadd_rn(acc[j], __fmul_rn(w, r[j]));
    }
}

__device__ __forceinline__ float bf16_to_f32(uint16_t h)
{
    return __uint_as_float(((uint32_t)h) << 16);
}

// fp32 -> bf16 round-to-nearest-even (NaN kept quiet).
__device__ __forceinline__ uint16_t f32_to_bf16(float f)
{
    uint32_t u = __float_as_uint(f);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);
    u += 0x7fffu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}

}  // namespace coset
