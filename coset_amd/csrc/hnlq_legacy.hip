// hnlq_legacy.hip -- the paper's hierarchical encode/decode with the overload
// loop (coset/legacy/quant/functional.py:15-181, Algorithms 1 and 2), one
// 8-wide block per lane.
//
// Encode: xs = x / beta (+ dither); the chain y = Q(x_l), b = coords(y),
// x_l = y / q over M levels with the legacy (textbook) Q; the block
// overloads when Q(x_M) != 0.  While it overloads, protection is on and
// t < max_iter, xs = xs / 2^alpha and the chain reruns; T = t.  Outputs: the
// final chain's level words and/or float codes, T, the overload flag, and
// optionally the Algorithm 2 decode of the same codes.
// Decode: x_hat = sum_i q^i (G b_i - q Q(G b_i / q)) in fp32 from zero,
// minus dither, then (beta * x_hat) * (float)2^(alpha T).
// Every step is the reference's fp32 operation (project<true, false> is the
// legacy Q on one contiguous vector).
#include <math.h>

#include "codec_kernels.hpp"
#include "legacy.hpp"

namespace coset {

namespace {

__device__ __forceinline__ void load_block(const LegacyArgs& a, int64_t i, float x[8])
{
    if (a.x_dtype == DT_BF16) {
        const uint4 v = reinterpret_cast<const uint4*>(a.x)[i];
        const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            x[2 * j] = __uint_as_float(w[j] << 16);
            x[2 * j + 1] = __uint_as_float(w[j] & 0xffff0000u);
        }
    } else {
        const float4* p = reinterpret_cast<const float4*>(a.x) + 2 * i;
        const float4 u = p[0], v = p[1];
        x[0] = u.x; x[1] = u.y; x[2] = u.z; x[3] = u.w;
        x[4] = v.x; x[5] = v.y; x[6] = v.z; x[7] = v.w;
    }
}

// One level's legacy residual accumulated as the reference's
// x_hat += q^i * x_i (fp32, no contraction).
template <int Q>
__device__ __forceinline__ void add_residual(const int b[8], float qf, float w, float acc[8])
{
    float gb[8], r[8];
    lattice_point(b, gb);
    residual_from_point<true, false, Q>(gb, qf, r);
#pragma unroll
    for (int j = 0; j < 8; ++j) acc[j] = __fadd_rn(acc[j], __fmul_rn(w, r[j]));
}

__device__ __forceinline__ void store_decoded(const LegacyArgs& a, int64_t i, const float acc[8], int t)
{
    const float s = a.scale_T[min(max(t, 0), kLegacyMaxT)];
    float o[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        float v = acc[j];
        if (a.dither) v = __fsub_rn(v, a.dither[a.dither_stride * i + j]);
        o[j] = __fmul_rn(__fmul_rn(a.beta, v), s);
    }
    float4* p = reinterpret_cast<float4*>(a.out) + 2 * i;
    p[0] = make_float4(o[0], o[1], o[2], o[3]);
    p[1] = make_float4(o[4], o[5], o[6], o[7]);
}

}  // namespace

template <int Q, bool DECODE_ONLY>
__global__ void __launch_bounds__(256) hnlq_legacy_kernel(LegacyArgs a)
{
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= a.n) return;
    const int q = Q > 0 ? Q : a.q;
    const float qf = (float)q;
    const int M = a.M;
    const int wb = word_bytes(q);

    if (DECODE_ONLY) {
        float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
        float w = 1.f;
        for (int m = 0; m < M; ++m) {
            int b[8];
            if (a.codes_in_f32) {
                const float* cp = a.codes_in_f32 + ((size_t)i * M + m) * 8;
#pragma unroll
                for (int j = 0; j < 8; ++j) b[j] = (int)cp[j];
            } else {
                const uint32_t word = wb == 2 ? reinterpret_cast<const uint16_t*>(a.packed_in)[(size_t)i * M + m]
                                              : reinterpret_cast<const uint32_t*>(a.packed_in)[(size_t)i * M + m];
                unpack_word<Q>(word, q, b);
            }
            add_residual<Q>(b, qf, w, acc);
            w = __fmul_rn(w, qf);
        }
        store_decoded(a, i, acc, a.T_in ? a.T_in[i] : 0);
        return;
    }

    float xs[8];
    load_block(a, i, xs);
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        xs[j] = a.beta_is_pow2 ? __fmul_rn(xs[j], a.beta_inv) : __fdiv_rn(xs[j], a.beta);
        if (a.dither) xs[j] = __fadd_rn(xs[j], a.dither[a.dither_stride * i + j]);
    }
    int t = 0;
    bool ov;
    float acc[8];
    for (;;) {
        // one chain (functional.py:83-116), writing this chain's codes
        float xl[8], y[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            xl[j] = xs[j];
            acc[j] = 0.f;
        }
        float w = 1.f;
        for (int m = 0; m < M; ++m) {
            int b[8];
            project<true, false>(xl, y);
            lattice_digits<Q>(y, q, b);
            if (a.packed) {
                const uint32_t word = pack_word<Q>(b, q);
                if (wb == 2)
                    reinterpret_cast<uint16_t*>(a.packed)[(size_t)i * M + m] = (uint16_t)word;
                else
                    reinterpret_cast<uint32_t*>(a.packed)[(size_t)i * M + m] = word;
            }
            if (a.codes_f32) {
                float4* cp = reinterpret_cast<float4*>(a.codes_f32 + ((size_t)i * M + m) * 8);
                cp[0] = make_float4((float)b[0], (float)b[1], (float)b[2], (float)b[3]);
                cp[1] = make_float4((float)b[4], (float)b[5], (float)b[6], (float)b[7]);
            }
            if (a.out) {
                add_residual<Q>(b, qf, w, acc);
                w = __fmul_rn(w, qf);
            }
#pragma unroll
            for (int j = 0; j < 8; ++j) xl[j] = div_q<Q>(y[j], qf);
        }
        project<true, false>(xl, y);
        ov = false;
#pragma unroll
        for (int j = 0; j < 8; ++j) ov = ov || !(fabsf(y[j]) <= 1e-8f);  // allclose(Q, 0, atol=1e-8); NaN fails
        if (!(a.protect && ov && t < a.max_iter)) break;
        ++t;
#pragma unroll
        for (int j = 0; j < 8; ++j) xs[j] = __fdiv_rn(xs[j], a.two_alpha);
    }
    if (a.T) a.T[i] = t;
    if (a.overload) a.overload[i] = ov ? 1 : 0;
    if (a.out) store_decoded(a, i, acc, t);
}

hipError_t launch_legacy(const LegacyArgs& a, bool decode_only, hipStream_t s)
{
    if (a.n == 0) return hipSuccess;
    dim3 grid((unsigned)((a.n + 255) / 256)), block(256);
#define COSET_LEGACY(QQ)                                                                                  \
    if (decode_only)                                                                                      \
        hipLaunchKernelGGL((hnlq_legacy_kernel<QQ, true>), grid, block, 0, s, a);                         \
    else                                                                                                  \
        hipLaunchKernelGGL((hnlq_legacy_kernel<QQ, false>), grid, block, 0, s, a);
    switch (a.q) {
    case 2: COSET_LEGACY(2) break;
    case 4: COSET_LEGACY(4) break;
    case 8: COSET_LEGACY(8) break;
    case 16: COSET_LEGACY(16) break;
    default: COSET_LEGACY(0) break;
    }
#undef COSET_LEGACY
    return hipGetLastError();
}

}  // namespace coset
