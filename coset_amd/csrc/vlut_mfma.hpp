// vlut_mfma.hpp -- device helpers and launch entry points shared by the
// matrix-core vLUT kernels (vlut.hip: tile kernel and reduce; vlut_rows.hip:
// rows kernel; vlut_wide.hip: wide and deep kernels).
#pragma once

#include "codec_kernels.hpp"
#include "lsq.hpp"
#include "vlut.hpp"

namespace coset {

typedef _Float16 half2_t __attribute__((ext_vector_type(2)));
typedef _Float16 half4_t __attribute__((ext_vector_type(4)));
typedef short bf16x4_t __attribute__((ext_vector_type(4)));
typedef float float4_t __attribute__((ext_vector_type(4)));

constexpr int kMfmaRows = 64;
constexpr int kMfmaKB = 16;              // k-blocks per step
constexpr int kMfmaK = kMfmaKB * 8;      // 128 K values per step
constexpr int kMfmaLd = kMfmaK + 8;      // row pitch in halves (16-byte aligned, skews banks)
constexpr int kMfmaMaxSteps = 4;         // steps per workgroup: its K range is <= 64 k-blocks
constexpr int kSwarSlots = 512 + kMaxCoarseVlut;

// two halves (bit patterns 0x64bb) from bytes k, k+1 of w
__device__ __forceinline__ uint32_t bytes_to_f16_bits(uint32_t w, bool upper)
{
    return __builtin_amdgcn_perm(0x64646464u, w, upper ? 0x04030402u : 0x04010400u);
}

typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));

constexpr int kRowsWaves = 8;

template <int Q, int M, int WN>
__device__ __forceinline__ void load_pair(const VlutMatmulArgs& p, int fmt, int64_t row, int64_t kb, int64_t kb_total,
                                          uint32_t w[WN])
{
    const int64_t i0 = vlut_word_index(fmt, row, kb, 0, kb_total, M);
    if (fmt == VLUT_DECODED) {
        const uint2 v = *reinterpret_cast<const uint2*>(reinterpret_cast<const uint32_t*>(p.words) + i0);
        w[0] = v.x;
        w[1 % WN] = v.y;
    } else if (fmt == VLUT_RAW) {
        const uint16_t* src = reinterpret_cast<const uint16_t*>(p.words) + i0;
        constexpr uint32_t kMask = Q == 2 ? 0xffu : 0xffffu;  // q^8 - 1: map bounds for any input
#pragma unroll
        for (int m = 0; m < M; ++m) {
            const uint32_t x = src[m] & kMask;
            w[m] = ((uint32_t)p.map[x] << 16) | x;
        }
    } else {
        const uint32_t* src = reinterpret_cast<const uint32_t*>(p.words) + i0;
        if (M == 2) {
            const uint2 v = *reinterpret_cast<const uint2*>(src);
            w[0] = v.x;
            w[1 % M] = v.y;
        } else if (M == 4) {
            const uint4 v = *reinterpret_cast<const uint4*>(src);
            w[0] = v.x;
            w[1 % M] = v.y;
            w[2 % M] = v.z;
            w[3 % M] = v.w;
        } else {
#pragma unroll
            for (int m = 0; m < M; ++m) w[m] = src[m];
        }
    }
}

// Eight biased bytes (x0: coordinates 0-3, x1: 4-7) minus the bias as 8
// halves (fp16) or bf16 values, exact.
template <bool BF16>
__device__ __forceinline__ uint4 bytes_to_operand(uint32_t x0, uint32_t x1, _Float16 f16_off, float f32_off)
{
    uint32_t hv[4];
    if (BF16) {
        float f[8];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            f[j] = (float)((x0 >> (8 * j)) & 0xffu) - f32_off;
            f[4 + j] = (float)((x1 >> (8 * j)) & 0xffu) - f32_off;
        }
#pragma unroll
        for (int j = 0; j < 4; ++j)
            hv[j] = __builtin_amdgcn_perm(__float_as_uint(f[2 * j + 1]), __float_as_uint(f[2 * j]), 0x07060302u);
    } else {
        const uint32_t raw[4] = {bytes_to_f16_bits(x0, false), bytes_to_f16_bits(x0, true),
                                 bytes_to_f16_bits(x1, false), bytes_to_f16_bits(x1, true)};
#pragma unroll
        for (int j = 0; j < 4; ++j)
            hv[j] = __builtin_bit_cast(uint32_t, __builtin_bit_cast(half2_t, raw[j]) - (half2_t){f16_off, f16_off});
    }
    return make_uint4(hv[0], hv[1], hv[2], hv[3]);
}

// One pair of the 6-byte format (vlut.hpp) from its 48 bits (lo: bits 0-31,
// hi: bits 32-47 in its low half; the upper half is ignored) as the bytes
// 2 x_hat + 2 off (x0: coordinates 0-3, x1: 4-7).  Fields 0-5 are the low 6
// bits of the six bytes; the bytes' top two bits carry field 6 (bytes 0-2)
// and v7 = field 7 | parity << 5 (bytes 3-5), each gathered into 6
// contiguous bits by one multiply (the three 2-bit pieces land 2 bits apart
// and the cross terms fall elsewhere: no carries).  Then 2 f + p per byte
// (at most 2 * 63 + 1).
__device__ __forceinline__ void d6_bytes(uint32_t lo, uint32_t hi, uint32_t& x0, uint32_t& x1)
{
    const uint32_t f6 = __builtin_amdgcn_ubfe((lo & 0x00c0c0c0u) * 4161u, 18, 6);
    const uint32_t y = __builtin_amdgcn_alignbit(hi, lo, 30);   // lo bits 30-31, then hi
    const uint32_t v7 = __builtin_amdgcn_ubfe((y & 0x00030303u) * 4161u, 12, 6);
    const uint32_t pm = (v7 >> 5) * 0x01010101u;
    const uint32_t b1 = (hi & 0x3f3fu) | (f6 << 16) | ((v7 & 31u) << 24);
    x0 = ((lo & 0x3f3f3f3fu) << 1) + pm;
    x1 = (b1 << 1) + pm;
}

// Pair j (0..7) of a lane's 6-byte chunk w[12] (384 bits, pair j at bit 48 j).
__device__ __forceinline__ void d6_pair(const uint32_t* w, int j, uint32_t& x0, uint32_t& x1)
{
    const int i = 3 * (j >> 1);
    if (j & 1)
        d6_bytes(__builtin_amdgcn_alignbit(w[i + 2], w[i + 1], 16), w[i + 2] >> 16, x0, x1);
    else
        d6_bytes(w[i], w[i + 1], x0, x1);
}

// 2 x_hat of one pair as 8 halves (fp16) or bf16 values, exact.
template <int Q, int M, bool BF16>
__device__ __forceinline__ uint4 decode_pair_swar(const uint64_t* s_tab, const uint32_t w[M], _Float16 f16_off,
                                                  float f32_off)
{
    uint32_t x0 = 0u, x1 = 0u;
#pragma unroll
    for (int m = M - 1; m >= 0; --m) {
        const uint32_t v = w[m];
        const uint2 tl = *reinterpret_cast<const uint2*>(&s_tab[256 + (v & 0xffu)]);
        const uint2 tc = *reinterpret_cast<const uint2*>(&s_tab[512 + (v >> 16)]);
        uint32_t l0 = tl.x + tc.x, l1 = tl.y + tc.y;
        if (Q != 2) {
            const uint2 th = *reinterpret_cast<const uint2*>(&s_tab[(v >> 8) & 0xffu]);
            l0 += th.x;
            l1 += th.y;
        }
        x0 = x0 * Q + l0;
        x1 = x1 * Q + l1;
    }
    return bytes_to_operand<BF16>(x0, x1, f16_off, f32_off);
}

// The three bf16 planes of the exact split a = h1 + h2 + h3, h1 the top 16 bits of a, h2 those of
// a - h1, h3 those of a - h1 - h2.  Each difference is exact (it keeps the
// bits the truncation dropped), and a - h1 - h2 has at most 8 significant
// bits, so h3 holds it exactly (for |a| above the bf16 subnormal range,
// ~1e-33).  Infinities go to h1 whole, a NaN to h1 as a quiet NaN, with
// h2 = h3 = 0, so the products see the value itself.
__device__ __forceinline__ void split3(float a, uint16_t& h1, uint16_t& h2, uint16_t& h3)
{
    const uint32_t u = __float_as_uint(a);
    if ((u & 0x7f800000u) == 0x7f800000u) {
        h1 = (u & 0x007fffffu) ? (uint16_t)0x7fc0u : (uint16_t)(u >> 16);
        h2 = h3 = 0;
        return;
    }
    h1 = (uint16_t)(u >> 16);
    const float r1 = __fsub_rn(a, __uint_as_float((uint32_t)h1 << 16));
    h2 = (uint16_t)(__float_as_uint(r1) >> 16);
    const float r2 = __fsub_rn(r1, __uint_as_float((uint32_t)h2 << 16));
    h3 = (uint16_t)(__float_as_uint(r2) >> 16);
}

// The same with bias[o] already loaded (b; used where bias is non-null).
__device__ __forceinline__ float vlut_epilogue_b(float y, float b, const float* bias, const float* lsq_alpha,
                                                 int lsq_qmax)
{
    if (bias) y = __fadd_rn(y, b);
    if (lsq_alpha) y = lsq_value(y, lsq_scale(lsq_alpha, lsq_qmax));
    return y;
}

// Output epilogue: + bias[o], then the LSQ activation quantizer (fp32, the
// reference's order: the value F.linear(x, W, b) followed by actq,
// coset/core/layers.py:472-484).
__device__ __forceinline__ float vlut_epilogue(float y, int64_t o, const float* bias, const float* lsq_alpha,
                                               int lsq_qmax)
{
    if (bias) y = __fadd_rn(y, bias[o]);
    if (lsq_alpha) y = lsq_value(y, lsq_scale(lsq_alpha, lsq_qmax));
    return y;
}


constexpr int kWideRT = 1;                            // row tiles of 16 per wave
constexpr int kWideNW = 8;                            // waves per workgroup
constexpr int kWideRows = 16 * kWideRT * kWideNW;     // rows per workgroup
constexpr int kWideTokens = 64;
constexpr int kWideStageKq = 4;                       // k-quads (4 k-blocks of 8, 32 K) per stage
constexpr int kWideActStride = 32 * kWideStageKq + 8; // halves per token row in LDS (16-byte pad)
constexpr int kDeepRT = 4;                          // row tiles of 16 per wave
constexpr int kDeepNW = 8;                          // waves per workgroup (split K)
constexpr int kDeepRows = 16 * kDeepRT;             // 64 rows per workgroup
constexpr int kDeepTokens = 64;
constexpr int kDeepKqWave = 4;                      // at most 4 k-quads (128 K) per wave
constexpr int kDeepKqWg = kDeepKqWave * kDeepNW;    // at most 32 k-quads (1024 K) per workgroup
constexpr int kDeepStride = 32 * kDeepKqWg + 8;     // halves per token row in LDS (16-byte pad)

// Launch the rows, wide or deep kernel of a plan (q in {2, 4}; the byte
// tables must cover M).  The wide and deep kernels with splits > 1 write
// split-major partials and leave the reduce to the caller.
hipError_t vlut_launch_rows(const VlutMatmulArgs& p, int splits, hipStream_t s);
// The rows kernel stages its activations in LDS (a wave's K range of at most
// two chunks) for this K and split count; with act_planes set and B <= 16
// it then splits fp32 activations into their planes itself.
bool vlut_rows_staged(int64_t K, int splits);
hipError_t vlut_launch_wide(const VlutMatmulArgs& p, int splits, hipStream_t s);
hipError_t vlut_launch_deep(const VlutMatmulArgs& p, int splits, hipStream_t s);

}  // namespace coset
