// hnlq_codec.hip -- fused E8 HNLQ encode / decode / round-trip kernels.
//
// Replaces the M-level loops of e8_encode (coset/core/e8/codecs.py:63-83) and
// E8Decoder._full_decode (codecs.py:139-180), including the layer-convention
// scaling of HNLQLinearQAT._quantize_weights (coset/core/layers.py:428-463).
//
// One thread owns one 8-wide block: two 16-byte loads (fp32) or one (bf16),
// M projections to encode, M more to decode, then packed level words and the
// decoded block are written with 16-byte stores.  Blocks are contiguous in
// HBM, so a wavefront reads and writes contiguous 2 KiB (fp32) spans.
//
// Scaling conventions
//   SCALE_CODEC  x_s = x / beta;        out = dec * beta           (codecs.py:64,175)
//   SCALE_LAYER  x_s = x * beta_row;    out = clamp(dec / beta_row, +-clip)
//                                                                 (layers.py:431,455,463)
#include <algorithm>
#include <type_traits>

#include "codec_kernels.hpp"
#include "tables.hpp"

namespace coset {

// 2 r(b) of one level word through the decode tables (q = 2, 4):
// 2 G b from the digits, minus q (2 c) for the word's coarse point.
template <int Q>
__device__ __forceinline__ void two_r_tables(uint32_t w, const uint16_t* map, const uint64_t* coarse, int out[8])
{
    w &= (Q == 2 ? 0xffu : 0xffffu);   // the map's bounds for any input word
    int b[8];
    unpack_word<Q>(w, Q, b);
    const uint64_t c = coarse[map[w]];
    out[0] = 4 * b[0] - 2 * b[1] + b[7];
#pragma unroll
    for (int j = 1; j < 6; ++j) out[j] = 2 * (b[j] - b[j + 1]) + b[7];
    out[6] = 2 * b[6] + b[7];
    out[7] = b[7];
#pragma unroll
    for (int j = 0; j < 8; ++j) out[j] -= Q * (int)(int8_t)(uint8_t)(c >> (8 * j));
}

// Tiles whose theta-derived beta one workgroup of 256 blocks can touch when a
// tile spans at least 64 blocks.
constexpr int kWgTiles = 256 / 64 + 2;

// WGBETA: layer scaling with beta derived from theta and tiles of at least
// 64 blocks -- the workgroup derives the beta of each tile it touches once,
// in LDS, instead of every block deriving its own.
// aux_out[i] = aux_in[i] in out_dtype (fp32 -> bf16 round to nearest even,
// as torch's cast)
__device__ __forceinline__ void aux_cast(const CodecArgs& a, int64_t i)
{
    const float v = a.aux_in[i];
    if (a.out_dtype == DT_BF16)
        reinterpret_cast<uint16_t*>(a.aux_out)[i] = f32_to_bf16(v);
    else
        reinterpret_cast<float*>(a.aux_out)[i] = v;
}

__global__ void __launch_bounds__(256) aux_cast_kernel(CodecArgs a)
{
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < a.aux_n) aux_cast(a, i);
}

// MM > 0: the level count fixed at compile time (the layer quantizer's M = 2
// round trip through the decode tables): every level is encoded first, then
// the levels' table reads are issued together, so a block waits for one
// round of map reads and one of coarse-point reads instead of one per level.
template <int Q, int MODE, bool WGBETA, int MM = 0>
__global__ void __launch_bounds__(256) hnlq_codec_kernel(CodecArgs a)
{
    int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i == 0 && a.step_counter) *a.step_counter += 1;
    if (a.aux_out && i < a.aux_n) aux_cast(a, i);
    // q = 8, 16: the decode table of residual_table, one entry per Z + 2q
    constexpr bool kRtab = (Q == 8 || Q == 16) && MODE != MODE_ENCODE;
    __shared__ uint4 s_rtab[kRtab ? 7 * Q : 1];
    if constexpr (kRtab) {
        if (threadIdx.x < 7 * Q) s_rtab[threadIdx.x] = dyadic_table_entry<Q>((int)threadIdx.x - 2 * Q);
        __syncthreads();
    }
    const int q = Q > 0 ? Q : a.q;
    const float qf = (float)q;
    const int M = MM > 0 ? MM : a.M;

    auto load_block = [&](int64_t il, float xl[8]) {
        if (a.x_dtype == DT_BF16) {
            uint4 v = reinterpret_cast<const uint4*>(a.x)[il];
            uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                xl[2 * j] = __uint_as_float(w[j] << 16);
                xl[2 * j + 1] = __uint_as_float(w[j] & 0xffff0000u);
            }
        } else {
            const float4* p = reinterpret_cast<const float4*>(a.x) + 2 * il;
            float4 u = p[0], v = p[1];
            xl[0] = u.x; xl[1] = u.y; xl[2] = u.z; xl[3] = u.w;
            xl[4] = v.x; xl[5] = v.y; xl[6] = v.z; xl[7] = v.w;
        }
    };
    float xl[8];
    float scale = 1.f;
    if constexpr (WGBETA) {
        // the block's input is loaded first (clamped to the last block), so its
        // latency overlaps the tile betas' derivation; the workgroup's blocks
        // span tiles t0 .. t0 + kWgTiles - 1 at most
        if (MODE != MODE_DECODE) load_block(i < a.n ? i : a.n - 1, xl);
        __shared__ float s_beta[kWgTiles];
        const int64_t b0 = (int64_t)blockIdx.x * blockDim.x;
        const int64_t t0 = b0 / a.blocks_per_row;
        const int64_t t = t0 + threadIdx.x;
        if (threadIdx.x < kWgTiles && t * a.blocks_per_row < a.n) {
            float lo, hi, sg;
            theta_beta_terms(a.tb, t, &lo, &hi, &sg);
            const float span = __fsub_rn(hi, lo);
            s_beta[threadIdx.x] = __fadd_rn(lo, __fmul_rn(sg, span));
            const int64_t first = t * a.blocks_per_row;   // the workgroup holding it records beta
            if (first >= b0 && first < b0 + blockDim.x) {
                if (a.beta_out) a.beta_out[t] = s_beta[threadIdx.x];
                if (a.dbdt_out) a.dbdt_out[t] = __fmul_rn(__fmul_rn(span, __fsub_rn(1.f, sg)), sg);
            }
        }
        __syncthreads();
        if (i >= a.n) return;
        scale = s_beta[i / a.blocks_per_row - t0];
    } else {
        if (i >= a.n) return;
        if (a.scale_mode == SCALE_CODEC)
            scale = a.beta;
        else if (a.scale_mode == SCALE_LAYER)
            scale = layer_scale(a, i);
        if (MODE != MODE_DECODE) load_block(i, xl);
    }

    float acc[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) acc[j] = 0.f;

    if (MODE != MODE_DECODE) {
        if (a.scale_mode == SCALE_CODEC) {
            if (a.beta_is_pow2) {
#pragma unroll
                for (int j = 0; j < 8; ++j) xl[j] = __fmul_rn(xl[j], a.beta_inv);
            } else {
#pragma unroll
                for (int j = 0; j < 8; ++j) xl[j] = __fdiv_rn(xl[j], scale);
            }
        } else if (a.scale_mode == SCALE_LAYER) {
#pragma unroll
            for (int j = 0; j < 8; ++j) xl[j] = __fmul_rn(xl[j], scale);
        }
        if (a.dither) {
#pragma unroll
            for (int j = 0; j < 8; ++j)
                xl[j] = __fadd_rn(xl[j], a.dither[a.dither_stride * i + j]);
        }

        if constexpr (MM > 0 && MODE == MODE_ROUNDTRIP && (Q == 2 || Q == 4)) {
            uint32_t words[MM];
#pragma unroll
            for (int m = 0; m < MM; ++m) {
                int b[8];
                encode_level<Q>(xl, a.fast_projection, q, b);
                words[m] = pack_word<Q>(b, q);
                if (a.packed) reinterpret_cast<uint16_t*>(a.packed)[(size_t)i * MM + m] = (uint16_t)words[m];
                if (a.codes_f32) {
                    float4* cp = reinterpret_cast<float4*>(a.codes_f32 + ((size_t)i * MM + m) * 8);
                    cp[0] = make_float4((float)b[0], (float)b[1], (float)b[2], (float)b[3]);
                    cp[1] = make_float4((float)b[4], (float)b[5], (float)b[6], (float)b[7]);
                }
#pragma unroll
                for (int j = 0; j < 8; ++j) xl[j] = div_q<Q>(xl[j], qf);
            }
            // 2 r of each level as two_r_tables computes it, the table reads first
            constexpr uint32_t kMask = Q == 2 ? 0xffu : 0xffffu;
            uint16_t cid[MM];
            uint64_t cc[MM];
#pragma unroll
            for (int m = 0; m < MM; ++m) cid[m] = a.dec_map[words[m] & kMask];
#pragma unroll
            for (int m = 0; m < MM; ++m) cc[m] = a.dec_coarse[cid[m]];
            float w = 1.f;
#pragma unroll
            for (int m = 0; m < MM; ++m) {
                int b[8], r2[8];
                unpack_word<Q>(words[m] & kMask, Q, b);
                r2[0] = 4 * b[0] - 2 * b[1] + b[7];
#pragma unroll
                for (int j = 1; j < 6; ++j) r2[j] = 2 * (b[j] - b[j + 1]) + b[7];
                r2[6] = 2 * b[6] + b[7];
                r2[7] = b[7];
#pragma unroll
                for (int j = 0; j < 8; ++j) {
                    const float r = 0.5f * (float)(r2[j] - Q * (int)(int8_t)(uint8_t)(cc[m] >> (8 * j)));
                    acc[j] = __fadd_rn(acc[j], __fmul_rn(w, r));
                }
                w = __fmul_rn(w, qf);
            }
        } else {
        float w = 1.f;
        for (int m = 0; m < M; ++m) {
            int b[8];
            encode_level<Q>(xl, a.fast_projection, q, b);
            uint32_t word = pack_word<Q>(b, q);
            if (a.packed) {  // level words stored as produced: [n, M]
                if (word_bytes(q) == 2)
                    reinterpret_cast<uint16_t*>(a.packed)[(size_t)i * M + m] = (uint16_t)word;
                else
                    reinterpret_cast<uint32_t*>(a.packed)[(size_t)i * M + m] = word;
            }
            if (a.codes_f32) {
                float4* cp = reinterpret_cast<float4*>(a.codes_f32 + ((size_t)i * M + m) * 8);
                cp[0] = make_float4((float)b[0], (float)b[1], (float)b[2], (float)b[3]);
                cp[1] = make_float4((float)b[4], (float)b[5], (float)b[6], (float)b[7]);
            }
            if (MODE == MODE_ROUNDTRIP) {
                float r[8];
                if ((Q == 2 || Q == 4) && a.dec_map) {
                    // exact: 2 r is an integer, r a half-integer
                    int r2[8];
                    two_r_tables<Q>(word, a.dec_map, a.dec_coarse, r2);
#pragma unroll
                    for (int j = 0; j < 8; ++j) r[j] = 0.5f * (float)r2[j];
                } else if constexpr (kRtab) {
                    residual_table<Q>(b, s_rtab, r);  // both distance rules agree on this grid
                } else {
                    if (a.strided)
                        level_residual<true, Q>(b, qf, r);
                    else
                        level_residual<false, Q>(b, qf, r);
                }
                add_level<Q>(acc, w, r);
                w = __fmul_rn(w, qf);
            }
#pragma unroll
            for (int j = 0; j < 8; ++j) xl[j] = div_q<Q>(xl[j], qf);
        }
        }
    } else {
        float w = 1.f;
        for (int m = 0; m < M; ++m) {
            float gb[8], r[8];
            if (a.codes_in_f32) {
                const float4* cp = reinterpret_cast<const float4*>(a.codes_in_f32 + ((size_t)i * M + m) * 8);
                float4 u = cp[0], v = cp[1];
                float bf[8] = {u.x, u.y, u.z, u.w, v.x, v.y, v.z, v.w};
                lattice_point_f(bf, gb);
            } else {
                uint32_t word;
                if (word_bytes(q) == 2)
                    word = reinterpret_cast<const uint16_t*>(a.packed_in)[(size_t)i * M + m];
                else
                    word = reinterpret_cast<const uint32_t*>(a.packed_in)[(size_t)i * M + m];
                if ((Q == 2 || Q == 4) && a.dec_map) {
                    int r2[8];
                    two_r_tables<Q>(word, a.dec_map, a.dec_coarse, r2);
#pragma unroll
                    for (int j = 0; j < 8; ++j) acc[j] = __fadd_rn(acc[j], __fmul_rn(w, 0.5f * (float)r2[j]));
                    w = __fmul_rn(w, qf);
                    continue;
                }
                int b[8];
                unpack_word<Q>(word, q, b);
                if constexpr (kRtab) {
                    residual_table<Q>(b, s_rtab, r);
                    add_level<Q>(acc, w, r);
                    w = __fmul_rn(w, qf);
                    continue;
                }
                lattice_point(b, gb);
            }
            if (a.strided)
                residual_from_point<false, true, Q>(gb, qf, r);
            else
                residual_from_point<false, false, Q>(gb, qf, r);
            add_level<Q>(acc, w, r);
            w = __fmul_rn(w, qf);
        }
    }

    if (MODE == MODE_ENCODE || !a.out) return;
    float o[8];
    if (a.scale_mode == SCALE_CODEC) {
#pragma unroll
        for (int j = 0; j < 8; ++j) o[j] = __fmul_rn(acc[j], scale);
    } else if (a.scale_mode == SCALE_LAYER) {
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            float v = __fdiv_rn(acc[j], scale);
            o[j] = fminf(fmaxf(v, -a.clip), a.clip);
            if (v != v) o[j] = v;  // torch.clamp propagates NaN
        }
    } else {
#pragma unroll
        for (int j = 0; j < 8; ++j) o[j] = acc[j];
    }
    if (a.out_dtype == DT_BF16) {
        uint4 v;
        v.x = f32_to_bf16(o[0]) | ((uint32_t)f32_to_bf16(o[1]) << 16);
        v.y = f32_to_bf16(o[2]) | ((uint32_t)f32_to_bf16(o[3]) << 16);
        v.z = f32_to_bf16(o[4]) | ((uint32_t)f32_to_bf16(o[5]) << 16);
        v.w = f32_to_bf16(o[6]) | ((uint32_t)f32_to_bf16(o[7]) << 16);
        reinterpret_cast<uint4*>(a.out)[i] = v;
    } else {
        float4* p = reinterpret_cast<float4*>(a.out) + 2 * i;
        p[0] = make_float4(o[0], o[1], o[2], o[3]);
        p[1] = make_float4(o[4], o[5], o[6], o[7]);
    }
}

// The layer quantizer's round trip with per-row betas, stored or derived from
// theta (SCALE_LAYER: HNLQLinearQAT._quantize_weights, coset/core/layers.py:428-463) for
// q = 8, 16 and M <= 4, with the level count and input dtype fixed at
// compile time, so a block runs straight through without the generic
// kernel's per-call branches and the register copies at their joins:
//  - the block's row from the launcher's 32-bit multiplier (blocks < 2^32);
//  - x * beta, then per level the encoder (the fast projection first, its
//    range checked once) and the level's residual from its digits through
//    the workgroup's LDS table of per-coordinate quantities
//    (dyadic_level_acc: residual_dyadic's values, summed in integers);
//  - dec / beta from one correctly rounded reciprocal per block and one or
//    two residual corrections (div_by_recip: one where the decoded sums stay
//    within its checked half-integer range), clamped by one med3.  That takes
//    |beta| in [2^-64, 2^64] -- the decoded sums are half-integers below 2^46
//    here, so every quantity stays normal -- and clip > 0 (the launcher's
//    condition); the sums are finite, so no quotient is NaN.  Other betas
//    (zero, tiny, huge, non-finite) take the IEEE divide and torch.clamp's NaN
//    rule, as the generic kernel does for every block.
template <int Q, int M, bool XBF16, bool THETA>
__global__ void __launch_bounds__(256) hnlq_layer_rt_kernel(CodecArgs a)
{
    static_assert(Q == 4 || Q == 8 || Q == 16, "the table decode's q within the codec's q <= 16");
    static_assert(M >= 1 && M <= 4, "level words stored as one vector");
    // q = 4 decodes each level through the L2-resident cid map and coarse
    // points (two_r_tables' values; measured faster here than the LDS table
    // of dyadic_level_acc, which q = 8, 16 take)
    constexpr bool kGdec = Q == 4;
    constexpr int kSteps = Q <= 8 || M <= 3 ? 1 : 2;
    constexpr int kLog2Q = Q == 4 ? 2 : Q == 8 ? 3 : 4;
    constexpr int kOff = Q * (((1 << (kLog2Q * M)) - 1) / (Q - 1));  // q sum_m q^m
    using Word = std::conditional_t<(Q <= 4), uint16_t, uint32_t>;  // word_bytes(q)
    // the decode table of dyadic_level_acc, one entry per Z + 2q
    __shared__ uint4 s_tab[kGdec ? 1 : 7 * Q];
    if (!kGdec && threadIdx.x < 7 * Q) s_tab[threadIdx.x] = dyadic_table_entry<Q>((int)threadIdx.x - 2 * Q);
    // THETA: the betas of the rows this workgroup's blocks span (rows of at
    // least 64 blocks: kWgTiles of them at most), derived from theta once
    // per row as the generic kernel does, and recorded with d beta / d theta
    // by the workgroup holding the row's first block
    __shared__ float s_beta[THETA ? kWgTiles : 1];
    const int64_t b0 = (int64_t)blockIdx.x * blockDim.x;
    uint32_t t0 = 0;
    if constexpr (THETA) {
        t0 = u32div((uint32_t)b0, a.row_div);
        const int64_t t = (int64_t)t0 + threadIdx.x;
        if (threadIdx.x < kWgTiles && t * a.blocks_per_row < a.n) {
            float lo, hi, sg;
            theta_beta_terms(a.tb, t, &lo, &hi, &sg);
            const float span = __fsub_rn(hi, lo);
            s_beta[threadIdx.x] = __fadd_rn(lo, __fmul_rn(sg, span));
            const int64_t first = t * a.blocks_per_row;
            if (first >= b0 && first < b0 + blockDim.x) {
                if (a.beta_out) a.beta_out[t] = s_beta[threadIdx.x];
                if (a.dbdt_out) a.dbdt_out[t] = __fmul_rn(__fmul_rn(span, __fsub_rn(1.f, sg)), sg);
            }
        }
    }
    __syncthreads();
    const int64_t i = b0 + threadIdx.x;
    if (i == 0 && a.step_counter) *a.step_counter += 1;
    // the side cast (the layer's bias) in the same launch: one more launch
    // would be one more dependent node in a captured step
    if (a.aux_out && i < a.aux_n) aux_cast(a, i);
    if (i >= a.n) return;
    const uint32_t row = u32div((uint32_t)i, a.row_div);
    const float beta = THETA ? s_beta[row - t0] : a.beta_row[row];
    float xl[8];
    if constexpr (XBF16) {
        const uint4 v = reinterpret_cast<const uint4*>(a.x)[i];
        const uint32_t u[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            xl[2 * j] = __uint_as_float(u[j] << 16);
            xl[2 * j + 1] = __uint_as_float(u[j] & 0xffff0000u);
        }
    } else {
        const float4* p = reinterpret_cast<const float4*>(a.x) + 2 * i;
        const float4 u = p[0], v = p[1];
        xl[0] = u.x; xl[1] = u.y; xl[2] = u.z; xl[3] = u.w;
        xl[4] = v.x; xl[5] = v.y; xl[6] = v.z; xl[7] = v.w;
    }
#pragma unroll
    for (int j = 0; j < 8; ++j) xl[j] = __fmul_rn(xl[j], beta);

    Word* pw = a.packed ? reinterpret_cast<Word*>(a.packed) + (size_t)i * M : nullptr;
    // the fast projection's range condition holds at every level once it
    // holds for the first: each level's input is the last one divided by q
    const bool in_range = fast_in_range(xl);
    // 2 x_hat = sum_m q^m (2 r_m) in integers (the float sum of the levels
    // is exact on these half-integers, so its value is the same)
    int acc2[8];
    if constexpr (kGdec) {
        // every level encoded first, then the levels' map reads and coarse
        // point reads issued together (two_r_tables' values: 2 r = 2 G b -
        // q c); acc2 takes the same q sum_m q^m offset as the table path
        uint32_t words[M];
#pragma unroll
        for (int m = 0; m < M; ++m) {
            if (m > 0) {
#pragma unroll
                for (int j = 0; j < 8; ++j) xl[j] = div_q<Q>(xl[j], (float)Q);
            }
            int b[8];
            encode_level<Q>(xl, 1, Q, b, in_range);
            words[m] = pack_word<Q>(b, Q);
        }
        if (pw) {
            if constexpr (M == 2) {
                *reinterpret_cast<uint32_t*>(pw) = words[0] | words[1] << 16;
            } else {
#pragma unroll
                for (int m = 0; m < M; ++m) pw[m] = (Word)words[m];
            }
        }
        uint16_t cid[M];
        uint64_t cc[M];
#pragma unroll
        for (int m = 0; m < M; ++m) cid[m] = a.dec_map[words[m]];
#pragma unroll
        for (int m = 0; m < M; ++m) cc[m] = a.dec_coarse[cid[m]];
#pragma unroll
        for (int j = 0; j < 8; ++j) acc2[j] = kOff;
#pragma unroll
        for (int m = 0; m < M; ++m) {
            int b[8], r2[8];
            unpack_word<Q>(words[m], Q, b);
            r2[0] = 4 * b[0] - 2 * b[1] + b[7];
#pragma unroll
            for (int j = 1; j < 6; ++j) r2[j] = 2 * (b[j] - b[j + 1]) + b[7];
            r2[6] = 2 * b[6] + b[7];
            r2[7] = b[7];
#pragma unroll
            for (int j = 0; j < 8; ++j)
                acc2[j] += (r2[j] - Q * (int)(int8_t)(uint8_t)(cc[m] >> (8 * j))) << (m * kLog2Q);
        }
    } else {
        {
            int b[8];
            encode_level<Q>(xl, 1, Q, b, in_range);
            if (pw) pw[0] = (Word)pack_word<Q>(b, Q);
            dyadic_level_acc<Q, true>(b, s_tab, 0, acc2);
        }
#pragma unroll 1
        for (int m = 1; m < M; ++m) {
#pragma unroll
            for (int j = 0; j < 8; ++j) xl[j] = div_q<Q>(xl[j], (float)Q);
            int b[8];
            encode_level<Q>(xl, 1, Q, b, in_range);
            if (pw) pw[m] = (Word)pack_word<Q>(b, Q);
            dyadic_level_acc<Q, false>(b, s_tab, m * kLog2Q, acc2);
        }
    }
    float acc[8];  // +0 where the sum is zero, as the float sum of the levels
#pragma unroll
    for (int j = 0; j < 8; ++j) acc[j] = 0.5f * (float)(acc2[j] - kOff);
    if (!a.out) return;

    float o[8];
    const float ab = fabsf(beta);
    if (ab >= 0x1p-64f && ab <= 0x1p64f) {
        const float y = __fdiv_rn(1.f, beta);
#pragma unroll
        for (int j = 0; j < 8; ++j)
            o[j] = __builtin_amdgcn_fmed3f(div_by_recip<kSteps>(acc[j], beta, y), -a.clip, a.clip);
    } else {
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const float v = __fdiv_rn(acc[j], beta);
            o[j] = fminf(fmaxf(v, -a.clip), a.clip);
            if (v != v) o[j] = v;  // torch.clamp propagates NaN
        }
    }
    if (a.out_dtype == DT_BF16) {
        uint4 v;
        v.x = f32_to_bf16(o[0]) | ((uint32_t)f32_to_bf16(o[1]) << 16);
        v.y = f32_to_bf16(o[2]) | ((uint32_t)f32_to_bf16(o[3]) << 16);
        v.z = f32_to_bf16(o[4]) | ((uint32_t)f32_to_bf16(o[5]) << 16);
        v.w = f32_to_bf16(o[6]) | ((uint32_t)f32_to_bf16(o[7]) << 16);
        reinterpret_cast<uint4*>(a.out)[i] = v;
    } else {
        float4* p = reinterpret_cast<float4*>(a.out) + 2 * i;
        p[0] = make_float4(o[0], o[1], o[2], o[3]);
        p[1] = make_float4(o[4], o[5], o[6], o[7]);
    }
}

// Calls the layer round-trip kernel takes (its static_asserts, the domain of
// its division and row index; it always tries the fast projection first);
// g_codec_plain = 0 keeps them on the generic kernel.
static bool layer_rt_supported(const CodecArgs& a, int mode)
{
    // betas stored per row, or derived from theta per row of at least 64
    // blocks (fp32 weights: the layer quantizer's input)
    const bool betas = a.use_theta ? a.blocks_per_row >= 64 && a.x_dtype == DT_F32 : a.beta_row != nullptr;
    return g_codec_plain && a.fast_projection && mode == MODE_ROUNDTRIP && a.scale_mode == SCALE_LAYER && betas &&
           (a.q == 8 || a.q == 16 ||
            (a.q == 4 && a.dec_map && ((uintptr_t)a.packed & 3u) == 0)) &&
           a.M >= 1 && a.M <= 4 &&
           !a.dither && !a.codes_f32 &&
           (a.x_dtype == DT_F32 || a.x_dtype == DT_BF16) && (a.out_dtype == DT_F32 || a.out_dtype == DT_BF16) &&
           a.clip > 0.f && a.n <= (int64_t)0xffffffffLL && a.blocks_per_row >= 1 &&
           a.blocks_per_row <= (int64_t)0xffffffffLL && (!a.aux_out || a.aux_n <= a.n);
}

static hipError_t launch_layer_rt(const CodecArgs& args, hipStream_t s)
{
    CodecArgs a = args;
    a.row_div = u32div_of((uint32_t)a.blocks_per_row);
    const dim3 grid((unsigned)((a.n + 255) / 256)), block(256);
    const bool bf = a.x_dtype == DT_BF16;
#define COSET_LAYER(QQ, MM)                                                                          \
    if (a.use_theta) hipLaunchKernelGGL((hnlq_layer_rt_kernel<QQ, MM, false, true>), grid, block, 0, s, a); \
    else if (bf) hipLaunchKernelGGL((hnlq_layer_rt_kernel<QQ, MM, true, false>), grid, block, 0, s, a);     \
    else hipLaunchKernelGGL((hnlq_layer_rt_kernel<QQ, MM, false, false>), grid, block, 0, s, a);            \
    break;
#define COSET_LAYER_Q(QQ)                     \
    switch (a.M) {                            \
    case 1: COSET_LAYER(QQ, 1)                \
    case 2: COSET_LAYER(QQ, 2)                \
    case 3: COSET_LAYER(QQ, 3)                \
    default: COSET_LAYER(QQ, 4)               \
    }                                         \
    break;
    switch (a.q) {
    case 4: COSET_LAYER_Q(4)
    case 8: COSET_LAYER_Q(8)
    default: COSET_LAYER_Q(16)
    }
#undef COSET_LAYER_Q
#undef COSET_LAYER
    return hipGetLastError();
}

// The forward of a small QAT layer in one launch (the layer's F.linear after
// its fused quantizer, coset/core/layers.py:428-484, under no_grad): workgroup
// o derives row o's beta from theta, quantizes the row into LDS with the
// quantizer's own operations (x * beta, two levels encoded, each decoded
// through the tables, sum, / beta, clamp: the W_q values the quantizer
// writes), then computes y[t, o] = sum_k x[t, k] W_q[o, k] + bias[o] for the
// tokens, each as the sum of 256 / P fixed-order partial sums (P the tokens
// rounded up to a power of two) added in order.  fp32 throughout.
constexpr int kHeadMaxCols = 8192;
constexpr int kHeadMaxTokens = 64;

struct HeadArgs {
    const float* W;          // [rows, cols]
    int64_t cols;
    ThetaBeta tb;            // one theta per row
    float clip;
    const float* x;          // [tokens, cols]
    int tokens, tpt;         // tpt: threads per token (256 / P)
    const float* bias;       // nullable [rows]
    float* y;                // [tokens, rows]
    int64_t rows;
    int64_t* step_counter;   // nullable: incremented once per launch
    const uint16_t* map;     // decode tables
    const uint64_t* coarse;
    int fast;
};

template <int Q>
__global__ void __launch_bounds__(256) qat_head_fwd_kernel(HeadArgs h)
{
    __shared__ __align__(16) float s_wq[kHeadMaxCols];
    __shared__ float s_part[256];
    __shared__ float s_beta;
    const int64_t o = blockIdx.x;
    const int tid = threadIdx.x;
    if (tid == 0) {
        float lo, hi, sg;
        theta_beta_terms(h.tb, o, &lo, &hi, &sg);
        s_beta = __fadd_rn(lo, __fmul_rn(sg, __fsub_rn(hi, lo)));
        if (o == 0 && h.step_counter) *h.step_counter += 1;
    }
    __syncthreads();
    const float scale = s_beta;
    const float qf = (float)Q;
    for (int64_t j = tid; j < h.cols / 8; j += blockDim.x) {
        const float4* p = reinterpret_cast<const float4*>(h.W + o * h.cols) + 2 * j;
        const float4 u = p[0], v = p[1];
        float xl[8] = {u.x, u.y, u.z, u.w, v.x, v.y, v.z, v.w};
#pragma unroll
        for (int e = 0; e < 8; ++e) xl[e] = __fmul_rn(xl[e], scale);
        uint32_t words[2];
#pragma unroll
        for (int m = 0; m < 2; ++m) {
            int b[8];
            encode_level<Q>(xl, h.fast, Q, b);
            words[m] = pack_word<Q>(b, Q);
#pragma unroll
            for (int e = 0; e < 8; ++e) xl[e] = div_q<Q>(xl[e], qf);
        }
        float acc[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) acc[e] = 0.f;
        float w = 1.f;
#pragma unroll
        for (int m = 0; m < 2; ++m) {
            int r2[8];
            two_r_tables<Q>(words[m], h.map, h.coarse, r2);
#pragma unroll
            for (int e = 0; e < 8; ++e) acc[e] = __fadd_rn(acc[e], __fmul_rn(w, 0.5f * (float)r2[e]));
            w = __fmul_rn(w, qf);
        }
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            const float q = __fdiv_rn(acc[e], scale);
            float c = fminf(fmaxf(q, -h.clip), h.clip);
            if (q != q) c = q;  // torch.clamp propagates NaN
            s_wq[8 * j + e] = c;
        }
    }
    __syncthreads();
    // token t = tid / tpt sums the columns 4 (part + tpt i) .. + 3 in order
    const int t = tid / h.tpt, part = tid % h.tpt;
    float sum = 0.f;
    if (t < h.tokens) {
        const float* xr = h.x + (int64_t)t * h.cols;
        for (int64_t k = 4 * part; k < h.cols; k += 4 * h.tpt) {
            const float4 xv = *reinterpret_cast<const float4*>(xr + k);
            const float4 wv = *reinterpret_cast<const float4*>(s_wq + k);
            sum = __fmaf_rn(xv.x, wv.x, sum);
            sum = __fmaf_rn(xv.y, wv.y, sum);
            sum = __fmaf_rn(xv.z, wv.z, sum);
            sum = __fmaf_rn(xv.w, wv.w, sum);
        }
    }
    s_part[tid] = sum;
    __syncthreads();
    if (tid < h.tokens) {
        float v = s_part[tid * h.tpt];
        for (int i = 1; i < h.tpt; ++i) v = __fadd_rn(v, s_part[tid * h.tpt + i]);
        if (h.bias) v = __fadd_rn(v, h.bias[o]);
        h.y[(int64_t)tid * h.rows + o] = v;
    }
}

hipError_t launch_qat_head(const float* W, int64_t rows, int64_t cols, const ThetaBeta& tb, float clip, int q,
                           const float* x, int tokens, const float* bias, float* y, int64_t* step_counter,
                           hipStream_t s)
{
    if (rows <= 0 || tokens <= 0) return hipSuccess;
    if ((q != 2 && q != 4) || cols <= 0 || cols % 8 || cols > kHeadMaxCols || tokens > kHeadMaxTokens)
        return hipErrorInvalidValue;
    const DecodeTables* t = nullptr;
    hipError_t e = get_decode_tables(q, 0, &t);
    if (e != hipSuccess) return e;
    HeadArgs h{};
    h.W = W;
    h.cols = cols;
    h.tb = tb;
    h.clip = clip;
    h.x = x;
    h.tokens = tokens;
    int p2 = 1;
    while (p2 < tokens) p2 *= 2;
    h.tpt = 256 / p2;
    h.bias = bias;
    h.y = y;
    h.rows = rows;
    h.step_counter = step_counter;
    h.map = t->cid_map;
    h.coarse = t->coarse;
    h.fast = g_fast_projection;
    if (q == 4)
        hipLaunchKernelGGL(qat_head_fwd_kernel<4>, dim3((unsigned)rows), dim3(256), 0, s, h);
    else
        hipLaunchKernelGGL(qat_head_fwd_kernel<2>, dim3((unsigned)rows), dim3(256), 0, s, h);
    return hipGetLastError();
}

template <int MODE>
static hipError_t launch_mode(const CodecArgs& a, hipStream_t s)
{
    dim3 block(256);
    dim3 grid((unsigned)((std::max<int64_t>(a.n, a.aux_out ? a.aux_n : 0) + 255) / 256));
    const bool wg_beta = a.scale_mode == SCALE_LAYER && a.use_theta && a.blocks_per_row >= 64;
#define COSET_Q(QQ) \
    if (wg_beta && MODE == MODE_ROUNDTRIP && (QQ == 2 || QQ == 4) && a.M == 2 && a.dec_map) \
        hipLaunchKernelGGL((hnlq_codec_kernel<QQ, MODE, true, 2>), grid, block, 0, s, a); \
    else if (wg_beta) hipLaunchKernelGGL((hnlq_codec_kernel<QQ, MODE, true>), grid, block, 0, s, a); \
    else hipLaunchKernelGGL((hnlq_codec_kernel<QQ, MODE, false>), grid, block, 0, s, a); \
    break;
    switch (a.q) {
    case 2: COSET_Q(2)
    case 4: COSET_Q(4)
    case 8: COSET_Q(8)
    case 16: COSET_Q(16)
    default: COSET_Q(0)
    }
#undef COSET_Q
    return hipGetLastError();
}

int g_codec_path = 0;
int g_fast_projection = 1;

hipError_t launch_codec(const CodecArgs& args, int mode, hipStream_t s)
{
    CodecArgs a = args;
    a.fast_projection = g_fast_projection;
    bool lut = lut_path_supported(a, mode) &&
               (g_codec_path == 2 || (g_codec_path == 0 && a.n >= kLutMinBlocks));
    if (a.aux_out && a.aux_n > 0 && (lut || a.n == 0)) {
        // the table kernels take no side cast: it gets its own launch
        hipLaunchKernelGGL(aux_cast_kernel, dim3((unsigned)((a.aux_n + 255) / 256)), dim3(256), 0, s, a);
        hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
        a.aux_out = nullptr;
    }
    if (a.n == 0) return hipSuccess;
    if (lut) return launch_codec_lut(a, mode, s);
    if (g_codec_path == 0 && (a.q == 2 || a.q == 4) && mode != MODE_ENCODE) {
        // layer-sized calls: the generic kernel decodes through the tables
        // (one map and one coarse-point read per level, both L2-resident)
        const DecodeTables* t = nullptr;
        hipError_t e = get_decode_tables(a.q, 0, &t);
        if (e != hipSuccess) return e;
        a.dec_map = t->cid_map;
        a.dec_coarse = t->coarse;
    }
    return launch_codec_generic(a, mode, s);
}

hipError_t launch_codec_generic(const CodecArgs& a, int mode, hipStream_t s)
{
    if (a.n == 0) return hipSuccess;  // (launch_codec has already done a side cast of an empty codec call)
    if (layer_rt_supported(a, mode)) return launch_layer_rt(a, s);
    switch (mode) {
    case MODE_ENCODE: return launch_mode<MODE_ENCODE>(a, s);
    case MODE_DECODE: return launch_mode<MODE_DECODE>(a, s);
    default: return launch_mode<MODE_ROUNDTRIP>(a, s);
    }
}

}  // namespace coset
