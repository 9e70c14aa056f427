// vlut_wide.hip -- the matrix-core wide and deep kernels of the vLUT matmul
// (batches above 32 tokens); the shared decode helpers are in vlut_mfma.hpp.
#include "vlut_mfma.hpp"

namespace coset {

// ---------------------------------------------------------------- MFMA wide kernel
// Tile: 128 output rows (8 row tiles of 16, one per wave) x 64 tokens per
// workgroup, K split over grid.y (partials [split][B][rows]), token tiles of
// 64 over grid.z.  The activations of a stage (64 tokens x 128 K) are loaded
// once per workgroup, two 16-byte loads per thread, and shared by the 8
// waves through LDS (double-buffered, one LDS-only barrier per stage); each
// wave decodes its own row tile's weight pairs into the B operand as the rows
// kernel does and runs 4 MFMAs (one per 16-token tile) per k-quad.  Every
// global load is unconditional (clamped; what lies outside the matrix or the
// workgroup's K range has zero activations), so the waits before a stage
// leave the next stage's loads in flight.

template <int Q, int M, bool BF16, int FMT, int RT, int NW>
__global__ void __launch_bounds__(NW * 64) vlut_wide_kernel(VlutMatmulArgs p)
{
    constexpr int WN = FMT == VLUT_DECODED ? 2 : M;  // uint32 per pair
    constexpr int T = NW * 64;                       // threads
    constexpr int P = 4 * kWideStageKq;              // 16-byte k-block chunks per token and stage
    constexpr int AL = kWideTokens * P / T;          // activation loads per thread and stage
    static_assert(kWideTokens * P % T == 0, "whole activation loads per thread");
    __shared__ uint64_t s_tab[FMT == VLUT_DECODED ? 1 : kSwarSlots];
    __shared__ __align__(16) uint16_t s_act[2][kWideTokens][kWideActStride];

    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, g = lane >> 4;
    const int64_t kb_total = p.K / 8;
    const int64_t kq_total = (kb_total + 3) / 4;
    const int64_t kq_wg = (kq_total + gridDim.y - 1) / gridDim.y;
    const int64_t kq_begin = blockIdx.y * kq_wg;
    const int64_t kq_end = min(kq_total, kq_begin + kq_wg);
    const int64_t rt0 = ((int64_t)blockIdx.x * NW + wave) * RT;  // first row tile of this wave
    const int64_t t_base = (int64_t)blockIdx.z * kWideTokens;
    const uint16_t* act = reinterpret_cast<const uint16_t*>(p.act);
    const int bias = FMT == VLUT_DECODED ? kVlutDecodedBias : p.swar_bias;
    const _Float16 f16_off = (_Float16)(1024 + bias);
    const float f32_off = (float)bias;

    // this thread's share of a stage's activations: chunks threadIdx.x + T i
    // (token c / P, k-block c % P of the stage, 16 bytes each)
    struct Act {
        uint4 v[AL];
    };
    const int a_part = threadIdx.x % P;
    auto load_act = [&](int64_t kq0, Act& ac) {
#pragma unroll
        for (int i = 0; i < AL; ++i) {
            const int tok = (threadIdx.x + T * i) / P;
            const int64_t kb = 4 * kq0 + a_part;
            const bool ok = t_base + tok < p.B && kb < kb_total && kq0 + a_part / 4 < kq_end;
            const uint4 v =
                *reinterpret_cast<const uint4*>(act + (ok ? (t_base + tok) * p.K + kb * 8 : 0));
            // zeroed through a mask the compiler cannot trace back to ok: a
            // select would let it branch around the load, and the waits after
            // a conditional load drain the queue
            uint32_t m;
            __asm__("v_mov_b32 %0, %1" : "=v"(m) : "v"(ok ? ~0u : 0u));
            ac.v[i] = make_uint4(v.x & m, v.y & m, v.z & m, v.w & m);
        }
    };
    struct W {
        uint32_t w[RT][kWideStageKq][WN];
    };
    auto load_w = [&](int64_t kq0, W& ws) {
#pragma unroll
        for (int t = 0; t < RT; ++t) {
            const int64_t r0 = (rt0 + t) * 16, row = r0 + (lane & 15);
            // rows that hold weights (whole tiles in the tiled formats)
            const bool rows_ok = (FMT == VLUT_TILED || FMT == VLUT_DECODED) ? r0 < p.rows : row < p.rows;
#pragma unroll
            for (int j = 0; j < kWideStageKq; ++j) {
                const int64_t kb = 4 * (kq0 + j) + g;
                const bool ok = rows_ok && kb < kb_total;
                // outside the matrix: pair (0, 0) instead, under zero
                // activations or an output that is not stored
                load_pair<Q, M, WN>(p, FMT, ok ? row : 0, ok ? kb : 0, kb_total, ws.w[t][j]);
            }
        }
    };
    float4_t acc[RT][4];
#pragma unroll
    for (int t = 0; t < RT; ++t)
#pragma unroll
        for (int s = 0; s < 4; ++s) acc[t][s] = (float4_t){0.f, 0.f, 0.f, 0.f};

    if (FMT != VLUT_DECODED) {
        for (int i = threadIdx.x; i < 512 + p.n_coarse; i += blockDim.x) s_tab[i] = p.swar[i];
    }
    const int stages = (int)((kq_end - kq_begin + kWideStageKq - 1) / kWideStageKq);
    W w_now, w_next;
    Act a_next;
    load_act(kq_begin, a_next);
    load_w(kq_begin, w_now);
    for (int st = 0; st < stages; ++st) {
        const int64_t kq0 = kq_begin + (int64_t)st * kWideStageKq;
        const int buf = st & 1;
#pragma unroll
        for (int i = 0; i < AL; ++i)
            *reinterpret_cast<uint4*>(&s_act[buf][(threadIdx.x + T * i) / P][a_part * 8]) = a_next.v[i];
        lds_barrier();
        // the next stage's loads go out before this stage's products
        const int64_t kq1 = st + 1 < stages ? kq0 + kWideStageKq : kq0;
        load_act(kq1, a_next);
        load_w(kq1, w_next);
        __asm__ volatile("" ::: "memory");  // the loads stay ahead of the products
        uint4 av_all[kWideStageKq][4];
#pragma unroll
        for (int j = 0; j < kWideStageKq; ++j)
#pragma unroll
            for (int s = 0; s < 4; ++s)
                av_all[j][s] = *reinterpret_cast<const uint4*>(&s_act[buf][16 * s + (lane & 15)][(4 * j + g) * 8]);
#pragma unroll
        for (int j = 0; j < kWideStageKq; ++j) {
#pragma unroll
            for (int t = 0; t < RT; ++t) {
                uint4 bw;
                if constexpr (FMT == VLUT_DECODED)
                    bw = bytes_to_operand<BF16>(w_now.w[t][j][0], w_now.w[t][j][1 % WN], f16_off, f32_off);
                else
                    bw = decode_pair_swar<Q, M, BF16>(s_tab, w_now.w[t][j], f16_off, f32_off);
#pragma unroll
                for (int s = 0; s < 4; ++s) {
                    const uint4 av = av_all[j][s];
                    if (BF16)
                        acc[t][s] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
                            __builtin_bit_cast(bf16x8_t, av), __builtin_bit_cast(bf16x8_t, bw), acc[t][s], 0, 0, 0);
                    else
                        acc[t][s] = __builtin_amdgcn_mfma_f32_16x16x32_f16(
                            __builtin_bit_cast(half8_t, av), __builtin_bit_cast(half8_t, bw), acc[t][s], 0, 0, 0);
                }
            }
        }
        w_now = w_next;
    }

    // D[token = 16 s + 4 (lane / 16) + i][row = lane % 16]
#pragma unroll
    for (int t = 0; t < RT; ++t) {
        const int64_t o = (rt0 + t) * 16 + (lane & 15);
        if (o >= p.rows) continue;
        const float sc = p.scale ? (p.scale_mode == 0 ? p.scale[o] : 1.f / p.scale[o]) : 1.f;
#pragma unroll
        for (int s = 0; s < 4; ++s)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int64_t tok = t_base + 16 * s + 4 * g + i;
                if (tok >= p.B) continue;
                if (gridDim.y == 1)
                    p.out[tok * p.rows + o] =
                        vlut_epilogue(acc[t][s][i] * 0.5f * sc, o, p.bias, p.lsq_alpha, p.lsq_qmax);
                else
                    p.partial[((int64_t)blockIdx.y * p.B + tok) * p.rows + o] = acc[t][s][i];
            }
    }
}

// ---------------------------------------------------------------- MFMA deep kernel
// Tile: 64 output rows x 64 tokens per workgroup of 8 waves; K split over
// grid.y (partials [split][B][rows]) and, inside the workgroup, over the 8
// waves.  Each wave owns all 4 row tiles of 16 rows (4 weight operands per
// k-quad) and all 4 token tiles, so every activation operand read from LDS
// feeds 4 MFMAs (the wide kernel's one-row-tile waves re-read all 64 tokens'
// activations per 16 rows).  The workgroup issues every load of its K slice
// up front -- activations (64 tokens x up to 1024 K, 128 KiB) straight into
// LDS, the waves' weight pairs into registers -- then runs the products; the 8 waves'
// partial tiles are summed in LDS in wave order, so a split writes one
// partial (or, unsplit, the output) and the sums are deterministic.

// 16 zero bytes, the source of activation chunks outside the matrix
static __device__ uint4 g_vlut_zero16;

template <int Q, int M, bool BF16, int FMT>
__global__ void __launch_bounds__(kDeepNW * 64) vlut_deep_kernel(VlutMatmulArgs p)
{
    constexpr int WN = FMT == VLUT_DECODED ? 2 : M;  // uint32 per pair
    constexpr bool D6 = FMT == VLUT_DECODED6;
    constexpr bool DEC = FMT == VLUT_DECODED || D6;   // no table reads
    constexpr int T = kDeepNW * 64;
    constexpr int CH = 4 * kDeepKqWg;                // 16-byte activation chunks per token row
    constexpr int AL = kDeepTokens * CH / T;         // activation loads per thread
    static_assert(kDeepTokens * CH % T == 0, "whole activation loads per thread");
    static_assert(kDeepNW * kDeepRows * kDeepTokens * 4 <= kDeepTokens * kDeepStride * 2,
                  "the cross-wave sum fits in the activation buffer");
    static_assert(kDeepStride * 2 % 16 == 0, "16-byte aligned token rows");
    __shared__ __align__(16) uint16_t s_act[kDeepTokens * kDeepStride];
    __shared__ uint64_t s_tab[DEC ? 1 : kSwarSlots];

    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, g = lane >> 4;
    const int64_t kb_total = p.K / 8;
    const int64_t kq_total = (kb_total + 3) / 4;
    // <= kDeepKqWg (the plan's splits); the 6-byte format's slices start on a
    // chunk of 8 k-quads and every wave takes half a chunk (4 k-quads); the
    // others' slices are whole multiples of 16 k-quads, so every wave's range
    // starts on an even k-quad (the 8-byte decoded format's 16-byte loads)
    constexpr int64_t KA = D6 ? kD6Steps : 2 * kDeepNW;
    const int64_t kq_wg = ((kq_total + gridDim.y - 1) / gridDim.y + KA - 1) / KA * KA;
    const int64_t kq_begin = blockIdx.y * kq_wg;
    const int64_t kq_end = min(kq_total, kq_begin + kq_wg);
    const int kqw = D6 ? kDeepKqWave : (int)((kq_wg + kDeepNW - 1) / kDeepNW);   // k-quads per wave, <= 4
    static_assert(!D6 || 2 * kDeepKqWave == kD6Steps, "a wave's k-quads are half a chunk");
    const int64_t rb = (int64_t)blockIdx.x * kDeepRows;
    const int64_t t_base = (int64_t)blockIdx.z * kDeepTokens;
    const uint16_t* act = reinterpret_cast<const uint16_t*>(p.act);
    const int bias = FMT == VLUT_DECODED ? kVlutDecodedBias : D6 ? p.d6_bias : p.swar_bias;
    const _Float16 f16_off = (_Float16)(1024 + bias);
    const float f32_off = (float)bias;

    // activations of the workgroup's K slice, loaded straight into LDS
    // (global_load_lds, 16 bytes a lane: lane l's chunk lands 16 l bytes after
    // the wave's base, which is uniform because a wave's 64 chunks c =
    // threadIdx.x + T i lie in one token row, CH = 128 chunks long).  Chunk c
    // is (token c / CH, local k-block c % CH); outside the matrix or the slice
    // the lane reads 16 zero bytes instead.
    static_assert(CH % 64 == 0 && T % 64 == 0, "a wave's chunks share one token row");
#pragma unroll
    for (int i = 0; i < AL; ++i) {
        const int c = threadIdx.x + T * i;
        const int c0 = c - lane;
        const int tok = c / CH, kbl = c % CH;
        const int64_t kb = 4 * kq_begin + kbl;
        const bool ok = t_base + tok < p.B && kb < kb_total && kq_begin + kbl / 4 < kq_end;
        const uint4* src = ok ? reinterpret_cast<const uint4*>(act + (t_base + tok) * p.K + kb * 8) : &g_vlut_zero16;
        __builtin_amdgcn_global_load_lds(src, &s_act[(c0 / CH) * kDeepStride + (c0 % CH) * 8], 16, 0, 0);
    }
    // this wave's weight pairs: row tiles rt, k-quads kq_begin + wave * kqw + j
    uint32_t w[D6 ? 1 : kDeepRT][D6 ? 1 : kDeepKqWave][WN];
    uint32_t w6[D6 ? kDeepRT : 1][kD6Words];   // 6-byte format: half a chunk per row tile (words 0-5)
#pragma unroll
    for (int rt = 0; rt < kDeepRT; ++rt) {
        const int64_t r0 = rb + 16 * rt, row = r0 + (lane & 15);
        const bool rows_ok = (FMT == VLUT_TILED || DEC) ? r0 < p.rows : row < p.rows;
        if constexpr (D6) {
            // k-quads kq0 .. kq0 + 3: the first or second half of a chunk (outside
            // the matrix or the slice: the first half of row tile 0's chunk 0)
            const int64_t kq0 = kq_begin + (int64_t)wave * kDeepKqWave;
            const bool ok = rows_ok && kq0 < kq_end;
            const uint32_t* src = reinterpret_cast<const uint32_t*>(p.words) +
                                  vlut_word_index(FMT, ok ? row : (lane & 15), ok ? 4 * kq0 + g : g, 0, kb_total, M) +
                                  (ok ? (kq0 % kD6Steps) * kD6Words / kD6Steps : 0);
            const uint4 v0 = *reinterpret_cast<const uint4*>(src);   // 24-byte halves: 8-byte aligned
            const uint2 v1 = *reinterpret_cast<const uint2*>(src + 4);
            w6[rt][0] = v0.x; w6[rt][1] = v0.y; w6[rt][2] = v0.z; w6[rt][3] = v0.w; w6[rt][4] = v1.x; w6[rt][5] = v1.y;
#pragma unroll
            for (int i = 6; i < kD6Words; ++i) w6[rt][i] = 0u;
        } else if constexpr (FMT == VLUT_DECODED) {
            // k-quads j, j + 1 of the wave (kq_begin and kqw are even) in one
            // 16-byte load; past the range, pair (0, 0) under zero activations
#pragma unroll
            for (int j = 0; j < kDeepKqWave; j += 2) {
                const int64_t kq = kq_begin + (int64_t)wave * kqw + j;
                const int64_t kb = 4 * kq + g;
                const bool ok = rows_ok && j < kqw && kq < kq_end && kb < kb_total;
                const uint4 v = *reinterpret_cast<const uint4*>(reinterpret_cast<const uint32_t*>(p.words) +
                                                                vlut_word_index(FMT, ok ? row : 0, ok ? kb : 0, 0,
                                                                                kb_total, M));
                w[rt][j][0] = v.x;
                w[rt][j][1 % WN] = v.y;
                w[rt][j + 1][0] = v.z;
                w[rt][j + 1][1 % WN] = v.w;
            }
        } else {
#pragma unroll
            for (int j = 0; j < kDeepKqWave; ++j) {
                const int64_t kq = kq_begin + (int64_t)wave * kqw + j;
                const int64_t kb = 4 * kq + g;
                const bool ok = rows_ok && j < kqw && kq < kq_end && kb < kb_total;
                load_pair<Q, M, WN>(p, FMT, ok ? row : 0, ok ? kb : 0, kb_total, w[rt][j]);
            }
        }
    }
    if (!DEC) {
        for (int i = threadIdx.x; i < 512 + p.n_coarse; i += T) s_tab[i] = p.swar[i];
    }
    // the LDS writes of global_load_lds complete with the loads (vmcnt)
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();

    float4_t acc[kDeepRT][4];
#pragma unroll
    for (int rt = 0; rt < kDeepRT; ++rt)
#pragma unroll
        for (int s = 0; s < 4; ++s) acc[rt][s] = (float4_t){0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int j = 0; j < kDeepKqWave; ++j) {
        const int kql = wave * kqw + j;
        if (j >= kqw || kq_begin + kql >= kq_end) break;   // wave-uniform
        uint4 a[4];
#pragma unroll
        for (int s = 0; s < 4; ++s)
            a[s] = *reinterpret_cast<const uint4*>(&s_act[(16 * s + (lane & 15)) * kDeepStride + kql * 32 + 8 * g]);
#pragma unroll
        for (int rt = 0; rt < kDeepRT; ++rt) {
            uint4 bw;
            if constexpr (D6) {
                uint32_t x0, x1;
                d6_pair(w6[rt], j, x0, x1);
                bw = bytes_to_operand<BF16>(x0, x1, f16_off, f32_off);
            } else if constexpr (FMT == VLUT_DECODED) {
                bw = bytes_to_operand<BF16>(w[rt][j][0], w[rt][j][1 % WN], f16_off, f32_off);
            } else {
                bw = decode_pair_swar<Q, M, BF16>(s_tab, w[rt][j], f16_off, f32_off);
            }
#pragma unroll
            for (int s = 0; s < 4; ++s) {
                if (BF16)
                    acc[rt][s] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
                        __builtin_bit_cast(bf16x8_t, a[s]), __builtin_bit_cast(bf16x8_t, bw), acc[rt][s], 0, 0, 0);
                else
                    acc[rt][s] = __builtin_amdgcn_mfma_f32_16x16x32_f16(
                        __builtin_bit_cast(half8_t, a[s]), __builtin_bit_cast(half8_t, bw), acc[rt][s], 0, 0, 0);
            }
        }
    }

    // the 8 waves' tiles summed in wave order through LDS (the activation
    // buffer, no longer read).  Element i of acc[rt][s] in lane l is
    // D[token 16 s + 4 (l / 16) + i][row 16 rt + l % 16]; a wave stores it
    // at red[((wave * 16 + rt * 4 + s) * 4 + i) * 64 + l], where rows
    // 4 r .. 4 r + 3 of a row tile and token are 4 consecutive floats
    __syncthreads();
    float* red = reinterpret_cast<float*>(s_act);
#pragma unroll
    for (int rt = 0; rt < kDeepRT; ++rt)
#pragma unroll
        for (int s = 0; s < 4; ++s)
#pragma unroll
            for (int i = 0; i < 4; ++i) red[((wave * 16 + rt * 4 + s) * 4 + i) * 64 + lane] = acc[rt][s][i];
    __syncthreads();
    // thread e: token t = e / 16 of the tile and its rows 4 (e % 16) .. + 3,
    // so 16 threads write one token's 64 rows as 16-byte stores
    for (int e = threadIdx.x; e < kDeepTokens * (kDeepRows / 4); e += T) {
        const int t = e >> 4, q = e & 15;
        const int s = t >> 4, g = (t >> 2) & 3, i = t & 3;
        const int rt = q >> 2, r4 = 4 * (q & 3);
        float sum[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int wv = 0; wv < kDeepNW; ++wv) {
            const float4 v = *reinterpret_cast<const float4*>(&red[((wv * 16 + rt * 4 + s) * 4 + i) * 64 + 16 * g + r4]);
            sum[0] += v.x;
            sum[1] += v.y;
            sum[2] += v.z;
            sum[3] += v.w;
        }
        const int64_t tok = t_base + t, o0 = rb + 16 * rt + r4;
        if (tok >= p.B || o0 >= p.rows) continue;
        float* dst;
        if (gridDim.y == 1) {
            dst = p.out + tok * p.rows + o0;
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                const int64_t o = o0 + k < p.rows ? o0 + k : p.rows - 1;
                const float sc = p.scale ? (p.scale_mode == 0 ? p.scale[o] : 1.f / p.scale[o]) : 1.f;
                sum[k] = vlut_epilogue(sum[k] * 0.5f * sc, o, p.bias, p.lsq_alpha, p.lsq_qmax);
            }
        } else {
            dst = p.partial + ((int64_t)blockIdx.y * p.B + tok) * p.rows + o0;
        }
        if (o0 + 3 < p.rows && ((uintptr_t)dst & 15) == 0) {
            *reinterpret_cast<float4*>(dst) = make_float4(sum[0], sum[1], sum[2], sum[3]);
        } else {
#pragma unroll
            for (int k = 0; k < 4; ++k)
                if (o0 + k < p.rows) dst[k] = sum[k];
        }
    }
}

namespace {

template <int Q, int M, bool BF16>
void launch_wide_fmt(const VlutMatmulArgs& p, int splits, hipStream_t s)
{
    dim3 grid((unsigned)((p.rows + kWideRows - 1) / kWideRows), (unsigned)splits,
              (unsigned)((p.B + kWideTokens - 1) / kWideTokens));
#define COSET_WIDE(F) \
    hipLaunchKernelGGL((vlut_wide_kernel<Q, M, BF16, F, kWideRT, kWideNW>), grid, dim3(kWideNW * 64), 0, s, p)
    switch (p.prepared) {
    case VLUT_RAW: COSET_WIDE(VLUT_RAW); break;
    case VLUT_PREPARED: COSET_WIDE(VLUT_PREPARED); break;
    case VLUT_DECODED: COSET_WIDE(VLUT_DECODED); break;
    default: COSET_WIDE(VLUT_TILED); break;
    }
#undef COSET_WIDE
}

template <int Q>
hipError_t dispatch_wide(const VlutMatmulArgs& p, int splits, hipStream_t s)
{
    const bool bf = p.act_dtype == DT_BF16;
    switch (p.M) {
#define COSET_M(MM) \
    case MM: \
        if constexpr (Q == 2 || MM <= 2) { \
            if (bf) launch_wide_fmt<Q, MM, true>(p, splits, s); else launch_wide_fmt<Q, MM, false>(p, splits, s); \
            return hipGetLastError(); \
        } \
        return hipErrorInvalidValue;
    COSET_M(1) COSET_M(2) COSET_M(3) COSET_M(4)
#undef COSET_M
    default: return hipErrorInvalidValue;
    }
}

template <int Q, int M, bool BF16>
void launch_deep_fmt(const VlutMatmulArgs& p, int splits, hipStream_t s)
{
    dim3 grid((unsigned)((p.rows + kDeepRows - 1) / kDeepRows), (unsigned)splits,
              (unsigned)((p.B + kDeepTokens - 1) / kDeepTokens));
#define COSET_DEEP(F) hipLaunchKernelGGL((vlut_deep_kernel<Q, M, BF16, F>), grid, dim3(kDeepNW * 64), 0, s, p)
    switch (p.prepared) {
    case VLUT_RAW: COSET_DEEP(VLUT_RAW); break;
    case VLUT_PREPARED: COSET_DEEP(VLUT_PREPARED); break;
    case VLUT_DECODED: COSET_DEEP(VLUT_DECODED); break;
    case VLUT_DECODED6: COSET_DEEP(VLUT_DECODED6); break;
    default: COSET_DEEP(VLUT_TILED); break;
    }
#undef COSET_DEEP
}

template <int Q>
hipError_t dispatch_deep(const VlutMatmulArgs& p, int splits, hipStream_t s)
{
    const bool bf = p.act_dtype == DT_BF16;
    switch (p.M) {
#define COSET_M(MM) \
    case MM: \
        if constexpr (Q == 2 || MM <= 2) { \
            if (bf) launch_deep_fmt<Q, MM, true>(p, splits, s); else launch_deep_fmt<Q, MM, false>(p, splits, s); \
            return hipGetLastError(); \
        } \
        return hipErrorInvalidValue;
    COSET_M(1) COSET_M(2) COSET_M(3) COSET_M(4)
#undef COSET_M
    default: return hipErrorInvalidValue;
    }
}

}  // namespace

hipError_t vlut_launch_wide(const VlutMatmulArgs& p, int splits, hipStream_t s)
{
    return p.q == 4 ? dispatch_wide<4>(p, splits, s) : dispatch_wide<2>(p, splits, s);
}

hipError_t vlut_launch_deep(const VlutMatmulArgs& p, int splits, hipStream_t s)
{
    return p.q == 4 ? dispatch_deep<4>(p, splits, s) : dispatch_deep<2>(p, splits, s);
}

}  // namespace coset
