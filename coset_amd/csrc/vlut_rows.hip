// vlut_rows.hip -- the matrix-core rows kernel of the vLUT matmul (batches
// up to 32 tokens); the shared decode helpers are in vlut_mfma.hpp.
#include "vlut_mfma.hpp"

namespace coset {

// ---------------------------------------------------------------- MFMA rows kernel
// Tile: 16 output rows per workgroup, K split over its 8 waves (and over
// grid.y when the row tiles alone cannot fill the GPU), up to 16 * NTILE
// tokens (grid.z beyond).  In each step lane l owns row l % 16 and k-block
// 4 kq + l / 16: it decodes that pair's 2 x_hat through the byte tables
// straight into its 8-half B operand of one 16x16x32 MFMA, and takes
// act[token][8 kb, 8 kb + 8) as its A operand.  Any assignment of K
// positions to (lane group, operand slot) works as long as A and B use the
// same one, which holds since both come from the same kb.  In the tiled
// format a step's 64 word groups are one contiguous run.  The waves' sums
// meet in LDS; with one K split the workgroup writes the output.
// Activations: with TB = 0 every lane loads its A operand from global memory
// (16 tokens x 64 bytes per wave load).  With TB > 0 (one 16-token tile, at
// most TB tokens) each wave copies its chunk's K slice of every token into
// LDS rows of its own with whole-row loads (two tokens x 512 bytes per wave
// load) and reads its A operands from there: fewer, coalesced loads, and no
// barrier, since no other wave touches those rows and a wave's LDS
// operations complete in order.  A chunk's activation loads are issued ahead
// of its weight loads.  The staged kernels take a wave's K range of at most
// two chunks (kRowsStageKq k-quads) in one piece.
constexpr int kRowsStageKq = 16;                             // k-quads of a wave's staged slice (two chunks)
constexpr int kRowsStageRow = 4 * kRowsStageKq * 16 + 16;    // bytes per staged token row (64 k-blocks, 16-byte pad)

// SPLIT (staged, bf16): act is fp32 [planes_b, K] and the staging writes
// each token's three bf16 planes (split3) to token rows b, planes_b + b and
// 2 planes_b + b, so the kernel multiplies the planes as 3 planes_b tokens
// without a separate split launch.
template <int Q, int M, bool BF16, int NTILE, int FMT, int TB, bool SPLIT = false>
__global__ void __launch_bounds__(kRowsWaves * 64) vlut_rows_kernel(VlutMatmulArgs p)
{
    constexpr int CH = 8 / NTILE;  // steps per prefetch chunk
    static_assert(TB == 0 || (NTILE == 1 && TB <= 16), "staged activations: one 16-token tile");
    static_assert(!SPLIT || (TB > 0 && BF16), "the split staging writes bf16 token rows");
    static_assert(TB == 0 || 2 * CH == kRowsStageKq, "a staged wave range is two chunks");
    constexpr bool DEC = FMT == VLUT_DECODED || FMT == VLUT_DECODED6;  // no table reads
    // raw words: the cid map (q^8 16-bit entries, 128 KiB at q = 4) staged in
    // LDS where it fits beside the kernel's other buffers (one 16-token tile,
    // at most one staged token), so a word's coarse point costs LDS reads
    // instead of a gather from global memory that waits on the word's load
    constexpr int kMapN = Q == 2 ? 256 : 65536;
    constexpr int kLdsOther = (DEC ? 8 : kSwarSlots * 8) + kRowsWaves * NTILE * 4 * 64 * 4 +
                              (TB == 0 ? 16 : kRowsWaves * TB * kRowsStageRow);
    constexpr bool LMAP = FMT == VLUT_RAW && kLdsOther + 2 * kMapN <= 160 * 1024;
    __shared__ uint64_t s_tab[DEC ? 1 : kSwarSlots];
    __shared__ float s_red[kRowsWaves][NTILE * 4][64];
    __shared__ __align__(16) unsigned char s_stage[TB == 0 ? 16 : kRowsWaves * TB * kRowsStageRow];
    __shared__ __align__(16) uint16_t s_map[LMAP ? kMapN : 8];

    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, g = lane >> 4;
    const int64_t kb_total = p.K / 8;
    const int64_t kq_total = (kb_total + 3) / 4;
    // split and wave ranges start on an even k-quad (the 8-byte decoded format
    // keeps a lane's two k-quads 2i, 2i + 1 together; every format aligns the
    // same way, so they sum in the same order) or, for the 6-byte format, on
    // a chunk of 8 k-quads
    constexpr int64_t KA = FMT == VLUT_DECODED6 ? kD6Steps : 2;
    const int64_t kq_wg = ((kq_total + gridDim.y - 1) / gridDim.y + KA - 1) / KA * KA;
    const int64_t kq_begin = blockIdx.y * kq_wg;
    const int64_t kq_end = min(kq_total, kq_begin + kq_wg);
    const int64_t kq_wave = ((kq_end - kq_begin + kRowsWaves - 1) / kRowsWaves + KA - 1) / KA * KA;
    const int64_t w0 = kq_begin + wave * kq_wave;
    const int64_t w1 = min(kq_end, w0 + kq_wave);
    const int64_t r0 = (int64_t)blockIdx.x * 16;
    const int64_t row = r0 + (lane & 15);
    const int64_t t_base = (int64_t)blockIdx.z * 16 * NTILE;
    const uint16_t* act = reinterpret_cast<const uint16_t*>(p.act);
    const int bias = FMT == VLUT_DECODED ? kVlutDecodedBias : FMT == VLUT_DECODED6 ? p.d6_bias : p.swar_bias;
    const _Float16 f16_off = (_Float16)(1024 + bias);
    const float f32_off = (float)bias;
    constexpr int WN = FMT == VLUT_DECODED ? 2 : M;  // uint32 per pair
    constexpr int W6 = FMT == VLUT_DECODED6 ? CH * kD6Words / kD6Steps : 1;  // 6-byte format: uint32 per lane and chunk
    static_assert(FMT != VLUT_DECODED6 || (CH * kD6Words) % kD6Steps == 0, "whole words per chunk");
    // the epilogue's per-row scale and bias, loaded with the first loads: a
    // thread's outputs all lie in row r0 + threadIdx.x % 16.  The division of
    // scale_mode 1 waits for its load, so it is done in the epilogue: here it
    // would hold back every weight load behind one memory round trip.
    const int64_t o_ep = min(r0 + (int64_t)(threadIdx.x & 15), p.rows - 1);
    const float sc_raw = p.scale ? p.scale[o_ep] : 1.f;
    const float bias_ep = p.bias ? p.bias[o_ep] : 0.f;

    struct Chunk {
        uint32_t w[FMT == VLUT_DECODED6 ? 1 : CH][WN];
        uint32_t w6[W6];                   // 6-byte format: the lane's steps of the chunk
        uint4 a[TB == 0 ? CH : 1][NTILE];  // A operands (TB = 0), masked in run
    };
    // Every load is unconditional, with a clamped address where it lies
    // outside the matrix, the wave's K range or the batch, and its value is
    // masked where it is used: the number of loads issued after a chunk's is
    // then the same on every path, so the wait for that chunk leaves the later
    // loads in flight.  (Weights of an out-of-range k-block meet zero
    // activations, and rows past the matrix are never written.)
    auto load = [&](int64_t c0, Chunk& ck) {
        if constexpr (FMT == VLUT_DECODED6) {
            // steps c0 .. c0 + CH - 1 of one chunk (c0 is a multiple of CH and the
            // wave's range starts on a chunk); past the wave's range, chunk 0
            const bool ok = c0 < w1;
            const uint32_t* src = reinterpret_cast<const uint32_t*>(p.words) +
                                  vlut_word_index(FMT, ok ? row : r0, ok ? 4 * c0 + g : g, 0, kb_total, M) +
                                  (ok ? (c0 % kD6Steps) * kD6Words / kD6Steps : 0);
            if constexpr (W6 == 12) {
                const uint4 v0 = reinterpret_cast<const uint4*>(src)[0], v1 = reinterpret_cast<const uint4*>(src)[1],
                            v2 = reinterpret_cast<const uint4*>(src)[2];
                const uint32_t v[12] = {v0.x, v0.y, v0.z, v0.w, v1.x, v1.y, v1.z, v1.w, v2.x, v2.y, v2.z, v2.w};
#pragma unroll
                for (int i = 0; i < 12; ++i) ck.w6[i] = v[i];
            } else if constexpr (W6 == 6) {
                const uint4 v0 = *reinterpret_cast<const uint4*>(src);  // 24-byte offsets: 8-byte aligned
                const uint2 v1 = *reinterpret_cast<const uint2*>(src + 4);
                ck.w6[0] = v0.x; ck.w6[1] = v0.y; ck.w6[2] = v0.z; ck.w6[3] = v0.w; ck.w6[4] = v1.x; ck.w6[5] = v1.y;
            } else {
#pragma unroll
                for (int i = 0; i < W6; ++i) ck.w6[i] = src[i];
            }
        }
#pragma unroll
        for (int st = 0; st < CH; ++st) {
            const int64_t kq = c0 + st;
            const int64_t kb = 4 * kq + g;
            const bool ok = kq < w1 && kb < kb_total && (FMT == VLUT_TILED || DEC || row < p.rows);
            if constexpr (FMT == VLUT_DECODED && CH % 2 == 0) {
                // steps st, st + 1 (k-quads 2i, 2i + 1: c0 is even) in one 16-byte load;
                // the second may lie past the range (padding or masked activations)
                if (st % 2 == 0) {
                    const uint4 v = *reinterpret_cast<const uint4*>(reinterpret_cast<const uint32_t*>(p.words) +
                                                                    vlut_word_index(FMT, ok ? row : r0, ok ? kb : 0,
                                                                                    0, kb_total, M));
                    ck.w[st][0] = v.x;
                    ck.w[st][1 % WN] = v.y;
                    ck.w[st + 1][0] = v.z;
                    ck.w[st + 1][1 % WN] = v.w;
                }
            } else if constexpr (LMAP) {
                // the words alone; their cids come from s_map when the pair is decoded
                const uint16_t* src = reinterpret_cast<const uint16_t*>(p.words) +
                                      vlut_word_index(FMT, ok ? row : r0, ok ? kb : 0, 0, kb_total, M);
                constexpr uint32_t kMask = kMapN - 1;  // map bounds for any input
#pragma unroll
                for (int m = 0; m < M; ++m) ck.w[st][m] = src[m] & kMask;
            } else if constexpr (FMT != VLUT_DECODED6) {
                load_pair<Q, M, WN>(p, FMT, ok ? row : r0, ok ? kb : 0, kb_total, ck.w[st]);
            }
            if constexpr (TB == 0) {
#pragma unroll
                for (int s = 0; s < NTILE; ++s) {
                    const int64_t tok = t_base + 16 * s + (lane & 15);
                    const bool oka = kq < w1 && kb < kb_total && tok < p.B;
                    ck.a[st][s] = *reinterpret_cast<const uint4*>(act + (oka ? tok * p.K + kb * 8 : 0));
                }
            }
        }
    };
    // the decode tables into LDS (every workgroup's own copy), then a barrier;
    // the map's 16-byte loads (16 a thread at q = 4) all go out before the
    // first store, so the staging waits for one round trip
    auto stage_tables = [&]() {
        if constexpr (!DEC) {
            // the <a, c> table's loads go out unconditionally (clamped index;
            // 512 + n_coarse <= kSwarSlots entries), then the stores, so the
            // staging waits for one round trip, not one per loop iteration
            constexpr int kThreads = kRowsWaves * 64;
            constexpr int kTabPer = (kSwarSlots + kThreads - 1) / kThreads;
            const int n_tab = 512 + p.n_coarse;
            uint64_t tv[kTabPer];
#pragma unroll
            for (int j = 0; j < kTabPer; ++j) {
                const int i = (int)threadIdx.x + j * kThreads;
                tv[j] = p.swar[i < n_tab ? i : 0];
            }
            if constexpr (LMAP) {
                constexpr int kVec = kMapN / 8;
                const uint4* src = reinterpret_cast<const uint4*>(p.map);
                uint4* dst = reinterpret_cast<uint4*>(s_map);
                if constexpr (kVec >= kThreads) {
                    static_assert(kVec % kThreads == 0, "whole rounds of map loads");
                    constexpr int kPer = kVec / kThreads;
                    uint4 v[kPer];
#pragma unroll
                    for (int j = 0; j < kPer; ++j) v[j] = src[j * kThreads + threadIdx.x];
#pragma unroll
                    for (int j = 0; j < kPer; ++j) dst[j * kThreads + threadIdx.x] = v[j];
                } else {
                    for (int i = threadIdx.x; i < kVec; i += kThreads) dst[i] = src[i];
                }
            }
#pragma unroll
            for (int j = 0; j < kTabPer; ++j) {
                const int i = (int)threadIdx.x + j * kThreads;
                if (i < n_tab) s_tab[i] = tv[j];
            }
            __syncthreads();
        }
    };
    float4_t acc[NTILE];
#pragma unroll
    for (int s = 0; s < NTILE; ++s) acc[s] = (float4_t){0.f, 0.f, 0.f, 0.f};
    auto run = [&](const Chunk& ck, int64_t c0) {
#pragma unroll
        for (int st = 0; st < CH; ++st) {
            uint4 a[NTILE];
            const int64_t kq = c0 + st, kb = 4 * kq + g;
            if constexpr (TB > 0) {
                // token lane % 16 (rows at or past the batch were not written: masked),
                // local k-block 4 (kq - w0) + lane / 16 (zeros past the wave's range)
                const int tok = lane & 15;
                const int tr = tok < TB ? tok : TB - 1;
                const uint4 v = *reinterpret_cast<const uint4*>(
                    &s_stage[(wave * TB + tr) * kRowsStageRow + (4 * (int)(kq - w0) + g) * 16]);
                a[0] = t_base + tok < p.B ? v : make_uint4(0u, 0u, 0u, 0u);
            } else {
#pragma unroll
                for (int s = 0; s < NTILE; ++s) {
                    const bool oka = kq < w1 && kb < kb_total && t_base + 16 * s + (lane & 15) < p.B;
                    a[s] = oka ? ck.a[st][s] : make_uint4(0u, 0u, 0u, 0u);
                }
            }
            uint4 bw;
            if constexpr (FMT == VLUT_DECODED6) {
                // step st of the loaded words: pair (c0 + st) % 8 of the chunk, i.e.
                // pair st of the CH loaded (CH divides 8)
                uint32_t x0, x1;
                uint32_t w12[12];
#pragma unroll
                for (int i = 0; i < 12; ++i) w12[i] = i < W6 ? ck.w6[i] : 0u;
                d6_pair(w12, st, x0, x1);
                bw = bytes_to_operand<BF16>(x0, x1, f16_off, f32_off);
            } else if constexpr (FMT == VLUT_DECODED) {
                bw = bytes_to_operand<BF16>(ck.w[st][0], ck.w[st][1 % WN], f16_off, f32_off);
            } else if constexpr (LMAP) {
                uint32_t wv[M];
#pragma unroll
                for (int m = 0; m < M; ++m) wv[m] = ((uint32_t)s_map[ck.w[st][m]] << 16) | ck.w[st][m];
                bw = decode_pair_swar<Q, M, BF16>(s_tab, wv, f16_off, f32_off);
            } else {
                bw = decode_pair_swar<Q, M, BF16>(s_tab, ck.w[st], f16_off, f32_off);
            }
#pragma unroll
            for (int s = 0; s < NTILE; ++s) {
                if (BF16)
                    acc[s] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, a[s]),
                                                                    __builtin_bit_cast(bf16x8_t, bw), acc[s], 0, 0, 0);
                else
                    acc[s] = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(half8_t, a[s]),
                                                                   __builtin_bit_cast(half8_t, bw), acc[s], 0, 0, 0);
            }
        }
    };

    Chunk c_a, c_b;
    if constexpr (SPLIT) {
        // each fp32 token's K slice, 32 bytes a lane, then both chunks'
        // weights; the three planes of a lane's 8 values go to the token's
        // three rows (3 planes_b <= TB, checked by the host)
        constexpr int NB = TB / 3;
        const float* act32 = static_cast<const float*>(p.act);
        const int64_t nb = p.planes_b;
        float4 av[NB][2];
#pragma unroll
        for (int b = 0; b < NB; ++b) {
            const int64_t kb = 4 * w0 + lane;
            const bool ok = b < nb && kb < 4 * w1 && kb < kb_total;
            const float4* src = reinterpret_cast<const float4*>(act32 + (ok ? b * p.K + kb * 8 : 0));
            av[b][0] = src[0];
            av[b][1] = src[1];
        }
        load(w0, c_a);
        load(w0 + CH, c_b);
#pragma unroll
        for (int b = 0; b < NB; ++b) {
            if (b >= nb) break;   // uniform
            const int64_t kb = 4 * w0 + lane;
            const bool ok = kb < 4 * w1 && kb < kb_total;
            const float v[8] = {av[b][0].x, av[b][0].y, av[b][0].z, av[b][0].w,
                                av[b][1].x, av[b][1].y, av[b][1].z, av[b][1].w};
            uint16_t h[3][8];
#pragma unroll
            for (int j = 0; j < 8; ++j) split3(ok ? v[j] : 0.f, h[0][j], h[1][j], h[2][j]);
#pragma unroll
            for (int pl = 0; pl < 3; ++pl)
                *reinterpret_cast<uint4*>(&s_stage[(wave * TB + pl * (int)nb + b) * kRowsStageRow + lane * 16]) =
                    make_uint4((uint32_t)h[pl][0] | ((uint32_t)h[pl][1] << 16),
                               (uint32_t)h[pl][2] | ((uint32_t)h[pl][3] << 16),
                               (uint32_t)h[pl][4] | ((uint32_t)h[pl][5] << 16),
                               (uint32_t)h[pl][6] | ((uint32_t)h[pl][7] << 16));
        }
        stage_tables();
        run(c_a, w0);
        run(c_b, w0 + CH);
    } else if constexpr (TB > 0) {
        // the wave's K slice (at most two chunks, checked by the host) of every
        // token, 16 bytes a lane and one load per token, then both chunks'
        // weights; the activations go to the wave's LDS rows as they arrive
        uint4 av[TB];
#pragma unroll
        for (int t = 0; t < TB; ++t) {
            const int64_t kb = 4 * w0 + lane;
            const bool ok = t_base + t < p.B && kb < 4 * w1 && kb < kb_total;
            av[t] = *reinterpret_cast<const uint4*>(act + (ok ? (t_base + t) * p.K + kb * 8 : 0));
        }
        load(w0, c_a);
        load(w0 + CH, c_b);
#pragma unroll
        for (int t = 0; t < TB; ++t) {
            const int64_t kb = 4 * w0 + lane;
            const bool ok = t_base + t < p.B && kb < 4 * w1 && kb < kb_total;
            uint32_t m;
            __asm__("v_mov_b32 %0, %1" : "=v"(m) : "v"(ok ? ~0u : 0u));
            *reinterpret_cast<uint4*>(&s_stage[(wave * TB + t) * kRowsStageRow + lane * 16]) =
                make_uint4(av[t].x & m, av[t].y & m, av[t].z & m, av[t].w & m);
        }
        stage_tables();
        run(c_a, w0);
        run(c_b, w0 + CH);
    } else {
        // ping-pong over chunks; the chunk after the wave's last is loaded too
        // (clamped and masked, never used), which keeps every load unconditional
        int64_t c0 = w0;
        load(c0, c_a);
        // the tables are staged while the first chunk's loads are in flight
        stage_tables();
        for (; c0 < w1; c0 += 2 * CH) {
            const int64_t c1 = c0 + CH;
            load(c1, c_b);
            run(c_a, c0);
            if (c1 >= w1) break;
            load(c1 + CH, c_a);
            run(c_b, c1);
        }
    }

    // D[token = 16 s + 4 (lane / 16) + i][row = lane % 16]; sum the waves
#pragma unroll
    for (int s = 0; s < NTILE; ++s)
#pragma unroll
        for (int i = 0; i < 4; ++i) s_red[wave][s * 4 + i][lane] = acc[s][i];
    __syncthreads();
    const float sc_ep = p.scale && p.scale_mode != 0 ? 1.f / sc_raw : sc_raw;
    if (p.planes_b > 0) {
        // one split and one token tile (t_base = 0) hold all three planes:
        // output (b, o) sums each plane's waves as below, scales it, adds the
        // planes in order and takes the epilogue
        const int64_t nb = p.planes_b;
        for (int e = threadIdx.x; e < nb * 16; e += blockDim.x) {
            const int64_t b = e >> 4, o = r0 + (e & 15);
            if (o >= p.rows) continue;
            const float sc = sc_ep;
            float y[3];
#pragma unroll
            for (int pl = 0; pl < 3; ++pl) {
                const int t = (int)(pl * nb + b);
                const int si = 4 * (t >> 4) + (t & 3), ln = 16 * ((t >> 2) & 3) + (e & 15);
                float v = 0.f;
#pragma unroll
                for (int w = 0; w < kRowsWaves; ++w) v += s_red[w][si][ln];
                y[pl] = v * 0.5f * sc;
            }
            p.out[b * p.rows + o] =
                vlut_epilogue_b(__fadd_rn(__fadd_rn(y[0], y[1]), y[2]), bias_ep, p.bias, p.lsq_alpha, p.lsq_qmax);
        }
        return;
    }
    for (int e = threadIdx.x; e < NTILE * 256; e += blockDim.x) {
        const int si = e >> 6, ln = e & 63;
        float v = 0.f;
#pragma unroll
        for (int w = 0; w < kRowsWaves; ++w) v += s_red[w][si][ln];
        const int64_t tok = t_base + 16 * (si >> 2) + 4 * (ln >> 4) + (si & 3);
        const int64_t o = r0 + (ln & 15);
        if (tok >= p.B || o >= p.rows) continue;
        if (gridDim.y == 1) {
            p.out[tok * p.rows + o] = vlut_epilogue_b(v * 0.5f * sc_ep, bias_ep, p.bias, p.lsq_alpha, p.lsq_qmax);
        } else {
            p.partial[(tok * p.rows + o) * gridDim.y + blockIdx.y] = v;
        }
    }
}

namespace {


template <int Q, int M, bool BF16, int NTILE, int TB, bool SPLIT = false>
void launch_rows_fmt(const VlutMatmulArgs& p, int splits, hipStream_t s)
{
    dim3 grid((unsigned)((p.rows + 15) / 16), (unsigned)splits, (unsigned)((p.B + 16 * NTILE - 1) / (16 * NTILE)));
#define COSET_ROWS(F) \
    hipLaunchKernelGGL((vlut_rows_kernel<Q, M, BF16, NTILE, F, TB, SPLIT>), grid, dim3(kRowsWaves * 64), 0, s, p)
    switch (p.prepared) {
    case VLUT_RAW: COSET_ROWS(VLUT_RAW); break;
    case VLUT_PREPARED: COSET_ROWS(VLUT_PREPARED); break;
    case VLUT_DECODED: COSET_ROWS(VLUT_DECODED); break;
    case VLUT_DECODED6: COSET_ROWS(VLUT_DECODED6); break;
    default: COSET_ROWS(VLUT_TILED); break;
    }
#undef COSET_ROWS
}

template <int Q, int M>
hipError_t launch_rows(const VlutMatmulArgs& p, int splits, hipStream_t s)
{
    if constexpr (Q == 2 || M <= 2) {
        const bool bf = p.act_dtype == DT_BF16;
        // the staged kernels take a wave's whole K range (at most kRowsStageKq k-quads) at once
        const bool staged = vlut_rows_staged(p.K, splits);
        // raw q = 4 words above one token: the kernels without staged activations,
        // whose LDS holds the cid map beside their other buffers
        const bool raw_map = Q == 4 && p.prepared == VLUT_RAW;
        if (p.act_planes) {   // fp32 activations split by the staging: one tile, one split
            if (!staged || splits != 1 || p.planes_b <= 0 || p.B != 3 * p.planes_b || p.B > 15)
                return hipErrorInvalidValue;
            if (p.B <= 6) launch_rows_fmt<Q, M, true, 1, 8, true>(p, splits, s);
            else launch_rows_fmt<Q, M, true, 1, 16, true>(p, splits, s);
        } else if (staged && p.B == 1) {  // staged activations, one token
            if (bf) launch_rows_fmt<Q, M, true, 1, 1>(p, splits, s); else launch_rows_fmt<Q, M, false, 1, 1>(p, splits, s);
        } else if (staged && p.B <= 8 && !raw_map) {  // staged activations, up to 8 tokens
            if (bf) launch_rows_fmt<Q, M, true, 1, 8>(p, splits, s); else launch_rows_fmt<Q, M, false, 1, 8>(p, splits, s);
        } else if (staged && p.B <= 16 && !raw_map) {  // staged activations, up to 16 tokens
            if (bf) launch_rows_fmt<Q, M, true, 1, 16>(p, splits, s); else launch_rows_fmt<Q, M, false, 1, 16>(p, splits, s);
        } else if (p.B <= 16) {
            if (bf) launch_rows_fmt<Q, M, true, 1, 0>(p, splits, s); else launch_rows_fmt<Q, M, false, 1, 0>(p, splits, s);
        } else if (p.B <= 32) {
            if (bf) launch_rows_fmt<Q, M, true, 2, 0>(p, splits, s); else launch_rows_fmt<Q, M, false, 2, 0>(p, splits, s);
        } else {
            if (bf) launch_rows_fmt<Q, M, true, 4, 0>(p, splits, s); else launch_rows_fmt<Q, M, false, 4, 0>(p, splits, s);
        }
        return hipGetLastError();
    }
    return hipErrorInvalidValue;
}

template <int Q>
hipError_t dispatch_rows(const VlutMatmulArgs& p, int splits, hipStream_t s)
{
    switch (p.M) {
    case 1: return launch_rows<Q, 1>(p, splits, s);
    case 2: return launch_rows<Q, 2>(p, splits, s);
    case 3: return launch_rows<Q, 3>(p, splits, s);
    case 4: return launch_rows<Q, 4>(p, splits, s);
    default: return hipErrorInvalidValue;
    }
}

}  // namespace

bool vlut_rows_staged(int64_t K, int splits)
{
    const int64_t kq_total = (K / 8 + 3) / 4;
    const int64_t kq_wg = (kq_total + splits - 1) / splits;
    return (kq_wg + kRowsWaves - 1) / kRowsWaves <= kRowsStageKq;
}

hipError_t vlut_launch_rows(const VlutMatmulArgs& p, int splits, hipStream_t s)
{
    return p.q == 4 ? dispatch_rows<4>(p, splits, s) : dispatch_rows<2>(p, splits, s);
}

}  // namespace coset
