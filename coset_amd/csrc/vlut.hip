// vlut.hip -- value lookup tables (vLUTs) of the E8 HNLQ codes.
//
// Reference definition (coset/legacy/quant/vlut.py:72-117, 217-238;
// tests/legacy/test_one_sided_vlut_pytest.py:22-43): for a query a in R^8
//   vLUT_a[idx(b)] = <a, r(b)>,   r(b) = G b - q P(G b / q)
// over all b in [0,q)^8, idx(b) = sum_j b_j q^(7-j), and for an encoded block
//   <a, x_hat> = sum_m q^m vLUT_a[idx(b_m)].
// P is the legacy textbook rule for the legacy vLUT and the core rule for
// tables that match e8_decode.
//
// Kernels
//   vlut_build_kernel      full one-sided tables, one thread per entry
//   vlut_dot_kernel        sum_m q^m vLUT[idx_m] over encoded blocks
//   vlut_lds_kernel        matmul out[t,o] = s_o sum_k sum_m q^m vLUT_{a_tk}[idx]
//                          with per-(token, k-block) tables in LDS, factorized
//                          over the coordinate pairs of r:
//                            vLUT_a[idx(b)] = sum_p <(a_2p, a_2p+1), r_p(b)>
//                          (289 floats instead of q^8 = 65536 at q = 4)
//   vlut_mfma_kernel       same product by decoding 2 x_hat (exact in fp16/bf16)
//                          into LDS and multiplying on the matrix cores
//                          (for (q, M) whose byte tables would overflow)
//   vlut_reduce_kernel     sums the split-K partials and applies s_o (the
//                          _sm kernels: split-major partials, summed in order)
// The byte-table matrix-core kernels live in vlut_rows.hip (up to 32 tokens)
// and vlut_wide.hip (wide and deep kernels, more tokens), with the helpers
// they share in vlut_mfma.hpp.
#include <algorithm>

#include "codec_kernels.hpp"
#include "tables.hpp"
#include "vlut.hpp"
#include "lsq.hpp"
#include "vlut_mfma.hpp"

namespace coset {

// ---------------------------------------------------------------- helpers
__device__ __forceinline__ float load_act(const void* p, int dt, int64_t i)
{
    if (dt == DT_F32) return reinterpret_cast<const float*>(p)[i];
    uint16_t h = reinterpret_cast<const uint16_t*>(p)[i];
    if (dt == DT_BF16) return __uint_as_float((uint32_t)h << 16);
    return (float)__builtin_bit_cast(_Float16, h);
}

// load_act in two steps, so the load can be issued ahead of others and
// converted once they are in flight: the element's bits, then its value.
__device__ __forceinline__ uint32_t load_act_bits(const void* p, int dt, int64_t i)
{
    if (dt == DT_F32) return reinterpret_cast<const uint32_t*>(p)[i];
    return reinterpret_cast<const uint16_t*>(p)[i];
}

__device__ __forceinline__ float act_value(uint32_t bits, int dt)
{
    if (dt == DT_F32) return __uint_as_float(bits);
    if (dt == DT_BF16) return __uint_as_float(bits << 16);
    return (float)__builtin_bit_cast(_Float16, (uint16_t)bits);
}

// 2 r(b) from the level word with the decode tables: U - q*(2c), U = 2Gb.
template <int Q>
__device__ __forceinline__ void two_r_lut(uint32_t w, const uint16_t* map, const uint64_t* coarse, int out[8])
{
    int b[8];
    unpack_word<Q>(w, Q, b);
    uint64_t c = coarse[map[w]];
    out[0] = 4 * b[0] - 2 * b[1] + b[7];
#pragma unroll
    for (int j = 1; j < 6; ++j) out[j] = 2 * (b[j] - b[j + 1]) + b[7];
    out[6] = 2 * b[6] + b[7];
    out[7] = b[7];
#pragma unroll
    for (int j = 0; j < 8; ++j) out[j] -= Q * (int)(int8_t)(uint8_t)(c >> (8 * j));
}

// Level word index i of the weight tensor -> (idx, coarse id).
__device__ __forceinline__ void load_word(const VlutMatmulArgs& p, int64_t i, uint32_t* idx, uint32_t* cid)
{
    if (p.prepared != VLUT_RAW) {
        uint32_t v = reinterpret_cast<const uint32_t*>(p.words)[i];
        *idx = v & 0xffffu;
        *cid = v >> 16;
    } else {
        uint32_t w = reinterpret_cast<const uint16_t*>(p.words)[i] & (p.q == 2 ? 0xffu : 0xffffu);  // map bounds
        *idx = w;
        *cid = p.map[w];
    }
}

// One thread per output word: the raw word of (row, kb, m) or, past the
// matrix in the tiled formats, the word 0 (which decodes to 0), stored as
// cid << 16 | word, or as its pair ids (VLUT_PAIRS).
__global__ void __launch_bounds__(256) vlut_prepare_kernel(const uint16_t* words, int64_t rows, int64_t kb_total,
                                                          int M, int fmt, int64_t n_out, const uint16_t* map,
                                                          const uint32_t* pair_map, uint32_t mask, uint32_t* out)
{
    int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n_out) return;
    uint32_t w = 0;
    if (fmt == VLUT_PAIRS) {  // [rows / 64][kb][M][64 rows]
        const int64_t rest = i >> 6;
        const int m = (int)(rest % M);
        const int64_t kb = (rest / M) % kb_total;
        const int64_t row = (rest / M / kb_total) * 64 + (i & 63);
        if (row < rows) w = words[(row * kb_total + kb) * M + m];
    } else if (fmt == VLUT_TILED) {
        const int m = (int)(i % M);
        const int64_t e = i / M;  // entry
        const int lane = (int)(e & 63);
        const int64_t tile = e >> 6;
        const int64_t kq = (kb_total + 3) / 4;
        const int64_t row = (tile / kq) * 16 + (lane & 15);
        const int64_t kb = (tile % kq) * 4 + (lane >> 4);
        if (row < rows && kb < kb_total) w = words[(row * kb_total + kb) * M + m];
    } else {
        w = words[i];
    }
    w &= mask;  // q^8 - 1: map bounds for any input
    out[i] = fmt == VLUT_PAIRS ? pair_map[w] : ((uint32_t)map[w] << 16) | w;
}

// ---------------------------------------------------------------- build
template <int Q>
__global__ void __launch_bounds__(256) vlut_build_kernel(const float* a, int64_t n_queries, uint32_t n_codes,
                                                        int q, int legacy, const uint16_t* map,
                                                        const uint64_t* coarse, float* vlut)
{
    int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (gid >= n_queries * (int64_t)n_codes) return;
    int64_t qi = gid / n_codes;
    uint32_t idx = (uint32_t)(gid - qi * n_codes);
    float r[8];
    if (Q == 2 || Q == 4) {
        int t[8];
        two_r_lut<Q>(idx, map, coarse, t);
#pragma unroll
        for (int j = 0; j < 8; ++j) r[j] = 0.5f * (float)t[j];
    } else {
        int b[8];
        float gb[8];
        unpack_word<0>(idx, q, b);
        lattice_point(b, gb);
        // the legacy vLUT projects one 8-vector at a time (contiguous rule)
        if (legacy)
            residual_from_point<true, false>(gb, (float)q, r);
        else
            residual_from_point<false, true>(gb, (float)q, r);
    }
    const float* av = a + 8 * qi;
    float acc = 0.f;
#pragma unroll
    for (int j = 0; j < 8; ++j) acc = __fmaf_rn(av[j], r[j], acc);
    vlut[gid] = acc;
}

// ---------------------------------------------------------------- lookup
__global__ void __launch_bounds__(256) vlut_dot_kernel(const void* words, int word_bytes_, int64_t n, int M,
                                                      int q, uint32_t n_codes, const float* vlut, float* out)
{
    int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    float acc = 0.f, w = 1.f;
    for (int m = 0; m < M; ++m) {
        uint32_t idx = word_bytes_ == 2 ? reinterpret_cast<const uint16_t*>(words)[i * M + m]
                                        : reinterpret_cast<const uint32_t*>(words)[i * M + m];
        idx = min(idx, n_codes - 1u);  // table bounds for any input
        acc = __fmaf_rn(w, vlut[idx], acc);
        w *= (float)q;
    }
    out[i] = acc;
}

// ---------------------------------------------------------------- LDS vLUT matmul
// out[t, o] = s_o sum_k sum_m q^m <a_tk, r(b_okm)>, the inner products read
// from per-(token, k-block) tables in LDS.  The coordinate pairs of r take
// few values (tables.hpp: pair_vals), so one table is four sub-tables
//   T[72 p + id] = a_2p r_2p(id) + a_2p+1 r_2p+1(id)     p = 0..3
// (289 floats; 261 used at q = 4) and a level word costs four lookups:
//   vLUT_a[idx(b)] = <a, r(b)> = sum_p T[72 p + id_p(b)].
// Workgroup: 4 waves x 2 or 4 tiles of 64 rows (512 or 1024 rows) x a K range (grid.y
// splits) x TT tokens (grid.z); a lane owns one row of each of its wave's
// tiles.  The tables of a k-block are interleaved in planes of VW = min(TT,
// 4) tokens, entry-major (plane h: T[(72 p + id) VW + c] for token h VW + c),
// so one lookup instruction reads an entry for VW tokens at once (16 bytes a
// lane at VW = 4, with consecutive ids 16 bytes apart over the banks): a
// quarter of the gather instructions of one table per token, the same bytes.
// Lanes with the same id share the read.  The
// K range runs in chunks of KB k-blocks: the chunk's activations and level
// words are loaded (the words as pair ids; one 256-byte read per wave and
// word in the pairs format), the activations staged and the tables built
// while the word loads are in flight, then the tables are read.
constexpr int kLdsWaves = 4;
// 64-row tiles per wave: 2 (512 rows per workgroup), or 4 (1024 rows) from
// 32 tokens on, where each table built serves twice the rows -- the builds,
// one per (row group, token, k-block), take more time than the lookups there
__host__ __device__ constexpr int lds_tiles(int64_t B) { return B >= 32 ? 4 : 2; }
__host__ __device__ constexpr int64_t lds_rows(int64_t B) { return kLdsWaves * lds_tiles(B) * 64; }
constexpr int kLdsTable = 4 * kPairSlots + 1;         // floats per (token, k-block) table

// 1, 2 or 4 consecutive table entries (one per token) as one LDS read
template <int N>
struct LdsVec {
    typedef float type __attribute__((ext_vector_type(N)));
    static __device__ __forceinline__ float at(const type& v, int c) { return v[c]; }
    static __device__ __forceinline__ void set(type& v, int c, float x) { v[c] = x; }
};
template <>
struct LdsVec<1> {
    typedef float type;
    static __device__ __forceinline__ float at(const type& v, int) { return v; }
    static __device__ __forceinline__ void set(type& v, int, float x) { v = x; }
};

template <int TT>
struct LdsChunk {
    static constexpr int KB = TT >= 8 ? 4 : 8;  // k-blocks per chunk
};

// PAIRS: the weight is in the pairs format; otherwise the level words
// (raw, row-major or tiled) are loaded first and their pair ids gathered
// from pair_map after, each phase issued whole (no load waits behind a
// per-word branch).
template <int Q, int M, int TT, int kLdsTiles, bool PAIRS>
__global__ void __launch_bounds__(kLdsWaves * 64) vlut_lds_kernel(VlutMatmulArgs p)
{
    constexpr int kLdsRows = kLdsWaves * kLdsTiles * 64;  // rows per workgroup
    constexpr int KB = LdsChunk<TT>::KB;
    constexpr int NTAB = TT * KB;  // tables per chunk; s_act holds token t, k-block j at t * KB + j
    constexpr int VW = TT < 4 ? TT : 4;  // tokens per lookup
    using vecw_t = typename LdsVec<VW>::type;
    __shared__ __align__(16) float s_tab[NTAB * kLdsTable];
    __shared__ float2 s_pv[4 * kPairSlots];
    __shared__ __align__(8) float s_act[NTAB * 8];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int64_t kb_total = p.K / 8;
    const int64_t kb_wg = (kb_total + gridDim.y - 1) / gridDim.y;
    const int64_t kb_begin = blockIdx.y * kb_wg;
    const int64_t kb_end = min(kb_total, kb_begin + kb_wg);
    const int64_t t0 = (int64_t)blockIdx.z * TT;
    const int64_t row0 = (int64_t)blockIdx.x * kLdsRows + wave * (kLdsTiles * 64) + lane;  // the lane's first row

    for (int i = threadIdx.x; i < 4 * kPairSlots; i += blockDim.x) s_pv[i] = p.pair_vals[i];

    float acc[kLdsTiles][TT];
#pragma unroll
    for (int i = 0; i < kLdsTiles; ++i)
#pragma unroll
        for (int t = 0; t < TT; ++t) acc[i][t] = 0.f;

    constexpr int kActPerThread = (NTAB * 8 + kLdsWaves * 64 - 1) / (kLdsWaves * 64);
    for (int64_t kc = kb_begin; kc < kb_end; kc += KB) {
        // the chunk's activations first: loads complete in order, so the
        // LDS staging below then waits for these alone, with the level words
        // still in flight through the table build
        uint32_t av[kActPerThread];  // bits (0 outside the matrix and the range: the value 0 in every dtype)
#pragma unroll
        for (int u = 0; u < kActPerThread; ++u) {
            const int e = threadIdx.x + u * kLdsWaves * 64;
            const int t = e / (8 * KB), j = (e / 8) % KB;
            const int64_t kb = kc + j;
            const bool ok = e < NTAB * 8 && t0 + t < p.B && kb < kb_end;
            // an index in the matrix for every lane, the bits dropped after
            const int64_t ai = ok ? (t0 + t) * p.K + kb * 8 + (e % 8) : 0;
            const uint32_t bits = load_act_bits(p.act, p.act_dtype, ai);
            av[u] = ok ? bits : 0u;
        }
        // the chunk's level words; indices clamped into the matrix (those
        // lanes' rows are never stored, their k-blocks have zero tables)
        uint32_t pw[kLdsTiles][KB][M];
        auto each_word = [&](auto&& f) {
#pragma unroll
            for (int i = 0; i < kLdsTiles; ++i) {
                const int64_t row = min(row0 + 64 * i, p.rows - 1);
#pragma unroll
                for (int j = 0; j < KB; ++j) {
                    const int64_t kb = min(kc + j, kb_total - 1);
#pragma unroll
                    for (int m = 0; m < M; ++m) f(pw[i][j][m], row, kb, m);
                }
            }
        };
        if constexpr (PAIRS) {
            const uint32_t* w32 = reinterpret_cast<const uint32_t*>(p.words);
            each_word([&](uint32_t& w, int64_t row, int64_t kb, int m) {
                w = w32[vlut_word_index(VLUT_PAIRS, row, kb, m, kb_total, M)];
            });
        } else {
            if (p.prepared == VLUT_RAW) {
                const uint16_t* w16 = reinterpret_cast<const uint16_t*>(p.words);
                each_word([&](uint32_t& w, int64_t row, int64_t kb, int m) {
                    w = w16[(row * kb_total + kb) * M + m];
                });
            } else {
                const uint32_t* w32 = reinterpret_cast<const uint32_t*>(p.words);
                const int fmt = p.prepared;
                each_word([&](uint32_t& w, int64_t row, int64_t kb, int m) {
                    w = w32[vlut_word_index(fmt, row, kb, m, kb_total, M)];
                });
            }
            const uint32_t mask = Q == 2 ? 0xffu : 0xffffu;  // map bounds for any input
            each_word([&](uint32_t& w, int64_t, int64_t, int) { w = p.pair_map[w & mask]; });
        }
        __syncthreads();  // the previous chunk's lookups are done with the tables
#pragma unroll
        for (int u = 0; u < kActPerThread; ++u) {
            const int e = threadIdx.x + u * kLdsWaves * 64;
            if (e < NTAB * 8) s_act[e] = act_value(av[u], p.act_dtype);
        }
        __syncthreads();
        // table item it = jh kLdsTable + slot: the VW entries of plane h of
        // k-block j (jh = j (TT / VW) + h) at that slot, tokens h VW + c, at
        // (jh kLdsTable + slot) VW + c.  A thread's items step by the
        // workgroup size, so (jh, slot) advance without a division.
        static_assert(kLdsWaves * 64 < kLdsTable, "one wrap of the slot per step");
        {
            int jh = 0, slot = threadIdx.x;
            for (int it = threadIdx.x; it < (NTAB / VW) * kLdsTable; it += kLdsWaves * 64) {
                const int j = jh / (TT / VW), h = jh % (TT / VW);
                const int pp = (slot >= kPairSlots) + (slot >= 2 * kPairSlots) + (slot >= 3 * kPairSlots);
                const bool live = slot < 4 * kPairSlots;
                const float2 r = s_pv[live ? slot : 0];
                vecw_t v;
#pragma unroll
                for (int c = 0; c < VW; ++c) {
                    const float2 a = *reinterpret_cast<const float2*>(s_act + ((h * VW + c) * KB + j) * 8 + 2 * pp);
                    LdsVec<VW>::set(v, c, live ? __fmaf_rn(a.y, r.y, a.x * r.x) : 0.f);
                }
                *reinterpret_cast<vecw_t*>(s_tab + it * VW) = v;
                slot += kLdsWaves * 64;
                if (slot >= kLdsTable) {
                    slot -= kLdsTable;
                    ++jh;
                }
            }
        }
        __syncthreads();
#pragma unroll
        for (int j = 0; j < KB; ++j) {
#pragma unroll
            for (int i = 0; i < kLdsTiles; ++i) {
                float qm = 1.f;
#pragma unroll
                for (int m = 0; m < M; ++m) {
                    const uint32_t w = pw[i][j][m];
                    // ids below the sub-table size for any input word
                    const uint32_t id0 = min(w & 0xffu, kPairSlots - 1u);
                    const uint32_t id1 = min((w >> 8) & 0xffu, kPairSlots - 1u) + kPairSlots;
                    const uint32_t id2 = min((w >> 16) & 0xffu, kPairSlots - 1u) + 2 * kPairSlots;
                    const uint32_t id3 = min(w >> 24, kPairSlots - 1u) + 3 * kPairSlots;
#pragma unroll
                    for (int h = 0; h < TT / VW; ++h) {
                        const float* T = s_tab + (j * (TT / VW) + h) * kLdsTable * VW;
                        const vecw_t x0 = *reinterpret_cast<const vecw_t*>(T + id0 * VW);
                        const vecw_t x1 = *reinterpret_cast<const vecw_t*>(T + id1 * VW);
                        const vecw_t x2 = *reinterpret_cast<const vecw_t*>(T + id2 * VW);
                        const vecw_t x3 = *reinterpret_cast<const vecw_t*>(T + id3 * VW);
#pragma unroll
                        for (int c = 0; c < VW; ++c) {
                            const float v = (LdsVec<VW>::at(x0, c) + LdsVec<VW>::at(x1, c)) +
                                            (LdsVec<VW>::at(x2, c) + LdsVec<VW>::at(x3, c));
                            acc[i][h * VW + c] = __fmaf_rn(qm, v, acc[i][h * VW + c]);
                        }
                    }
                    qm *= (float)Q;
                }
            }
        }
    }
    // one store per (row, token): the output itself when the K range is
    // whole, else the split's partial
#pragma unroll
    for (int i = 0; i < kLdsTiles; ++i) {
        const int64_t row = row0 + 64 * i;
        if (row >= p.rows) continue;
        const float sc = gridDim.y > 1 || !p.scale ? 1.f : (p.scale_mode == 0 ? p.scale[row] : 1.f / p.scale[row]);
#pragma unroll
        for (int t = 0; t < TT; ++t) {
            if (t0 + t >= p.B) break;
            if (gridDim.y == 1)
                p.out[(t0 + t) * p.rows + row] = vlut_epilogue(acc[i][t] * sc, row, p.bias, p.lsq_alpha, p.lsq_qmax);
            else
                p.partial[((int64_t)blockIdx.y * p.B + t0 + t) * p.rows + row] = acc[i][t];
        }
    }
}

// ---------------------------------------------------------------- MFMA matmul
// Tile: 64 output rows x up to NT tokens per workgroup (4 waves, one 16-row
// slice each), K split over grid.y.  A step covers 16 k-blocks (128 K):
// every thread decodes 4 (row, k-block) pairs to 8 halves of 2*x_hat in LDS,
// the activation tile [NT x 128] is staged in LDS with 16-byte loads, then
// each wave runs 8 K-slices of 16x16x16 MFMAs per 16-token sub-tile.  All
// level words of the workgroup are loaded before the first step.
//
// Decode (SWAR): the three byte tables of 2r (tables.hpp) are added as two
// 32-bit words per level, levels combine as acc = acc*q + L_m, and each byte
// b = 2x + bias becomes a half through the bit pattern 0x64bb (= 1024 + b)
// minus (1024 + bias), exact as every value is an integer below 2048.
// Decode (integer): 2x = sum_m q^m (2Gb - q (2c)) with the digits unpacked,
// for the (q, M) whose bytes would overflow.
template <int Q, int M, bool BF16, bool SWAR, int NT>
__global__ void __launch_bounds__(256) vlut_mfma_kernel(VlutMatmulArgs p)
{
    constexpr int kTSub = NT / 16;
    __shared__ __align__(16) uint16_t s_b[kMfmaRows][kMfmaLd];
    __shared__ __align__(16) uint16_t s_a[NT][kMfmaLd];
    __shared__ uint64_t s_tab[SWAR ? kSwarSlots : kMaxCoarseVlut];
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;

    const int64_t kb_total = p.K / 8;
    const int64_t ks_len = ((kb_total + gridDim.y - 1) / gridDim.y + kMfmaKB - 1) / kMfmaKB * kMfmaKB;
    const int64_t k_begin = blockIdx.y * ks_len;
    const int64_t k_end = min(kb_total, k_begin + ks_len);
    const int n_steps = (int)min((int64_t)kMfmaMaxSteps, (k_end - k_begin + kMfmaKB - 1) / kMfmaKB);
    const int64_t r0 = (int64_t)blockIdx.x * kMfmaRows;
    const int64_t t_base = (int64_t)blockIdx.z * NT;
    const int nt = (int)min((int64_t)NT, p.B - t_base);
    const int n_tsub = (nt + 15) / 16;
    const uint16_t* act = reinterpret_cast<const uint16_t*>(p.act);

    // (row pr/16, k-block pr%16) pairs, 4 per thread per step; a word is kept
    // as cid << 16 | idx, all-ones marking a pair outside the matrix
    uint32_t words[kMfmaMaxSteps][4][M];
#pragma unroll
    for (int st = 0; st < kMfmaMaxSteps; ++st) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int pr = threadIdx.x + 256 * i;
            const int64_t row = r0 + (pr >> 4);
            const int64_t kb = k_begin + st * kMfmaKB + (pr & 15);
            const bool ok = st < n_steps && row < p.rows && kb < k_end;
#pragma unroll
            for (int m = 0; m < M; ++m) {
                uint32_t v = 0xffffffffu;
                if (ok) {
                    const int64_t wi = vlut_word_index(p.prepared, row, kb, m, kb_total, M);
                    if (p.prepared != VLUT_RAW) {
                        v = reinterpret_cast<const uint32_t*>(p.words)[wi];
                    } else {
                        const uint32_t w = reinterpret_cast<const uint16_t*>(p.words)[wi];
                        v = ((uint32_t)p.map[w] << 16) | w;
                    }
                }
                words[st][i][m] = v;
            }
        }
    }

    float4_t acc[kTSub];
#pragma unroll
    for (int s = 0; s < kTSub; ++s) acc[s] = (float4_t){0.f, 0.f, 0.f, 0.f};

    // tables are staged while the word loads are in flight
    if (SWAR) {
        for (int i = threadIdx.x; i < 512 + p.n_coarse; i += 256) s_tab[i] = p.swar[i];
    } else {
        for (int i = threadIdx.x; i < p.n_coarse; i += 256) s_tab[i] = p.coarse[i];
    }
    const _Float16 f16_off = (_Float16)(1024 + p.swar_bias);
    const float f32_off = (float)p.swar_bias;

    uint4 av[NT / 16];
    auto load_act_tile = [&](int st) {
#pragma unroll
        for (int j = 0; j < NT / 16; ++j) {
            const int idx = threadIdx.x + 256 * j;
            const int tok = idx >> 4, seg = idx & 15;
            const int64_t kb = k_begin + st * kMfmaKB + seg;
            av[j] = make_uint4(0u, 0u, 0u, 0u);
            if (st < n_steps && tok < nt && kb < k_end)
                av[j] = *reinterpret_cast<const uint4*>(act + (t_base + tok) * p.K + kb * 8);
        }
    };
    load_act_tile(0);

#pragma unroll
    for (int st = 0; st < kMfmaMaxSteps; ++st) {
        if (st >= n_steps) break;
        __syncthreads();  // the previous step's MFMAs are done with s_a / s_b (first step: s_tab is written)
#pragma unroll
        for (int j = 0; j < NT / 16; ++j) {
            const int idx = threadIdx.x + 256 * j;
            *reinterpret_cast<uint4*>(&s_a[idx >> 4][(idx & 15) * 8]) = av[j];
        }
        if (st + 1 < n_steps) load_act_tile(st + 1);  // in flight during decode and MFMAs
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const bool ok = words[st][i][0] != 0xffffffffu;
            uint32_t hv[4];
            if (SWAR) {
                uint32_t x0 = 0u, x1 = 0u;
#pragma unroll
                for (int m = M - 1; m >= 0; --m) {
                    const uint32_t v = ok ? words[st][i][m] : 0u;
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
                if (BF16) {
                    float f[8];
#pragma unroll
                    for (int j = 0; j < 4; ++j) {
                        f[j] = (float)((x0 >> (8 * j)) & 0xffu) - f32_off;
                        f[4 + j] = (float)((x1 >> (8 * j)) & 0xffu) - f32_off;
                    }
#pragma unroll
                    for (int j = 0; j < 4; ++j)  // exact: small integers
                        hv[j] = __builtin_amdgcn_perm(__float_as_uint(f[2 * j + 1]), __float_as_uint(f[2 * j]),
                                                      0x07060302u);
                } else {
                    const uint32_t raw[4] = {bytes_to_f16_bits(x0, false), bytes_to_f16_bits(x0, true),
                                             bytes_to_f16_bits(x1, false), bytes_to_f16_bits(x1, true)};
#pragma unroll
                    for (int j = 0; j < 4; ++j) {
                        half2_t h = __builtin_bit_cast(half2_t, raw[j]) - (half2_t){f16_off, f16_off};
                        hv[j] = __builtin_bit_cast(uint32_t, h);
                    }
                }
            } else {
                int two_x[8];
#pragma unroll
                for (int j = 0; j < 8; ++j) two_x[j] = 0;
                int wq = 1;
#pragma unroll
                for (int m = 0; m < M; ++m) {
                    const uint32_t v = ok ? words[st][i][m] : 0u;
                    int b[8];
                    unpack_word<Q>(v & 0xffffu, Q, b);
                    const uint64_t c = s_tab[v >> 16];
                    int u[8];
                    u[0] = 4 * b[0] - 2 * b[1] + b[7];
#pragma unroll
                    for (int j = 1; j < 6; ++j) u[j] = 2 * (b[j] - b[j + 1]) + b[7];
                    u[6] = 2 * b[6] + b[7];
                    u[7] = b[7];
#pragma unroll
                    for (int j = 0; j < 8; ++j) two_x[j] += wq * (u[j] - Q * (int)(int8_t)(uint8_t)(c >> (8 * j)));
                    wq *= Q;
                }
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    uint32_t lo, hi;
                    if (BF16) {  // exact: |2x| < 256
                        lo = __float_as_uint((float)two_x[2 * j]) >> 16;
                        hi = __float_as_uint((float)two_x[2 * j + 1]) >> 16;
                    } else {     // exact: |2x| < 2048
                        _Float16 l = (_Float16)two_x[2 * j], h = (_Float16)two_x[2 * j + 1];
                        lo = __builtin_bit_cast(uint16_t, l);
                        hi = __builtin_bit_cast(uint16_t, h);
                    }
                    hv[j] = lo | (hi << 16);
                }
            }
            const int pr = threadIdx.x + 256 * i;
            *reinterpret_cast<uint4*>(&s_b[pr >> 4][(pr & 15) * 8]) =
                ok ? make_uint4(hv[0], hv[1], hv[2], hv[3]) : make_uint4(0u, 0u, 0u, 0u);
        }
        __syncthreads();
        // D[token][row] += A[token][k] * B[k][row]
        const int brow = wave * 16 + (lane & 15);
#pragma unroll
        for (int kk = 0; kk < kMfmaK / 16; ++kk) {
            const int kof = kk * 16 + 4 * (lane >> 4);
            uint2 bv = *reinterpret_cast<const uint2*>(&s_b[brow][kof]);
#pragma unroll
            for (int s = 0; s < kTSub; ++s) {
                if (s >= n_tsub) break;
                uint2 a2 = *reinterpret_cast<const uint2*>(&s_a[s * 16 + (lane & 15)][kof]);
                if (BF16) {
                    acc[s] = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(__builtin_bit_cast(bf16x4_t, a2),
                                                                      __builtin_bit_cast(bf16x4_t, bv), acc[s], 0, 0, 0);
                } else {
                    acc[s] = __builtin_amdgcn_mfma_f32_16x16x16f16(__builtin_bit_cast(half4_t, a2),
                                                                  __builtin_bit_cast(half4_t, bv), acc[s], 0, 0, 0);
                }
            }
        }
    }
    // D[token = 16 s + 4 (lane/16) + i][row = 16 wave + lane%16]
    const int64_t row = r0 + wave * 16 + (lane & 15);
    if (row < p.rows) {
#pragma unroll
        for (int s = 0; s < kTSub; ++s) {
            if (s >= n_tsub) break;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                int64_t tok = t_base + s * 16 + 4 * (lane >> 4) + i;
                if (tok < p.B) p.partial[(tok * p.rows + row) * gridDim.y + blockIdx.y] = acc[s][i];
            }
        }
    }
}

// ---------------------------------------------------------------- reduce
__global__ void __launch_bounds__(256) vlut_reduce_kernel(const float* partial, int splits, int64_t B,
                                                         int64_t rows, const float* scale, int scale_mode,
                                                         float mult, const float* bias, const float* lsq_alpha,
                                                         int lsq_qmax, float* out)
{
    int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= B * rows) return;
    int64_t o = i % rows;
    const float* pp = partial + i * splits;  // the splits of one output are contiguous
    float acc = 0.f;
    int s = 0;
    if ((splits & 3) == 0) {
        for (; s < splits; s += 4) {
            float4 v = *reinterpret_cast<const float4*>(pp + s);
            acc += (v.x + v.y) + (v.z + v.w);
        }
    }
    for (; s < splits; ++s) acc += pp[s];
    float sc = scale ? (scale_mode == 0 ? scale[o] : 1.f / scale[o]) : 1.f;
    out[i] = vlut_epilogue(acc * mult * sc, o, bias, lsq_alpha, lsq_qmax);
}

// Same for partials stored split-major, [splits][B][rows] (the wide kernel);
// the splits are summed in order.
__global__ void __launch_bounds__(256) vlut_reduce_sm_kernel(const float* partial, int splits, int64_t B,
                                                            int64_t rows, const float* scale, int scale_mode,
                                                            float mult, const float* bias, const float* lsq_alpha,
                                                            int lsq_qmax, float* out)
{
    int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= B * rows) return;
    int64_t o = i % rows;
    const int64_t n = B * rows;
    float acc = 0.f;
    for (int s = 0; s < splits; ++s) acc += partial[s * n + i];
    float sc = scale ? (scale_mode == 0 ? scale[o] : 1.f / scale[o]) : 1.f;
    out[i] = vlut_epilogue(acc * mult * sc, o, bias, lsq_alpha, lsq_qmax);
}

// The same with four consecutive outputs (one token, rows o..o+3; rows % 4
// == 0) per thread: 16-byte loads of every split's partials and one 16-byte
// store; each output's splits are still summed in order.
__global__ void __launch_bounds__(256) vlut_reduce_sm4_kernel(const float* partial, int splits, int64_t B,
                                                             int64_t rows, const float* scale, int scale_mode,
                                                             float mult, const float* bias, const float* lsq_alpha,
                                                             int lsq_qmax, float* out)
{
    const int64_t n4 = B * rows / 4;
    const int64_t i4 = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i4 >= n4) return;
    const float4* p4 = reinterpret_cast<const float4*>(partial);
    float acc[4] = {0.f, 0.f, 0.f, 0.f};
    for (int s = 0; s < splits; ++s) {
        const float4 v = p4[s * n4 + i4];
        acc[0] += v.x;
        acc[1] += v.y;
        acc[2] += v.z;
        acc[3] += v.w;
    }
    const int64_t o0 = (4 * i4) % rows;
    float r[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int64_t o = o0 + j;
        const float sc = scale ? (scale_mode == 0 ? scale[o] : 1.f / scale[o]) : 1.f;
        r[j] = vlut_epilogue(acc[j] * mult * sc, o, bias, lsq_alpha, lsq_qmax);
    }
    reinterpret_cast<float4*>(out)[i4] = make_float4(r[0], r[1], r[2], r[3]);
}

// The same sums for the deep kernel's partials with workgroup (x, y) taking
// the 64 rows of row group x for tokens 16 y .. 16 y + 15, one quad a
// thread: x runs on the XCD whose workgroups wrote that row group's
// partials (both grids deal workgroups to the 8 XCDs by x mod 8 when there
// are a multiple of 8 row groups), so its reads hit that XCD's L2.
__global__ void __launch_bounds__(256) vlut_reduce_rg4_kernel(const float* partial, int splits, int64_t B,
                                                             int64_t rows, const float* scale, int scale_mode,
                                                             float mult, const float* bias, const float* lsq_alpha,
                                                             int lsq_qmax, float* out)
{
    const int64_t rq = rows / 4, n4 = B * rq;
    const int64_t qd = (int64_t)blockIdx.x * 16 + (threadIdx.x & 15);
    const int64_t tok = (int64_t)blockIdx.y * 16 + (threadIdx.x >> 4);
    if (qd >= rq || tok >= B) return;
    const float4* p4 = reinterpret_cast<const float4*>(partial);
    const int64_t i4 = tok * rq + qd, o0 = 4 * qd;
    float acc[4] = {0.f, 0.f, 0.f, 0.f};
    for (int s = 0; s < splits; ++s) {
        const float4 v = p4[s * n4 + i4];
        acc[0] += v.x;
        acc[1] += v.y;
        acc[2] += v.z;
        acc[3] += v.w;
    }
    float r[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int64_t o = o0 + j;
        const float sc = scale ? (scale_mode == 0 ? scale[o] : 1.f / scale[o]) : 1.f;
        r[j] = vlut_epilogue(acc[j] * mult * sc, o, bias, lsq_alpha, lsq_qmax);
    }
    reinterpret_cast<float4*>(out)[i4] = make_float4(r[0], r[1], r[2], r[3]);
}

// The same for three planes of nb tokens (B = 3 nb, rows % 4 == 0): each
// plane's splits are summed and scaled as above, then the planes are added
// in order and the epilogue applied; out is [nb, rows].
__global__ void __launch_bounds__(256) vlut_reduce_planes4_kernel(const float* partial, int splits, int64_t nb,
                                                                 int64_t rows, const float* scale, int scale_mode,
                                                                 float mult, const float* bias,
                                                                 const float* lsq_alpha, int lsq_qmax, float* out)
{
    // workgroup (x, y): row group x (64 rows) of tokens 16 y .. 16 y + 15, as
    // in vlut_reduce_rg4_kernel
    const int64_t rq = rows / 4, m4 = nb * rq, n4 = 3 * m4;
    const int64_t qd = (int64_t)blockIdx.x * 16 + (threadIdx.x & 15);
    const int64_t tok = (int64_t)blockIdx.y * 16 + (threadIdx.x >> 4);
    if (qd >= rq || tok >= nb) return;
    const float4* p4 = reinterpret_cast<const float4*>(partial);
    const int64_t i4 = tok * rq + qd, o0 = 4 * qd;
    float y[3][4];
#pragma unroll
    for (int pl = 0; pl < 3; ++pl) {
        float acc[4] = {0.f, 0.f, 0.f, 0.f};
        for (int s = 0; s < splits; ++s) {
            const float4 v = p4[s * n4 + pl * m4 + i4];
            acc[0] += v.x;
            acc[1] += v.y;
            acc[2] += v.z;
            acc[3] += v.w;
        }
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int64_t o = o0 + j;
            const float sc = scale ? (scale_mode == 0 ? scale[o] : 1.f / scale[o]) : 1.f;
            y[pl][j] = acc[j] * mult * sc;
        }
    }
    float r[4];
#pragma unroll
    for (int j = 0; j < 4; ++j)
        r[j] = vlut_epilogue(__fadd_rn(__fadd_rn(y[0][j], y[1][j]), y[2][j]), o0 + j, bias, lsq_alpha, lsq_qmax);
    reinterpret_cast<float4*>(out)[i4] = make_float4(r[0], r[1], r[2], r[3]);
}

// The same for many splits and few outputs (the LDS-table kernel at small
// batches): a workgroup takes 16 output quads with 16 threads per quad, each
// summing every 16th split in order; the 16 sums of a quad are added in a
// fixed order through LDS, so the result is the same on every run.
constexpr int kReduceGroups = 16;

__global__ void __launch_bounds__(256) vlut_reduce_sm4g_kernel(const float* partial, int splits, int64_t B,
                                                              int64_t rows, const float* scale, int scale_mode,
                                                              float mult, const float* bias, const float* lsq_alpha,
                                                              int lsq_qmax, float* out, int64_t rg_rows)
{
    __shared__ float4 s_sum[kReduceGroups][16 + 1];
    const int quad = threadIdx.x & 15, g = threadIdx.x >> 4;
    const int64_t n4 = B * rows / 4;
    // rg_rows > 0: workgroup (x, y) takes 16 quads of token y in row group
    // x % groups (chunk x / groups), so it runs on the XCD whose workgroups
    // wrote that row group's partials (the LDS-table kernel's workgroup x
    // takes rows rg_rows x ..; both grids deal workgroups to the 8 XCDs by
    // linear id mod 8); rg_rows = 0: the 16 quads 16 x .. of the flat order
    int64_t i4 = (int64_t)blockIdx.x * 16 + quad;
    bool live = i4 < n4;
    if (rg_rows > 0) {
        const int64_t groups = (rows + rg_rows - 1) / rg_rows;
        const int64_t rg = blockIdx.x % groups, q = (blockIdx.x / groups) * 16 + quad;
        live = q < rg_rows / 4 && rg * (rg_rows / 4) + q < rows / 4;
        i4 = (int64_t)blockIdx.y * (rows / 4) + rg * (rg_rows / 4) + q;
    }
    const float4* p4 = reinterpret_cast<const float4*>(partial);
    float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
    if (live) {
        for (int sp = g; sp < splits; sp += kReduceGroups) {
            const float4 v = p4[sp * n4 + i4];
            acc.x += v.x;
            acc.y += v.y;
            acc.z += v.z;
            acc.w += v.w;
        }
    }
    s_sum[g][quad] = acc;
    __syncthreads();
    if (g != 0 || !live) return;
    for (int k = 1; k < kReduceGroups; ++k) {
        const float4 v = s_sum[k][quad];
        acc.x += v.x;
        acc.y += v.y;
        acc.z += v.z;
        acc.w += v.w;
    }
    const float a[4] = {acc.x, acc.y, acc.z, acc.w};
    const int64_t o0 = (4 * i4) % rows;
    float r[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int64_t o = o0 + j;
        const float sc = scale ? (scale_mode == 0 ? scale[o] : 1.f / scale[o]) : 1.f;
        r[j] = vlut_epilogue(a[j] * mult * sc, o, bias, lsq_alpha, lsq_qmax);
    }
    reinterpret_cast<float4*>(out)[i4] = make_float4(r[0], r[1], r[2], r[3]);
}

// ---------------------------------------------------------------- launchers
namespace {

int lds_tokens(int64_t B)
{
    return B >= 8 ? 8 : (B >= 4 ? 4 : (B >= 2 ? 2 : 1));
}

template <int Q, int M, bool PAIRS>
void launch_lds_fmt(const VlutMatmulArgs& p, int splits, hipStream_t s)
{
    const int TT = lds_tokens(p.B);
    const int64_t rows_wg = lds_rows(p.B);
    dim3 grid((unsigned)((p.rows + rows_wg - 1) / rows_wg), (unsigned)splits, (unsigned)((p.B + TT - 1) / TT));
    dim3 block(kLdsWaves * 64);
    if (lds_tiles(p.B) == 4) {   // B >= 32: TT = 8
        hipLaunchKernelGGL((vlut_lds_kernel<Q, M, 8, 4, PAIRS>), grid, block, 0, s, p);
        return;
    }
    switch (TT) {
    case 8: hipLaunchKernelGGL((vlut_lds_kernel<Q, M, 8, 2, PAIRS>), grid, block, 0, s, p); break;
    case 4: hipLaunchKernelGGL((vlut_lds_kernel<Q, M, 4, 2, PAIRS>), grid, block, 0, s, p); break;
    case 2: hipLaunchKernelGGL((vlut_lds_kernel<Q, M, 2, 2, PAIRS>), grid, block, 0, s, p); break;
    default: hipLaunchKernelGGL((vlut_lds_kernel<Q, M, 1, 2, PAIRS>), grid, block, 0, s, p); break;
    }
}

template <int Q, int M>
hipError_t launch_lds(const VlutMatmulArgs& p, int splits, hipStream_t s)
{
    if (p.prepared == VLUT_PAIRS)
        launch_lds_fmt<Q, M, true>(p, splits, s);
    else
        launch_lds_fmt<Q, M, false>(p, splits, s);
    return hipGetLastError();
}

template <int Q, int M, bool SWAR, int NT>
void launch_mfma_nt(const VlutMatmulArgs& p, int splits, hipStream_t s)
{
    dim3 grid((unsigned)((p.rows + kMfmaRows - 1) / kMfmaRows), (unsigned)splits, (unsigned)((p.B + NT - 1) / NT));
    if (p.act_dtype == DT_BF16)
        hipLaunchKernelGGL((vlut_mfma_kernel<Q, M, true, SWAR, NT>), grid, dim3(256), 0, s, p);
    else
        hipLaunchKernelGGL((vlut_mfma_kernel<Q, M, false, SWAR, NT>), grid, dim3(256), 0, s, p);
}

template <int Q, int M>
hipError_t launch_mfma(const VlutMatmulArgs& p, int splits, hipStream_t s)
{
    // byte decode where the tables allow it (q = 4: M <= 2, q = 2: M <= 4)
    // the byte decode of this kernel is superseded by vlut_rows_kernel
    launch_mfma_nt<Q, M, false, 64>(p, splits, s);
    return hipGetLastError();
}

template <int Q>
hipError_t dispatch_m(const VlutMatmulArgs& p, int method, int splits, hipStream_t s)
{
    switch (p.M) {
#define COSET_M(MM) \
    case MM: return method == VLUT_METHOD_MFMA ? launch_mfma<Q, MM>(p, splits, s) : launch_lds<Q, MM>(p, splits, s);
    COSET_M(1) COSET_M(2) COSET_M(3) COSET_M(4)
#undef COSET_M
    default: return hipErrorInvalidValue;
    }
}

}  // namespace

hipError_t vlut_build(const float* a, int64_t n_queries, int q, int legacy, float* vlut, hipStream_t s)
{
    uint32_t n = 1;
    for (int i = 0; i < 8; ++i) n *= (uint32_t)q;
    int64_t total = n_queries * (int64_t)n;
    if (total == 0) return hipSuccess;
    dim3 grid((unsigned)((total + 255) / 256));
    if (q == 2 || q == 4) {
        const DecodeTables* t = nullptr;
        hipError_t e = get_decode_tables(q, legacy, &t);
        if (e != hipSuccess) return e;
        if (q == 4)
            hipLaunchKernelGGL(vlut_build_kernel<4>, grid, dim3(256), 0, s, a, n_queries, n, q, legacy, t->cid_map, t->coarse, vlut);
        else
            hipLaunchKernelGGL(vlut_build_kernel<2>, grid, dim3(256), 0, s, a, n_queries, n, q, legacy, t->cid_map, t->coarse, vlut);
    } else {
        hipLaunchKernelGGL(vlut_build_kernel<0>, grid, dim3(256), 0, s, a, n_queries, n, q, legacy,
                           (const uint16_t*)nullptr, (const uint64_t*)nullptr, vlut);
    }
    return hipGetLastError();
}

hipError_t vlut_dot(const void* words, int64_t n, int M, int q, const float* vlut, float* out, hipStream_t s)
{
    if (n == 0) return hipSuccess;
    uint32_t n_codes = 1;
    for (int i = 0; i < 8; ++i) n_codes *= (uint32_t)q;
    hipLaunchKernelGGL(vlut_dot_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, words, word_bytes(q), n,
                       M, q, n_codes, vlut, out);
    return hipGetLastError();
}

int g_vlut_swar = 1;
int g_vlut_splits = 0;
int g_vlut_deep = 1;

namespace {

int device_cu_count()
{
    static int cached[64] = {0};
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
    if (!cached[dev]) {
        int n = 0;
        if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
        cached[dev] = n;
    }
    return cached[dev];
}

}  // namespace

VlutPlan vlut_plan(int64_t rows, int64_t B, int64_t K, int q, int M, int method)
{
    const int64_t kb = K / 8;
    if (method == VLUT_METHOD_LDS) {
        // 512- or 1024-row, TT-token workgroups, with K splits for two per
        // CU (each keeping at least one k-block)
        const int TT = lds_tokens(B);
        const int64_t groups = ((rows + lds_rows(B) - 1) / lds_rows(B)) * ((B + TT - 1) / TT);
        int64_t splits = g_vlut_splits > 0 ? g_vlut_splits
                                           : (2 * device_cu_count() + groups - 1) / std::max<int64_t>(1, groups);
        return {VK_LDS, (int)std::max<int64_t>(1, std::min<int64_t>(splits, kb))};
    }
    const bool swar = g_vlut_swar && ((q == 2 && M <= 4) || (q == 4 && M <= 2));
    if (swar && B > 32 && g_vlut_deep) {
        // 64-row, 64-token workgroups, at most 32 k-quads each: enough K
        // splits for that, and more (down to one k-quad per workgroup) to
        // fill the CUs
        const int64_t kq_total = (kb + 3) / 4;
        const int64_t groups = ((rows + kDeepRows - 1) / kDeepRows) * ((B + kDeepTokens - 1) / kDeepTokens);
        const int64_t min_splits = (kq_total + kDeepKqWg - 1) / kDeepKqWg;
        int64_t splits = g_vlut_splits > 0 ? g_vlut_splits
                                           : std::max<int64_t>(1, device_cu_count() / std::max<int64_t>(1, groups));
        splits = std::max(min_splits, std::min<int64_t>(splits, kq_total));
        return {VK_MFMA_DEEP, (int)splits};
    }
    if (swar && B > 32) {
        // 128-row, 64-token workgroups sharing the activations through LDS,
        // with K splits to fill the CUs (each keeping at least one stage)
        const int64_t groups = ((rows + kWideRows - 1) / kWideRows) * ((B + kWideTokens - 1) / kWideTokens);
        const int64_t max_splits = std::max<int64_t>(1, ((kb + 3) / 4) / kWideStageKq);
        int64_t splits = g_vlut_splits > 0 ? g_vlut_splits
                                           : std::max<int64_t>(1, device_cu_count() / std::max<int64_t>(1, groups));
        return {VK_MFMA_WIDE, (int)std::max<int64_t>(1, std::min<int64_t>(splits, max_splits))};
    }
    if (swar) {
        // one workgroup of 16 rows per CU when the rows allow, else K splits
        // (each keeping at least one 4-k-block step per wave)
        const int64_t row_tiles = (rows + 15) / 16;
        const int64_t max_splits = std::max<int64_t>(1, ((kb + 3) / 4) / kRowsWaves);
        int64_t splits = g_vlut_splits > 0 ? g_vlut_splits
                                           : (device_cu_count() + row_tiles - 1) / std::max<int64_t>(1, row_tiles);
        return {VK_MFMA_ROWS, (int)std::max<int64_t>(1, std::min<int64_t>(splits, max_splits))};
    }
    // every workgroup covers at most kMfmaMaxSteps * 16 k-blocks; beyond
    // that minimum, small batches take more splits (more workgroups in
    // flight) since their partial sums are cheap
    int64_t min_splits = (kb + kMfmaKB * kMfmaMaxSteps - 1) / (kMfmaKB * kMfmaMaxSteps);
    int64_t max_splits = (kb + kMfmaKB - 1) / kMfmaKB;
    int64_t row_tiles = (rows + kMfmaRows - 1) / kMfmaRows;
    int64_t want = B <= 16 ? 2048 : 512;
    int64_t splits = g_vlut_splits > 0 ? g_vlut_splits
                                       : std::max<int64_t>(min_splits, want / std::max<int64_t>(1, row_tiles));
    return {VK_MFMA_TILE, (int)std::max<int64_t>(1, std::min<int64_t>(std::max(splits, min_splits), max_splits))};
}

// One tile entry (pair) per thread: 2 x_hat = sum_m q^m 2 r(b_m) with the
// integer decode, stored as bytes + 128; padding pairs decode to 0.
template <int Q>
__global__ void __launch_bounds__(256) vlut_prepare_decoded_kernel(const uint16_t* words, int64_t rows,
                                                                  int64_t kb_total, int M, int64_t n_pairs,
                                                                  const uint16_t* map, const uint64_t* coarse,
                                                                  uint32_t mask, uint32_t* out)
{
    // pair e: [row tile][k-quad pair][lane][k-quad % 2] (vlut.hpp)
    const int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (e >= n_pairs) return;
    const int half = (int)(e & 1);
    const int lane = (int)((e >> 1) & 63);
    const int64_t tile = e >> 7;
    const int64_t kq2 = ((kb_total + 3) / 4 + 1) / 2;
    const int64_t row = (tile / kq2) * 16 + (lane & 15);
    const int64_t kb = ((tile % kq2) * 2 + half) * 4 + (lane >> 4);
    int acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    if (row < rows && kb < kb_total) {
        int qm = 1;
        for (int m = 0; m < M; ++m) {
            int r2[8];
            two_r_lut<Q>(words[(row * kb_total + kb) * M + m] & mask, map, coarse, r2);
#pragma unroll
            for (int j = 0; j < 8; ++j) acc[j] += qm * r2[j];
            qm *= Q;
        }
    }
    uint32_t lo = 0u, hi = 0u;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        lo |= (uint32_t)(acc[j] + kVlutDecodedBias) << (8 * j);
        hi |= (uint32_t)(acc[4 + j] + kVlutDecodedBias) << (8 * j);
    }
    out[2 * e] = lo;
    out[2 * e + 1] = hi;
}

// VLUT_DECODED6 (vlut.hpp): one thread per (row tile, chunk, lane) writes
// the lane's 8 pairs as 12 words.
template <int Q>
__global__ void __launch_bounds__(256) vlut_prepare_decoded6_kernel(const uint16_t* words, int64_t rows,
                                                                   int64_t kb_total, int M, int64_t n_lanes,
                                                                   const uint16_t* map, const uint64_t* coarse,
                                                                   uint32_t mask, int off, uint32_t* out)
{
    const int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (e >= n_lanes) return;
    const int lane = (int)(e & 63);
    const int64_t chunks = ((kb_total + 3) / 4 + kD6Steps - 1) / kD6Steps;
    const int64_t rt = (e >> 6) / chunks, ch = (e >> 6) % chunks;
    const int64_t row = rt * 16 + (lane & 15);
    uint32_t w[kD6Words];
#pragma unroll
    for (int i = 0; i < kD6Words; ++i) w[i] = 0u;
    for (int st = 0; st < kD6Steps; ++st) {
        const int64_t kb = (ch * kD6Steps + st) * 4 + (lane >> 4);
        int acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
        if (row < rows && kb < kb_total) {
            int qm = 1;
            for (int m = 0; m < M; ++m) {
                int r2[8];
                two_r_lut<Q>(words[(row * kb_total + kb) * M + m] & mask, map, coarse, r2);
#pragma unroll
                for (int j = 0; j < 8; ++j) acc[j] += qm * r2[j];
                qm *= Q;
            }
        }
        // fields f_j = floor(2 x_hat_j / 2) + off and the parity p (shared by
        // the 8: x_hat is in E8), laid out as d6_bytes (vlut_mfma.hpp) reads them
        uint32_t f[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) f[j] = (uint32_t)((acc[j] >> 1) + off);
        const uint32_t v7 = f[7] | ((uint32_t)(acc[0] & 1) << 5);
        const uint32_t top[6] = {f[6] & 3u, (f[6] >> 2) & 3u, (f[6] >> 4) & 3u, v7 & 3u, (v7 >> 2) & 3u, v7 >> 4};
        uint64_t v = 0;
#pragma unroll
        for (int i = 0; i < 6; ++i) v |= (uint64_t)(f[i] | (top[i] << 6)) << (8 * i);
        const int b0 = 48 * st;  // bit offset in the lane's 384 bits
#pragma unroll
        for (int i = 0; i < kD6Words; ++i) {
            const int lo = 32 * i;
            if (lo + 32 <= b0 || lo >= b0 + 48) continue;
            w[i] |= lo >= b0 ? (uint32_t)(v >> (lo - b0)) : (uint32_t)(v << (b0 - lo));
        }
    }
    uint4* dst = reinterpret_cast<uint4*>(out + e * kD6Words);
    dst[0] = make_uint4(w[0], w[1], w[2], w[3]);
    dst[1] = make_uint4(w[4], w[5], w[6], w[7]);
    dst[2] = make_uint4(w[8], w[9], w[10], w[11]);
}

hipError_t vlut_prepare(const uint16_t* words, int64_t rows, int64_t kb, int M, int q, int legacy, int fmt,
                        uint32_t* prepared, hipStream_t s)
{
    const int64_t n = vlut_prepared_words(rows, kb, M, fmt);
    if (n == 0) return hipSuccess;
    const DecodeTables* t = nullptr;
    hipError_t e = get_decode_tables(q, legacy, &t);
    if (e != hipSuccess) return e;
    if (fmt == VLUT_DECODED6) {
        const int off = decoded6_offset(*t, M);
        if (off < 0 || (q != 2 && q != 4)) return hipErrorInvalidValue;  // fields would overflow
        const int64_t lanes = n / kD6Words;
        const dim3 grid((unsigned)((lanes + 255) / 256)), block(256);
        if (q == 4)
            hipLaunchKernelGGL(vlut_prepare_decoded6_kernel<4>, grid, block, 0, s, words, rows, kb, M, lanes,
                               t->cid_map, t->coarse, t->n_codes - 1u, off, prepared);
        else
            hipLaunchKernelGGL(vlut_prepare_decoded6_kernel<2>, grid, block, 0, s, words, rows, kb, M, lanes,
                               t->cid_map, t->coarse, t->n_codes - 1u, off, prepared);
        return hipGetLastError();
    }
    if (fmt == VLUT_DECODED) {
        if (M > t->swar_max_m || (q != 2 && q != 4)) return hipErrorInvalidValue;  // bytes would overflow
        const int64_t pairs = n / 2;
        const dim3 grid((unsigned)((pairs + 255) / 256)), block(256);
        if (q == 4)
            hipLaunchKernelGGL(vlut_prepare_decoded_kernel<4>, grid, block, 0, s, words, rows, kb, M, pairs,
                               t->cid_map, t->coarse, t->n_codes - 1u, prepared);
        else
            hipLaunchKernelGGL(vlut_prepare_decoded_kernel<2>, grid, block, 0, s, words, rows, kb, M, pairs,
                               t->cid_map, t->coarse, t->n_codes - 1u, prepared);
        return hipGetLastError();
    }
    hipLaunchKernelGGL(vlut_prepare_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, words, rows, kb, M, fmt,
                       n, t->cid_map, t->pair_map, t->n_codes - 1u, prepared);
    return hipGetLastError();
}


// One fp32 activation per thread (four a thread), split by split3 (vlut_mfma.hpp).
__global__ void __launch_bounds__(256) vlut_split_kernel(const float* __restrict__ act, int64_t n4,
                                                        uint16_t* __restrict__ planes, int64_t plane)
{
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n4) return;
    const float4 v = reinterpret_cast<const float4*>(act)[i];
    const float a[4] = {v.x, v.y, v.z, v.w};
    uint16_t h[3][4];
#pragma unroll
    for (int j = 0; j < 4; ++j) split3(a[j], h[0][j], h[1][j], h[2][j]);
#pragma unroll
    for (int p = 0; p < 3; ++p)
        *reinterpret_cast<uint2*>(planes + p * plane + 4 * i) =
            make_uint2((uint32_t)h[p][0] | ((uint32_t)h[p][1] << 16), (uint32_t)h[p][2] | ((uint32_t)h[p][3] << 16));
}

// out[b, o] = epilogue((y[b, o] + y[B + b, o]) + y[2B + b, o]) over the three
// planes' scaled outputs y [3B, rows]
__global__ void __launch_bounds__(256) vlut_split_sum_kernel(const float* __restrict__ y, int64_t B, int64_t rows,
                                                            const float* bias, const float* lsq_alpha, int lsq_qmax,
                                                            float* __restrict__ out)
{
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    const int64_t n = B * rows;
    if (i >= n) return;
    const float v = __fadd_rn(__fadd_rn(y[i], y[n + i]), y[2 * n + i]);
    out[i] = vlut_epilogue(v, i % rows, bias, lsq_alpha, lsq_qmax);
}

namespace {

constexpr int64_t align64(int64_t n) { return (n + 63) / 64 * 64; }

}  // namespace

int64_t vlut_split_workspace_floats(int64_t B, int64_t rows, int64_t K, int q, int M)
{
    const int64_t planes = align64(3 * B * K / 2), outs = align64(3 * B * rows);
    return planes + outs + vlut_workspace_floats(vlut_plan(rows, 3 * B, K, q, M, VLUT_METHOD_MFMA), 3 * B, rows);
}

hipError_t vlut_matmul_split(VlutMatmulArgs p, float* workspace, hipStream_t s)
{
    if (p.B == 0 || p.rows == 0) return hipSuccess;
    const int64_t B = p.B, n = B * p.K;
    uint16_t* planes = reinterpret_cast<uint16_t*>(workspace);
    float* y = workspace + align64(3 * B * p.K / 2);
    float* inner = y + align64(3 * B * p.rows);
    VlutMatmulArgs q = p;
    q.act_dtype = DT_BF16;
    q.B = 3 * B;
    q.partial = inner;
    const VlutPlan plan = vlut_plan(p.rows, 3 * B, p.K, p.q, p.M, VLUT_METHOD_MFMA);
    // the plane sum goes into the plan's last kernel where that kernel holds
    // all three planes of an output: the rows kernel with one split and one
    // token tile, or the reduce of a split wide / deep kernel; a staged rows
    // kernel also splits the fp32 activations itself
    const bool v4 = p.rows % 4 == 0 && ((uintptr_t)p.out % 16) == 0 && ((uintptr_t)inner % 16) == 0;
    const bool rows1 = plan.kernel == VK_MFMA_ROWS && plan.splits == 1;
    if (rows1 && 3 * B <= 15 && vlut_rows_staged(p.K, 1)) {
        q.planes_b = B;
        q.act_planes = 1;   // q.act stays the fp32 activations
        return vlut_matmul(q, plan, s);
    }
    hipLaunchKernelGGL(vlut_split_kernel, dim3((unsigned)((n / 4 + 255) / 256)), dim3(256), 0, s,
                       static_cast<const float*>(p.act), n / 4, planes, n);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    q.act = planes;
    if ((rows1 && 3 * B <= 64) || ((plan.kernel == VK_MFMA_WIDE || plan.kernel == VK_MFMA_DEEP) && plan.splits > 1 && v4)) {
        q.planes_b = B;
        return vlut_matmul(q, plan, s);
    }
    q.out = y;
    q.bias = nullptr;
    q.lsq_alpha = nullptr;
    e = vlut_matmul(q, plan, s);
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(vlut_split_sum_kernel, dim3((unsigned)((B * p.rows + 255) / 256)), dim3(256), 0, s, y, B,
                       p.rows, p.bias, p.lsq_alpha, p.lsq_qmax, p.out);
    return hipGetLastError();
}

hipError_t vlut_matmul(VlutMatmulArgs p, const VlutPlan& plan, hipStream_t s)
{
    if (p.B == 0 || p.rows == 0) return hipSuccess;
    const int splits = plan.splits;
    if (vlut_workspace_floats(plan, p.B, p.rows) > 0 && !p.partial) return hipErrorInvalidValue;
    if (plan.kernel == VK_MFMA_TILE) {
        int64_t kb = p.K / 8;
        if ((kb + splits - 1) / splits > (int64_t)kMfmaKB * kMfmaMaxSteps) return hipErrorInvalidValue;
    }
    const DecodeTables* t = nullptr;
    hipError_t e = get_decode_tables(p.q, p.legacy, &t);
    if (e != hipSuccess) return e;
    p.map = t->cid_map;
    p.coarse = t->coarse;
    p.n_coarse = t->n_coarse;
    p.swar = t->swar;
    p.swar_ok = p.M <= t->swar_max_m && g_vlut_swar;
    p.swar_bias = p.swar_ok ? t->swar_bias[p.M] : 0;
    p.pair_map = t->pair_map;
    p.pair_vals = t->pair_vals;
    if (p.prepared == VLUT_DECODED && plan.kernel != VK_MFMA_ROWS && plan.kernel != VK_MFMA_WIDE &&
        plan.kernel != VK_MFMA_DEEP)
        return hipErrorInvalidValue;
    if (p.prepared == VLUT_DECODED6) {
        // the rows and deep kernels read the 6-byte format
        const int off = decoded6_offset(*t, p.M);
        if (off < 0 || (plan.kernel != VK_MFMA_ROWS && plan.kernel != VK_MFMA_DEEP)) return hipErrorInvalidValue;
        p.d6_bias = 2 * off;
    }
    if (p.prepared == VLUT_PAIRS && plan.kernel != VK_LDS) return hipErrorInvalidValue;
    if (plan.kernel == VK_MFMA_WIDE || plan.kernel == VK_MFMA_DEEP || plan.kernel == VK_LDS) {
        if (plan.kernel == VK_LDS) {
            e = p.q == 4 ? dispatch_m<4>(p, VLUT_METHOD_LDS, splits, s) : dispatch_m<2>(p, VLUT_METHOD_LDS, splits, s);
        } else if (!p.swar_ok) {
            return hipErrorInvalidValue;
        } else if (plan.kernel == VK_MFMA_DEEP) {
            const int64_t kq_total = (p.K / 8 + 3) / 4;
            if ((kq_total + splits - 1) / splits > kDeepKqWg) return hipErrorInvalidValue;
            e = vlut_launch_deep(p, splits, s);
        } else {
            e = vlut_launch_wide(p, splits, s);
        }
        if (e != hipSuccess || splits == 1) return e;
        // split-major partials [splits, B, rows] of 2 x_hat products (MFMA) or of x_hat ones (LDS)
        const float mult = plan.kernel == VK_LDS ? 1.f : 0.5f;
        const int64_t nw = p.B * p.rows;
        const bool v4 = p.rows % 4 == 0 && ((uintptr_t)p.out % 16) == 0 && ((uintptr_t)p.partial % 16) == 0;
        if (p.planes_b > 0) {
            if (!v4 || plan.kernel == VK_LDS || p.B != 3 * p.planes_b) return hipErrorInvalidValue;
            hipLaunchKernelGGL(vlut_reduce_planes4_kernel,
                               dim3((unsigned)((p.rows + 63) / 64), (unsigned)((p.planes_b + 15) / 16)), dim3(256), 0, s, p.partial, splits, p.planes_b, p.rows, p.scale, p.scale_mode, mult,
                               p.bias, p.lsq_alpha, p.lsq_qmax, p.out);
        } else if (v4 && plan.kernel == VK_MFMA_DEEP) {
            hipLaunchKernelGGL(vlut_reduce_rg4_kernel, dim3((unsigned)((p.rows + 63) / 64), (unsigned)((p.B + 15) / 16)),
                               dim3(256), 0, s, p.partial, splits, p.B, p.rows, p.scale, p.scale_mode, mult, p.bias,
                               p.lsq_alpha, p.lsq_qmax, p.out);
        } else if (v4 && plan.kernel == VK_LDS)
        {
            const int64_t rg = lds_rows(p.B), groups = (p.rows + rg - 1) / rg;
            // by row group where the kernel put all of a row group's splits on one XCD
            if (groups % 8 == 0 && p.B <= 65535 && groups * (rg / 64) <= 0x7fffffff)
                hipLaunchKernelGGL(vlut_reduce_sm4g_kernel, dim3((unsigned)(groups * (rg / 64)), (unsigned)p.B),
                                   dim3(256), 0, s, p.partial, splits, p.B, p.rows, p.scale, p.scale_mode, mult,
                                   p.bias, p.lsq_alpha, p.lsq_qmax, p.out, rg);
            else
                hipLaunchKernelGGL(vlut_reduce_sm4g_kernel, dim3((unsigned)((nw / 4 + 15) / 16)), dim3(256), 0, s,
                                   p.partial, splits, p.B, p.rows, p.scale, p.scale_mode, mult, p.bias, p.lsq_alpha,
                                   p.lsq_qmax, p.out, (int64_t)0);
        }
        else if (v4)
            hipLaunchKernelGGL(vlut_reduce_sm4_kernel, dim3((unsigned)((nw / 4 + 255) / 256)), dim3(256), 0, s,
                               p.partial, splits, p.B, p.rows, p.scale, p.scale_mode, mult, p.bias, p.lsq_alpha,
                               p.lsq_qmax, p.out);
        else
            hipLaunchKernelGGL(vlut_reduce_sm_kernel, dim3((unsigned)((nw + 255) / 256)), dim3(256), 0, s, p.partial,
                               splits, p.B, p.rows, p.scale, p.scale_mode, mult, p.bias, p.lsq_alpha, p.lsq_qmax,
                               p.out);
        return hipGetLastError();
    }
    if (plan.kernel == VK_MFMA_ROWS) {
        if (!p.swar_ok) return hipErrorInvalidValue;
        e = vlut_launch_rows(p, splits, s);
        if (e != hipSuccess || splits == 1) return e;
    } else {
        e = p.q == 4 ? dispatch_m<4>(p, VLUT_METHOD_MFMA, splits, s) : dispatch_m<2>(p, VLUT_METHOD_MFMA, splits, s);
        if (e != hipSuccess) return e;
    }
    int64_t n = p.B * p.rows;
    hipLaunchKernelGGL(vlut_reduce_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, p.partial, splits,
                       p.B, p.rows, p.scale, p.scale_mode, 0.5f, p.bias, p.lsq_alpha, p.lsq_qmax, p.out);
    return hipGetLastError();
}

}  // namespace coset
