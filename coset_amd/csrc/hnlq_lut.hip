// hnlq_lut.hip -- E8 HNLQ codec for q in {2, 4} with table decode in LDS.
//
// Same contract and bit-exact results as hnlq_codec.hip (the generic path),
// but each decode level is two LDS lookups instead of a projection:
//   2r = 2Gb - q * (2c),  c = coarse[cid_map[idx]]    (tables.hip)
// 2Gb is integer arithmetic on the digits, and the level sum
// x_hat = sum_m q^m r_m (exact in the reference's fp32) is accumulated as
// integers and halved at the end.
//
// Launch: persistent grid, one 1024-thread workgroup per CU.  The q = 4 map
// (65536 x uint16 = 128 KiB) plus the coarse points (<= 8 KiB) fill most of
// the 160 KiB LDS of a gfx950 CU; every workgroup stages them once and then
// walks blocks: the general kernel with a grid stride, the fixed-format one
// in tiles handed out by a per-stream counter (so workgroups that run ahead
// take more tiles), and HBM sees one contiguous read of x and one write of
// the outputs.
#include <algorithm>
#include <map>
#include <atomic>
#include <mutex>
#include <utility>

#include "codec_kernels.hpp"
#include "counters.hpp"
#include "probes.hpp"
#include "tables.hpp"

namespace coset {

int g_codec_plain = 1;
int g_codec_dynamic = 1;

template <int Q>
struct LutShape {
    static constexpr int kCodes = Q * Q * Q * Q * Q * Q * Q * Q;
};

constexpr int kLutThreads = 1024;

// Tile counters of the dynamic schedule: a pair taken from the per-device
// counter ring (counters.hpp) for each launch -- [0] hands out tiles, [1]
// counts finished workgroups, and the workgroup that finishes last puts both
// back to zero and then releases the slot to the host.
constexpr int kTileBlocks = 2;        // blocks per thread in a dynamic tile
constexpr int kTileBlocksDecode = 2;  // the decoder's, whole next tile ahead (1, 4, 8 measured slower)
static __device__ __align__(256) unsigned g_counter_ring[kCounterRing];


// Copies the decode tables to LDS: the map (n_map uint4) and the byte or
// coarse table (n_tab uint64).  Each thread issues all its loads before any
// LDS store (one round trip to L2, not one per element), and each workgroup
// starts at its own offset so the CUs do not all request the same lines at
// once.  blockDim.x == kLutThreads.
template <int PM, int PT>
__device__ __forceinline__ void stage_tables(const uint4* __restrict__ g_map, uint4* s_map, int n_map,
                                             const uint64_t* __restrict__ g_tab, uint64_t* s_tab, int n_tab)
{
    // loads are unconditional (an index past the end reads the last element)
    // so none of them waits behind a branch; only the stores are predicated
    const unsigned salt = blockIdx.x * 2459u;
    const int rm = n_map > 0 ? (int)(salt % (unsigned)n_map) : 0;
    const int rt = n_tab > 0 ? (int)(salt % (unsigned)n_tab) : 0;
    auto at = [](int i, int r, int n) {
        if (i >= n) return n - 1;
        const int j = i + r;
        return j >= n ? j - n : j;
    };
    uint4 m[PM];
    uint64_t t[PT];
#pragma unroll
    for (int k = 0; k < PM; ++k) m[k] = g_map[at(threadIdx.x + k * kLutThreads, rm, n_map)];
    if (n_tab > 0) {
#pragma unroll
        for (int k = 0; k < PT; ++k) t[k] = g_tab[at(threadIdx.x + k * kLutThreads, rt, n_tab)];
    }
#pragma unroll
    for (int k = 0; k < PM; ++k) {
        const int i = threadIdx.x + k * kLutThreads;
        if (i < n_map) s_map[at(i, rm, n_map)] = m[k];
    }
#pragma unroll
    for (int k = 0; k < PT; ++k) {
        const int i = threadIdx.x + k * kLutThreads;
        if (i < n_tab) s_tab[at(i, rt, n_tab)] = t[k];
    }
}

// Block schedules of the persistent kernels.  Each walks blocks 0..n-1
// (n >= 1) of its workgroup's share, calling load(i, in) for a block's input
// into a register set and body(i, in) for the rest, with the next input in
// flight while a body runs.  Loads and stores share one in-order completion
// counter, so the wait before a body leaves the other set's loads and the
// last body's stores in flight only if their number is the same on every
// path into it: the loads are unconditional (past the end they read block
// n - 1), and the first step is peeled so each loop is entered as it is
// re-entered.  A partial last tile recomputes block n - 1 and stores the same
// values to it.  In the grid stride and the whole-tile schedule pro() runs
// once, by every thread of a workgroup that has work, after its first loads
// are issued (the decoder stages its LDS tables there, so the first input
// and the tables arrive together).

// Grid stride (no tile counter): one block ahead.  The loop runs on the
// workgroup's base index, so every lane of a wave takes every step (a lane
// past the end works on block n - 1), which the bodies' wave-wide stores
// assume.
template <typename In, typename Load, typename Body, typename Pro>
__device__ __forceinline__ void schedule_stride(int64_t n, Load& load, Body& body, Pro& pro)
{
    const int64_t last = n - 1;
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    auto blk = [&](int64_t b) {
        const int64_t i = b + threadIdx.x;
        return i < n ? i : last;
    };
    int64_t b = (int64_t)blockIdx.x * blockDim.x;
    if (b >= n) return;
    In in0, in1;
    load(blk(b), in0);
    int64_t b1 = b + stride;
    load(blk(b1), in1);
    pro();
    body(blk(b), in0);
    while (b1 < n) {
        const int64_t b2 = b1 + stride;
        load(blk(b2), in0);
        body(blk(b1), in1);
        if (b2 >= n) break;
        b1 = b2 + stride;
        load(blk(b1), in1);
        body(blk(b2), in0);
    }
}

// The counter pair's protocol: thread 0 takes tiles with atomicInc (the
// compiler rewrites a uniform-address atomicAdd into a wave reduction that
// waits for its result at once) two tiles ahead and publishes them through
// LDS behind an LDS-only barrier; when a workgroup has seen its last tile it
// counts itself done, and the last one resets the pair and then sets the
// slot's release flag (host memory, system scope): only after that does the
// host hand the pair to another launch.
__device__ __forceinline__ void tiles_first_two(unsigned* tiles, unsigned* s_tile, int64_t& t0, int64_t& t1)
{
    if (threadIdx.x == 0) {
        s_tile[2] = atomicInc(tiles, ~0u);
        s_tile[3] = atomicInc(tiles, ~0u);
    }
    lds_barrier();
    t0 = s_tile[2];
    t1 = s_tile[3];
}

__device__ __forceinline__ void tiles_done(unsigned* tiles, unsigned* release)
{
    if (threadIdx.x == 0 && atomicAdd(tiles + 1, 1u) == gridDim.x - 1) {
        atomicExch(tiles, 0u);
        atomicExch(tiles + 1, 0u);
        __threadfence_system();
        __hip_atomic_store(release, 1u, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_SYSTEM);
    }
}

// Dynamic tiles of KT x blockDim.x consecutive blocks (KT per thread,
// blockDim.x apart) with one block ahead; one LDS barrier per tile.
template <int KT, typename In, typename Load, typename Body>
__device__ __forceinline__ void schedule_tiles(int64_t n, TileCounters tc, unsigned* s_tile, Load& load, Body& body)
{
    static_assert(KT % 2 == 0 || KT == 1, "register sets alternate per block");
    unsigned* tiles = tc.pair;
    const int64_t last = n - 1;
    const int64_t ntiles = (n + KT * (int64_t)blockDim.x - 1) / (KT * (int64_t)blockDim.x);
    auto blk = [&](int64_t t, int j) {
        const int64_t b = (t * KT + j) * blockDim.x + threadIdx.x;
        return b < n ? b : last;
    };
    int64_t t0, t1;
    tiles_first_two(tiles, s_tile, t0, t1);
    In in0, in1;
    auto tile = [&](int64_t cur, int64_t nxt, In& s0, In& s1, int slot) {
#pragma unroll
        for (int j = 0; j < KT - 1; ++j) {
            load(blk(cur, j + 1), j % 2 ? s0 : s1);
            body(blk(cur, j), j % 2 ? s1 : s0);
        }
        In& now = (KT - 1) % 2 ? s1 : s0;
        In& ahead = (KT - 1) % 2 ? s0 : s1;
        unsigned grab = 0;
        if (threadIdx.x == 0) grab = atomicInc(tiles, ~0u);
        load(blk(nxt, 0), ahead);
        body(blk(cur, KT - 1), now);
        if (threadIdx.x == 0) s_tile[slot] = grab;
        lds_barrier();
        return (int64_t)s_tile[slot];
    };
    if (t0 < ntiles) {
        load(blk(t0, 0), in0);
        if constexpr (KT == 1) {
            int64_t t2 = tile(t0, t1, in0, in1, 0);
            while (t1 < ntiles) {
                const int64_t t3 = tile(t1, t2, in1, in0, 1);
                if (t2 >= ntiles) break;
                t1 = tile(t2, t3, in0, in1, 0);
                if (t3 >= ntiles) break;
                t2 = t1;
                t1 = t3;
            }
        } else {  // every tile starts in in0
            int64_t t2 = tile(t0, t1, in0, in1, 0);
            int slot = 1;
            while (t1 < ntiles) {
                const int64_t t3 = tile(t1, t2, in0, in1, slot);
                slot ^= 1;
                t1 = t2;
                t2 = t3;
            }
        }
    }
    tiles_done(tiles, tc.release);
}

// Dynamic tiles of KD blocks per thread with all of the next tile's inputs
// in flight while the current tile is processed (inputs of a few bytes).
template <int KD, typename In, typename Load, typename Body, typename Pro>
__device__ __forceinline__ void schedule_tiles_whole(int64_t n, TileCounters tc, unsigned* s_tile, Load& load,
                                                     Body& body, Pro& pro)
{
    unsigned* tiles = tc.pair;
    const int64_t last = n - 1;
    const int64_t ntiles = (n + KD * (int64_t)blockDim.x - 1) / (KD * (int64_t)blockDim.x);
    auto blk = [&](int64_t t, int j) {
        const int64_t b = (t * KD + j) * blockDim.x + threadIdx.x;
        return b < n ? b : last;
    };
    int64_t t0, t1;
    tiles_first_two(tiles, s_tile, t0, t1);
    In A[KD], B[KD];
    auto tile = [&](int64_t cur, int64_t nxt, In (&now)[KD], In (&ahead)[KD], int slot) {
        unsigned grab = 0;
        if (threadIdx.x == 0) grab = atomicInc(tiles, ~0u);
#pragma unroll
        for (int j = 0; j < KD; ++j) load(blk(nxt, j), ahead[j]);
        __asm__ volatile("" ::: "memory");  // the loads stay ahead of the bodies
#pragma unroll
        for (int j = 0; j < KD; ++j) body(blk(cur, j), now[j]);
        if (threadIdx.x == 0) s_tile[slot] = grab;
        lds_barrier();
        return (int64_t)s_tile[slot];
    };
    if (t0 < ntiles) {
#pragma unroll
        for (int j = 0; j < KD; ++j) load(blk(t0, j), A[j]);
    }
    pro();
    if (t0 < ntiles) {
        int64_t t2 = tile(t0, t1, A, B, 0);
        while (t1 < ntiles) {
            const int64_t t3 = tile(t1, t2, B, A, 1);
            if (t2 >= ntiles) break;
            t1 = tile(t2, t3, A, B, 0);
            if (t3 >= ntiles) break;
            t2 = t1;
            t1 = t3;
        }
    }
    tiles_done(tiles, tc.release);
}

// SWAR: each level's 2r comes from three byte tables (tables.hpp) added as
// two 32-bit words, levels are summed with shifts, and the bytes hold
// 2 x_hat + swar_bias; otherwise 2r = 2Gb - q (2c) from the unpacked digits.
template <int Q, int M, int MODE, bool SWAR>
__global__ void __launch_bounds__(kLutThreads) hnlq_lut_kernel(CodecArgs a, const uint16_t* __restrict__ g_map,
                                                            const uint64_t* __restrict__ g_tab,
                                                            int n_coarse, int swar_bias)
{
    constexpr int NC = LutShape<Q>::kCodes;
    __shared__ __align__(16) uint16_t s_map[NC];
    __shared__ uint64_t s_tab[SWAR ? 512 + kMaxCoarse : kMaxCoarse];

    if (MODE != MODE_ENCODE) {
        stage_tables<(NC / 8 + kLutThreads - 1) / kLutThreads,
                     ((SWAR ? 512 : 0) + kMaxCoarse + kLutThreads - 1) / kLutThreads>(
            reinterpret_cast<const uint4*>(g_map), reinterpret_cast<uint4*>(s_map), NC / 8, g_tab, s_tab,
            SWAR ? 512 + n_coarse : n_coarse);
        __syncthreads();
    }
    const float half_bias = 0.5f * (float)swar_bias;

    if (blockIdx.x == 0 && threadIdx.x == 0 && a.step_counter) *a.step_counter += 1;
    const float qf = (float)Q;
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < a.n; i += stride) {
        float scale = 1.f;
        if (a.scale_mode == SCALE_CODEC)
            scale = a.beta;
        else if (a.scale_mode == SCALE_LAYER)
            scale = layer_scale(a, i);

        // Level words are collected in one 64-bit register (M <= 4 words of
        // 16 bits); each level is encoded, then decoded from its digits.
        uint64_t pack = 0;
        float xl[8];
        if (MODE != MODE_DECODE) {
            if (a.x_dtype == DT_BF16) {
                uint4 v = reinterpret_cast<const uint4*>(a.x)[i];
                uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    xl[2 * j] = __uint_as_float(w[j] << 16);
                    xl[2 * j + 1] = __uint_as_float(w[j] & 0xffff0000u);
                }
            } else {
                const float4* p = reinterpret_cast<const float4*>(a.x) + 2 * i;
                float4 u = p[0], v = p[1];
                xl[0] = u.x; xl[1] = u.y; xl[2] = u.z; xl[3] = u.w;
                xl[4] = v.x; xl[5] = v.y; xl[6] = v.z; xl[7] = v.w;
            }
            if (a.scale_mode == SCALE_CODEC) {
                if (a.beta_is_pow2) {
                    if (a.beta_inv != 1.f) {  // x / 1 = x
#pragma unroll
                        for (int j = 0; j < 8; ++j) xl[j] = __fmul_rn(xl[j], a.beta_inv);
                    }
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
        } else {
            const uint16_t* pw = reinterpret_cast<const uint16_t*>(a.packed_in) + (size_t)i * M;
            if (M == 2) {
                pack = *reinterpret_cast<const uint32_t*>(pw);
            } else if (M == 4) {
                pack = *reinterpret_cast<const uint64_t*>(pw);
            } else {
#pragma unroll
                for (int m = 0; m < M; ++m) pack |= (uint64_t)pw[m] << (16 * m);
            }
        }

        int acc2[8];  // sum_m q^m * 2 r_m, exact integers
#pragma unroll
        for (int j = 0; j < 8; ++j) acc2[j] = 0;
        uint32_t sw0 = 0u, sw1 = 0u;  // SWAR: bytes 0-3 / 4-7 of sum_m q^m (2 r_m + bias)
        int wq = 1;
#pragma unroll
        for (int m = 0; m < M; ++m) {
            int b[8];
            uint32_t word;
            if (MODE != MODE_DECODE) {
                encode_level<Q>(xl, a.fast_projection, Q, b);
                word = pack_word<Q>(b, Q);
                pack |= (uint64_t)word << (16 * m);
                if (a.codes_f32) {
                    float4* cp = reinterpret_cast<float4*>(a.codes_f32 + ((size_t)i * M + m) * 8);
                    cp[0] = make_float4((float)b[0], (float)b[1], (float)b[2], (float)b[3]);
                    cp[1] = make_float4((float)b[4], (float)b[5], (float)b[6], (float)b[7]);
                }
                if (m + 1 < M) {
#pragma unroll
                    for (int j = 0; j < 8; ++j) xl[j] = div_q<Q>(xl[j], qf);
                }
            } else {
                word = (uint32_t)(pack >> (16 * m)) & (uint32_t)(NC - 1);  // table bounds for any input
                unpack_word<Q>(word, Q, b);
            }
            if (MODE != MODE_ENCODE && SWAR) {
                const uint2 tl = *reinterpret_cast<const uint2*>(&s_tab[256 + (word & 0xffu)]);
                const uint2 tc = *reinterpret_cast<const uint2*>(&s_tab[512 + s_map[word]]);
                uint32_t l0 = tl.x + tc.x, l1 = tl.y + tc.y;
                if (Q != 2) {
                    const uint2 th = *reinterpret_cast<const uint2*>(&s_tab[(word >> 8) & 0xffu]);
                    l0 += th.x;
                    l1 += th.y;
                }
                sw0 += l0 * (uint32_t)wq;  // q^m: a shift, no byte overflows (checked when tables are built)
                sw1 += l1 * (uint32_t)wq;
                wq *= Q;
            } else if (MODE != MODE_ENCODE) {
                int u[8];  // 2 G b
                u[0] = 4 * b[0] - 2 * b[1] + b[7];
#pragma unroll
                for (int j = 1; j < 6; ++j) u[j] = 2 * (b[j] - b[j + 1]) + b[7];
                u[6] = 2 * b[6] + b[7];
                u[7] = b[7];
                uint64_t c = s_tab[s_map[word]];
#pragma unroll
                for (int j = 0; j < 8; ++j) {
                    int two_c = (int)(int8_t)(uint8_t)(c >> (8 * j));
                    acc2[j] += wq * (u[j] - Q * two_c);
                }
                wq *= Q;
            }
        }
        if (MODE != MODE_DECODE && a.packed) {
            uint16_t* pw = reinterpret_cast<uint16_t*>(a.packed) + (size_t)i * M;
            if (M == 1) {
                pw[0] = (uint16_t)pack;
            } else if (M == 2) {
                *reinterpret_cast<uint32_t*>(pw) = (uint32_t)pack;
            } else {
#pragma unroll
                for (int m = 0; m < M; ++m) pw[m] = (uint16_t)(pack >> (16 * m));
            }
        }
        if (MODE == MODE_ENCODE) continue;

        if (!a.out) continue;
        float o[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            float v;
            if (SWAR) {  // (byte - bias) / 2, exact
                const uint32_t w = j < 4 ? sw0 : sw1;
                v = __fmaf_rn((float)((w >> (8 * (j & 3))) & 0xffu), 0.5f, -half_bias);
            } else {
                v = __fmul_rn((float)acc2[j], 0.5f);  // exact
            }
            if (a.scale_mode == SCALE_CODEC) {
                if (a.beta != 1.f) v = __fmul_rn(v, scale);  // x * 1 = x
            } else if (a.scale_mode == SCALE_LAYER) {
                v = __fdiv_rn(v, scale);
                v = (v != v) ? v : fminf(fmaxf(v, -a.clip), a.clip);  // clamp keeps NaN
            }
            o[j] = v;
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
}

typedef float f32x4_nt __attribute__((ext_vector_type(4)));

// Streaming (non-temporal) stores of the outputs, which nothing reads back
// in the same launch: 2^24-block round trip 203.9 -> 200.3 us on one box
// (non-temporal loads of the input measured slower and are not used).
__device__ __forceinline__ void store_nt(void* p, const float4& v)
{
    __builtin_nontemporal_store(__builtin_bit_cast(f32x4_nt, v), static_cast<f32x4_nt*>(p));
}

__device__ __forceinline__ void store_nt(uint32_t* p, uint32_t v)
{
    __builtin_nontemporal_store(v, p);
}

// Stores one block's 8 decoded floats (32 bytes) through the wave's 1 KiB
// LDS slice st: half the wave at a time writes its blocks' 32 bytes there
// and the whole wave reads them back 16 bytes a lane, so each of the two
// stores writes 32 consecutive blocks (1 KiB) rather than every lane 32
// bytes.  Every lane is active and the lanes of a wave hold consecutive
// blocks clamped to n - 1 (the schedules' contract), so lane q's block is
// min(i_0 + q, n - 1), i_0 being lane 0's.  LDS operations of one wave
// complete in order, so the slice needs no barrier, only compiler fences:
// a lane reads what other lanes wrote, which a single lane's view of
// memory does not show.
__device__ __forceinline__ void store_out_wave(float* out, int64_t n, int64_t i, const float o[8], float4* st)
{
    const int lane = threadIdx.x & 63;
    const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)i);
    const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)((uint64_t)i >> 32));
    const int64_t i0 = (int64_t)(((uint64_t)hi << 32) | lo);
    const int64_t room = n - 1 - i0;
    const int lim = room < 63 ? (int)room : 63;
    char* dst = reinterpret_cast<char*>(out + 8 * i0);
#pragma unroll
    for (int h = 0; h < 2; ++h) {
        if ((lane >> 5) == h) {
            st[2 * (lane & 31)] = make_float4(o[0], o[1], o[2], o[3]);
            st[2 * (lane & 31) + 1] = make_float4(o[4], o[5], o[6], o[7]);
        }
        __asm__ volatile("" ::: "memory");
        const float4 v = st[lane];
        __asm__ volatile("" ::: "memory");
        const uint32_t q = min(32 * h + (lane >> 1), lim);
        store_nt(dst + (q * 32u + (lane & 1) * 16u), v);  // 32-bit lane offset
    }
}

// The float code tensor [n, 2, 8] of the two level words of a block (low 16
// bits: level 0), 64 bytes a block, through the wave's 1 KiB LDS slice as
// in store_out_wave: a quarter of the wave at a time writes its blocks'
// codes there and the whole wave reads them back 16 bytes a lane, so each
// of the four stores writes 16 consecutive blocks (1 KiB).  NT: the stores
// are non-temporal (measured faster for the encoder, whose only other output
// is the packed words, and slower beside the decoded-block stores of the
// round trip).
template <int Q, bool NT>
__device__ __forceinline__ void store_codes_wave(float* codes, int64_t n, int64_t i, uint32_t words, uint4* st)
{
    uint32_t e[4][4];  // e[chunk][dword]: chunk c = level c / 2, coordinates 4 (c % 2) ..
#pragma unroll
    for (int m = 0; m < 2; ++m) {
        int b[8];
        unpack_word<Q>((words >> (16 * m)) & 0xffffu, Q, b);
#pragma unroll
        for (int d = 0; d < 8; ++d) e[2 * m + d / 4][d % 4] = __float_as_uint((float)b[d]);
    }
    const int lane = threadIdx.x & 63;
    const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)i);
    const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)((uint64_t)i >> 32));
    const int64_t i0 = (int64_t)(((uint64_t)hi << 32) | lo);
    const int64_t room = n - 1 - i0;
    const int lim = room < 63 ? (int)room : 63;
    char* dst = reinterpret_cast<char*>(codes + 16 * i0);
#pragma unroll
    for (int h = 0; h < 4; ++h) {
        if ((lane >> 4) == h) {
#pragma unroll
            for (int c = 0; c < 4; ++c) st[4 * (lane & 15) + c] = make_uint4(e[c][0], e[c][1], e[c][2], e[c][3]);
        }
        __asm__ volatile("" ::: "memory");
        const uint4 v = st[lane];
        __asm__ volatile("" ::: "memory");
        const uint32_t q = min(16 * h + (lane >> 2), lim);
        char* p = dst + (q * 64u + (lane & 3) * 16u);  // 32-bit lane offset
        if constexpr (NT)
            store_nt(p, __builtin_bit_cast(float4, v));
        else
            *reinterpret_cast<uint4*>(p) = v;
    }
}

// Same contract for the common case, with everything the general kernel
// decides per block fixed at compile time: fp32 input and output, no scale
// or a codec beta = 2^k (x / beta == x * 2^-k exactly; SCALED false when
// beta = 1), no dither, byte-table decode, the encoder's fast projection
// on; the float code tensor is an optional output (CODES).  The loop is
// unrolled twice so the next block's input loads into the other register
// set while the current block is processed.
// One encoder level straight to its word idx(b).  On the fast path each
// digit (the low bits of a row) is funnelled into the top of an accumulator
// as the accumulator shifts right, one v_alignbit per digit.
template <int Q>
__device__ __forceinline__ uint32_t encode_level_word(const float xl[8], bool in_range)
{
    static_assert(Q == 2 || Q == 4, "byte-table formats");
    constexpr int L = Q == 2 ? 1 : 2;
    int c[8];
    const bool ok = fast_rows(xl, c, in_range);
#pragma unroll
    for (int i = 0; i < 8; ++i) __asm__ volatile("" : "+v"(c[i]));  // rows computed ahead of the fallback
    if (ok) {
        uint32_t acc = 0u;
#pragma unroll
        for (int j = 7; j >= 0; --j) acc = __builtin_amdgcn_alignbit((uint32_t)c[j], acc, L);
        return acc >> (32 - 8 * L);  // digit 0 highest: sum_j b_j Q^(7-j)
    }
    float y[8];
    int b[8];
    project<false, false>(xl, y);
    lattice_digits<Q>(y, Q, b);
    return pack_word<Q>(b, Q);
}

// PROBE (measurement, the round trip only): 0 is the codec; 1 keeps the
// launch, table staging, tile schedule, loads and stores but writes each
// block's input back out and a word folded from its bits, with no lattice
// arithmetic -- the streaming ceiling of this kernel's access pattern; 2 is
// 1 without the table staging.
template <int Q, int M, int MODE, bool SCALED, bool CODES, bool PK, int PROBE = 0>
__global__ void __launch_bounds__(kLutThreads) hnlq_plain_kernel(CodecArgs a, const uint16_t* __restrict__ g_map,
                                                              const uint64_t* __restrict__ g_tab, int n_coarse,
                                                              int swar_bias, TileCounters tc)
{
    constexpr int NC = LutShape<Q>::kCodes;
    __shared__ __align__(16) uint16_t s_map[NC];
    __shared__ uint64_t s_tab[512 + kMaxCoarse];
    __shared__ unsigned s_tile[4];
    __shared__ float4 s_stage[MODE == MODE_ENCODE && !CODES ? 1 : kLutThreads / 64][64];  // store_*_wave
    auto stage = [&]() {
        stage_tables<(NC / 8 + kLutThreads - 1) / kLutThreads, (512 + kMaxCoarse + kLutThreads - 1) / kLutThreads>(
            reinterpret_cast<const uint4*>(g_map), reinterpret_cast<uint4*>(s_map), NC / 8, g_tab, s_tab,
            512 + n_coarse);
    };
    // The decoder stages its tables after the first tile's loads are issued
    // (an LDS-only barrier: the loads stay in flight), 2.5 us sooner per
    // launch at 2^24 blocks; the round trip stages them first (measured
    // faster that way on the same box).
    static_assert(PROBE == 0 || (MODE == MODE_ROUNDTRIP && M == 2 && PK && !CODES && !SCALED), "probe: C2's outputs");
    if constexpr (MODE == MODE_ROUNDTRIP && PROBE != 2) {
        stage();
        __syncthreads();
    }
    auto pro = [&]() {
        if constexpr (MODE == MODE_DECODE) {
            stage();
            lds_barrier();
        }
    };
    const float half_bias = 0.5f * (float)swar_bias;
    const float4* xs = reinterpret_cast<const float4*>(a.x);
    const int64_t n = a.n;

    struct In {
        float4 u, v;
        uint64_t w;
    };
    auto load = [&](int64_t i, In& in) {
        if (MODE != MODE_DECODE) {
            in.u = xs[2 * i];
            in.v = xs[2 * i + 1];
        } else {
            const uint16_t* pw = reinterpret_cast<const uint16_t*>(a.packed_in) + (size_t)i * M;
            if (M == 2) {
                in.w = *reinterpret_cast<const uint32_t*>(pw);
            } else if (M == 4) {
                in.w = *reinterpret_cast<const uint64_t*>(pw);
            } else {
                uint64_t w = 0;
#pragma unroll
                for (int m = 0; m < M; ++m) w |= (uint64_t)pw[m] << (16 * m);
                in.w = w;
            }
        }
    };
    auto body = [&](int64_t i, const In& in) {
        if constexpr (PROBE != 0) {
            const uint32_t f = __float_as_uint(in.u.x) ^ __float_as_uint(in.u.y) ^ __float_as_uint(in.u.z) ^
                               __float_as_uint(in.u.w) ^ __float_as_uint(in.v.x) ^ __float_as_uint(in.v.y) ^
                               __float_as_uint(in.v.z) ^ __float_as_uint(in.v.w);
            *reinterpret_cast<uint32_t*>(reinterpret_cast<uint16_t*>(a.packed) + (size_t)i * 2) = f;
            const float o[8] = {in.u.x, in.u.y, in.u.z, in.u.w, in.v.x, in.v.y, in.v.z, in.v.w};
            store_out_wave(static_cast<float*>(a.out), n, i, o, s_stage[threadIdx.x >> 6]);
            return;
        }
        float xl[8] = {in.u.x, in.u.y, in.u.z, in.u.w, in.v.x, in.v.y, in.v.z, in.v.w};
        uint64_t pack = MODE == MODE_DECODE ? in.w : 0;
        if (MODE != MODE_DECODE && SCALED) {
#pragma unroll
            for (int j = 0; j < 8; ++j) xl[j] = __fmul_rn(xl[j], a.beta_inv);
        }
        // level m's input is xl * Q^-m exactly, so max |x_m| < 2^21 is
        // max |x_0| < 2^21 Q^m
        float amax = 0.f;
        if (MODE != MODE_DECODE) {
            amax = fabsf(xl[0]);
#pragma unroll
            for (int j = 1; j < 8; ++j) amax = fmaxf(amax, fabsf(xl[j]));
        }
        uint32_t sw0 = 0u, sw1 = 0u;
        float lim = kFastMaxAbs;
#pragma unroll
        for (int m = 0; m < M; ++m) {
            uint32_t word;
            if (MODE != MODE_DECODE) {
                word = encode_level_word<Q>(xl, amax < lim);
                lim *= (float)Q;
                pack |= (uint64_t)word << (16 * m);
                if (CODES && M != 2) {  // the reference's float code tensor [n, M, 8]
                    int b[8];
                    unpack_word<Q>(word, Q, b);
                    float4* cp = reinterpret_cast<float4*>(a.codes_f32 + ((size_t)i * M + m) * 8);
                    cp[0] = make_float4((float)b[0], (float)b[1], (float)b[2], (float)b[3]);
                    cp[1] = make_float4((float)b[4], (float)b[5], (float)b[6], (float)b[7]);
                }
                if (m + 1 < M) {
#pragma unroll
                    for (int j = 0; j < 8; ++j) xl[j] = __fmul_rn(xl[j], 1.0f / (float)Q);  // exact: Q = 2^k
                }
            } else {
                word = (uint32_t)(pack >> (16 * m)) & (uint32_t)(NC - 1);  // table bounds for any input
            }
            if (MODE != MODE_ENCODE) {
                const uint2 tl = *reinterpret_cast<const uint2*>(&s_tab[256 + (word & 0xffu)]);
                const uint2 tc = *reinterpret_cast<const uint2*>(&s_tab[512 + s_map[word]]);
                uint32_t l0 = tl.x + tc.x, l1 = tl.y + tc.y;
                if (Q != 2) {
                    const uint2 th = *reinterpret_cast<const uint2*>(&s_tab[(word >> 8) & 0xffu]);
                    l0 += th.x;
                    l1 += th.y;
                }
                constexpr int L = Q == 2 ? 1 : 2;
                sw0 += l0 << (L * m);  // q^m, no byte overflows (checked when the tables are built)
                sw1 += l1 << (L * m);
            }
        }
        if (MODE != MODE_DECODE && CODES && M == 2)
            store_codes_wave<Q, MODE == MODE_ENCODE>(a.codes_f32, n, i, (uint32_t)pack, reinterpret_cast<uint4*>(s_stage[threadIdx.x >> 6]));
        if (MODE != MODE_DECODE && PK) {
            uint16_t* pw = reinterpret_cast<uint16_t*>(a.packed) + (size_t)i * M;
            if (M == 1) {
                pw[0] = (uint16_t)pack;
            } else if (M == 2) {
                store_nt(reinterpret_cast<uint32_t*>(pw), (uint32_t)pack);
            } else if (M == 4) {
                *reinterpret_cast<uint64_t*>(pw) = pack;
            } else {
#pragma unroll
                for (int m = 0; m < M; ++m) pw[m] = (uint16_t)(pack >> (16 * m));
            }
        }
        if (MODE == MODE_ENCODE) return;
        float o[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const uint32_t w = j < 4 ? sw0 : sw1;
            o[j] = __fmaf_rn((float)((w >> (8 * (j & 3))) & 0xffu), 0.5f, -half_bias);  // (byte - bias) / 2, exact
            if (SCALED) o[j] = __fmul_rn(o[j], a.beta);
        }
        // staged whole-line stores measured faster for the decoder and the
        // round trip with packed words, direct stores for the round trip
        // without them (A/B on one box, 2^24 blocks: 1.2 and 2.7 us)
        if constexpr (MODE == MODE_DECODE || PK) {
            store_out_wave(static_cast<float*>(a.out), n, i, o, s_stage[threadIdx.x >> 6]);
        } else {
            float4* p = reinterpret_cast<float4*>(a.out) + 2 * i;
            store_nt(p, make_float4(o[0], o[1], o[2], o[3]));
            store_nt(p + 1, make_float4(o[4], o[5], o[6], o[7]));
        }
    };

    // every store of a body is unconditional (see the schedules above)
    if constexpr (MODE == MODE_DECODE) {
        if (tc.pair) {
            schedule_tiles_whole<kTileBlocksDecode, In>(n, tc, s_tile, load, body, pro);
            return;
        }
    }
    if constexpr (MODE != MODE_DECODE) {
        if (tc.pair) {
            // one block per thread and tile when the float codes are written
            // (e8_encode 290 -> 278 us at 2^24 blocks; two blocks measured
            // faster for the others, A/B on one box)
            schedule_tiles<CODES ? 1 : kTileBlocks, In>(n, tc, s_tile, load, body);
            return;
        }
    }
    schedule_stride<In>(n, load, body, pro);
}

namespace {

// Per-device counter rings: the pairs' device address, the release flags
// (coherent host memory, and their device address) and the host bookkeeping.
constexpr int kRingDevices = 64;
std::mutex g_ring_mu;
unsigned* g_ring_pairs[kRingDevices] = {nullptr};
unsigned* g_ring_release_dev[kRingDevices] = {nullptr};
CounterRing* g_ring[kRingDevices] = {nullptr};

CounterRing* device_ring(int dev)
{
    std::lock_guard<std::mutex> lock(g_ring_mu);
    if (!g_ring[dev]) {
        void* p = nullptr;
        if (hipGetSymbolAddress(&p, HIP_SYMBOL(g_counter_ring)) != hipSuccess || !p) {
            (void)hipGetLastError();
            return nullptr;
        }
        // the kernels write the flags with system-scope stores; every slot starts free
        void* h = nullptr;
        if (hipHostMalloc(&h, kCounterSlots * sizeof(uint32_t), hipHostMallocCoherent) != hipSuccess || !h) {
            (void)hipGetLastError();
            return nullptr;
        }
        void* hd = nullptr;
        if (hipHostGetDevicePointer(&hd, h, 0) != hipSuccess || !hd) {
            (void)hipGetLastError();
            (void)hipHostFree(h);
            return nullptr;
        }
        uint32_t* flags = static_cast<uint32_t*>(h);
        for (uint32_t i = 0; i < kCounterSlots; ++i) flags[i] = 1u;
        CounterRing* r = new CounterRing;
        r->release = flags;
        g_ring_pairs[dev] = static_cast<unsigned*>(p);
        g_ring_release_dev[dev] = static_cast<unsigned*>(hd);
        g_ring[dev] = r;
    }
    return g_ring[dev];
}

}  // namespace

// A counter pair of the current device's ring for one launch on stream s
// (counters.hpp), or none (pair null: the static schedule) while s captures a
// graph (a replayed graph keeps the counters it was captured with and may
// run beside later launches), while every slot is held by a launch still in
// flight, or when the ring cannot be set up.
TileCounters take_counters(hipStream_t s)
{
    const TileCounters none{nullptr, nullptr, -1};
    hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing(s, &cap) != hipSuccess) {
        (void)hipGetLastError();  // the query's own error, not the launch's
        return none;
    }
    if (cap != hipStreamCaptureStatusNone) return none;
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kRingDevices) return none;
    CounterRing* r = device_ring(dev);
    if (!r) return none;
    const int64_t slot = ring_acquire(*r);
    if (slot < 0) return none;
    return TileCounters{g_ring_pairs[dev] + 2 * slot, g_ring_release_dev[dev] + slot, slot};
}

// Hands back the slot of a launch that failed to start (its kernel never
// releases it); call on the device the slot was taken on.
void return_counters(const TileCounters& tc)
{
    if (!tc.pair || tc.slot < 0) return;
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kRingDevices) return;
    CounterRing* r = g_ring[dev];
    if (r) ring_release(*r, tc.slot);
}

namespace {

int cu_count()
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

// Byte tables hold q^M-weighted sums for q = 2 (M <= 4) and q = 4 (M <= 2);
// the encoder alone needs no tables.
template <int Q, int M, int MODE>
hipError_t launch_plain(const CodecArgs& a, int grid, const uint16_t* map, const uint64_t* sw, int nc, int bias,
                        hipStream_t s)
{
    if constexpr (MODE == MODE_ENCODE || Q == 2 || M <= 2) {
        const bool scaled = a.scale_mode == SCALE_CODEC && a.beta != 1.f;
        const bool codes = MODE != MODE_DECODE && a.codes_f32;
        const TileCounters tiles = g_codec_dynamic ? take_counters(s) : TileCounters{nullptr, nullptr, -1};
        // packed words are always written by the encoder, optional in the
        // round trip (e8_quantize asks for the decoded blocks only)
        const bool pk = MODE == MODE_ENCODE || (MODE == MODE_ROUNDTRIP && a.packed);
#define COSET_PLAIN(SC, CO, P) \
    hipLaunchKernelGGL((hnlq_plain_kernel<Q, M, MODE, SC, CO, P>), dim3(grid), dim3(kLutThreads), 0, s, a, map, sw, nc, \
                       bias, tiles)
        if constexpr (MODE == MODE_DECODE) {
            if (scaled) COSET_PLAIN(true, false, false); else COSET_PLAIN(false, false, false);
        } else if constexpr (MODE == MODE_ENCODE) {
            if (scaled) {
                if (codes) COSET_PLAIN(true, true, true); else COSET_PLAIN(true, false, true);
            } else {
                if (codes) COSET_PLAIN(false, true, true); else COSET_PLAIN(false, false, true);
            }
        } else if (pk) {
            if (scaled) {
                if (codes) COSET_PLAIN(true, true, true); else COSET_PLAIN(true, false, true);
            } else {
                if (codes) COSET_PLAIN(false, true, true); else COSET_PLAIN(false, false, true);
            }
        } else {
            if (scaled) {
                if (codes) COSET_PLAIN(true, true, false); else COSET_PLAIN(true, false, false);
            } else {
                if (codes) COSET_PLAIN(false, true, false); else COSET_PLAIN(false, false, false);
            }
        }
#undef COSET_PLAIN
        const hipError_t e = hipGetLastError();
        if (e != hipSuccess) return_counters(tiles);
        return e;
    }
    return hipErrorInvalidValue;
}

template <int Q, int MODE>
hipError_t launch_q(const CodecArgs& a, const DecodeTables* t, hipStream_t s)
{
    int64_t need = (a.n + kLutThreads - 1) / kLutThreads;
    int grid = (int)std::min<int64_t>(need, (int64_t)cu_count());
    const uint16_t* map = t ? t->cid_map : nullptr;
    int nc = t ? t->n_coarse : 0;
    const bool swar = t && a.M <= t->swar_max_m;
    const uint64_t* tab = t ? (swar ? t->swar : t->coarse) : nullptr;
    const int bias = swar ? t->swar_bias[a.M] : 0;
    // the plain kernel: fp32 in and out, no scale or a codec beta = 2^k, no
    // dither, no step counter, byte tables for the decode, and the encoder's
    // fast projection on (it is a compile-time constant there), and the
    // mode's outputs present (its stores are unconditional; the round trip's
    // packed words are a compile-time option)
    const bool plain = (MODE == MODE_DECODE || (a.x_dtype == DT_F32 && a.fast_projection)) &&
                       (MODE == MODE_ENCODE || a.out_dtype == DT_F32) &&
                       (a.scale_mode == SCALE_NONE || (a.scale_mode == SCALE_CODEC && a.beta_is_pow2)) &&
                       !a.dither && !a.step_counter && (MODE == MODE_ENCODE || swar) &&
                       (MODE != MODE_ENCODE || a.packed) && (MODE == MODE_ENCODE || a.out) && g_codec_plain;
    if (plain) {
        const uint64_t* sw = t ? t->swar : nullptr;
        switch (a.M) {
        case 1: return launch_plain<Q, 1, MODE>(a, grid, map, sw, nc, bias, s);
        case 2: return launch_plain<Q, 2, MODE>(a, grid, map, sw, nc, bias, s);
        case 3: return launch_plain<Q, 3, MODE>(a, grid, map, sw, nc, bias, s);
        case 4: return launch_plain<Q, 4, MODE>(a, grid, map, sw, nc, bias, s);
        default: return hipErrorInvalidValue;
        }
    }
#define COSET_LUT(MM, SW) \
    hipLaunchKernelGGL((hnlq_lut_kernel<Q, MM, MODE, SW>), dim3(grid), dim3(kLutThreads), 0, s, a, map, tab, nc, bias)
    switch (a.M) {
    case 1: if (swar) COSET_LUT(1, true); else COSET_LUT(1, false); break;
    case 2: if (swar) COSET_LUT(2, true); else COSET_LUT(2, false); break;
    case 3: if (Q == 2 && swar) COSET_LUT(3, Q == 2); else COSET_LUT(3, false); break;
    case 4: if (Q == 2 && swar) COSET_LUT(4, Q == 2); else COSET_LUT(4, false); break;
    default: return hipErrorInvalidValue;
    }
#undef COSET_LUT
    return hipGetLastError();
}

}  // namespace

hipError_t launch_c2_stream_probe(const float* x, int64_t n, uint32_t* packed, float* out, int staged, hipStream_t s)
{
    CodecArgs a{};
    a.x = x;
    a.x_dtype = DT_F32;
    a.n = n;
    a.q = 4;
    a.M = 2;
    a.packed = packed;
    a.out = out;
    a.out_dtype = DT_F32;
    const DecodeTables* t = nullptr;
    hipError_t e = get_decode_tables(4, 0, &t);
    if (e != hipSuccess) return e;
    const int grid = (int)std::min<int64_t>((n + kLutThreads - 1) / kLutThreads, (int64_t)cu_count());
    const TileCounters tiles = g_codec_dynamic ? take_counters(s) : TileCounters{nullptr, nullptr, -1};
    if (staged)
        hipLaunchKernelGGL((hnlq_plain_kernel<4, 2, MODE_ROUNDTRIP, false, false, true, 1>), dim3(grid),
                           dim3(kLutThreads), 0, s, a, t->cid_map, t->swar, t->n_coarse, t->swar_bias[2], tiles);
    else
        hipLaunchKernelGGL((hnlq_plain_kernel<4, 2, MODE_ROUNDTRIP, false, false, true, 2>), dim3(grid),
                           dim3(kLutThreads), 0, s, a, t->cid_map, t->swar, t->n_coarse, t->swar_bias[2], tiles);
    e = hipGetLastError();
    if (e != hipSuccess) return_counters(tiles);
    return e;
}

bool lut_path_supported(const CodecArgs& a, int mode)
{
    if (a.q != 2 && a.q != 4) return false;
    if (a.M < 1 || a.M > 4) return false;
    if (mode == MODE_DECODE && a.codes_in_f32) return false;  // float codes may be off-grid
    return true;
}

hipError_t launch_codec_lut(const CodecArgs& a, int mode, hipStream_t s)
{
    const DecodeTables* t = nullptr;
    if (mode != MODE_ENCODE) {
        hipError_t e = get_decode_tables(a.q, 0, &t);
        if (e != hipSuccess) return e;
    }
    if (a.q == 4) {
        switch (mode) {
        case MODE_ENCODE: return launch_q<4, MODE_ENCODE>(a, t, s);
        case MODE_DECODE: return launch_q<4, MODE_DECODE>(a, t, s);
        default: return launch_q<4, MODE_ROUNDTRIP>(a, t, s);
        }
    }
    switch (mode) {
    case MODE_ENCODE: return launch_q<2, MODE_ENCODE>(a, t, s);
    case MODE_DECODE: return launch_q<2, MODE_DECODE>(a, t, s);
    default: return launch_q<2, MODE_ROUNDTRIP>(a, t, s);
    }
}

}  // namespace coset
