// gemm_tn.hip -- dW_q = gy^T x, the weight-gradient product of the QAT
// layer's F.linear (coset/core/layers.py:478; its autograd runs this product
// in the reference), on gfx950's matrix cores.
//
// Both operands keep the token dimension K outermost (gy [K, M], x [K, N],
// row-major), so each 16-byte global load holds 8 consecutive output rows
// (or columns) of one token, while a 16x16x32 MFMA operand wants 8
// consecutive tokens per lane.  Each 32-token slice is staged in LDS as it
// lies in memory ([k][m], m contiguous) and read back with
// ds_read_b64_tr_b16: within each 16-lane group, lane i receives element i
// of the four 8-byte rows that lanes 4j + i / 4 (j = 0..3) addressed, so
// lanes r = 0..15 addressing (k0 + r / 4, m0 + 4 (r % 4)) give lane i the
// four tokens k0..k0+3 of row m0 + i -- the MFMA layout (lane l: row l % 16,
// tokens 8 (l / 16) .. + 7 from two such reads).
//
// One workgroup of NW = 8 waves per 64 x 64 output tile (each token row of a
// tile is one whole 128-byte line; partial lines cost the L2 about a third
// of its delivery rate) and per K split.  The waves share no data: wave w
// takes the 32-token slices w, w + NW, ... of the workgroup's K range, stages
// each in an LDS slice of its own and multiplies it, so the main loop has no
// barrier (a wave's LDS operations complete in order, so a slice is
// overwritten only after its reads), and the waves' loads, LDS traffic and
// MFMAs overlap freely.  Slices s + 1 .. s + D are in flight in registers
// while slice s is multiplied; the loop is unrolled over the wave's MY
// slices, a compile-time count, so the compiler's waits leave those loads in
// flight.  At the end the waves' 64 x 64 partial tiles meet in LDS and are
// summed in wave order; with several K splits each workgroup writes its fp32
// partial tile and gemm_tn_reduce_kernel adds the splits in split order.
// Every summation order is fixed, so the result is deterministic.  Tiles are
// handed to the XCDs in compact blocks (workgroup b runs on XCD b % 8), so
// the tiles sharing an operand panel share an L2.
#include <algorithm>
#include <type_traits>
#include <utility>

#include "gemm.hpp"

namespace coset {
namespace {

typedef short s16x4_t __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8_gt __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef unsigned int u32x4_t __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) s16x4_t lds_s16x4_t;
typedef __attribute__((address_space(3))) char lds_char_t;

constexpr int kTnWaves = 8;     // waves per workgroup
constexpr int kTnD = 1;         // slices in flight per wave, in registers while the previous one is multiplied from LDS
constexpr int kTnSlice = 32;    // tokens per slice (one MFMA K step)
constexpr int kTnCsCols = 64;   // columns of A per column-sum workgroup

// The layout of one output tile size T (64 or 96 rows and columns per
// workgroup).  LDS row pitch of a T-wide operand slice: 2T bytes + 32, so the
// four 32-byte row pieces one 16-lane group of a transposing read touches
// (rows k..k+3: offsets 0, P, 2P, 3P mod 256 = 0, 160, 64, 224 for T = 64 and
// 0, 224, 192, 160 for T = 96) fall in distinct bank windows.
template <int T>
struct TnShape {
    static_assert(T == 64 || T == 96, "tile sizes of the kernel");
    static constexpr int kPitch = 2 * T + 32;
    static constexpr int kWaveLds = 2 * kTnSlice * kPitch;     // A and B slices of one wave
    static constexpr int kLds = kTnWaves * kWaveLds;           // 80 KiB (T = 64), 112 KiB (T = 96)
    static constexpr int kCh = T / 8;                          // 16-byte chunks per row
    static constexpr int kLoads = kTnSlice * kCh / 64;         // loads per lane, slice and operand
    static constexpr int kMt = T / 16;                         // MFMA tiles per dimension
    static constexpr int kRp = T + 4;                          // epilogue row pitch (floats)
    static constexpr int kHt = 2;                              // row tiles per epilogue pass
    static_assert(kTnWaves * 16 * kHt * kRp * 4 <= kLds, "epilogue fits the slices");
    static_assert(kMt % kHt == 0, "whole epilogue passes");
};

// f(s0 + I, integral_constant<I>) for I = 0, 1, ...: the register slot of each
// step is a compile-time index
template <class F, int... I>
__device__ __forceinline__ void unroll_steps(F& f, int s0, std::integer_sequence<int, I...>)
{
    (f(s0 + I, std::integral_constant<int, I>{}), ...);
}

__device__ __forceinline__ uint16_t f32_to_bf16_rne(float f)
{
    uint32_t u = __float_as_uint(f);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);   // NaN stays a (quiet) NaN
    u += 0x7fffu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}

// 8 consecutive outputs: fp32 (OUT 0, 2) or bf16 (OUT 1)
template <int OUT>
__device__ __forceinline__ void store8(void* C, int64_t idx, const float v[8])
{
    if (OUT == 1) {
        uint32_t h[4];
#pragma unroll
        for (int q = 0; q < 4; ++q)
            h[q] = (uint32_t)f32_to_bf16_rne(v[2 * q]) | ((uint32_t)f32_to_bf16_rne(v[2 * q + 1]) << 16);
        *reinterpret_cast<uint4*>(static_cast<uint16_t*>(C) + idx) = make_uint4(h[0], h[1], h[2], h[3]);
    } else {
        float4* dst = reinterpret_cast<float4*>(static_cast<float*>(C) + idx);
        dst[0] = make_float4(v[0], v[1], v[2], v[3]);
        dst[1] = make_float4(v[4], v[5], v[6], v[7]);
    }
}

// Column sums of one 64-column block of A (cols <= 64 of them, M being a
// multiple of 32) over one split's K range (kRows tokens from k0), for the
// workgroups past the tiles: thread t sums column
// chunk t % 8 (8 columns, one 16-byte load per token) over the tokens
// t / 8, t / 8 + 64, ... in order, 8 loads in flight; then the 64 row groups'
// sums of each column are added in group order.  Deterministic; fp32.
template <int MY>
__device__ __forceinline__ void tn_colsum_block(const uint16_t* __restrict__ A, int64_t lda, int64_t m0, int cols,
                                                int64_t k0, float* __restrict__ out, char* lds)
{
    constexpr int kRows = kTnWaves * MY * kTnSlice;
    constexpr int kIter = kRows / 64;
    const int tid = threadIdx.x, c = tid & 7, rg = tid >> 3;
    // a last block of cols < 64 columns: the chunks past it re-read chunk 0
    // (inside the matrix) and their sums are not used
    const uint16_t* p = A + (k0 + rg) * lda + m0 + (8 * c < cols ? 8 * c : 0);
    float s[8];
#pragma unroll
    for (int q = 0; q < 8; ++q) s[q] = 0.f;
#pragma unroll 8
    for (int it = 0; it < kIter; ++it) {
        const u32x4_t v = *reinterpret_cast<const u32x4_t*>(p + (int64_t)it * 64 * lda);
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            s[2 * q] += __uint_as_float(v[q] << 16);
            s[2 * q + 1] += __uint_as_float(v[q] & 0xffff0000u);
        }
    }
    float* red = reinterpret_cast<float*>(lds);   // [64 row groups][64 columns]
#pragma unroll
    for (int q = 0; q < 8; ++q) red[rg * kTnCsCols + 8 * c + q] = s[q];
    __syncthreads();
    if (tid < cols) {
        float v = red[tid];
        for (int grp = 1; grp < 64; ++grp) v += red[grp * kTnCsCols + tid];
        out[m0 + tid] = v;
    }
}

// OUT: 0 fp32 C, 1 bf16 C (one K split, C with leading dimension ldc), 2 the
// fp32 partial tile of split blockIdx.y at C + blockIdx.y * M * ldc.  MY: the
// 32-token slices of each wave (the split's K range is kTnWaves * MY * 32).
// CS: also the column sums of A, colsum[m] = sum_k A[k, m] (the bias
// gradient when A is the output gradient), by M / 64 more workgroups past the
// tiles, one per 64-column block and split (tn_colsum_block); they run beside
// the tiles on CUs the tiles leave free.  fp32 to colsum (one split) or split
// blockIdx.y's partial to colsum + blockIdx.y * M.
template <int T, int OUT, int MY, bool CS>
__global__ void __launch_bounds__(kTnWaves * 64) gemm_tn_kernel(const uint16_t* __restrict__ A, int64_t lda,
                                                                const uint16_t* __restrict__ B, int64_t ldb,
                                                                void* __restrict__ C, int64_t ldc, int64_t M,
                                                                int tiles_n, int xcd_m, int xcd_n,
                                                                float* __restrict__ colsum)
{
    using S = TnShape<T>;
    __shared__ __align__(16) char lds[S::kLds];
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int g = lane >> 4, r = lane & 15;

    if (CS && (int64_t)blockIdx.x >= (M / T) * tiles_n) {
        const int64_t cb = (int64_t)blockIdx.x - (M / T) * tiles_n;
        // past the blocks: padding that keeps the grid a multiple of 8
        if (cb * kTnCsCols < M)
            tn_colsum_block<MY>(A, lda, cb * kTnCsCols, (int)std::min<int64_t>(kTnCsCols, M - cb * kTnCsCols), (int64_t)blockIdx.y * kTnWaves * MY * kTnSlice,
                                colsum + (OUT == 2 ? (int64_t)blockIdx.y * M : 0), lds);
        return;
    }
    int tm, tn;
    if (xcd_m > 0) {
        // workgroup b runs on XCD b % 8 (tiles % 8 == 0, so every split's
        // tiles map alike): XCD x takes block x of xcd_m x xcd_n tiles (blocks
        // row-major over the tile grid), tile b / 8 of it
        const int b = blockIdx.x, x = b & 7, j = b >> 3;
        const int blocks_n = tiles_n / xcd_n;
        tm = (x / blocks_n) * xcd_m + j / xcd_n;
        tn = (x % blocks_n) * xcd_n + j % xcd_n;
    } else {
        tm = blockIdx.x / tiles_n;
        tn = blockIdx.x % tiles_n;
    }
    const int64_t m0 = (int64_t)tm * T, n0 = (int64_t)tn * T;
    // this wave's slices: k = (blockIdx.y * kTnWaves * MY + wave + i * kTnWaves) * 32, i < MY
    const int64_t k_wave = ((int64_t)blockIdx.y * kTnWaves * MY + wave) * kTnSlice;

    // a slice is 32 rows of 2T bytes per operand: chunk e = j * 64 + lane is
    // row e / (T / 8), 16-byte piece e % (T / 8)
    u32x4_t ra[kTnD][S::kLoads], rb[kTnD][S::kLoads];
    auto gload = [&](int i, u32x4_t (&xa)[S::kLoads], u32x4_t (&xb)[S::kLoads]) __attribute__((always_inline)) {
        const int ii = i < MY ? i : MY - 1;   // past the last slice: repeat it (loaded, never used)
        const int64_t k0 = k_wave + (int64_t)ii * kTnWaves * kTnSlice;
#pragma unroll
        for (int j = 0; j < S::kLoads; ++j) {
            const int e = j * 64 + lane, row = e / S::kCh, c = e % S::kCh;
            xa[j] = *reinterpret_cast<const u32x4_t*>(A + (k0 + row) * lda + m0 + 8 * c);
            xb[j] = *reinterpret_cast<const u32x4_t*>(B + (k0 + row) * ldb + n0 + 8 * c);
        }
    };
    char* wl = lds + wave * S::kWaveLds;
    auto swrite = [&](const u32x4_t (&xa)[S::kLoads], const u32x4_t (&xb)[S::kLoads]) __attribute__((always_inline)) {
#pragma unroll
        for (int j = 0; j < S::kLoads; ++j) {
            const int e = j * 64 + lane, row = e / S::kCh, c = e % S::kCh;
            *reinterpret_cast<u32x4_t*>(wl + row * S::kPitch + 16 * c) = xa[j];
            *reinterpret_cast<u32x4_t*>(wl + (kTnSlice + row) * S::kPitch + 16 * c) = xb[j];
        }
    };

    f32x4_t acc[S::kMt][S::kMt];
#pragma unroll
    for (int i = 0; i < S::kMt; ++i)
#pragma unroll
        for (int j = 0; j < S::kMt; ++j) acc[i][j] = (f32x4_t){0.f, 0.f, 0.f, 0.f};

    // two transposing reads per operand tile: rows (tokens) 8 g + r / 4 and 4
    // more, columns 16 i + 4 (r % 4)
    const lds_char_t* rbase = (const lds_char_t*)wl + (8 * g + (r >> 2)) * S::kPitch + 8 * (r & 3);
    auto compute = [&]() __attribute__((always_inline)) {
        s16x4_t a[S::kMt][2], b[S::kMt][2];
#pragma unroll
        for (int i = 0; i < S::kMt; ++i)
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                a[i][h] = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4_t*)(rbase + h * 4 * S::kPitch + 32 * i));
                b[i][h] = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                    (lds_s16x4_t*)(rbase + (kTnSlice + h * 4) * S::kPitch + 32 * i));
            }
#pragma unroll
        for (int i = 0; i < S::kMt; ++i) {
            const bf16x8_gt av =
                __builtin_bit_cast(bf16x8_gt, __builtin_shufflevector(a[i][0], a[i][1], 0, 1, 2, 3, 4, 5, 6, 7));
#pragma unroll
            for (int j = 0; j < S::kMt; ++j) {
                const bf16x8_gt bv =
                    __builtin_bit_cast(bf16x8_gt, __builtin_shufflevector(b[j][0], b[j][1], 0, 1, 2, 3, 4, 5, 6, 7));
                acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(av, bv, acc[i][j], 0, 0, 0);
            }
        }
    };

    // slice i sits in register slot i % D until the step that stages it in
    // the wave's LDS slice (whose earlier reads were issued before, and a
    // wave's LDS operations complete in order) and multiplies it; the slot is
    // refilled with slice i + D in between
#pragma unroll
    for (int d = 0; d < kTnD; ++d) gload(d, ra[d], rb[d]);
    auto step = [&](int i, auto dc) __attribute__((always_inline)) {
        constexpr int d = decltype(dc)::value;
        swrite(ra[d], rb[d]);
        gload(i + kTnD, ra[d], rb[d]);
        if (i < MY) compute();
        __builtin_amdgcn_sched_barrier(0);   // keeps each step's loads in program order
    };
#pragma unroll
    for (int i0 = 0; i0 < MY; i0 += kTnD) unroll_steps(step, i0, std::make_integer_sequence<int, kTnD>{});
    __syncthreads();

    // epilogue: the waves' tiles meet in LDS (S::kHt row tiles at a time) and
    // each output is the sum of the waves' values in wave order
    float* red = reinterpret_cast<float*>(lds);
    void* out = OUT == 2 ? static_cast<void*>(static_cast<float*>(C) + (int64_t)blockIdx.y * M * ldc) : C;
    for (int i0 = 0; i0 < S::kMt; i0 += S::kHt) {
        // D[row 4 g + e][column r] of tile (i, j) -> red[wave][16 (i - i0) + 4 g + e][16 j + r]
#pragma unroll
        for (int i = 0; i < S::kHt; ++i)
#pragma unroll
            for (int j = 0; j < S::kMt; ++j)
#pragma unroll
                for (int e = 0; e < 4; ++e)
                    red[(wave * 16 * S::kHt + 16 * i + 4 * g + e) * S::kRp + 16 * j + r] = acc[i0 + i][j][e];
        __syncthreads();
        constexpr int kChunks = 16 * S::kHt * S::kCh;   // 8 consecutive columns each
        for (int idx = tid; idx < kChunks; idx += kTnWaves * 64) {
            const int row = idx / S::kCh, c = idx % S::kCh;
            float v[8];
#pragma unroll
            for (int w = 0; w < kTnWaves; ++w) {
                const float4* src = reinterpret_cast<const float4*>(&red[(w * 16 * S::kHt + row) * S::kRp + 8 * c]);
                const float4 x0 = src[0], x1 = src[1];
                const float xv[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
#pragma unroll
                for (int q = 0; q < 8; ++q) v[q] = w == 0 ? xv[q] : v[q] + xv[q];
            }
            store8<OUT>(out, (m0 + 16 * i0 + row) * ldc + n0 + 8 * c, v);
        }
        __syncthreads();
    }
}

// C = sum over splits of the fp32 partials [splits, M, N], in split order;
// 8 consecutive outputs per thread (N % 8 == 0).  With colsum: the threads
// past C also sum the column sums' partials [splits, M] (after the tiles'
// partials in the workspace) into colsum.
template <int OUT>
__global__ void __launch_bounds__(256) gemm_tn_reduce_kernel(const float* __restrict__ part, int splits, int64_t M,
                                                             int64_t N, void* __restrict__ C, int64_t ldc,
                                                             float* __restrict__ colsum)
{
    const int64_t i = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) * 8;
    const int64_t mn = M * N;
    if (i >= mn) {
        const int64_t m = i - mn;
        if (!colsum || m >= M) return;
        const float* cp = part + splits * mn;
        for (int q = 0; q < 8; ++q) {
            float v = cp[m + q];
            for (int sp = 1; sp < splits; ++sp) v += cp[sp * M + m + q];
            colsum[m + q] = v;
        }
        return;
    }
    float v[8];
    for (int s = 0; s < splits; ++s) {
        const float4* src = reinterpret_cast<const float4*>(part + s * mn + i);
        const float4 x0 = src[0], x1 = src[1];
        const float xv[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
#pragma unroll
        for (int q = 0; q < 8; ++q) v[q] = s == 0 ? xv[q] : v[q] + xv[q];
    }
    store8<OUT>(C, (i / N) * ldc + i % N, v);
}

template <int T, int MY, bool CS>
hipError_t launch_tn(const uint16_t* A, int64_t lda, const uint16_t* B, int64_t ldb, void* C, int64_t ldc,
                     int out_bf16, int64_t M, int64_t N, const GemmTnPlan& plan, float* partial, float* colsum,
                     hipStream_t s)
{
    const int tiles_n = (int)(N / T);
    // the column-sum workgroups, padded to a multiple of 8 so that every
    // split's tiles keep their XCDs
    const int64_t cs_wg = CS ? ((M + kTnCsCols - 1) / kTnCsCols + 7) / 8 * 8 : 0;
    const dim3 grid((unsigned)((M / T) * tiles_n + cs_wg), (unsigned)plan.splits);
    const dim3 block(kTnWaves * 64);
    if (plan.splits == 1) {
        if (out_bf16)
            hipLaunchKernelGGL((gemm_tn_kernel<T, 1, MY, CS>), grid, block, 0, s, A, lda, B, ldb, C, ldc, M, tiles_n,
                               plan.xcd_m, plan.xcd_n, colsum);
        else
            hipLaunchKernelGGL((gemm_tn_kernel<T, 0, MY, CS>), grid, block, 0, s, A, lda, B, ldb, C, ldc, M, tiles_n,
                               plan.xcd_m, plan.xcd_n, colsum);
        return hipGetLastError();
    }
    // split partials: the tiles' [splits, M, N], then the column sums' [splits, M]
    hipLaunchKernelGGL((gemm_tn_kernel<T, 2, MY, CS>), grid, block, 0, s, A, lda, B, ldb, (void*)partial, N, M, tiles_n,
                       plan.xcd_m, plan.xcd_n, partial + (int64_t)plan.splits * M * N);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    const int64_t threads = (M * N + (CS ? M : 0)) / 8;
    const dim3 rgrid((unsigned)((threads + 255) / 256));
    if (out_bf16)
        hipLaunchKernelGGL((gemm_tn_reduce_kernel<1>), rgrid, dim3(256), 0, s, partial, plan.splits, M, N, C, ldc,
                           CS ? colsum : nullptr);
    else
        hipLaunchKernelGGL((gemm_tn_reduce_kernel<0>), rgrid, dim3(256), 0, s, partial, plan.splits, M, N, C, ldc,
                           CS ? colsum : nullptr);
    return hipGetLastError();
}

template <int T, int MY>
hipError_t launch_tn_cs(const uint16_t* A, int64_t lda, const uint16_t* B, int64_t ldb, void* C, int64_t ldc,
                        int out_bf16, int64_t M, int64_t N, const GemmTnPlan& plan, float* partial, float* colsum,
                        hipStream_t s)
{
    return colsum ? launch_tn<T, MY, true>(A, lda, B, ldb, C, ldc, out_bf16, M, N, plan, partial, colsum, s)
                  : launch_tn<T, MY, false>(A, lda, B, ldb, C, ldc, out_bf16, M, N, plan, partial, nullptr, s);
}

}  // namespace

namespace {

GemmTnPlan plan_for_tile(int64_t M, int64_t N, int64_t K, int T)
{
    GemmTnPlan p{0, 1, 0, 0, 0};
    if (M <= 0 || N <= 0 || K <= 0 || M % T || N % T) return p;
    // one round of workgroups (one per CU of MI355X's 256): larger grids are
    // left to the library GEMM, which covers them with larger tiles
    const int64_t tiles = (M / T) * (N / T);
    if (tiles > 256) return p;
    // K splits while the tiles leave most CUs idle; each wave then takes MY
    // slices, MY one of the compiled counts
    int splits = 1;
    while (tiles * splits * 2 <= 256) splits *= 2;
    for (; splits >= 1; splits /= 2) {
        if (K % ((int64_t)splits * kTnWaves * kTnSlice)) continue;
        const int64_t my = K / ((int64_t)splits * kTnWaves * kTnSlice);
        if (my == 4 || my == 8 || my == 16 || my == 32) {
            p.my = (int)my;
            break;
        }
    }
    if (p.my == 0) return p;
    p.tile = T;
    p.splits = splits;
    // XCD blocks: 8 blocks of tiles / 8 tiles, the most compact shape (fewest
    // operand panels per block) that tiles the grid
    const int64_t tm = M / T, tn = N / T;
    if (tiles % 8 == 0) {
        const int64_t per = tiles / 8;
        int64_t best = -1;
        for (int64_t bm = 1; bm <= per; ++bm) {
            if (per % bm || tm % bm) continue;
            const int64_t bn = per / bm;
            if (tn % bn) continue;
            if (best < 0 || bm + bn < best) {
                best = bm + bn;
                p.xcd_m = (int)bm;
                p.xcd_n = (int)bn;
            }
        }
    }
    return p;
}

}  // namespace

int g_gemm_tn_tile = 0;

GemmTnPlan gemm_tn_plan(int64_t M, int64_t N, int64_t K)
{
    // 64 x 64 tiles where they fit in one round, else 96 x 96 (products of up
    // to 256 tiles of 96, such as the 3072-wide layers' 768 x 3072 dW: 576
    // tiles of 64); g_gemm_tn_tile forces one of them
    if (g_gemm_tn_tile == 64 || g_gemm_tn_tile == 96) return plan_for_tile(M, N, K, g_gemm_tn_tile);
    const GemmTnPlan p = plan_for_tile(M, N, K, 64);
    return p.tile > 0 ? p : plan_for_tile(M, N, K, 96);
}

int64_t gemm_tn_workspace_floats(const GemmTnPlan& p, int64_t M, int64_t N)
{
    return p.tile > 0 && p.splits > 1 ? (int64_t)p.splits * (M * N + M) : 0;
}

hipError_t gemm_tn_bf16(const uint16_t* A, int64_t lda, const uint16_t* B, int64_t ldb, void* C, int64_t ldc,
                        int out_dtype, int64_t M, int64_t N, int64_t K, const GemmTnPlan& plan, float* workspace,
                        float* colsum, hipStream_t s)
{
    const int ob = out_dtype == 1;
    if ((plan.tile != 64 && plan.tile != 96) || (plan.splits > 1 && !workspace)) return hipErrorInvalidValue;
    (void)K;   // the plan's slice count fixes the K range of each launch
#define COSET_TN(TT)                                                                                        \
    switch (plan.my) {                                                                                      \
    case 4: return launch_tn_cs<TT, 4>(A, lda, B, ldb, C, ldc, ob, M, N, plan, workspace, colsum, s);      \
    case 8: return launch_tn_cs<TT, 8>(A, lda, B, ldb, C, ldc, ob, M, N, plan, workspace, colsum, s);      \
    case 16: return launch_tn_cs<TT, 16>(A, lda, B, ldb, C, ldc, ob, M, N, plan, workspace, colsum, s);    \
    case 32: return launch_tn_cs<TT, 32>(A, lda, B, ldb, C, ldc, ob, M, N, plan, workspace, colsum, s);    \
    default: return hipErrorInvalidValue;                                                                   \
    }
    if (plan.tile == 96) {
        COSET_TN(96)
    }
    COSET_TN(64)
#undef COSET_TN
}

}  // namespace coset
