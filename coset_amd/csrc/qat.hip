// qat.hip -- backward of the QAT weight quantizer (straight-through estimator).
//
// Forward (coset/core/layers.py:428-463):
//   W_q = clamp(Q / beta, -clip, clip),   Q = STE(dec(enc(W * beta)))
// Autograd of that chain, given g = dL/dW_q (layers.py:62-95 for the STE):
//   m      = (-clip <= Q/beta <= clip)        clamp backward
//   gq     = (g * m) / beta                    div backward, to Q
//   dW     = gq * beta                         STE identity, then mul backward
//   dbeta  = sum_tile( gq * W ) + sum_tile( -(g*m) * ((Q/beta)/beta) )
// The forward kernel (hnlq_codec / hnlq_lut, SCALE_LAYER) saves the packed
// level words; here Q is re-decoded from them (for q = 2, 4, 8, 16 through a
// per-coordinate table in LDS, projections otherwise), so the backward reads
// g, W and 0.5 B/weight of codes and makes no dependent global loads.
//
// One workgroup per tile (row tiling: a tile is an output row of
// blocks_per_tile 8-wide blocks) reduces dbeta with a wave reduction and one
// LDS pass; block tiling (one block per tile) needs no reduction.
#include <hip/hip_fp16.h>

#include "codec_kernels.hpp"
#include "tables.hpp"

namespace coset {

struct QatBwdArgs {
    const void* g;         // [rows, cols] fp32 or bf16
    int g_dtype;
    const float* W;        // [rows, cols]
    const void* packed;    // [n_blocks, M] level words
    const float* beta;     // [n_tiles]
    int64_t n_blocks;
    int64_t blocks_per_tile;
    float clip;
    int q, M, strided;
    float* dW;             // [rows, cols]
    float* dbeta;          // [n_tiles]
    const float* dbdt;     // [n_tiles] d beta / d theta, or null
    float* dtheta;         // [n_tiles] when dbdt is given
};

// dL/dtheta = dL/dbeta * (beta_max - beta_min) s (1 - s), s = sigmoid(theta);
// the factor was recorded by the forward kernel.
__device__ __forceinline__ void write_dtheta(const QatBwdArgs& a, int64_t t, float dbeta)
{
    if (a.dbdt) a.dtheta[t] = __fmul_rn(dbeta, a.dbdt[t]);
}

// q = 2, 4, 8, 16: each workgroup's table of dyadic_table_entry, one entry
// per Z + 2q (built at the kernel's start), else unused
template <int Q>
struct BwdTab {
    static constexpr bool kOn = Q == 2 || Q == 4 || Q == 8 || Q == 16;
    static constexpr int kEntries = kOn ? 7 * Q : 1;
};

template <int Q>
__device__ __forceinline__ void build_bwd_tab(uint4* tab)
{
    if constexpr (BwdTab<Q>::kOn) {
        if (threadIdx.x < 7 * Q) tab[threadIdx.x] = dyadic_table_entry<Q>((int)threadIdx.x - 2 * Q);
        __syncthreads();
    }
}

// Unscaled quantized block Q = sum_m q^m r_m from packed words.
template <int Q>
__device__ __forceinline__ void decode_q(const QatBwdArgs& a, int64_t blk, const uint4* tab, float out[8])
{
    const int q = Q > 0 ? Q : a.q;
    const float qf = (float)q;
    if constexpr (Q == 2 || Q == 4) {
        // 2 Q = sum_m q^m (2 r_m) in integers: dyadic_level_acc adds
        // q^m (2 r_m + q); q sum_m q^m comes off at the end
        constexpr int kLog2Q = Q == 2 ? 1 : 2;
        int acc2[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) acc2[j] = 0;
        int off = 0;
        for (int m = 0; m < a.M; ++m) {
            const uint32_t w = reinterpret_cast<const uint16_t*>(a.packed)[blk * a.M + m] & (Q == 2 ? 0xffu : 0xffffu);
            int b[8];
            unpack_word<Q>(w, q, b);
            dyadic_level_acc<Q, false>(b, tab, m * kLog2Q, acc2);
            off += Q << (m * kLog2Q);
        }
#pragma unroll
        for (int j = 0; j < 8; ++j) out[j] = __fmul_rn((float)(acc2[j] - off), 0.5f);
    } else {
        float acc[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) acc[j] = 0.f;
        float wf = 1.f;
        for (int m = 0; m < a.M; ++m) {
            uint32_t w = word_bytes(q) == 2 ? reinterpret_cast<const uint16_t*>(a.packed)[blk * a.M + m]
                                            : reinterpret_cast<const uint32_t*>(a.packed)[blk * a.M + m];
            int b[8];
            float r[8];
            unpack_word<Q>(w, q, b);
            if constexpr (BwdTab<Q>::kOn)  // both rules agree on the dyadic grid
                residual_table<Q>(b, tab, r);
            else if (!a.strided)
                level_residual<false, Q>(b, qf, r);
            else
                level_residual<true, Q>(b, qf, r);
            add_level<Q>(acc, wf, r);
            wf = __fmul_rn(wf, qf);
        }
#pragma unroll
        for (int j = 0; j < 8; ++j) out[j] = acc[j];
    }
}

// Gradients of one block; returns its dbeta contribution.
template <int Q>
__device__ __forceinline__ float block_grad(const QatBwdArgs& a, int64_t blk, float beta, const uint4* tab)
{
    float Qv[8], g[8], w[8];
    decode_q<Q>(a, blk, tab, Qv);
    if (a.g_dtype == DT_BF16) {
        uint4 v = reinterpret_cast<const uint4*>(a.g)[blk];
        uint32_t u[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            g[2 * j] = __uint_as_float(u[j] << 16);
            g[2 * j + 1] = __uint_as_float(u[j] & 0xffff0000u);
        }
    } else {
        const float4* p = reinterpret_cast<const float4*>(a.g) + 2 * blk;
        float4 u = p[0], v = p[1];
        g[0] = u.x; g[1] = u.y; g[2] = u.z; g[3] = u.w;
        g[4] = v.x; g[5] = v.y; g[6] = v.z; g[7] = v.w;
    }
    {
        const float4* p = reinterpret_cast<const float4*>(a.W) + 2 * blk;
        float4 u = p[0], v = p[1];
        w[0] = u.x; w[1] = u.y; w[2] = u.z; w[3] = u.w;
        w[4] = v.x; w[5] = v.y; w[6] = v.z; w[7] = v.w;
    }
    float d_mul = 0.f, d_div = 0.f;
    float dw[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        float wq = __fdiv_rn(Qv[j], beta);
        float gm = (wq >= -a.clip && wq <= a.clip) ? g[j] : 0.f;
        float gq = __fdiv_rn(gm, beta);
        dw[j] = __fmul_rn(gq, beta);
        d_mul = __fmaf_rn(gq, w[j], d_mul);
        d_div = __fmaf_rn(-gm, __fdiv_rn(wq, beta), d_div);
    }
    float4* o = reinterpret_cast<float4*>(a.dW) + 2 * blk;
    o[0] = make_float4(dw[0], dw[1], dw[2], dw[3]);
    o[1] = make_float4(dw[4], dw[5], dw[6], dw[7]);
    return d_mul + d_div;
}

template <int Q>
__global__ void __launch_bounds__(256) qat_bwd_tile_kernel(QatBwdArgs a)
{
    __shared__ uint4 s_tab[BwdTab<Q>::kEntries];
    build_bwd_tab<Q>(s_tab);
    const int64_t tile = blockIdx.x;
    const float beta = a.beta[tile];
    const int64_t b0 = tile * a.blocks_per_tile;
    float part = 0.f;
    for (int64_t k = threadIdx.x; k < a.blocks_per_tile; k += blockDim.x)
        part += block_grad<Q>(a, b0 + k, beta, s_tab);
    // wave reduction, then across the 4 waves
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) part += __shfl_down(part, off, 64);
    __shared__ float s_part[4];
    if ((threadIdx.x & 63) == 0) s_part[threadIdx.x >> 6] = part;
    __syncthreads();
    if (threadIdx.x == 0) {
        float db = (s_part[0] + s_part[1]) + (s_part[2] + s_part[3]);
        a.dbeta[tile] = db;
        write_dtheta(a, tile, db);
    }
}

template <int Q>
__global__ void __launch_bounds__(256) qat_bwd_block_kernel(QatBwdArgs a)
{
    __shared__ uint4 s_tab[BwdTab<Q>::kEntries];
    build_bwd_tab<Q>(s_tab);
    int64_t blk = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (blk >= a.n_blocks) return;
    float db = block_grad<Q>(a, blk, a.beta[blk], s_tab);
    a.dbeta[blk] = db;
    write_dtheta(a, blk, db);
}

template <int Q>
static hipError_t launch_bwd_q(const QatBwdArgs& a, hipStream_t s)
{
    if (a.blocks_per_tile == 1) {
        hipLaunchKernelGGL(qat_bwd_block_kernel<Q>, dim3((unsigned)((a.n_blocks + 255) / 256)), dim3(256), 0, s, a);
    } else {
        int64_t tiles = a.n_blocks / a.blocks_per_tile;
        hipLaunchKernelGGL(qat_bwd_tile_kernel<Q>, dim3((unsigned)tiles), dim3(256), 0, s, a);
    }
    return hipGetLastError();
}

// ---------------------------------------------------------------------------
// Statistics update (HNLQLinearQAT._gather_stats, coset/core/layers.py:366-379)
// over tiles of n contiguous weights (row tiling: a row; block tiling: one
// 8-wide block):
//   sigma = std(tile) + 1e-8,  xmax = max |tile| + 1e-8
//   sigma_ema = sigma_ema * m + (1 - m) * sigma   (and xmax_ema likewise)
// The standard deviation follows the reference's CPU arithmetic: the
// unbiased variance accumulated in double, its double square root rounded
// once to fp32; the rest are single fp32 operations in the reference's order
// with the scalars rounded to fp32.  Two passes in double (mean, then the
// squared deviations) keep the variance exact to ~1e-16 relative, so the
// fp32 result matches a double-accumulating reduction in any order.
struct StatsArgs {
    const float* W;
    int64_t tiles, n;           // tiles of n weights
    float m, one_minus_m, eps;  // fp32 roundings of m, 1 - m, 1e-8
    float* sigma_ema;
    float* xmax_ema;
};

__device__ __forceinline__ void stats_write(const StatsArgs& a, int64_t t, double m2, float amax)
{
    float sd = (float)sqrt(m2 / (double)(a.n - 1));
    float s1 = __fadd_rn(sd, a.eps);
    float x1 = __fadd_rn(amax, a.eps);
    a.sigma_ema[t] = __fadd_rn(__fmul_rn(a.sigma_ema[t], a.m), __fmul_rn(a.one_minus_m, s1));
    a.xmax_ema[t] = __fadd_rn(__fmul_rn(a.xmax_ema[t], a.m), __fmul_rn(a.one_minus_m, x1));
}

// max(a, b) that returns a NaN operand (the reference's Tensor.amax
// propagates NaN; fmaxf would drop it)
__device__ __forceinline__ float max_nan(float a, float b)
{
    return (b > a || b != b) ? b : a;
}

// one workgroup (256 threads) per tile
__global__ void __launch_bounds__(256) qat_stats_tile_kernel(StatsArgs a)
{
    const int64_t t = blockIdx.x;
    const float* w = a.W + t * a.n;
    __shared__ double s_d[4];
    __shared__ float s_f[4];
    double sum = 0.0;
    float amax = 0.f;
    for (int64_t i = threadIdx.x; i < a.n; i += blockDim.x) {
        float v = w[i];
        sum += (double)v;
        amax = max_nan(amax, fabsf(v));
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
        sum += __shfl_down(sum, off, 64);
        amax = max_nan(amax, __shfl_down(amax, off, 64));
    }
    if ((threadIdx.x & 63) == 0) {
        s_d[threadIdx.x >> 6] = sum;
        s_f[threadIdx.x >> 6] = amax;
    }
    __syncthreads();
    const double mean = ((s_d[0] + s_d[1]) + (s_d[2] + s_d[3])) / (double)a.n;
    amax = max_nan(max_nan(s_f[0], s_f[1]), max_nan(s_f[2], s_f[3]));
    __syncthreads();
    double m2 = 0.0;
    for (int64_t i = threadIdx.x; i < a.n; i += blockDim.x) {
        double d = (double)w[i] - mean;
        m2 += d * d;
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) m2 += __shfl_down(m2, off, 64);
    if ((threadIdx.x & 63) == 0) s_d[threadIdx.x >> 6] = m2;
    __syncthreads();
    if (threadIdx.x == 0) stats_write(a, t, (s_d[0] + s_d[1]) + (s_d[2] + s_d[3]), amax);
}

// one thread per 8-wide tile (block tiling)
__global__ void __launch_bounds__(256) qat_stats_block_kernel(StatsArgs a)
{
    const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (t >= a.tiles) return;
    const float4* p = reinterpret_cast<const float4*>(a.W + t * 8);
    float4 u = p[0], v = p[1];
    float x[8] = {u.x, u.y, u.z, u.w, v.x, v.y, v.z, v.w};
    double sum = 0.0;
    float amax = 0.f;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        sum += (double)x[j];
        amax = max_nan(amax, fabsf(x[j]));
    }
    const double mean = sum / 8.0;
    double m2 = 0.0;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        double d = (double)x[j] - mean;
        m2 += d * d;
    }
    stats_write(a, t, m2, amax);
}

// ---------------------------------------------------------------------------
// Bias gradient of the layer's product y = x W_q^T + b (coset/core/layers.py:
// 478): db[c] = sum_t g[t, c] over the tokens, accumulated in fp32 in a fixed
// order whatever g's dtype (fp32, bf16 or fp16).  Stage 1: workgroups of 256
// threads = 64 column threads (8 consecutive columns each: one 16-byte bf16
// load or two fp32 loads) x 4 row threads, over a chunk of kColsumChunk rows,
// write one fp32 partial per (chunk, column); stage 2 adds the chunks'
// partials of a column in order.  Deterministic: no atomics.
constexpr int kColsumChunk = 64;

template <int DT>
__device__ __forceinline__ void load8(const void* g, int64_t idx, float v[8])
{
    if (DT == DT_F32) {
        const float4* p = reinterpret_cast<const float4*>(reinterpret_cast<const float*>(g) + idx);
        float4 a = p[0], b = p[1];
        v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w; v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
    } else {
        uint4 u = *reinterpret_cast<const uint4*>(reinterpret_cast<const uint16_t*>(g) + idx);
        uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            if (DT == DT_BF16) {
                v[2 * j] = __uint_as_float(w[j] << 16);
                v[2 * j + 1] = __uint_as_float(w[j] & 0xffff0000u);
            } else {
                v[2 * j] = __half2float(__ushort_as_half((unsigned short)(w[j] & 0xffffu)));
                v[2 * j + 1] = __half2float(__ushort_as_half((unsigned short)(w[j] >> 16)));
            }
        }
    }
}

template <int DT>
__global__ void __launch_bounds__(256) colsum_partial_kernel(const void* g, int64_t rows, int64_t cols,
                                                             float* partial)
{
    const int64_t c8 = (int64_t)blockIdx.x * 64 + (threadIdx.x & 63);
    const int rt = threadIdx.x >> 6;
    const int64_t r0 = (int64_t)blockIdx.y * kColsumChunk;
    const int64_t r1 = r0 + kColsumChunk < rows ? r0 + kColsumChunk : rows;
    float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    const bool live = 8 * c8 < cols;
    if (live) {
        for (int64_t r = r0 + rt; r < r1; r += 4) {
            float v[8];
            load8<DT>(g, r * cols + 8 * c8, v);
#pragma unroll
            for (int j = 0; j < 8; ++j) acc[j] = __fadd_rn(acc[j], v[j]);
        }
    }
    __shared__ float s[3][64][9];
    if (rt > 0) {
#pragma unroll
        for (int j = 0; j < 8; ++j) s[rt - 1][threadIdx.x & 63][j] = acc[j];
    }
    __syncthreads();
    if (rt == 0 && live) {
        float* out = partial + (int64_t)blockIdx.y * cols + 8 * c8;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const int l = threadIdx.x & 63;
            out[j] = __fadd_rn(__fadd_rn(acc[j], s[0][l][j]), __fadd_rn(s[1][l][j], s[2][l][j]));
        }
    }
}

// Stage 2: 64 columns per workgroup, the chunks split over 4 thread rows
// (each sums its run of chunks with its loads in flight together), the 4
// runs then added in order.
__global__ void __launch_bounds__(256) colsum_final_kernel(const float* partial, int64_t chunks, int64_t cols,
                                                           float* out)
{
    const int64_t c = (int64_t)blockIdx.x * 64 + (threadIdx.x & 63);
    const int part = threadIdx.x >> 6;
    const int64_t per = (chunks + 3) / 4;
    const int64_t k0 = part * per, k1 = k0 + per < chunks ? k0 + per : chunks;
    float s = 0.f;
    if (c < cols) {
        int64_t k = k0;
        for (; k + 4 <= k1; k += 4) {
            const float v0 = partial[k * cols + c], v1 = partial[(k + 1) * cols + c];
            const float v2 = partial[(k + 2) * cols + c], v3 = partial[(k + 3) * cols + c];
            s = __fadd_rn(__fadd_rn(__fadd_rn(__fadd_rn(s, v0), v1), v2), v3);
        }
        for (; k < k1; ++k) s = __fadd_rn(s, partial[k * cols + c]);
    }
    __shared__ float s_part[3][64];
    if (part > 0) s_part[part - 1][threadIdx.x & 63] = s;
    __syncthreads();
    if (part == 0 && c < cols) {
        const int l = threadIdx.x & 63;
        out[c] = __fadd_rn(__fadd_rn(__fadd_rn(s, s_part[0][l]), s_part[1][l]), s_part[2][l]);
    }
}

int64_t colsum_workspace_floats(int64_t rows, int64_t cols)
{
    return ((rows + kColsumChunk - 1) / kColsumChunk) * cols;
}

hipError_t launch_colsum(const void* g, int dtype, int64_t rows, int64_t cols, float* out, float* workspace,
                         hipStream_t s)
{
    if (cols == 0) return hipSuccess;
    if (rows == 0) {
        hipLaunchKernelGGL(colsum_final_kernel, dim3((unsigned)((cols + 63) / 64)), dim3(256), 0, s,
                           (const float*)workspace, (int64_t)0, cols, out);
        return hipGetLastError();
    }
    const int64_t chunks = (rows + kColsumChunk - 1) / kColsumChunk;
    dim3 grid((unsigned)((cols / 8 + 63) / 64), (unsigned)chunks);
    if (dtype == DT_F32)
        hipLaunchKernelGGL(colsum_partial_kernel<DT_F32>, grid, dim3(256), 0, s, g, rows, cols, workspace);
    else if (dtype == DT_BF16)
        hipLaunchKernelGGL(colsum_partial_kernel<DT_BF16>, grid, dim3(256), 0, s, g, rows, cols, workspace);
    else
        hipLaunchKernelGGL(colsum_partial_kernel<DT_F16>, grid, dim3(256), 0, s, g, rows, cols, workspace);
    hipLaunchKernelGGL(colsum_final_kernel, dim3((unsigned)((cols + 63) / 64)), dim3(256), 0, s,
                       (const float*)workspace, chunks, cols, out);
    return hipGetLastError();
}

hipError_t launch_qat_stats(const float* W, int64_t tiles, int64_t n, double momentum, float* sigma_ema,
                            float* xmax_ema, hipStream_t s)
{
    if (tiles == 0) return hipSuccess;
    StatsArgs a{};
    a.W = W;
    a.tiles = tiles;
    a.n = n;
    a.m = (float)momentum;
    a.one_minus_m = (float)(1.0 - momentum);
    a.eps = 1e-8f;
    a.sigma_ema = sigma_ema;
    a.xmax_ema = xmax_ema;
    if (n == 8)
        hipLaunchKernelGGL(qat_stats_block_kernel, dim3((unsigned)((tiles + 255) / 256)), dim3(256), 0, s, a);
    else
        hipLaunchKernelGGL(qat_stats_tile_kernel, dim3((unsigned)tiles), dim3(256), 0, s, a);
    return hipGetLastError();
}

hipError_t launch_qat_bwd(const void* g, int g_dtype, const float* W, const void* packed,
                          const float* beta, int64_t n_blocks, int64_t blocks_per_tile, float clip,
                          int q, int M, float* dW, float* dbeta, const float* dbdt, float* dtheta,
                          hipStream_t s)
{
    if (n_blocks == 0) return hipSuccess;
    QatBwdArgs a{};
    a.dbdt = dbdt;
    a.dtheta = dtheta;
    a.g = g;
    a.g_dtype = g_dtype;
    a.W = W;
    a.packed = packed;
    a.beta = beta;
    a.n_blocks = n_blocks;
    a.blocks_per_tile = blocks_per_tile;
    a.clip = clip;
    a.q = q;
    a.M = M;
    a.strided = n_blocks > 1;
    a.dW = dW;
    a.dbeta = dbeta;
    switch (q) {
    case 2: return launch_bwd_q<2>(a, s);
    case 4: return launch_bwd_q<4>(a, s);
    case 8: return launch_bwd_q<8>(a, s);
    case 16: return launch_bwd_q<16>(a, s);
    default: return launch_bwd_q<0>(a, s);
    }
}

}  // namespace coset
