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
// level words; here Q is re-decoded from them (tables for q = 2, 4,
// projections otherwise), so the backward reads g, W and 0.5 B/weight of codes.
//
// One workgroup per tile (row tiling: a tile is an output row of
// blocks_per_tile 8-wide blocks) reduces dbeta with a wave reduction and one
// LDS pass; block tiling (one block per tile) needs no reduction.
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
    const uint16_t* map;   // decode tables (q = 2, 4) or null
    const uint64_t* coarse;
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

// Unscaled quantized block Q = sum_m q^m r_m from packed words.
template <int Q>
__device__ __forceinline__ void decode_q(const QatBwdArgs& a, int64_t blk, float out[8])
{
    const int q = Q > 0 ? Q : a.q;
    const float qf = (float)q;
    if (Q == 2 || Q == 4) {
        int acc2[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) acc2[j] = 0;
        int wq = 1;
        for (int m = 0; m < a.M; ++m) {
            uint32_t w = reinterpret_cast<const uint16_t*>(a.packed)[blk * a.M + m] & (Q == 2 ? 0xffu : 0xffffu);
            int b[8];
            unpack_word<Q>(w, q, b);
            int u[8];
            u[0] = 4 * b[0] - 2 * b[1] + b[7];
#pragma unroll
            for (int j = 1; j < 6; ++j) u[j] = 2 * (b[j] - b[j + 1]) + b[7];
            u[6] = 2 * b[6] + b[7];
            u[7] = b[7];
            uint64_t c = a.coarse[a.map[w]];
#pragma unroll
            for (int j = 0; j < 8; ++j) acc2[j] += wq * (u[j] - Q * (int)(int8_t)(uint8_t)(c >> (8 * j)));
            wq *= Q;
        }
#pragma unroll
        for (int j = 0; j < 8; ++j) out[j] = __fmul_rn((float)acc2[j], 0.5f);
    } else {
        float acc[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) acc[j] = 0.f;
        float wf = 1.f;
        for (int m = 0; m < a.M; ++m) {
            uint32_t w = word_bytes(q) == 2 ? reinterpret_cast<const uint16_t*>(a.packed)[blk * a.M + m]
                                            : reinterpret_cast<const uint32_t*>(a.packed)[blk * a.M + m];
            int b[8];
            float gb[8], r[8];
            unpack_word<Q>(w, q, b);
            lattice_point(b, gb);
            if (a.strided)
                residual_from_point<false, true, Q>(gb, qf, r);
            else
                residual_from_point<false, false, Q>(gb, qf, r);
#pragma unroll
            for (int j = 0; j < 8; ++j) acc[j] = __fadd_rn(acc[j], __fmul_rn(wf, r[j]));
            wf = __fmul_rn(wf, qf);
        }
#pragma unroll
        for (int j = 0; j < 8; ++j) out[j] = acc[j];
    }
}

// Gradients of one block; returns its dbeta contribution.
template <int Q>
__device__ __forceinline__ float block_grad(const QatBwdArgs& a, int64_t blk, float beta)
{
    float Qv[8], g[8], w[8];
    decode_q<Q>(a, blk, Qv);
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
    const int64_t tile = blockIdx.x;
    const float beta = a.beta[tile];
    const int64_t b0 = tile * a.blocks_per_tile;
    float part = 0.f;
    for (int64_t k = threadIdx.x; k < a.blocks_per_tile; k += blockDim.x) part += block_grad<Q>(a, b0 + k, beta);
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
    int64_t blk = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (blk >= a.n_blocks) return;
    float db = block_grad<Q>(a, blk, a.beta[blk]);
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
    if (q == 2 || q == 4) {
        const DecodeTables* t = nullptr;
        hipError_t e = get_decode_tables(q, 0, &t);
        if (e != hipSuccess) return e;
        a.map = t->cid_map;
        a.coarse = t->coarse;
        return q == 4 ? launch_bwd_q<4>(a, s) : launch_bwd_q<2>(a, s);
    }
    switch (q) {
    case 8: return launch_bwd_q<8>(a, s);
    case 16: return launch_bwd_q<16>(a, s);
    default: return launch_bwd_q<0>(a, s);
    }
}

}  // namespace coset
