// d4.hip -- the D4 variant: lattice operators and the fused QAT weight
// quantizer of the D4 layer.
//
// D4 (coset/core/d4/lattice.py:14-146): G has the columns (-1,-1,0,0),
// (1,-1,0,0), (0,1,-1,0), (0,0,1,-1); its fp32 inverse is exact (entries
// +-1/2, +-1).  Closest point: f = custom_round(x), kept when sum(f) is even,
// else g_x(x), which moves the first worst coordinate by +1 when x_k >= 0
// and f_k < x_k and by -1 otherwise (the same rule as the core E8 g_x):
// dn_candidate<4> of e8_core.hpp.
//
// The D4 layer (create_d4_hnlq_linear, coset/core/d4/layers.py:14-68)
// quantizes 4-wide blocks by the projection alone (d4_quantize ignores q):
//   W_q = clamp(P(W * beta_t) / beta_t, -clip, clip)
// with beta_t given or derived from theta as in the E8 layer
// (coset/core/layers.py:381-396, 418-463).  The backward recomputes P(W beta)
// (a few operations per block, cheaper than storing it) and applies the
// straight-through estimator's autograd:
//   m = (-clip <= P/beta <= clip),  dW = ((g m) / beta) beta,
//   dbeta_t = sum_t ((g m) / beta) W - (g m) ((P / beta) / beta).
#include "codec_kernels.hpp"

namespace coset {

namespace {

constexpr float kD4Ginv[4][4] = {{-0.5f, -0.5f, -0.5f, -0.5f},
                                 {0.5f, -0.5f, -0.5f, -0.5f},
                                 {-0.f, -0.f, -1.f, -1.f},
                                 {-0.f, -0.f, -0.f, -1.f}};

__device__ __forceinline__ void d4_project(const float x[4], float y[4]) { dn_candidate<4, false>(x, y); }

__device__ __forceinline__ float4 ld4(const float* p, int64_t i) { return reinterpret_cast<const float4*>(p)[i]; }

__device__ __forceinline__ void st4(float* p, int64_t i, const float v[4])
{
    reinterpret_cast<float4*>(p)[i] = make_float4(v[0], v[1], v[2], v[3]);
}

// round(G^-1 x) mod q (coset/core/base.py:134-154): the products with the
// exact inverse in fp32, summed in column order, torch.round (half to even)
// and torch.remainder's sign rule.
__device__ __forceinline__ void d4_encode_coords(const float x[4], int q, float b[4])
{
    const float qf = (float)q;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        float c = __fmul_rn(kD4Ginv[i][0], x[0]);
#pragma unroll
        for (int j = 1; j < 4; ++j) c = __fadd_rn(c, __fmul_rn(kD4Ginv[i][j], x[j]));
        float m = fmodf(rintf(c), qf);
        if (m != 0.f && m < 0.f) m = __fadd_rn(m, qf);
        b[i] = m;
    }
}

// G b (coset/core/base.py:156-176): y0 = -b0 + b1, y1 = -b0 - b1 + b2,
// y2 = -b2 + b3, y3 = -b3, in fp32.
__device__ __forceinline__ void d4_decode_coords(const float b[4], float y[4])
{
    y[0] = __fadd_rn(-b[0], b[1]);
    y[1] = __fadd_rn(__fsub_rn(-b[0], b[1]), b[2]);
    y[2] = __fadd_rn(-b[2], b[3]);
    y[3] = -b[3];
}

// One kernel per operator.  (Built as one run-time switch over the four
// bodies, the decode arm came out of hipcc without its y[3] computation.)
template <int OP>
__global__ void __launch_bounds__(256) d4_lattice_op_kernel(const float* in, int64_t n, int q, float* out)
{
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    const float4 v = ld4(in, i);
    const float x[4] = {v.x, v.y, v.z, v.w};
    float y[4];
    if constexpr (OP == OP_G_X)
        dn_candidate<4, false, true>(x, y);
    else if constexpr (OP == OP_PROJECT)
        d4_project(x, y);
    else if constexpr (OP == OP_ENCODE_COORDS)
        d4_encode_coords(x, q, y);
    else
        d4_decode_coords(x, y);
    st4(out, i, y);
}

struct D4QatArgs {
    const float* W;       // [n_blocks, 4]
    int64_t n_blocks, blocks_per_tile;
    float clip;
    const float* beta;    // [tiles], or null with use_theta
    int use_theta;
    ThetaBeta tb;
    float* beta_out;      // nullable [tiles]
    float* dbdt_out;      // nullable [tiles]
    int64_t* step_counter;
    void* Wq;             // [n_blocks, 4] fp32 or bf16
    int wq_dtype;
    // backward
    const void* g;        // [n_blocks, 4] fp32 or bf16
    int g_dtype;
    const float* dbdt;    // nullable [tiles]
    float* dW;
    float* dbeta;
    float* dtheta;
};

__device__ __forceinline__ float tile_beta(const D4QatArgs& a, int64_t blk)
{
    const int64_t t = blk / a.blocks_per_tile;
    if (!a.use_theta) return a.beta[t];
    float lo, hi, sg;
    theta_beta_terms(a.tb, t, &lo, &hi, &sg);
    const float span = __fsub_rn(hi, lo);
    const float b = __fadd_rn(lo, __fmul_rn(sg, span));
    if (blk == t * a.blocks_per_tile) {  // one thread per tile records beta and its derivative
        if (a.beta_out) a.beta_out[t] = b;
        if (a.dbdt_out) a.dbdt_out[t] = __fmul_rn(__fmul_rn(span, __fsub_rn(1.f, sg)), sg);
    }
    return b;
}

__device__ __forceinline__ float clamp_clip(float v, float clip)
{
    return v != v ? v : fminf(fmaxf(v, -clip), clip);
}

__global__ void __launch_bounds__(256) d4_qat_fwd_kernel(D4QatArgs a)
{
    const int64_t blk = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (blk == 0 && a.step_counter) *a.step_counter += 1;
    if (blk >= a.n_blocks) return;
    const float beta = tile_beta(a, blk);
    const float4 v = ld4(a.W, blk);
    const float x[4] = {__fmul_rn(v.x, beta), __fmul_rn(v.y, beta), __fmul_rn(v.z, beta), __fmul_rn(v.w, beta)};
    float p[4], wq[4];
    d4_project(x, p);
#pragma unroll
    for (int j = 0; j < 4; ++j) wq[j] = clamp_clip(__fdiv_rn(p[j], beta), a.clip);
    if (a.wq_dtype == DT_BF16) {
        uint2 o;
        o.x = f32_to_bf16(wq[0]) | ((uint32_t)f32_to_bf16(wq[1]) << 16);
        o.y = f32_to_bf16(wq[2]) | ((uint32_t)f32_to_bf16(wq[3]) << 16);
        reinterpret_cast<uint2*>(a.Wq)[blk] = o;
    } else {
        st4(reinterpret_cast<float*>(a.Wq), blk, wq);
    }
}

// Gradients of one block; returns its dbeta contribution.
__device__ __forceinline__ float d4_block_grad(const D4QatArgs& a, int64_t blk, float beta)
{
    const float4 v = ld4(a.W, blk);
    const float w[4] = {v.x, v.y, v.z, v.w};
    float g[4];
    if (a.g_dtype == DT_BF16) {
        const uint2 u = reinterpret_cast<const uint2*>(a.g)[blk];
        g[0] = __uint_as_float(u.x << 16);
        g[1] = __uint_as_float(u.x & 0xffff0000u);
        g[2] = __uint_as_float(u.y << 16);
        g[3] = __uint_as_float(u.y & 0xffff0000u);
    } else {
        const float4 u = ld4(reinterpret_cast<const float*>(a.g), blk);
        g[0] = u.x; g[1] = u.y; g[2] = u.z; g[3] = u.w;
    }
    float x[4], p[4], dw[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) x[j] = __fmul_rn(w[j], beta);
    d4_project(x, p);
    float d_mul = 0.f, d_div = 0.f;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const float wq = __fdiv_rn(p[j], beta);
        const float gm = (wq >= -a.clip && wq <= a.clip) ? g[j] : 0.f;
        const float gq = __fdiv_rn(gm, beta);
        dw[j] = __fmul_rn(gq, beta);
        d_mul = __fmaf_rn(gq, w[j], d_mul);
        d_div = __fmaf_rn(-gm, __fdiv_rn(wq, beta), d_div);
    }
    st4(a.dW, blk, dw);
    return d_mul + d_div;
}

__device__ __forceinline__ void write_dbeta(const D4QatArgs& a, int64_t t, float db)
{
    a.dbeta[t] = db;
    if (a.dbdt) a.dtheta[t] = __fmul_rn(db, a.dbdt[t]);
}

__global__ void __launch_bounds__(256) d4_qat_bwd_tile_kernel(D4QatArgs a)
{
    const int64_t tile = blockIdx.x;
    const float beta = a.beta[tile];
    const int64_t b0 = tile * a.blocks_per_tile;
    float part = 0.f;
    for (int64_t k = threadIdx.x; k < a.blocks_per_tile; k += blockDim.x) part += d4_block_grad(a, b0 + k, beta);
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) part += __shfl_down(part, off, 64);
    __shared__ float s_part[4];
    if ((threadIdx.x & 63) == 0) s_part[threadIdx.x >> 6] = part;
    __syncthreads();
    if (threadIdx.x == 0) write_dbeta(a, tile, (s_part[0] + s_part[1]) + (s_part[2] + s_part[3]));
}

__global__ void __launch_bounds__(256) d4_qat_bwd_block_kernel(D4QatArgs a)
{
    const int64_t blk = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (blk >= a.n_blocks) return;
    write_dbeta(a, blk, d4_block_grad(a, blk, a.beta[blk]));
}

}  // namespace

hipError_t launch_d4_lattice_op(int op, const float* in, int64_t n, int q, float* out, hipStream_t s)
{
    if (n == 0) return hipSuccess;
    const dim3 grid((unsigned)((n + 255) / 256)), block(256);
    switch (op) {
    case OP_G_X: hipLaunchKernelGGL(d4_lattice_op_kernel<OP_G_X>, grid, block, 0, s, in, n, q, out); break;
    case OP_PROJECT: hipLaunchKernelGGL(d4_lattice_op_kernel<OP_PROJECT>, grid, block, 0, s, in, n, q, out); break;
    case OP_ENCODE_COORDS:
        hipLaunchKernelGGL(d4_lattice_op_kernel<OP_ENCODE_COORDS>, grid, block, 0, s, in, n, q, out);
        break;
    case OP_DECODE_COORDS:
        hipLaunchKernelGGL(d4_lattice_op_kernel<OP_DECODE_COORDS>, grid, block, 0, s, in, n, q, out);
        break;
    default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

hipError_t launch_d4_qat_fwd(const float* W, int64_t n_blocks, int64_t blocks_per_tile, const float* beta,
                             const ThetaBeta* tb, float clip, void* Wq, int wq_dtype, float* beta_out,
                             float* dbdt_out, int64_t* step_counter, hipStream_t s)
{
    D4QatArgs a{};
    a.W = W;
    a.n_blocks = n_blocks;
    a.blocks_per_tile = blocks_per_tile;
    a.clip = clip;
    a.beta = beta;
    a.use_theta = tb != nullptr;
    if (tb) a.tb = *tb;
    a.beta_out = beta_out;
    a.dbdt_out = dbdt_out;
    a.step_counter = step_counter;
    a.Wq = Wq;
    a.wq_dtype = wq_dtype;
    const int64_t grid = (n_blocks + 255) / 256;
    hipLaunchKernelGGL(d4_qat_fwd_kernel, dim3((unsigned)(grid > 0 ? grid : 1)), dim3(256), 0, s, a);
    return hipGetLastError();
}

hipError_t launch_d4_qat_bwd(const void* g, int g_dtype, const float* W, const float* beta, const float* dbdt,
                             int64_t n_blocks, int64_t blocks_per_tile, float clip, float* dW, float* dbeta,
                             float* dtheta, hipStream_t s)
{
    if (n_blocks == 0) return hipSuccess;
    D4QatArgs a{};
    a.W = W;
    a.n_blocks = n_blocks;
    a.blocks_per_tile = blocks_per_tile;
    a.clip = clip;
    a.beta = beta;
    a.g = g;
    a.g_dtype = g_dtype;
    a.dbdt = dbdt;
    a.dW = dW;
    a.dbeta = dbeta;
    a.dtheta = dtheta;
    if (blocks_per_tile == 1)
        hipLaunchKernelGGL(d4_qat_bwd_block_kernel, dim3((unsigned)((n_blocks + 255) / 256)), dim3(256), 0, s, a);
    else
        hipLaunchKernelGGL(d4_qat_bwd_tile_kernel, dim3((unsigned)(n_blocks / blocks_per_tile)), dim3(256), 0, s, a);
    return hipGetLastError();
}

}  // namespace coset
