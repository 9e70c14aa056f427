// lsq.hip -- the LSQ activation quantizer (coset/core/layers.py:117-137, with
// ste_clip / ste_round of layers.py:20-26) as one forward and one backward
// pass over the activations.
//
// Forward, the reference's fp32 operations in its order, on float(x):
//   a   = relu(alpha) + 1e-8
//   xc  = (x - x) + clamp(x, -a, a)          ste_clip (value)
//   s   = a / qmax
//   y   = xc / s
//   yq  = (y - y) + round_half_even(y)       ste_round (value)
//   out = yq * s                             rounded once to x's dtype
// The (x - x) and (y - y) terms are kept: they make +-inf inputs NaN and
// turn a rounded -0 into +0, as in the reference.
// Backward, the autograd of that chain for g = dL/dout:
//   dx     = (g * s) / s                     mul, then div backward
//   dL/ds  = sum g * yq + sum -(g * s) * ((xc / s) / s)
//   dalpha = relu(alpha) > 0 ? (dL/ds) / qmax : 0
// (the clamp bounds are detached in ste_clip, so they carry no gradient).
// The two sums go per thread, per workgroup in a fixed tree, and over the
// workgroup partials in double in one workgroup: deterministic.
#include <hip/hip_fp16.h>
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "codec_kernels.hpp"
#include "lsq.hpp"

namespace coset {

namespace {

constexpr int kLsqThreads = 256;
constexpr int kLsqMaxGroups = 2048;

__device__ __forceinline__ float load_elem(const void* p, int dt, int64_t i)
{
    if (dt == DT_F32) return reinterpret_cast<const float*>(p)[i];
    const uint16_t h = reinterpret_cast<const uint16_t*>(p)[i];
    return dt == DT_BF16 ? bf16_to_f32(h) : __half2float(__ushort_as_half(h));
}

__device__ __forceinline__ void store_elem(void* p, int dt, int64_t i, float v)
{
    if (dt == DT_F32)
        reinterpret_cast<float*>(p)[i] = v;
    else if (dt == DT_BF16)
        reinterpret_cast<uint16_t*>(p)[i] = f32_to_bf16(v);
    else
        reinterpret_cast<uint16_t*>(p)[i] = __half_as_ushort(__float2half_rn(v));
}

__global__ void __launch_bounds__(kLsqThreads) lsq_fwd_kernel(const void* x, int dt, int64_t n, const float* alpha,
                                                             int qmax, void* out)
{
    const LsqScale c = lsq_scale(alpha, qmax);
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) {
        const LsqElem e = lsq_elem(load_elem(x, dt, i), c);
        store_elem(out, dt, i, __fmul_rn(e.yq, c.s));
    }
}

__device__ __forceinline__ float block_sum(float v, float* sh)
{
    // wave64 butterfly, then the waves' sums in LDS (fixed order)
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, 64);
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    __syncthreads();
    if (lane == 0) sh[wave] = v;
    __syncthreads();
    float t = 0.f;
    if (threadIdx.x == 0)
        for (int w = 0; w < kLsqThreads / 64; ++w) t += sh[w];
    return t;
}

__global__ void __launch_bounds__(kLsqThreads) lsq_bwd_kernel(const void* x, const void* g, int dt, int64_t n,
                                                             const float* alpha, int qmax, void* dx,
                                                             float* partial)
{
    __shared__ float sh[kLsqThreads / 64];
    const LsqScale c = lsq_scale(alpha, qmax);
    float s1 = 0.f, s2 = 0.f;
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) {
        const LsqElem e = lsq_elem(load_elem(x, dt, i), c);
        const float gi = load_elem(g, dt, i);
        const float gs = __fmul_rn(gi, c.s);
        store_elem(dx, dt, i, __fdiv_rn(gs, c.s));
        s1 += __fmul_rn(gi, e.yq);
        s2 += __fmul_rn(-gs, __fdiv_rn(__fdiv_rn(e.xc, c.s), c.s));
    }
    const float t1 = block_sum(s1, sh);
    const float t2 = block_sum(s2, sh);
    if (threadIdx.x == 0) {
        partial[2 * blockIdx.x] = t1;
        partial[2 * blockIdx.x + 1] = t2;
    }
}

__global__ void __launch_bounds__(kLsqThreads) lsq_alpha_kernel(const float* partial, int groups, const float* alpha,
                                                               int qmax, float* d_alpha)
{
    __shared__ double sh[2][kLsqThreads];
    double a1 = 0.0, a2 = 0.0;
    for (int i = threadIdx.x; i < groups; i += blockDim.x) {
        a1 += (double)partial[2 * i];
        a2 += (double)partial[2 * i + 1];
    }
    sh[0][threadIdx.x] = a1;
    sh[1][threadIdx.x] = a2;
    __syncthreads();
    for (int w = kLsqThreads / 2; w >= 1; w >>= 1) {
        if (threadIdx.x < w) {
            sh[0][threadIdx.x] += sh[0][threadIdx.x + w];
            sh[1][threadIdx.x] += sh[1][threadIdx.x + w];
        }
        __syncthreads();
    }
    if (threadIdx.x == 0) {
        const LsqScale c = lsq_scale(alpha, qmax);
        const float ds = __fadd_rn((float)sh[0][0], (float)sh[1][0]);
        d_alpha[0] = c.pos ? __fdiv_rn(ds, (float)qmax) : 0.f;
    }
}

int lsq_groups(int64_t n)
{
    const int64_t need = (n + kLsqThreads * 4 - 1) / (kLsqThreads * 4);
    return (int)(need < 1 ? 1 : need > kLsqMaxGroups ? kLsqMaxGroups : need);
}

}  // namespace

int64_t lsq_workspace_floats(int64_t n) { return 2 * (int64_t)lsq_groups(n); }

hipError_t launch_lsq_fwd(const void* x, int dt, int64_t n, const float* alpha, int qmax, void* out, hipStream_t s)
{
    if (n == 0) return hipSuccess;
    hipLaunchKernelGGL(lsq_fwd_kernel, dim3(lsq_groups(n)), dim3(kLsqThreads), 0, s, x, dt, n, alpha, qmax, out);
    return hipGetLastError();
}

hipError_t launch_lsq_bwd(const void* x, const void* g, int dt, int64_t n, const float* alpha, int qmax, void* dx,
                          float* d_alpha, float* workspace, hipStream_t s)
{
    const int groups = lsq_groups(n);
    if (n > 0)
        hipLaunchKernelGGL(lsq_bwd_kernel, dim3(groups), dim3(kLsqThreads), 0, s, x, g, dt, n, alpha, qmax, dx,
                           workspace);
    hipLaunchKernelGGL(lsq_alpha_kernel, dim3(1), dim3(kLsqThreads), 0, s, workspace, n > 0 ? groups : 0, alpha,
                       qmax, d_alpha);
    return hipGetLastError();
}

}  // namespace coset
