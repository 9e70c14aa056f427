// probes.hip -- measurement kernels: the floors bench.py sets the codec and
// vLUT kernels against (no counterpart in the reference).
//   empty: a launch of a given grid, block and LDS size that does no work --
//          what a single launch costs from dispatch to completion;
//   read:  a stream of `bytes` from HBM into registers, L 16-byte loads per
//          thread all issued before any is used, one uint32 per workgroup
//          written (so the loads are live) -- the floor of a kernel that
//          reads a weight format of that size with that launch shape;
//   valu:  eight independent VALU chains per thread, 8 waves per workgroup
//          -- the sustained VALU issue rate the arithmetic-bound kernels
//          (C3) are set against.
// The C2 streaming probe (the codec kernel's own access pattern) is a
// variant of that kernel, in hnlq_lut.hip.
#include <hip/hip_runtime.h>

#include "probes.hpp"

namespace coset {

__global__ void probe_empty_kernel(uint32_t* out, uint32_t never)
{
    extern __shared__ uint32_t lds[];
    // never taken (the host passes 0): keeps the LDS allocation and the
    // output argument without doing work
    if (never && threadIdx.x == 0) out[blockIdx.x] = lds[0];
}

template <int L>
__global__ void probe_read_kernel(const uint4* __restrict__ src, int64_t n16, uint32_t* out)
{
    // workgroup b reads items [b * L * T, (b + 1) * L * T): item j of thread t
    // is b * L * T + j * T + t, so each wave load is 1 KiB contiguous
    const int64_t T = blockDim.x;
    const int64_t base = (int64_t)blockIdx.x * L * T + threadIdx.x;
    uint4 v[L];
#pragma unroll
    for (int j = 0; j < L; ++j) {
        const int64_t i = base + j * T;
        v[j] = src[i < n16 ? i : n16 - 1];
    }
    uint32_t x = 0u;
#pragma unroll
    for (int j = 0; j < L; ++j) x ^= v[j].x ^ v[j].y ^ v[j].z ^ v[j].w;
    // one word per workgroup: a wave-wide XOR, then lane 0 of wave 0
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) x ^= __shfl_xor(x, off, 64);
    if (threadIdx.x == 0) out[blockIdx.x] = x;
}

// KIND 0: 64 v_fma_f32 per iteration (8 steps x 8 chains), 1: 64 compares
// and 64 selects; the empty asm keeps each step's eight operations in place
template <int KIND>
__global__ void __launch_bounds__(512) probe_valu_kernel(float* out, int iters, float s)
{
    const float t0 = (float)threadIdx.x * 1e-3f;
    float a0 = t0, a1 = t0 + 1.f, a2 = t0 + 2.f, a3 = t0 + 3.f, a4 = t0 + 4.f, a5 = t0 + 5.f, a6 = t0 + 6.f,
          a7 = t0 + 7.f;
    for (int i = 0; i < iters; ++i) {
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            if (KIND == 0) {
                a0 = __builtin_fmaf(a0, s, 1.f); a1 = __builtin_fmaf(a1, s, 1.f);
                a2 = __builtin_fmaf(a2, s, 1.f); a3 = __builtin_fmaf(a3, s, 1.f);
                a4 = __builtin_fmaf(a4, s, 1.f); a5 = __builtin_fmaf(a5, s, 1.f);
                a6 = __builtin_fmaf(a6, s, 1.f); a7 = __builtin_fmaf(a7, s, 1.f);
            } else {
                a0 = a0 > s ? a1 : a2; a1 = a1 > s ? a2 : a3; a2 = a2 > s ? a3 : a4; a3 = a3 > s ? a4 : a5;
                a4 = a4 > s ? a5 : a6; a5 = a5 > s ? a6 : a7; a6 = a6 > s ? a7 : a0; a7 = a7 > s ? a0 : a1;
            }
            __asm__ volatile("" ::: "memory");
        }
    }
    out[(int64_t)blockIdx.x * blockDim.x + threadIdx.x] = a0 + a1 + a2 + a3 + a4 + a5 + a6 + a7;
}

hipError_t launch_probe_valu(int kind, int grid, int iters, float* out, hipStream_t s)
{
    if (kind == 0)
        hipLaunchKernelGGL(probe_valu_kernel<0>, dim3(grid), dim3(512), 0, s, out, iters, 0.999f);
    else
        hipLaunchKernelGGL(probe_valu_kernel<1>, dim3(grid), dim3(512), 0, s, out, iters, 0.999f);
    return hipGetLastError();
}

hipError_t launch_probe_empty(int grid, int threads, int lds_bytes, uint32_t* out, hipStream_t s)
{
    hipLaunchKernelGGL(probe_empty_kernel, dim3(grid), dim3(threads), lds_bytes, s, out, 0u);
    return hipGetLastError();
}

int probe_read_loads(int64_t bytes, int grid, int threads)
{
    const int64_t per = (int64_t)grid * threads * 16;
    const int64_t L = (bytes + per - 1) / per;
    return L <= 1 ? 1 : L <= 2 ? 2 : L <= 4 ? 4 : L <= 8 ? 8 : L <= 16 ? 16 : L <= 32 ? 32 : -1;
}

hipError_t launch_probe_read(const void* src, int64_t bytes, int grid, int threads, uint32_t* out, hipStream_t s)
{
    const int64_t n16 = bytes / 16;
    const uint4* p = static_cast<const uint4*>(src);
    switch (probe_read_loads(bytes, grid, threads)) {
    case 1: hipLaunchKernelGGL((probe_read_kernel<1>), dim3(grid), dim3(threads), 0, s, p, n16, out); break;
    case 2: hipLaunchKernelGGL((probe_read_kernel<2>), dim3(grid), dim3(threads), 0, s, p, n16, out); break;
    case 4: hipLaunchKernelGGL((probe_read_kernel<4>), dim3(grid), dim3(threads), 0, s, p, n16, out); break;
    case 8: hipLaunchKernelGGL((probe_read_kernel<8>), dim3(grid), dim3(threads), 0, s, p, n16, out); break;
    case 16: hipLaunchKernelGGL((probe_read_kernel<16>), dim3(grid), dim3(threads), 0, s, p, n16, out); break;
    case 32: hipLaunchKernelGGL((probe_read_kernel<32>), dim3(grid), dim3(threads), 0, s, p, n16, out); break;
    default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

}  // namespace coset
