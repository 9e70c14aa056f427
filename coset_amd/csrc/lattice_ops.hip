// lattice_ops.hip -- elementwise E8 lattice operators on the GPU.
//
// The building blocks of the codec exposed one by one, with the reference
// semantics of coset/core/base.py:134-202 (encode_coords, decode_coords,
// custom_round) and coset/core/e8/lattice.py:67-169 (g_x, projection);
// legacy=1 selects coset/legacy/lattices/e8.py:41-103.
#include "codec_kernels.hpp"

namespace coset {

__global__ void __launch_bounds__(256) custom_round_kernel(const float* in, int64_t n, float* out)
{
    int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) out[i] = custom_round(in[i]);
}

template <int OP, bool LEGACY>
__global__ void __launch_bounds__(256) block_op_kernel(const float* in, int64_t n, int q, float* out)
{
    int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    const float4* p = reinterpret_cast<const float4*>(in) + 2 * i;
    float4 u = p[0], v = p[1];
    float x[8] = {u.x, u.y, u.z, u.w, v.x, v.y, v.z, v.w};
    float y[8];
    if (OP == OP_G_X) {
        d8_candidate<LEGACY, true>(x, y);
    } else if (OP == OP_PROJECT) {
        project<LEGACY, false>(x, y);
    } else if (OP == OP_ENCODE_COORDS) {
        // round(G^-1 x) mod q; exact for x in (1/2)Z^8, fp32 row sums otherwise
        float suf = 0.f;
        float c[8];
        for (int r = 6; r >= 1; --r) {
            suf = __fadd_rn(suf, x[r]);
            c[r] = __fsub_rn(suf, __fmul_rn((float)(7 - r), x[7]));
        }
        suf = __fadd_rn(suf, x[0]);
        c[0] = __fsub_rn(__fmul_rn(0.5f, suf), __fmul_rn(3.5f, x[7]));
        c[7] = __fmul_rn(2.f, x[7]);
        float qf = (float)q;
        for (int r = 0; r < 8; ++r) {
            float k = rintf(c[r]);
            float m = fmodf(k, qf);
            y[r] = (m < 0.f) ? __fadd_rn(m, qf) : m;
        }
    } else {
        lattice_point_f(x, y);
    }
    float4* o = reinterpret_cast<float4*>(out) + 2 * i;
    o[0] = make_float4(y[0], y[1], y[2], y[3]);
    o[1] = make_float4(y[4], y[5], y[6], y[7]);
}

hipError_t launch_lattice_op(int op, int legacy, const float* in, int64_t n, int q,
                             float* out, hipStream_t s)
{
    if (n == 0) return hipSuccess;
    dim3 block(256);
    if (op == OP_CUSTOM_ROUND) {
        int64_t m = 8 * n;
        hipLaunchKernelGGL(custom_round_kernel, dim3((unsigned)((m + 255) / 256)), block, 0, s, in, m, out);
        return hipGetLastError();
    }
    dim3 grid((unsigned)((n + 255) / 256));
#define COSET_OP(OPV)                                                                        \
    if (legacy)                                                                              \
        hipLaunchKernelGGL((block_op_kernel<OPV, true>), grid, block, 0, s, in, n, q, out);  \
    else                                                                                     \
        hipLaunchKernelGGL((block_op_kernel<OPV, false>), grid, block, 0, s, in, n, q, out);
    switch (op) {
    case OP_G_X: COSET_OP(OP_G_X) break;
    case OP_PROJECT: COSET_OP(OP_PROJECT) break;
    case OP_ENCODE_COORDS: COSET_OP(OP_ENCODE_COORDS) break;
    default: COSET_OP(OP_DECODE_COORDS) break;
    }
#undef COSET_OP
    return hipGetLastError();
}

}  // namespace coset
