// lsq.hpp -- scalar steps of the LSQ activation quantizer
// (coset/core/layers.py:117-137), shared by the standalone kernels (lsq.hip)
// and the vLUT matmul epilogue (vlut.hip).  fp32 operations in the
// reference's order; see lsq.hip for the chain and its backward.
#pragma once

#include <hip/hip_runtime.h>

namespace coset {

struct LsqScale {
    float a;   // relu(alpha) + 1e-8
    float s;   // a / qmax
    bool pos;  // relu(alpha) > 0
};

__device__ __forceinline__ LsqScale lsq_scale(const float* alpha, int qmax)
{
    const float v = alpha[0];
    const float r = (v > 0.f || v != v) ? v : 0.f;  // relu, NaN kept
    LsqScale c;
    c.a = __fadd_rn(r, 1e-8f);
    c.s = __fdiv_rn(c.a, (float)qmax);
    c.pos = r > 0.f;
    return c;
}

struct LsqElem {
    float xc, y, yq;
};

__device__ __forceinline__ LsqElem lsq_elem(float x, const LsqScale& c)
{
    const float cl = x != x ? x : fminf(fmaxf(x, -c.a), c.a);
    LsqElem e;
    e.xc = __fadd_rn(__fsub_rn(x, x), cl);
    e.y = __fdiv_rn(e.xc, c.s);
    e.yq = __fadd_rn(__fsub_rn(e.y, e.y), rintf(e.y));
    return e;
}

// The quantized value of one activation.
__device__ __forceinline__ float lsq_value(float x, const LsqScale& c)
{
    return __fmul_rn(lsq_elem(x, c).yq, c.s);
}

}  // namespace coset
