// legacy.hpp -- launch descriptor of the paper's hierarchical encode/decode
// with the overload loop (hnlq_legacy.hip).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace coset {

constexpr int kLegacyMaxT = 63;  // largest scaling count T (max_iter bound)

struct LegacyArgs {
    int64_t n;                // blocks
    int q, M;
    float beta;               // x / beta on encode, beta * x_hat on decode
    int beta_is_pow2;         // beta = 2^k: x / beta == x * beta_inv exactly
    float beta_inv;
    float two_alpha;          // (float)2^alpha, the overload rescale divisor
    int max_iter, protect;    // max_scaling_iterations, !disable_overload_protection
    const void* x;            // encode input [n, 8] fp32 / bf16
    int x_dtype;
    const float* dither;      // nullable, [8] (stride 0) or [n, 8] (stride 8)
    int64_t dither_stride;
    void* packed;             // nullable [n, M] level words of the final chain
    float* codes_f32;         // nullable [n, M, 8]
    int32_t* T;               // nullable [n]
    uint8_t* overload;        // nullable [n]: the final chain overloads
    const void* packed_in;    // decode input (or codes_in_f32)
    const float* codes_in_f32;
    const int32_t* T_in;      // nullable: T = 0
    float* out;               // nullable decode output [n, 8] fp32
    float scale_T[kLegacyMaxT + 1];  // (float)2^(alpha t)
};

hipError_t launch_legacy(const LegacyArgs& a, bool decode_only, hipStream_t s);

}  // namespace coset
