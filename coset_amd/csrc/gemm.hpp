// gemm.hpp -- the weight-gradient product of the QAT layer's F.linear
// (coset/core/layers.py:478, whose autograd forms dW_q = gy^T x), on the
// matrix cores (gemm_tn.hip).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace coset {

// Launch shape of C[M, N] = A^T B for A [K, M], B [K, N] (both row-major,
// bf16, K the token dimension): `tile` x `tile` output tiles (0: the kernel
// does not take the shape), `splits` K ranges per tile (> 1: fp32 partials in
// a workspace, summed in split order by a second kernel), `my` 32-token
// slices per wave and split, and the blocks of tiles the XCDs take (xcd_m x
// xcd_n tiles each; 0: plain row-major order).
struct GemmTnPlan {
    int tile;
    int splits;
    int xcd_m, xcd_n;
    int my;
};

// The plan for this shape: tiles of 64 x 64 (M, N multiples of 64, at most 256
// tiles) where they fit, else of 96 x 96 (multiples of 96, at most 256
// tiles), K = 256 * splits * my for my in {4, 8, 16, 32}.
GemmTnPlan gemm_tn_plan(int64_t M, int64_t N, int64_t K);
// 0 (default): the plan's choice of tile; 64 or 96: only that tile size
extern int g_gemm_tn_tile;
// fp32 workspace the plan needs (splits x (M x N + M), or 0)
int64_t gemm_tn_workspace_floats(const GemmTnPlan& p, int64_t M, int64_t N);

// out_dtype: 0 fp32, 1 bf16 (round to nearest even).  ldc in elements.
// colsum (nullable): also colsum[m] = sum_k A[k, m] in fp32 (fixed order).
hipError_t gemm_tn_bf16(const uint16_t* A, int64_t lda, const uint16_t* B, int64_t ldb, void* C, int64_t ldc,
                        int out_dtype, int64_t M, int64_t N, int64_t K, const GemmTnPlan& plan, float* workspace,
                        float* colsum, hipStream_t s);

}  // namespace coset
