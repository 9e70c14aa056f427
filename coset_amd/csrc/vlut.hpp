// vlut.hpp -- launch descriptors of the vLUT kernels (vlut.hip).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace coset {

constexpr int kMaxCoarseVlut = 640;  // LDS table slots for <a, c> (637 at q = 4)

enum VlutMethod { VLUT_METHOD_AUTO = 0, VLUT_METHOD_LDS = 1, VLUT_METHOD_MFMA = 2 };

struct VlutMatmulArgs {
    const void* words;   // [rows, K/8, M] uint16 level words, or uint32 (cid << 16 | idx) when prepared
    int prepared;
    const float* scale;  // [rows] or null
    int scale_mode;      // 0: out *= scale[o]; 1: out /= scale[o]
    const void* act;     // [B, K] fp32 / bf16 / fp16
    int act_dtype;
    int64_t B, rows, K;
    int q, M, legacy;
    float* partial;      // [B, rows, splits] workspace
    float* out;          // [B, rows]
    // filled by the launcher
    const uint16_t* map;
    const uint64_t* coarse;
    int n_coarse;
    int kb_per_chunk;
    const uint64_t* swar;  // byte tables of the MFMA decode (tables.hpp)
    int swar_ok;
    int swar_bias;
};

// 0 forces the integer decode in the MFMA kernel (tests compare both)
extern int g_vlut_swar;
// > 0 forces the number of K splits (clamped to what the method allows)
extern int g_vlut_splits;

hipError_t vlut_build(const float* a, int64_t n_queries, int q, int legacy, float* vlut, hipStream_t s);
hipError_t vlut_dot(const void* words, int64_t n, int M, int q, const float* vlut, float* out, hipStream_t s);
int vlut_default_splits(int64_t rows, int64_t B, int64_t K, int method);
hipError_t vlut_matmul(VlutMatmulArgs p, int method, int splits, hipStream_t s);
// prepared[i] = cid(words[i]) << 16 | words[i]: the coarse-point id each level
// word decodes through, stored next to it so the matmul needs no map lookup.
hipError_t vlut_prepare(const uint16_t* words, int64_t n, int q, int legacy, uint32_t* prepared, hipStream_t s);

}  // namespace coset
