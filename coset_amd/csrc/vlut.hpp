// vlut.hpp -- launch descriptors of the vLUT kernels (vlut.hip).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace coset {

constexpr int kMaxCoarseVlut = 640;  // LDS table slots for <a, c> (637 at q = 4)

// VLUT_METHOD_MFMA_SPLIT is internal: method MFMA with fp32 activations,
// each split exactly into three bf16 planes that run on the matrix cores
enum VlutMethod { VLUT_METHOD_AUTO = 0, VLUT_METHOD_LDS = 1, VLUT_METHOD_MFMA = 2, VLUT_METHOD_MFMA_SPLIT = 3 };

// Weight formats (include/coset_amd.h): raw uint16 words, row-major
// prepared uint32 (cid << 16 | idx), tiled prepared (matrix-core fragments).
// VLUT_DECODED: per (row, k-block) pair the 8 bytes 2 x_hat + 128 of its
// M-level decode (exact for the byte-table formats, |2 x_hat| <= 127), in the
// tiled fragment order; two uint32 per pair.  VLUT_PAIRS: each level word
// replaced by its four coordinate-pair ids (pair_map, tables.hpp), laid out
// [rows / 64][kb][M][64 rows] (rows padded to 64 with the ids of word 0):
// the LDS-table kernel's format, one 256-byte read per wave and word.
enum VlutFormat { VLUT_RAW = 0, VLUT_PREPARED = 1, VLUT_TILED = 2, VLUT_DECODED = 3, VLUT_PAIRS = 4 };
constexpr int kVlutDecodedBias = 128;

struct VlutMatmulArgs {
    const void* words;   // [rows, K/8, M] (VLUT_RAW / VLUT_PREPARED) or tiles (the other formats)
    int prepared;        // VlutFormat
    const float* scale;  // [rows] or null
    int scale_mode;      // 0: out *= scale[o]; 1: out /= scale[o]
    const void* act;     // [B, K] fp32 / bf16 / fp16
    int act_dtype;
    int64_t B, rows, K;
    int q, M, legacy;
    float* partial;      // split-K partials, [splits, B, rows] (the tile kernel: [B, rows, splits])
    float* out;          // [B, rows]
    // epilogue after the scale: + bias[o] (nullable), then the LSQ activation
    // quantizer with parameter *lsq_alpha and lsq_qmax (nullable alpha: none)
    const float* bias;
    const float* lsq_alpha;
    int lsq_qmax;
    // > 0: act holds three planes of planes_b tokens each (B = 3 planes_b,
    // the fp32 activations' exact bf16 planes); out is [planes_b, rows] and
    // each output adds its three planes' scaled products in plane order
    // before the bias / LSQ epilogue.  Set by vlut_matmul_split only, for
    // plans whose last kernel holds all three planes of an output.
    int64_t planes_b;
    // with planes_b: 1 when act is the fp32 activations [planes_b, K]
    // themselves, which the rows kernel's staging splits into the planes
    // (staged rows plans only), 0 when act holds the bf16 planes
    int act_planes;
    // filled by the launcher
    const uint16_t* map;
    const uint64_t* coarse;
    int n_coarse;
    const uint64_t* swar;  // byte tables of the MFMA decode (tables.hpp)
    int swar_ok;
    int swar_bias;
    const uint32_t* pair_map;  // coordinate-pair ids and values (tables.hpp)
    const float2* pair_vals;
};

// 0 forces the integer decode in the MFMA kernel (tests compare both)
extern int g_vlut_swar;
// > 0 forces the number of K splits (clamped to what the method allows)
extern int g_vlut_splits;
// 1 (default): batches above 32 tokens take the deep kernel, 0 the wide one
extern int g_vlut_deep;

// Index of level word m of (row, k-block kb) in a weight of format fmt.
// (VLUT_DECODED: index of the pair's first uint32; m and M are ignored.)
__host__ __device__ inline int64_t vlut_word_index(int fmt, int64_t row, int64_t kb, int m, int64_t kb_total, int M)
{
    if (fmt == VLUT_PAIRS) return (((row >> 6) * kb_total + kb) * M + m) * 64 + (row & 63);
    if (fmt != VLUT_TILED && fmt != VLUT_DECODED) return (row * kb_total + kb) * M + m;
    const int64_t kq = (kb_total + 3) / 4;
    const int64_t entry = (((row >> 4) * kq + (kb >> 2)) * 64) + (row & 15) + 16 * (kb & 3);
    return fmt == VLUT_DECODED ? 2 * entry : entry * M + m;
}

__host__ __device__ inline int64_t vlut_prepared_words(int64_t rows, int64_t kb, int M, int fmt)
{
    if (fmt == VLUT_PAIRS) return ((rows + 63) / 64) * 64 * kb * M;
    if (fmt != VLUT_TILED && fmt != VLUT_DECODED) return rows * kb * M;
    return ((rows + 15) / 16) * ((kb + 3) / 4) * 64 * (fmt == VLUT_DECODED ? 2 : M);
}

// Launch plan of a matmul: kernel and K splits (splits > 1 needs a
// workspace of splits * B * rows floats and a reduce launch).
enum VlutKernel { VK_LDS = 0, VK_MFMA_TILE = 1, VK_MFMA_ROWS = 2, VK_MFMA_WIDE = 3, VK_MFMA_DEEP = 4 };
struct VlutPlan {
    int kernel;
    int splits;
};
VlutPlan vlut_plan(int64_t rows, int64_t B, int64_t K, int q, int M, int method);
// Workspace floats a plan needs: the split-K partials ([B, rows, splits],
// or [splits, B, rows] for the wide kernel), none when the rows or wide
// kernel runs unsplit and writes the output itself.
inline int64_t vlut_workspace_floats(const VlutPlan& plan, int64_t B, int64_t rows)
{
    if ((plan.kernel == VK_MFMA_ROWS || plan.kernel == VK_MFMA_WIDE || plan.kernel == VK_MFMA_DEEP ||
         plan.kernel == VK_LDS) &&
        plan.splits == 1)
        return 0;
    return (int64_t)plan.splits * B * rows;
}

hipError_t vlut_build(const float* a, int64_t n_queries, int q, int legacy, float* vlut, hipStream_t s);
hipError_t vlut_dot(const void* words, int64_t n, int M, int q, const float* vlut, float* out, hipStream_t s);
hipError_t vlut_matmul(VlutMatmulArgs p, const VlutPlan& plan, hipStream_t s);
// fp32 activations on the matrix cores: a = h1 + h2 + h3 with each h the
// bf16 truncation of what the previous ones leave (exact: 3 x 8 significant
// bits), the three planes multiplied as 3B tokens of bf16 and summed per
// output.  The workspace holds the planes, the planes' outputs and the inner
// product's own partials.
int64_t vlut_split_workspace_floats(int64_t B, int64_t rows, int64_t K, int q, int M);
hipError_t vlut_matmul_split(VlutMatmulArgs p, float* workspace, hipStream_t s);
// prepared = cid(word) << 16 | word for raw words [rows, kb, M]: the
// coarse-point id each level word decodes through, stored next to it so the
// matmul needs no map lookup; fmt VLUT_PREPARED keeps the layout,
// VLUT_TILED writes the fragment order (padding decodes to 0); VLUT_PAIRS
// writes pair_map[word] in that order, VLUT_DECODED the M-level decode.
hipError_t vlut_prepare(const uint16_t* words, int64_t rows, int64_t kb, int M, int q, int legacy, int fmt,
                        uint32_t* prepared, hipStream_t s);

}  // namespace coset
