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
// tiled fragment order with each lane's two k-quads 2i, 2i + 1 adjacent
// ([row tile][k-quad pair][lane][2 pairs], k-quads padded to even), so a
// lane reads two steps as one 16-byte load; two uint32 per pair.  VLUT_PAIRS: each level word
// replaced by its four coordinate-pair ids (pair_map, tables.hpp), laid out
// [rows / 64][kb][M][64 rows] (rows padded to 64 with the ids of word 0):
// the LDS-table kernel's format, one 256-byte read per wave and word.
// VLUT_DECODED6: the same decode in 6 bytes per pair.  2 x_hat is in E8, so
// its 8 coordinates share one parity p; coordinate j is stored as the field
// f_j = floor(2 x_hat_j / 2) + off, off from decoded6_offset (tables.hpp: 18
// at q = 4, M = 2): byte i (0..5) holds f_i in bits 0-5, and its bits 6-7
// hold bits 2i, 2i + 1 of f_6 (bytes 0-2) or bits 2(i - 3), 2(i - 3) + 1 of
// v7 = f_7 | p << 5 (bytes 3-5).  Layout: [row tile of 16][chunk of 8 k-quads][lane][8 steps x 6
// bytes], lane = row % 16 + 16 (kb % 4) and step = k-quad % 8 as in the tiled
// order, so each lane reads its chunk as three 16-byte loads.  Padding (rows
// to 16, k-quads to 8) holds x_hat = 0.
enum VlutFormat { VLUT_RAW = 0, VLUT_PREPARED = 1, VLUT_TILED = 2, VLUT_DECODED = 3, VLUT_PAIRS = 4,
                  VLUT_DECODED6 = 5 };
constexpr int kVlutDecodedBias = 128;
constexpr int kD6Steps = 8;                  // k-quads per chunk of the 6-byte format
constexpr int kD6Words = 12;                 // uint32 per lane and chunk (8 x 48 bits)

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
    int d6_bias;           // VLUT_DECODED6: byte bias of 2 x_hat (2 off)
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
// (VLUT_DECODED: index of the pair's first uint32; VLUT_DECODED6: of the
// first uint32 of the lane's chunk holding the pair; m and M are ignored.)
__host__ __device__ inline int64_t vlut_word_index(int fmt, int64_t row, int64_t kb, int m, int64_t kb_total, int M)
{
    if (fmt == VLUT_PAIRS) return (((row >> 6) * kb_total + kb) * M + m) * 64 + (row & 63);
    if (fmt == VLUT_DECODED6) {
        const int64_t chunks = ((kb_total + 3) / 4 + kD6Steps - 1) / kD6Steps;
        const int64_t lane = (row & 15) + 16 * (kb & 3);
        return (((row >> 4) * chunks + (kb >> 2) / kD6Steps) * 64 + lane) * kD6Words;
    }
    if (fmt != VLUT_TILED && fmt != VLUT_DECODED) return (row * kb_total + kb) * M + m;
    const int64_t kq = (kb_total + 3) / 4;
    const int64_t lane = (row & 15) + 16 * (kb & 3);
    if (fmt == VLUT_DECODED)
        return ((((row >> 4) * ((kq + 1) / 2) + (kb >> 3)) * 64 + lane) * 2 + ((kb >> 2) & 1)) * 2;
    const int64_t entry = (((row >> 4) * kq + (kb >> 2)) * 64) + lane;
    return entry * M + m;
}

__host__ __device__ inline int64_t vlut_prepared_words(int64_t rows, int64_t kb, int M, int fmt)
{
    if (fmt == VLUT_PAIRS) return ((rows + 63) / 64) * 64 * kb * M;
    if (fmt == VLUT_DECODED6) return ((rows + 15) / 16) * (((kb + 3) / 4 + kD6Steps - 1) / kD6Steps) * 64 * kD6Words;
    if (fmt != VLUT_TILED && fmt != VLUT_DECODED) return rows * kb * M;
    if (fmt == VLUT_DECODED) return ((rows + 15) / 16) * (((kb + 3) / 4 + 1) / 2) * 64 * 4;
    return ((rows + 15) / 16) * ((kb + 3) / 4) * 64 * M;
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
// writes pair_map[word] in that order, VLUT_DECODED the M-level decode,
// VLUT_DECODED6 the same in 6 bytes (hipErrorInvalidValue where it does not fit).
hipError_t vlut_prepare(const uint16_t* words, int64_t rows, int64_t kb, int M, int q, int legacy, int fmt,
                        uint32_t* prepared, hipStream_t s);

}  // namespace coset
