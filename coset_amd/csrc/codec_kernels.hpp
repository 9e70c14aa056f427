// codec_kernels.hpp -- launch descriptors shared by the HIP kernels and the C-ABI.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "e8_core.hpp"

namespace coset {

enum DType { DT_F32 = 0, DT_BF16 = 1, DT_F16 = 2 };
enum ScaleMode { SCALE_NONE = 0, SCALE_CODEC = 1, SCALE_LAYER = 2 };
enum CodecMode { MODE_ENCODE = 0, MODE_DECODE = 1, MODE_ROUNDTRIP = 2 };

constexpr int kMaxM = 8;

// Bytes of one packed level word: q^8 <= 65536 fits 16 bits.
__host__ __device__ inline int word_bytes(int q) { return q <= 4 ? 2 : 4; }

struct CodecArgs {
    int64_t n;               // blocks
    int q, M;
    int scale_mode;          // ScaleMode
    float beta;              // SCALE_CODEC
    int beta_is_pow2;        // beta = 2^k: x / beta == x * beta_inv exactly
    float beta_inv;
    const float* beta_row;   // SCALE_LAYER: [n / blocks_per_row]
    int64_t blocks_per_row;  // SCALE_LAYER
    float clip;              // SCALE_LAYER
    int strided;             // decode distances with the batched (fma) rule
    // encode input
    const void* x;           // [n, 8] fp32 or bf16
    int x_dtype;
    const float* dither;     // nullable; [8] (stride 0) or [n, 8] (stride 8)
    int64_t dither_stride;
    // encode outputs
    void* packed;            // nullable [n, M] words (uint16 if q <= 4 else uint32)
    float* codes_f32;        // nullable [n, M, 8]
    // decode inputs (MODE_DECODE)
    const void* packed_in;
    const float* codes_in_f32;
    // decode output
    void* out;               // nullable [n, 8] fp32 or bf16
    int out_dtype;
};

// Dispatch: the LDS-table kernel (hnlq_lut.hip) for q in {2, 4} and large
// n, the generic kernel (hnlq_codec.hip) otherwise.  codec_path overrides
// the choice: 0 automatic, 1 always generic, 2 table kernel when supported.
hipError_t launch_codec(const CodecArgs& a, int mode, hipStream_t s);
hipError_t launch_codec_generic(const CodecArgs& a, int mode, hipStream_t s);
bool lut_path_supported(const CodecArgs& a, int mode);
hipError_t launch_codec_lut(const CodecArgs& a, int mode, hipStream_t s);
extern int g_codec_path;
constexpr int64_t kLutMinBlocks = 1 << 16;

// Backward of the QAT weight quantizer (qat.hip).
hipError_t launch_qat_bwd(const void* g, int g_dtype, const float* W, const void* packed,
                          const float* beta, int64_t n_blocks, int64_t blocks_per_tile, float clip,
                          int q, int M, float* dW, float* dbeta, hipStream_t s);

// Elementwise lattice operators (custom_round, g_x, projection,
// encode_coords, decode_coords) over n blocks.
enum LatticeOp {
    OP_CUSTOM_ROUND = 0,
    OP_G_X = 1,
    OP_PROJECT = 2,
    OP_ENCODE_COORDS = 3,
    OP_DECODE_COORDS = 4,
};
hipError_t launch_lattice_op(int op, int legacy, const float* in, int64_t n, int q,
                             float* out, hipStream_t s);

}  // namespace coset
