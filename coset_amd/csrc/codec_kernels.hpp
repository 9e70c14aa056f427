// codec_kernels.hpp -- launch descriptors shared by the HIP kernels and the C-ABI.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "e8_core.hpp"
#include "e8_fast.hpp"
#include "fastdiv.hpp"

namespace coset {

enum DType { DT_F32 = 0, DT_BF16 = 1, DT_F16 = 2 };
enum ScaleMode { SCALE_NONE = 0, SCALE_CODEC = 1, SCALE_LAYER = 2 };
enum CodecMode { MODE_ENCODE = 0, MODE_DECODE = 1, MODE_ROUNDTRIP = 2 };

constexpr int kMaxM = 8;

// Bytes of one packed level word: q^8 <= 65536 fits 16 bits.
__host__ __device__ inline int word_bytes(int q) { return q <= 4 ? 2 : 4; }

// The layer's adaptive scale (coset/core/layers.py:381-396, 418-422) as the
// fp32 operation sequence torch runs on the device:
//   beta_min  = recip(c_eta_ginv * sigma) * c_min
//   beta_max  = min(recip(c_2ginv * xmax) * c_det, recip(c_2eta_ginv * sigma) * c_det)
//   beta_min  = min(beta_min, beta_max * 0.9)
//   beta      = beta_min + sigmoid(theta) * (beta_max - beta_min)
// with the Python-double constants rounded to fp32 as torch does.
struct ThetaBeta {
    const float* theta;      // [tiles]
    const float* sigma;      // [tiles] sigma_ema
    const float* xmax;       // [tiles] xmax_ema
    float c_min, c_eta_ginv, c_det, c_2ginv, c_2eta_ginv;
};

__device__ __forceinline__ void theta_beta_terms(const ThetaBeta& tb, int64_t t, float* bmin, float* bmax, float* sg)
{
    float sigma = tb.sigma[t], xmax = tb.xmax[t];
    float lo = __fmul_rn(__fdiv_rn(1.f, __fmul_rn(tb.c_eta_ginv, sigma)), tb.c_min);
    float hi_det = __fmul_rn(__fdiv_rn(1.f, __fmul_rn(tb.c_2ginv, xmax)), tb.c_det);
    float hi_prob = __fmul_rn(__fdiv_rn(1.f, __fmul_rn(tb.c_2eta_ginv, sigma)), tb.c_det);
    float hi = fminf(hi_det, hi_prob);
    lo = fminf(lo, __fmul_rn(hi, 0.9f));
    *bmin = lo;
    *bmax = hi;
    // sigmoid = 1 / (1 + e) in fp32 with e = exp(-theta) rounded once to
    // fp32 from a double-precision exp: the correctly rounded fp32 exp (but
    // for double-rounding cases), which is what torch's CPU sigmoid gives on
    // the reference's own layer goldens.
    *sg = __fdiv_rn(1.f, __fadd_rn(1.f, (float)exp(-(double)tb.theta[t])));
}

__device__ __forceinline__ float theta_beta(const ThetaBeta& tb, int64_t t)
{
    float lo, hi, sg;
    theta_beta_terms(tb, t, &lo, &hi, &sg);
    return __fadd_rn(lo, __fmul_rn(sg, __fsub_rn(hi, lo)));
}

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
    // SCALE_LAYER with beta derived in-kernel from theta (beta_row unused)
    int use_theta;
    ThetaBeta tb;
    float* beta_out;         // nullable [tiles]: the beta used, one write per tile
    float* dbdt_out;         // nullable [tiles]: d beta / d theta at that beta
    int64_t* step_counter;   // nullable: incremented once per launch
    int fast_projection;     // encoders try project_fast first (set by the launcher)
    // decode tables (tables.hpp, core rule; set by the launcher for q = 2, 4):
    // the generic kernel then decodes a level as 2 r = 2 G b - q (2 c[cid])
    // from the coarse-point id instead of running the projection
    const uint16_t* dec_map;
    const uint64_t* dec_coarse;
    // nullable: aux_out[i] = aux_in[i] in out_dtype for i < aux_n, written by
    // the same launch (the layer's bias in the GEMM's dtype)
    const float* aux_in;
    void* aux_out;
    int64_t aux_n;
    // SCALE_LAYER: floor(block / blocks_per_row) for blocks < 2^32 (set by
    // the launcher for the layer round-trip kernel)
    U32Div row_div;
};

// One encoder level (core rule, contiguous distances): the projection's
// fast path where its conditions hold, straight to the rows of G^-1 y, and
// the reference sequence for the lanes where they fail.  Digits are the rows
// mod q either way.  in_range is max |x_i| < 2^21 (fast_in_range).
template <int Q>
__device__ __forceinline__ void encode_level(const float x[8], int fast, int q, int b[8], bool in_range)
{
    int c[8];
    bool ok = false;
    if (fast) {
        ok = fast_rows<true>(x, c, in_range);  // condition (5) of e8_fast.hpp: tiny and zero coordinates stay fast
        // the rows stay computed here, ahead of the fallback branch: sunk past
        // it they would keep the argmax lane masks live across the fallback's
        // code
#pragma unroll
        for (int i = 0; i < 8; ++i) __asm__ volatile("" : "+v"(c[i]));
    }
    if (ok) {
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            if (Q > 0 && (Q & (Q - 1)) == 0) {
                b[i] = c[i] & (Q - 1);  // two's complement & == Python-style mod
            } else {
                const int qq = Q > 0 ? Q : q;
                const int m = c[i] % qq;
                b[i] = m < 0 ? m + qq : m;
            }
        }
    } else {
        float y[8];
        project<false, false>(x, y);
        lattice_digits<Q>(y, q, b);
    }
}

template <int Q>
__device__ __forceinline__ void encode_level(const float x[8], int fast, int q, int b[8])
{
    encode_level<Q>(x, fast, q, b, fast && fast_in_range(x));
}

// Per-block scale of SCALE_LAYER (reads beta_row or derives it from theta).
__device__ __forceinline__ float layer_scale(const CodecArgs& a, int64_t block)
{
    int64_t t = block / a.blocks_per_row;
    if (!a.use_theta) return a.beta_row[t];
    float lo, hi, sg;
    theta_beta_terms(a.tb, t, &lo, &hi, &sg);
    float span = __fsub_rn(hi, lo);
    float b = __fadd_rn(lo, __fmul_rn(sg, span));
    if (block == t * a.blocks_per_row) {  // one thread per tile records beta and its derivative
        if (a.beta_out) a.beta_out[t] = b;
        if (a.dbdt_out) a.dbdt_out[t] = __fmul_rn(__fmul_rn(span, __fsub_rn(1.f, sg)), sg);
    }
    return b;
}

// Dispatch: the LDS-table kernel (hnlq_lut.hip) for q in {2, 4} and large
// n, the generic kernel (hnlq_codec.hip) otherwise.  codec_path overrides
// the choice: 0 automatic, 1 always generic, 2 table kernel when supported.
hipError_t launch_codec(const CodecArgs& a, int mode, hipStream_t s);
// The forward of a small QAT layer (hnlq_codec.hip): W [rows, cols] fp32
// with one theta per row, q = 2 or 4, M = 2; x [tokens, cols] fp32 (tokens
// <= 64, cols <= 8192, cols % 8 == 0); y [tokens, rows] fp32.
hipError_t launch_qat_head(const float* W, int64_t rows, int64_t cols, const ThetaBeta& tb, float clip, int q,
                           const float* x, int tokens, const float* bias, float* y, int64_t* step_counter,
                           hipStream_t s);
hipError_t launch_codec_generic(const CodecArgs& a, int mode, hipStream_t s);
bool lut_path_supported(const CodecArgs& a, int mode);
hipError_t launch_codec_lut(const CodecArgs& a, int mode, hipStream_t s);
extern int g_codec_path;
extern int g_fast_projection;  // 1 (default): encoders use the fast projection where it is exact
extern int g_codec_plain;      // 1 (default): the table kernel's fixed-format variant where it applies
extern int g_codec_dynamic;    // 1 (default): the fixed-format kernel takes its tiles from a counter
constexpr int64_t kLutMinBlocks = 1 << 20;  // below it the table staging does not pay (layer-sized calls)
// A zeroed counter pair of the current device's counter ring (counters.hpp)
// for one launch on stream s, held until the launch's last workgroup puts the
// pair back to zero and stores 1 to *release; pair is null (static schedule)
// under graph capture or while every slot is held.
struct TileCounters {
    unsigned* pair;     // [0] hands out tiles, [1] counts finished workgroups
    unsigned* release;  // the slot's release flag (host memory, device address)
    int64_t slot;
};
TileCounters take_counters(hipStream_t s);
// Hands back the slot of a launch that failed to start.
void return_counters(const TileCounters& tc);

// Workgroup barrier that orders LDS only: waits for this wave's LDS
// operations, not for its loads and stores in flight (__syncthreads would
// drain those too).
__device__ __forceinline__ void lds_barrier()
{
    __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0); vmcnt, expcnt unrestricted
    __asm__ volatile("" ::: "memory");
    __builtin_amdgcn_s_barrier();
    __asm__ volatile("" ::: "memory");
}

// Backward of the QAT weight quantizer (qat.hip).
// dbdt (nullable): also write dtheta[t] = dbeta[t] * dbdt[t].
int64_t colsum_workspace_floats(int64_t rows, int64_t cols);
hipError_t launch_colsum(const void* g, int dtype, int64_t rows, int64_t cols, float* out, float* workspace,
                         hipStream_t s);
hipError_t launch_qat_stats(const float* W, int64_t tiles, int64_t n, double momentum, float* sigma_ema,
                            float* xmax_ema, hipStream_t s);
hipError_t launch_qat_bwd(const void* g, int g_dtype, const float* W, const void* packed,
                          const float* beta, int64_t n_blocks, int64_t blocks_per_tile, float clip,
                          int q, int M, float* dW, float* dbeta, const float* dbdt, float* dtheta,
                          hipStream_t s);

// D4 variant (d4.hip): lattice operators over [n, 4] blocks, and the D4
// layer's fused weight quantizer (tb non-null: beta from theta).
hipError_t launch_d4_lattice_op(int op, const float* in, int64_t n, int q, float* out, hipStream_t s);
hipError_t launch_d4_qat_fwd(const float* W, int64_t n_blocks, int64_t blocks_per_tile, const float* beta,
                             const ThetaBeta* tb, float clip, void* Wq, int wq_dtype, float* beta_out,
                             float* dbdt_out, int64_t* step_counter, hipStream_t s);
hipError_t launch_d4_qat_bwd(const void* g, int g_dtype, const float* W, const float* beta, const float* dbdt,
                             int64_t n_blocks, int64_t blocks_per_tile, float clip, float* dW, float* dbeta,
                             float* dtheta, hipStream_t s);

// LSQ activation quantizer (lsq.hip): forward, and backward with dalpha
// reduced through a caller-owned workspace of lsq_workspace_floats(n) floats.
int64_t lsq_workspace_floats(int64_t n);
hipError_t launch_lsq_fwd(const void* x, int dt, int64_t n, const float* alpha, int qmax, void* out, hipStream_t s);
hipError_t launch_lsq_bwd(const void* x, const void* g, int dt, int64_t n, const float* alpha, int qmax, void* dx,
                          float* d_alpha, float* workspace, hipStream_t s);

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
