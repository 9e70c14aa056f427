/*
 * coset_amd.h -- C ABI of the MI355X E8 HNLQ library (libcoset_amd.so).
 *
 * Plain pointers and sizes only.  Every buffer is device memory allocated by
 * the caller; `stream` is a hipStream_t (NULL = legacy default stream).  Calls
 * are asynchronous and stream-ordered; none synchronizes the host.  Return
 * value: COSET_OK (0) or a negative COSET_E* code; coset_last_error() then
 * holds a message for the calling thread.  Work runs on the calling thread's
 * current HIP device (hipSetDevice): the buffers and the stream passed in
 * must belong to it (per-device state -- decode tables, tile counters -- is
 * looked up from it).
 *
 * Packed code format: level word idx(b) = sum_j b_j q^(7-j) for the level's
 * digits b in [0,q)^8 (the reference vLUT index, coset/legacy/quant/vlut.py:
 * 217-238); words are stored [n_blocks, M] as uint16 when q <= 4 and uint32
 * when 4 < q <= 16 (coset_word_bytes).
 *
 * Reference interfaces replaced (paths in the mlsquare/coset tree):
 *   coset_e8_hnlq_encode     e8_encode             coset/core/e8/codecs.py:17-89
 *   coset_e8_hnlq_decode     e8_decode/_full_decode coset/core/e8/codecs.py:139-218
 *   coset_e8_hnlq_roundtrip  e8_quantize           coset/core/e8/codecs.py:221-286
 *                            and the quantize step of HNLQLinearQAT._quantize_weights
 *                                                  coset/core/layers.py:428-463
 *   coset_e8_lattice_op      Lattice.custom_round/encode_coords/decode_coords
 *                                                  coset/core/base.py:134-202,
 *                            E8Lattice.g_x/projection coset/core/e8/lattice.py:67-169,
 *                            legacy E8Lattice.g_x/Q coset/legacy/lattices/e8.py:41-103
 *   coset_e8_qat_fwd         HNLQLinearQAT._quantize_weights (scale, STE quantize,
 *                            unscale, clamp)       coset/core/layers.py:398-470
 *   coset_e8_qat_head_fwd    HNLQLinearQAT.forward of a small layer under no_grad
 *                            (quantizer + F.linear) coset/core/layers.py:428-484
 *   coset_e8_qat_bwd         autograd of that chain through the straight-through
 *                            estimator             coset/core/layers.py:62-110, 428-463
 *   coset_qat_stats_update   HNLQLinearQAT._gather_stats coset/core/layers.py:366-379
 *   coset_colsum             bias gradient of the layer's F.linear  coset/core/layers.py:478
 *   coset_gemm_tn            weight gradient of the layer's F.linear coset/core/layers.py:478
 *   coset_vlut_build_one_sided  vLUTManager.build_one_sided_vlut
 *                                                  coset/legacy/quant/vlut.py:72-117
 *   coset_vlut_lookup_dot    one-sided lookup sum  tests/legacy/test_one_sided_vlut_pytest.py:22-43
 *   coset_vlut_matmul        the same lookup over a weight matrix (the reference's
 *                            placeholder is QLinear._lut_matmul,
 *                                                  coset/legacy/nn/qlinear.py:272-281)
 */
#ifndef COSET_AMD_H
#define COSET_AMD_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define COSET_ABI_VERSION 3

enum {
    COSET_OK = 0,
    COSET_EINVAL = -1,       /* bad size, q, M, pointer or alignment */
    COSET_EUNSUPPORTED = -2, /* valid request this build does not handle */
    COSET_EHIP = -3          /* HIP runtime error (launch or device) */
};

enum { COSET_F32 = 0, COSET_BF16 = 1, COSET_F16 = 2 };

/* scale_mode: NONE uses x as is; CODEC divides by beta before encoding and
 * multiplies the decode by beta (codecs.py:64,175); LAYER multiplies by
 * beta_row[block / blocks_per_row] before encoding, divides the decode by it
 * and clamps to [-clip, clip] (layers.py:431,455,463). */
enum { COSET_SCALE_NONE = 0, COSET_SCALE_CODEC = 1, COSET_SCALE_LAYER = 2 };

/* op codes of coset_e8_lattice_op */
enum {
    COSET_OP_CUSTOM_ROUND = 0,
    COSET_OP_G_X = 1,
    COSET_OP_PROJECT = 2,
    COSET_OP_ENCODE_COORDS = 3,
    COSET_OP_DECODE_COORDS = 4
};

/* option keys of coset_set_option */
enum {
    COSET_OPT_CODEC_PATH = 1,  /* 0 automatic, 1 generic kernel, 2 LDS-table kernel (q = 2, 4) */
    COSET_OPT_VLUT_DECODE = 2, /* MFMA vLUT decode: 1 byte tables where they fit (default), 0 integer */
    COSET_OPT_VLUT_SPLITS = 3, /* vLUT K splits: 0 automatic, n > 0 forced (clamped to the valid range) */
    COSET_OPT_FAST_PROJECTION = 4, /* encoders: 1 fast projection where provably exact (default), 0 never */
    COSET_OPT_CODEC_PLAIN = 5,     /* 1 fixed-format codec kernels where a call qualifies (default: the table kernel's for fp32,
                                      beta = 2^k calls; the layer round trip's for stored or theta-derived betas at q = 4, 8, 16), 0 never */
    COSET_OPT_CODEC_DYNAMIC = 6,   /* fixed-format table kernel: 1 tiles from a counter run per launch (default), 0 grid stride */
    COSET_OPT_VLUT_DEEP = 7,       /* vLUT matmul above 32 tokens: 1 the 64-row deep kernel (default), 0 the 128-row wide one */
    COSET_OPT_GEMM_TN_TILE = 8     /* coset_gemm_tn output tiles: 0 64 x 64 where they fit, else 96 x 96 (default); 64 or 96 only that size */
};

int coset_abi_version(void);
const char* coset_last_error(void);
int coset_word_bytes(int q);

/* The paper's hierarchical quantizer with overload handling
 * (coset/legacy/quant/functional.py:15-181, Algorithms 1 and 2), per 8-wide
 * block: xs = x / beta (+ dither), level chain y = Q(x_l), x_l = y / q with
 * the legacy (textbook) Q; a block overloads when Q(x_M) != 0.  With protect
 * set, an overloading block is rescaled xs /= 2^alpha and re-encoded up to
 * max_iter (<= 63) times.  Outputs (each nullable): the final chain's level
 * words and float codes [n, M, 8], T [n] (int32 rescale count), overload
 * [n] (uint8, the final chain's flag; the core codecs have none, their T is
 * always 0 as in codecs.py:89) and decoded [n, 8]: Algorithm 2 of the same
 * codes.  Decode: x_hat = sum_i q^i r(b_i) with the legacy residual, minus
 * dither, times beta, times (float)2^(alpha T) (T NULL: T = 0). */
int coset_e8_legacy_encode(const void* x, int x_dtype, int64_t n_blocks, float beta, double alpha,
                           int max_iter, int protect, const float* dither, int64_t dither_stride,
                           int q, int M, void* packed, float* codes_f32, int32_t* T,
                           uint8_t* overload, float* decoded, void* stream);
int coset_e8_legacy_decode(const void* packed, const float* codes_f32, const int32_t* T,
                           int64_t n_blocks, float beta, double alpha, const float* dither,
                           int64_t dither_stride, int q, int M, float* out, void* stream);

/* Build the per-device constant tables (single-level decode and vLUT coarse
 * points for q = 2 and 4, core and legacy rules) on `device` (-1: current).
 * Blocking; call once before capturing HIP graphs.  Other entry points build
 * them on first use. */
int coset_init(int device);

/* Process-wide tuning/test knobs (see COSET_OPT_*). */
int coset_set_option(int key, int value);

/* Encode n_blocks 8-wide blocks (x: fp32 or bf16, 16-byte aligned).
 * dither (nullable, fp32): added after scaling; dither_stride 0 broadcasts one
 * [8] vector, 8 reads [n_blocks, 8].  Outputs (each nullable): packed words
 * and the reference's float code tensor [n_blocks, M, 8]. */
int coset_e8_hnlq_encode(const void* x, int x_dtype, int64_t n_blocks,
                         int scale_mode, float beta, const float* beta_row,
                         int64_t blocks_per_row, const float* dither, int64_t dither_stride,
                         int q, int M, void* packed, float* codes_f32, void* stream);

/* Decode from packed words or, when packed is NULL, from a float code tensor
 * codes_f32 [n_blocks, M, 8].  strided=1 reproduces the reference's batched
 * decode distance rule (any call on more than one block); it changes results
 * only for q that is not a power of two.  out: fp32 or bf16 [n_blocks, 8]. */
int coset_e8_hnlq_decode(const void* packed, const float* codes_f32, int64_t n_blocks,
                         int scale_mode, float beta, const float* beta_row,
                         int64_t blocks_per_row, float clip, int q, int M, int strided,
                         void* out, int out_dtype, void* stream);

/* Fused encode -> decode in one pass (one HBM read, one write).  Any of
 * packed, codes_f32, out may be NULL. */
int coset_e8_hnlq_roundtrip(const void* x, int x_dtype, int64_t n_blocks,
                            int scale_mode, float beta, const float* beta_row,
                            int64_t blocks_per_row, float clip,
                            const float* dither, int64_t dither_stride,
                            int q, int M, int strided,
                            void* packed, float* codes_f32, void* out, int out_dtype,
                            void* stream);

/* QAT weight quantizer forward (coset/core/layers.py:428-463 with the
 * injected e8_quantize, codecs.py:221-286):
 *   Wq = clamp(dec(enc(W * beta_t)) / beta_t, -clip, clip)
 * W fp32 [rows, cols] (cols % 8 == 0), beta_t = beta[block / blocks_per_tile]
 * (blocks_per_tile = cols/8 for row tiling, 1 for block tiling).  Writes Wq
 * (fp32 or bf16, nullable) and the packed level words (nullable) that
 * coset_e8_qat_bwd re-decodes. */
int coset_e8_qat_fwd(const float* W, int64_t rows, int64_t cols, const float* beta,
                     int64_t blocks_per_tile, float clip, int q, int M, void* Wq, int wq_dtype,
                     void* packed, void* stream);

/* QAT weight quantizer backward through the straight-through estimator
 * (StraightThroughQuantize.backward, coset/core/layers.py:86-95, and the
 * autograd of layers.py:431-463): from g = dL/dWq (fp32 or bf16) writes
 *   dW    = ((g*m)/beta)*beta,   m = (-clip <= Q/beta <= clip)
 *   dbeta[t] = sum_t ((g*m)/beta)*W - (g*m)*((Q/beta)/beta)
 * with Q re-decoded from `packed`.  dbeta has one entry per tile. */
int coset_e8_qat_bwd(const void* gWq, int g_dtype, const float* W, const void* packed,
                     const float* beta, int64_t rows, int64_t cols, int64_t blocks_per_tile,
                     float clip, int q, int M, float* dW, float* dbeta, void* stream);

/* Same forward with beta computed in the kernel from the layer's theta and
 * EMA buffers (coset/core/layers.py:381-396, 418-422: beta = beta_min +
 * sigmoid(theta)(beta_max - beta_min), one entry per tile), so a QAT step
 * needs no separate launches for the bounds.  beta_out and dbeta_dtheta_out
 * (nullable, [tiles]) receive the beta used and (beta_max - beta_min) s (1 - s),
 * s = sigmoid(theta); step_counter (nullable, int64 device scalar: the layer's
 * step_count buffer) is incremented once.  M_bounds is the layer's M (the
 * bounds' q^M); M is the codec depth (2: e8_quantize, codecs.py:245-254).
 * bias / bias_out (nullable, [rows]): the same launch also writes the
 * layer's fp32 bias in wq_dtype (round to nearest even), the operand of the
 * product that follows (layers.py:478), so no separate cast launch is needed. */
int coset_e8_qat_fwd_theta(const float* W, int64_t rows, int64_t cols, int64_t blocks_per_tile,
                           const float* theta, const float* sigma_ema, const float* xmax_ema, double delta0,
                           double eta, double gamma_inv, int M_bounds, float clip, int q, int M, void* Wq,
                           int wq_dtype, void* packed, float* beta_out, float* dbeta_dtheta_out,
                           int64_t* step_counter, const float* bias, void* bias_out, void* stream);

/* The forward of a small QAT layer in one launch: HNLQLinearQAT.forward
 * (coset/core/layers.py:472-484) with its fused quantizer
 * (coset_e8_qat_fwd_theta, row tiling: one theta per row, M = 2, q = 2 or 4)
 * and F.linear, y [tokens, rows] = x [tokens, cols] W_q^T + bias, fp32, for
 * inference-sized batches (tokens <= 64, cols % 8 == 0 and <= 8192; others
 * return COSET_EUNSUPPORTED).  W_q is the quantizer's, bit for bit; the
 * products are fp32 in a fixed order.  step_counter (nullable) is
 * incremented once; bias nullable. */
int coset_e8_qat_head_fwd(const float* W, int64_t rows, int64_t cols, const float* theta, const float* sigma_ema,
                          const float* xmax_ema, double delta0, double eta, double gamma_inv, int M_bounds, float clip,
                          int q, const float* x, int64_t tokens, const float* bias, float* y, int64_t* step_counter,
                          void* stream);

/* Backward of coset_e8_qat_fwd_theta: dW and dbeta as coset_e8_qat_bwd, plus
 * dtheta[t] = dbeta[t] * dbeta_dtheta[t] (the factor the forward recorded). */
int coset_e8_qat_bwd_theta(const void* gWq, int g_dtype, const float* W, const void* packed, const float* beta,
                           const float* dbeta_dtheta, int64_t rows, int64_t cols, int64_t blocks_per_tile,
                           float clip, int q, int M, float* dW, float* dbeta, float* dtheta, void* stream);

/* Bias gradient of the layer's product (F.linear in HNLQLinearQAT.forward,
 * coset/core/layers.py:478, whose autograd sums the output gradient over the
 * tokens): out[c] = sum_t g[t, c] for g [rows, cols] (fp32, bf16 or fp16,
 * cols % 8 == 0, 16-byte aligned), accumulated in fp32 in a fixed order
 * (deterministic).  workspace: caller-owned fp32 scratch of
 * coset_colsum_workspace_floats(rows, cols) floats. */
int64_t coset_colsum_workspace_floats(int64_t rows, int64_t cols);
int coset_colsum(const void* g, int dtype, int64_t rows, int64_t cols, float* out, float* workspace,
                 int64_t workspace_floats, void* stream);

/* Weight gradient of the layer's product (F.linear in HNLQLinearQAT.forward,
 * coset/core/layers.py:478, whose autograd forms grad_weight = gy^T x):
 * C[M, N] = A^T B for A = gy [K, M] and B = x [K, N], bf16, row-major with
 * leading dimensions lda, ldb (elements), accumulated in fp32 in a fixed
 * order (deterministic); C [M, N] (leading dimension ldc) in fp32
 * (out_dtype COSET_F32) or bf16 rounded to nearest even (COSET_BF16).  Shapes
 * the kernel takes (coset_gemm_tn_supported returns 1 for them): M and N
 * multiples of 64 with (M / 64) (N / 64) <= 256 (64 x 64 output tiles), or
 * else multiples of 96 with (M / 96) (N / 96) <= 256 (96 x 96 tiles), and
 * K = 256 s m for a power of two s (the K splits the launch plan picks) and
 * m in {4, 8, 16, 32} (e.g. K = 1024 .. 8192 in powers of two); others
 * return COSET_EUNSUPPORTED -- larger products are the library GEMM's
 * (COSET_OPT_GEMM_TN_TILE restricts the plan to one tile size).  Buffers
 * 16-byte aligned, lda, ldb, ldc multiples of 8.  colsum (nullable): also
 * colsum[m] = sum_k A[k, m], fp32, fixed order -- with A = gy, the bias
 * gradient of the same F.linear, in the same pass.  workspace: caller-owned
 * fp32 scratch of coset_gemm_tn_workspace_floats(M, N, K) floats (the split-K
 * partials; 0 when the launch plan has none, and workspace may then be
 * NULL). */
int coset_gemm_tn_supported(int64_t M, int64_t N, int64_t K);
int64_t coset_gemm_tn_workspace_floats(int64_t M, int64_t N, int64_t K);
int coset_gemm_tn(const void* A, int64_t lda, const void* B, int64_t ldb, void* C, int64_t ldc, int out_dtype,
                  int64_t M, int64_t N, int64_t K, float* colsum, float* workspace, int64_t workspace_floats,
                  void* stream);

/* The layer's periodic statistics update (HNLQLinearQAT._gather_stats,
 * coset/core/layers.py:366-379, run every stat_update_interval steps at
 * layers.py:408-413) over `tiles` tiles of tile_size contiguous fp32 weights
 * (row tiling: tile_size = in_features; block tiling: 8):
 *   sigma_ema[t] = sigma_ema[t] * m + (1 - m) * (std(tile) + 1e-8)
 *   xmax_ema[t]  = xmax_ema[t]  * m + (1 - m) * (max |tile| + 1e-8)
 * std unbiased; the reference's CPU arithmetic: variance in double, its
 * square root rounded once to fp32, the EMA in fp32 with m and 1 - m rounded
 * to fp32. */
int coset_qat_stats_update(const float* W, int64_t tiles, int64_t tile_size, double momentum, float* sigma_ema,
                           float* xmax_ema, void* stream);

/* One-sided vLUTs (coset/legacy/quant/vlut.py:72-117): for each query
 * a[i, 0:8] writes vlut[i, idx] = <a, r(b_idx)> for all q^8 level words in
 * lexicographic order, r(b) = G b - q P(G b / q).  legacy=1 uses the legacy
 * textbook P (what vLUTManager uses), legacy=0 the core rule of e8_decode.
 * q in [2, 8]. */
int coset_vlut_build_one_sided(const float* queries, int64_t n_queries, int q, int legacy, float* vlut,
                               void* stream);

/* out[i] = sum_m q^m vlut[words[i, m]] (tests/legacy/test_one_sided_vlut_pytest.py:22-43). */
int coset_vlut_lookup_dot(const void* words, int64_t n_blocks, int q, int M, const float* vlut, float* out,
                          void* stream);

/* Weight formats of coset_vlut_matmul (word_format):
 *   0  the uint16 level words [rows, K/8, M] as encoded (q^8 <= 65536)
 *   1  row-major prepared: uint32 cid << 16 | idx, same shape, cid the id of
 *      the coarse point c(b) the word decodes through, so the matmul reads it
 *      instead of gathering from the per-device map
 *   2  tiled prepared: the format-1 values in matrix-core fragment order:
 *      tiles of 16 rows x 4 k-blocks, tile (row / 16, kb / 4) at index
 *      (row / 16) * ceil(kb_total / 4) + kb / 4, 64 entries per tile (entry
 *      row % 16 + 16 * (kb % 4)) of M words each; rows are padded to 16 and
 *      k-blocks to 4 with the word 0, which decodes to 0.
 *   3  decoded: the same tile order with, per entry, the 8 bytes
 *      2 x_hat + 128 of the pair's M-level decode (two uint32, coordinates
 *      0-3 then 4-7; padding decodes to 0): the weight decoded once, at the
 *      footprint of format 2 for M = 2, so the matmul reads no tables.
 *      q = 4 with M <= 2 or q = 2 with M <= 4 (|2 x_hat| <= 127); matrix-core
 *      method only.
 *   4  pairs: each level word replaced by the ids of its residual's four
 *      coordinate pairs (r_2p, r_2p+1), one byte each (at most 72 distinct
 *      values per pair), the entries the LDS-table method looks up, laid out
 *      [ceil(rows / 64)][kb][M][64 rows] (padding rows hold the ids of word
 *      0, which decodes to 0); that method only (method 0 selects it).
 *   5  decoded6: the decode of format 3 in 6 bytes per pair (12.6 MB at
 *      4096 x 4096 against 16.8 MB).  2 x_hat lies in E8, so its coordinates
 *      share one parity p: coordinate j is stored as the 6-bit field
 *      f_j = floor(2 x_hat_j / 2) + off (f_7 < 32), off = 18 for q = 4, M = 2
 *      (core or legacy rule; other q, M where the ranges fit, else the
 *      prepare call returns COSET_EUNSUPPORTED).  Byte i (0-5) of a pair
 *      holds f_i in bits 0-5; bits 6-7 of bytes 0-2 hold f_6 (2 bits each,
 *      low first) and those of bytes 3-5 hold f_7 | p << 5.  Layout: [ceil(rows / 16)][ceil(kb / 32)][64
 *      lanes][8 pairs x 6 bytes]: lane row % 16 + 16 (kb % 4), pair
 *      (kb / 4) % 8, so a lane reads a chunk of 8 k-quads as three 16-byte
 *      loads; padding holds x_hat = 0.  Matrix-core method, rows (B <= 32)
 *      and deep (B > 32) kernels.
 * coset_vlut_prepared_words gives the uint32 count of a format; prepare
 * (once per weight) converts format-0 words [rows, kb, M] into format 1, 2,
 * 3, 4 or 5 for the core rule (legacy = 0) or the legacy one. */
int64_t coset_vlut_prepared_words(int64_t rows, int64_t kb, int M, int word_format);
int coset_vlut_prepare(const void* words, int64_t rows, int64_t kb, int M, int q, int legacy, int word_format,
                       uint32_t* prepared, void* stream);

/* vLUT matmul: out[t, o] = s_o * sum_k sum_m q^m vLUT_{act[t, 8k:8k+8]}[words[o, k, m]]
 * for level words of q in {2, 4}, M <= 4 in any word_format above (a
 * prepared format with the legacy flag it was prepared with), activations
 * [B, K] fp32/bf16/fp16, s_o = scale[o] (scale_mode 0), 1/scale[o] (1) or 1
 * (scale NULL).  method 1 keeps a per-(token, k-block) inner-product table in
 * LDS, factorized over the coordinate pairs of r: <a, r(b)> = sum_p
 * <(a_2p, a_2p+1), r_p(b)>, four lookups per level word (any activation
 * dtype); method 2 decodes 2*x_hat and runs the product on the matrix cores
 * (fp16/bf16 activations holding 2*x_hat exactly; fp32 activations as three
 * bf16 planes, a = h1 + h2 + h3 exactly, multiplied as 3B tokens and summed
 * per output, where bf16 holds 2*x_hat exactly); 0 picks 2 when it is
 * exact, and 1 for format 4.  workspace: caller-owned fp32 scratch of
 * coset_vlut_workspace_floats floats (0 is a valid size; query with method 1
 * for format 4).
 * The reference has no matmul routine; its placeholder QLinear._lut_matmul is
 * coset/legacy/nn/qlinear.py:272-281. */
int64_t coset_vlut_workspace_floats(int64_t B, int64_t rows, int64_t K, int q, int M, int act_dtype, int method);
int coset_vlut_matmul(const void* words, int word_format, const float* scale, int scale_mode, const void* act,
                      int act_dtype, int64_t B, int64_t rows, int64_t K, int q, int M, int legacy, int method,
                      float* workspace, int64_t workspace_floats, float* out, void* stream);

/* coset_vlut_matmul without a workspace argument, for callers that cannot
 * allocate (code under HIP graph capture, tight serving loops, harnesses
 * that forbid hipMalloc).  No counterpart in the reference (whose vLUT path
 * is Python on the CPU).  It allocates nothing: the split-K partials go to a
 * fixed per-device scratch array of coset_vlut_noalloc_scratch_floats()
 * floats (8 MiB), whose address coset_init(device) looks up once per device;
 * call coset_init on each device first (it also builds the decode tables,
 * which this entry point never builds).  A launch plan needing more scratch
 * is refused with COSET_EINVAL.  Every call on a device shares that
 * device's array: calls that overlap on one GPU (two streams at once) race
 * on it; calls on one stream are ordered and safe.  Nothing in the array
 * needs to start at zero (each launch writes every partial it reads). */
int64_t coset_vlut_noalloc_scratch_floats(void);
int coset_vlut_matmul_noalloc(const void* words, int word_format, const float* scale, int scale_mode,
                              const void* act, int act_dtype, int64_t B, int64_t rows, int64_t K, int q, int M,
                              int legacy, int method, float* out, void* stream);

/* Measurement probes (no counterpart in the reference: the floors bench.py
 * sets the kernels above against).
 *   coset_probe_empty: a launch of grid x threads with lds_bytes of LDS that
 *     does no work (out is never written) -- the cost of one launch.
 *   coset_probe_read: reads `bytes` (a multiple of 16) from src into
 *     registers at that launch shape, every load issued before any is used,
 *     and writes one uint32 per workgroup to out[grid] -- the floor of a
 *     kernel that reads a weight format of that size.
 *   coset_probe_c2_stream: the C2 round trip's kernel (coset_e8_hnlq_roundtrip
 *     at q = 4, M = 2, fp32, no scale) with its launch, tile schedule, loads
 *     and stores but no lattice arithmetic: out = x, packed[i] = the XOR of
 *     block i's eight words (staged != 0: with its decode-table staging) --
 *     the streaming ceiling of that access pattern.
 *   coset_probe_valu: `grid` 512-thread workgroups whose waves each run
 *     `iters` x 8 steps of eight independent VALU chains -- kind 0 fp32 FMA
 *     (64 v_fma_f32 per iteration), 1 compare + select (64 v_cmp_lt_f32 and
 *     64 v_cndmask_b32) -- and write one float per thread to out[grid * 512]:
 *     the sustained VALU issue rate of this part (wave instructions per SIMD
 *     per second = waves x instructions per wave / SIMDs / time). */
int coset_probe_empty(int grid, int threads, int lds_bytes, uint32_t* out, void* stream);
int coset_probe_read(const void* src, int64_t bytes, int grid, int threads, uint32_t* out, void* stream);
int coset_probe_c2_stream(const float* x, int64_t n_blocks, uint32_t* packed, float* out, int staged, void* stream);
int coset_probe_valu(int kind, int grid, int iters, float* out, void* stream);

/* D4 lattice operator over n_blocks fp32 [n, 4] blocks (coset/core/d4/lattice.py:62-146,
 * coset/core/base.py:134-176): COSET_OP_G_X, COSET_OP_PROJECT (closest point,
 * the reference's rule), COSET_OP_ENCODE_COORDS (round(G^-1 x) mod q),
 * COSET_OP_DECODE_COORDS (G b).  custom_round is elementwise: use
 * coset_e8_lattice_op. */
int coset_d4_lattice_op(int op, const float* in, int64_t n_blocks, int q, float* out, void* stream);

/* The D4 layer's weight quantizer (create_d4_hnlq_linear,
 * coset/core/d4/layers.py:14-68, which quantizes by projection only, with
 * HNLQLinearQAT._quantize_weights, coset/core/layers.py:428-463):
 *   Wq = clamp(P_D4(W * beta_t) / beta_t, -clip, clip)
 * W fp32 [rows, cols] (cols % 4 == 0), beta_t per tile of blocks_per_tile
 * 4-wide blocks (cols/4: row tiling, 1: block tiling); Wq fp32 or bf16. */
int coset_d4_qat_fwd(const float* W, int64_t rows, int64_t cols, const float* beta, int64_t blocks_per_tile,
                     float clip, void* Wq, int wq_dtype, void* stream);

/* Same with beta derived from theta and the EMA buffers as in
 * coset_e8_qat_fwd_theta (q and M_bounds give the bounds' q^M), writing the
 * beta used, d beta / d theta and incrementing step_counter (nullables). */
int coset_d4_qat_fwd_theta(const float* W, int64_t rows, int64_t cols, int64_t blocks_per_tile, const float* theta,
                           const float* sigma_ema, const float* xmax_ema, double delta0, double eta,
                           double gamma_inv, int q, int M_bounds, float clip, void* Wq, int wq_dtype,
                           float* beta_out, float* dbeta_dtheta_out, int64_t* step_counter, void* stream);

/* Backward of either forward (P recomputed from W and beta):
 *   dW = ((g m) / beta) beta, m = (-clip <= P/beta <= clip),
 *   dbeta[t] = sum_t ((g m) / beta) W - (g m) ((P / beta) / beta),
 * and with dbeta_dtheta non-NULL dtheta[t] = dbeta[t] * dbeta_dtheta[t]. */
int coset_d4_qat_bwd(const void* gWq, int g_dtype, const float* W, const float* beta, const float* dbeta_dtheta,
                     int64_t rows, int64_t cols, int64_t blocks_per_tile, float clip, float* dW, float* dbeta,
                     float* dtheta, void* stream);

/* LSQ activation quantizer forward (LSQActivation.forward with ste_clip and
 * ste_round, coset/core/layers.py:117-137, 20-26), over n values of x
 * (COSET_F32, COSET_BF16 or COSET_F16), computed in fp32 in the reference's
 * operation order and written once in x's dtype:
 *   a = relu(alpha) + 1e-8, s = a / qmax,
 *   out = ((y - y) + round(y)) * s,  y = ((x - x) + clamp(x, -a, a)) / s.
 * alpha: device pointer to the fp32 parameter (read on the device). */
int coset_lsq_fwd(const void* x, int dtype, int64_t n, const float* alpha, int qmax, void* out, void* stream);

/* Its backward (the autograd of the same chain): dx = (g s) / s in x's dtype
 * and d_alpha[0] = relu(alpha) > 0 ? (sum g yq - sum (g s)((xc / s) / s)) / qmax
 * : 0, written (not accumulated), summed in a fixed order through a
 * caller-owned workspace of coset_lsq_workspace_floats(n) floats. */
int64_t coset_lsq_workspace_floats(int64_t n);
int coset_lsq_bwd(const void* x, const void* g, int dtype, int64_t n, const float* alpha, int qmax, void* dx,
                  float* d_alpha, float* workspace, int64_t workspace_floats, void* stream);

/* coset_vlut_matmul with the layer's epilogue fused into the output write:
 * out = actq(matmul + bias[o]), the value of HNLQLinearQAT.forward
 * (F.linear then the LSQ activation quantizer, coset/core/layers.py:472-484).
 * bias: [rows] fp32 or NULL; lsq_alpha: device pointer to the LSQ parameter
 * (as coset_lsq_fwd, fp32 result) or NULL for no activation quantizer. */
int coset_vlut_linear(const void* words, int word_format, const float* scale, int scale_mode, const void* act,
                      int act_dtype, int64_t B, int64_t rows, int64_t K, int q, int M, int legacy, int method,
                      const float* bias, const float* lsq_alpha, int lsq_qmax, float* workspace,
                      int64_t workspace_floats, float* out, void* stream);

/* Elementwise lattice operator over n_blocks fp32 blocks (custom_round is
 * applied to all 8*n_blocks values).  legacy selects the legacy g_x rule. */
int coset_e8_lattice_op(int op, int legacy, const float* in, int64_t n_blocks, int q,
                        float* out, void* stream);

#ifdef __cplusplus
}
#endif

#endif
