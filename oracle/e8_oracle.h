/*
 * e8_oracle.h -- CPU restatement of the reference E8 HNLQ algorithm.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the parity checker for the HIP
 * product in coset_amd/.  Only tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py may load it.  The product never calls it.
 *
 * Every function follows one reference function (cited file:line, paths
 * relative to the mlsquare/coset tree) and reproduces its fp32 arithmetic
 * operation by operation: same operand order, no FMA contraction, IEEE
 * round-to-nearest-even, correctly rounded sqrt and divide.
 *
 * Code layout shared with the product: a block is 8 fp32 values; level codes
 * b in [0,q)^8 are int32 digits; the packed level word is the reference vLUT
 * index idx(b) = sum_j b_j q^(7-j) (coset/legacy/quant/vlut.py:217-238).
 */
#ifndef COSET_E8_ORACLE_H
#define COSET_E8_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* coset/core/base.py:179-202 */
float or_custom_round(float x);

/* coset/core/e8/lattice.py:67-112 (core g_x, "else -1" rule); legacy=1 selects
 * coset/legacy/lattices/e8.py:41-68 (flip toward x). */
void or_g_x(const float* x, int legacy, float* out);

/* coset/core/e8/lattice.py:114-169 (core) or coset/legacy/lattices/e8.py:70-103
 * (legacy Q) for n blocks. */
void or_projection(const float* x, int64_t n, int legacy, float* y);

/* coset/core/base.py:134-154 and 156-176 for n blocks. */
void or_encode_coords(const float* y, int64_t n, int q, int32_t* b);
void or_decode_coords(const int32_t* b, int64_t n, float* y);

/* Packed level word <-> digits. */
uint32_t or_pack_index(const int32_t* b, int q);
void or_unpack_index(uint32_t idx, int q, int32_t* b);

/* coset/core/e8/codecs.py:17-89 with LatticeConfig(beta, q, M), no dither.
 * codes: [n, M, 8] int32. */
void or_e8_encode(const float* x, int64_t n, float beta, int q, int M, int32_t* codes);

/* coset/core/e8/codecs.py:139-180: decode [n, M, 8] int32 codes.  As in the
 * reference, a batch of more than one block uses the strided-norm rule. */
void or_e8_decode(const int32_t* codes, int64_t n, float beta, int q, int M, float* out);

/* One level's residual r(b) = G b - q * P(G b / q) (codecs.py:164-166 core,
 * vlut.py:107-110 legacy).  strided=1 selects the fused-multiply-add norm of
 * the batched decode (reference e8_decode on more than one block); it only
 * changes results for q that is not a power of two. */
void or_residual(const int32_t* b, int q, int legacy, int strided, float* r);

/* Layer-convention quantize-dequantize (coset/core/layers.py:428-463 with
 * quantize_fn = e8_quantize-style encode/decode at the given M, beta 1.0):
 *   Wq = clamp(dec(enc(W * beta_row)) / beta_row, -clip, clip)
 * W is [rows, cols] fp32 row-major, cols % 8 == 0.  codes (nullable) gets
 * [rows*cols/8, M, 8].  qraw (nullable) gets the unscaled dec(enc(.)). */
void or_layer_quant(const float* W, int64_t rows, int64_t cols, const float* beta_row,
                    int q, int M, float clip, float* Wq, float* qraw, int32_t* codes);

/* coset/legacy/quant/vlut.py:72-117: vlut[i] = <a, r(b_i)> over the q^8 codes
 * in lexicographic order (last digit fastest).  Accumulates the 8-term dot in
 * double, then rounds once to fp32. */
void or_build_one_sided_vlut(const float* a, int q, int legacy, float* vlut);

/* Reference composition of the one-sided lookup (tests/legacy/
 * test_one_sided_vlut_pytest.py:22-43) across a weight matrix:
 *   out[t,o] = s_o * sum_k sum_m q^m <a[t, 8k:8k+8], r(b[o,k,m])>
 * with s_o = scale[o] (scale_mode 0: multiply) or 1/scale[o] (mode 1: divide).
 * codes: [rows, K/8, M] packed level words (uint32).  Accumulates in double. */
void or_vlut_matmul(const uint32_t* words, const float* scale, int scale_mode,
                    const float* act, int64_t B, int64_t rows, int64_t K,
                    int q, int M, int legacy, float* out);

/* All q^8 residuals r(b_i) (or_residual) in lexicographic order: R [q^8, 8]. */
void or_residual_table(int q, int legacy, int strided, float* R);

/* The one-sided vLUT method of coset/legacy/quant/vlut.py:72-117 with the
 * lookup sum of tests/legacy/test_one_sided_vlut_pytest.py:22-43, for one
 * activation row a [K] over k-blocks [kb0, kb1) of level words
 * [rows, kb_total, M]: per k-block it builds the query's table
 * T[i] = <a[8k:8k+8], R[i]> (R from or_residual_table; table: q^8 floats of
 * scratch) and adds sum_m q^m T[word[o, k, m]] to acc[o] (double).  The
 * residuals do not depend on the query, so they are computed once, not per
 * table as the reference's Python loop does.  CPU-baseline timing only. */
void or_vlut_onesided_accumulate(const uint32_t* words, int64_t rows, int64_t kb_total, int M, int q,
                                 const float* R, const float* a, int64_t kb0, int64_t kb1, float* table,
                                 double* acc);

/* coset/legacy/quant/functional.py:15-116 (encode with the overload loop,
 * the paper's Algorithm 1) for n 8-vectors: xs = x / beta (+ dither
 * [8] or [n, 8] by dither_stride 0 / 8), the chain y = Q(xs), xs = y / q
 * over M levels with the legacy Q, and while the chain overloads
 * (Q(x_M) != 0), protect is set and t < max_iter: xs /= two_alpha.
 * codes [n, M, 8]; T [n]; overload [n]: the final chain's flag. */
void or_legacy_encode(const float* x, int64_t n, float beta, float two_alpha, int max_iter, int protect,
                      const float* dither, int64_t dither_stride, int q, int M, int32_t* codes, int32_t* T,
                      uint8_t* overload);

/* coset/legacy/quant/functional.py:119-181 (decode, Algorithm 2): legacy
 * residuals summed with q^i in fp32, minus dither, times beta, times
 * scale_T[T] = (float)2^(alpha T). */
void or_legacy_decode(const int32_t* codes, const int32_t* T, int64_t n, float beta, const float* scale_T,
                      const float* dither, int64_t dither_stride, int q, int M, float* out);

/* D4 (coset/core/d4/lattice.py:62-146, d4/layers.py:46-47). */
void or_d4_g_x(const float* x, float* out);
void or_d4_projection(const float* x, int64_t n, float* y);
void or_d4_encode_coords(const float* y, int64_t n, int q, int32_t* b);
void or_d4_decode_coords(const int32_t* b, int64_t n, float* y);
void or_d4_layer_quant(const float* W, int64_t rows, int64_t cols, const float* beta, int64_t blocks_per_tile,
                       float clip, float* Wq);

#ifdef __cplusplus
}
#endif

#endif
