/*
 * e8_oracle.c -- CPU restatement of the reference E8 HNLQ path.
 *
 * TEST INFRASTRUCTURE ONLY (parity checker; never linked into the product).
 * Build: oracle/Makefile (gcc -O2 -ffp-contract=off, no fast-math) so that
 * every fp32 operation below is a single IEEE RNE operation, exactly like the
 * PyTorch CPU kernels the reference runs.
 *
 * Reference semantics being restated (paths relative to the mlsquare/coset
 * tree):
 *   custom_round        coset/core/base.py:179-202
 *   g_x (core)          coset/core/e8/lattice.py:67-112   (else-branch is -1)
 *   g_x (legacy)        coset/legacy/lattices/e8.py:41-68 (flip toward x)
 *   projection / Q      coset/core/e8/lattice.py:114-169, legacy e8.py:70-103
 *   encode_coords       coset/core/base.py:134-154
 *   decode_coords       coset/core/base.py:156-176
 *   e8_encode           coset/core/e8/codecs.py:17-89
 *   _full_decode        coset/core/e8/codecs.py:139-180
 *   layer quantization  coset/core/layers.py:428-463
 *   one-sided vLUT      coset/legacy/quant/vlut.py:72-156, 217-238
 *   D4 g_x / projection coset/core/d4/lattice.py:62-146
 *   D4 layer quantizer  coset/core/d4/layers.py:46-47 with layers.py:428-463
 */
#include "e8_oracle.h"

#include <math.h>
#include <string.h>

#define EPS_F32 1.1920928955078125e-07f /* torch.finfo(torch.float32).eps */

/* Generator matrix G (columns are the basis vectors listed as rows at
 * coset/core/e8/lattice.py:32-41) and its exact inverse. */
static const float G[8][8] = {
    {2.f, -1.f, 0.f, 0.f, 0.f, 0.f, 0.f, .5f},
    {0.f, 1.f, -1.f, 0.f, 0.f, 0.f, 0.f, .5f},
    {0.f, 0.f, 1.f, -1.f, 0.f, 0.f, 0.f, .5f},
    {0.f, 0.f, 0.f, 1.f, -1.f, 0.f, 0.f, .5f},
    {0.f, 0.f, 0.f, 0.f, 1.f, -1.f, 0.f, .5f},
    {0.f, 0.f, 0.f, 0.f, 0.f, 1.f, -1.f, .5f},
    {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 1.f, .5f},
    {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, .5f},
};
static const float GINV[8][8] = {
    {.5f, .5f, .5f, .5f, .5f, .5f, .5f, -3.5f},
    {0.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, -6.f},
    {0.f, 0.f, 1.f, 1.f, 1.f, 1.f, 1.f, -5.f},
    {0.f, 0.f, 0.f, 1.f, 1.f, 1.f, 1.f, -4.f},
    {0.f, 0.f, 0.f, 0.f, 1.f, 1.f, 1.f, -3.f},
    {0.f, 0.f, 0.f, 0.f, 0.f, 1.f, 1.f, -2.f},
    {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 1.f, -1.f},
    {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 2.f},
};

float or_custom_round(float x)
{
    /* y = x - sign(x) * eps ; floor(y + 0.5) */
    float s = (x > 0.f) ? 1.f : ((x < 0.f) ? -1.f : 0.f);
    float nudge = s * EPS_F32;
    float y = x - nudge;
    float t = y + 0.5f;
    return floorf(t);
}

/* First index of the maximum, like torch.argmax. */
static int first_argmax8(const float* d)
{
    int k = 0;
    float m = d[0];
    for (int i = 1; i < 8; ++i) {
        if (d[i] > m) {
            m = d[i];
            k = i;
        }
    }
    return k;
}

void or_g_x(const float* x, int legacy, float* out)
{
    float f[8], delta[8];
    for (int i = 0; i < 8; ++i) {
        f[i] = or_custom_round(x[i]);
        delta[i] = fabsf(x[i] - f[i]);
    }
    int k = first_argmax8(delta);
    memcpy(out, f, sizeof f);
    float xk = x[k], fk = f[k];
    int up;
    if (xk >= 0.f)
        up = fk < xk;
    else
        up = legacy ? (fk <= xk) : 0; /* core: every negative x_k takes -1 */
    out[k] = up ? fk + 1.f : fk - 1.f;
}

/* torch.sum(f) % 2 == 0 for integer-valued f (exact). */
static int even_sum8(const float* f)
{
    float s = 0.f;
    for (int i = 0; i < 8; ++i) s += f[i];
    double r = fmod((double)s, 2.0);
    return r == 0.0;
}

/* torch.norm(x - y, dim=-1) over 8 fp32.  A contiguous row (torch's
 * last-dim fast path) sums the rounded squares in order; a strided row (the
 * transposed view decode_coords returns, coset/core/base.py:176) goes through
 * the generic reduction, which accumulates acc = fma(e, e, acc) in order.
 * Both end in a correctly rounded sqrt. */
static float dist8(const float* x, const float* y, int strided)
{
    float acc = 0.f;
    for (int i = 0; i < 8; ++i) {
        float e = x[i] - y[i];
        if (strided) {
            acc = fmaf(e, e, acc);
        } else {
            float sq = e * e;
            acc = acc + sq;
        }
    }
    return sqrtf(acc);
}

static void project1(const float* x, int legacy, int strided, float* out)
{
    float f0[8], y0[8], xs[8], f1[8], y1[8];
    for (int i = 0; i < 8; ++i) f0[i] = or_custom_round(x[i]);
    if (even_sum8(f0))
        memcpy(y0, f0, sizeof y0);
    else
        or_g_x(x, legacy, y0);

    for (int i = 0; i < 8; ++i) xs[i] = x[i] - 0.5f;
    for (int i = 0; i < 8; ++i) f1[i] = or_custom_round(xs[i]);
    if (even_sum8(f1)) {
        for (int i = 0; i < 8; ++i) y1[i] = f1[i] + 0.5f;
    } else {
        float g1[8];
        or_g_x(xs, legacy, g1);
        for (int i = 0; i < 8; ++i) y1[i] = g1[i] + 0.5f;
    }
    float d0 = dist8(x, y0, strided);
    float d1 = dist8(x, y1, strided);
    if (d0 < d1)
        memcpy(out, y0, sizeof y0);
    else
        memcpy(out, y1, sizeof y1);
}

void or_projection(const float* x, int64_t n, int legacy, float* y)
{
    for (int64_t i = 0; i < n; ++i) project1(x + 8 * i, legacy, 0, y + 8 * i);
}

static int pymod_int(double v, int q)
{
    double r = fmod(v, (double)q);
    if (r < 0) r += q;
    return (int)r;
}

static void encode_coords1(const float* y, int q, int32_t* b)
{
    for (int r = 0; r < 8; ++r) {
        double acc = 0.0; /* exact: entries are in (1/2)Z with small magnitude */
        for (int c = 0; c < 8; ++c) acc += (double)GINV[r][c] * (double)y[c];
        b[r] = pymod_int(nearbyint(acc), q);
    }
}

void or_encode_coords(const float* y, int64_t n, int q, int32_t* b)
{
    for (int64_t i = 0; i < n; ++i) encode_coords1(y + 8 * i, q, b + 8 * i);
}

static void decode_coords1(const int32_t* b, float* y)
{
    for (int r = 0; r < 8; ++r) {
        double acc = 0.0;
        for (int c = 0; c < 8; ++c) acc += (double)G[r][c] * (double)b[c];
        y[r] = (float)acc;
    }
}

void or_decode_coords(const int32_t* b, int64_t n, float* y)
{
    for (int64_t i = 0; i < n; ++i) decode_coords1(b + 8 * i, y + 8 * i);
}

uint32_t or_pack_index(const int32_t* b, int q)
{
    uint32_t idx = 0;
    for (int j = 0; j < 8; ++j) idx = idx * (uint32_t)q + (uint32_t)b[j];
    return idx;
}

void or_unpack_index(uint32_t idx, int q, int32_t* b)
{
    for (int j = 7; j >= 0; --j) {
        b[j] = (int32_t)(idx % (uint32_t)q);
        idx /= (uint32_t)q;
    }
}

void or_residual(const int32_t* b, int q, int legacy, int strided, float* r)
{
    float gb[8], z[8], c[8];
    decode_coords1(b, gb);
    float qf = (float)q;
    for (int i = 0; i < 8; ++i) z[i] = gb[i] / qf;
    project1(z, legacy, strided, c);
    for (int i = 0; i < 8; ++i) r[i] = gb[i] - qf * c[i];
}

static void encode1(const float* xs, int q, int M, int32_t* codes)
{
    float xl[8], y[8];
    memcpy(xl, xs, sizeof xl);
    float qf = (float)q;
    for (int m = 0; m < M; ++m) {
        project1(xl, 0, 0, y);
        encode_coords1(y, q, codes + 8 * m);
        for (int i = 0; i < 8; ++i) xl[i] = xl[i] / qf;
    }
}

static void decode1(const int32_t* codes, int q, int M, int strided, float* acc)
{
    for (int i = 0; i < 8; ++i) acc[i] = 0.f;
    float w = 1.f;
    for (int m = 0; m < M; ++m) {
        float r[8];
        or_residual(codes + 8 * m, q, 0, strided, r);
        for (int i = 0; i < 8; ++i) acc[i] = acc[i] + w * r[i];
        w = w * (float)q;
    }
}

void or_e8_encode(const float* x, int64_t n, float beta, int q, int M, int32_t* codes)
{
    for (int64_t i = 0; i < n; ++i) {
        float xs[8];
        for (int j = 0; j < 8; ++j) xs[j] = x[8 * i + j] / beta;
        encode1(xs, q, M, codes + (size_t)8 * M * i);
    }
}

void or_e8_decode(const int32_t* codes, int64_t n, float beta, int q, int M, float* out)
{
    for (int64_t i = 0; i < n; ++i) {
        float acc[8];
        decode1(codes + (size_t)8 * M * i, q, M, n > 1, acc);
        for (int j = 0; j < 8; ++j) out[8 * i + j] = acc[j] * beta;
    }
}

void or_layer_quant(const float* W, int64_t rows, int64_t cols, const float* beta_row,
                    int q, int M, float clip, float* Wq, float* qraw, int32_t* codes)
{
    int64_t bpr = cols / 8;
    for (int64_t r = 0; r < rows; ++r) {
        float beta = beta_row[r];
        for (int64_t k = 0; k < bpr; ++k) {
            int64_t blk = r * bpr + k;
            const float* w = W + r * cols + 8 * k;
            float xs[8], acc[8];
            int32_t c[8 * 16];
            for (int j = 0; j < 8; ++j) xs[j] = w[j] * beta;
            encode1(xs, q, M, c);
            decode1(c, q, M, rows * bpr > 1, acc);
            for (int j = 0; j < 8; ++j) {
                float v = acc[j] / beta;
                if (qraw) qraw[8 * blk + j] = acc[j];
                if (v < -clip) v = -clip;
                if (v > clip) v = clip;
                Wq[8 * blk + j] = v;
            }
            if (codes) memcpy(codes + (size_t)8 * M * blk, c, sizeof(int32_t) * 8 * M);
        }
    }
}

void or_build_one_sided_vlut(const float* a, int q, int legacy, float* vlut)
{
    uint32_t n = 1;
    for (int j = 0; j < 8; ++j) n *= (uint32_t)q;
    for (uint32_t i = 0; i < n; ++i) {
        int32_t b[8];
        float r[8];
        or_unpack_index(i, q, b);
        or_residual(b, q, legacy, 0, r);
        double acc = 0.0;
        for (int j = 0; j < 8; ++j) acc += (double)a[j] * (double)r[j];
        vlut[i] = (float)acc;
    }
}

void or_residual_table(int q, int legacy, int strided, float* R)
{
    uint32_t n = 1;
    for (int j = 0; j < 8; ++j) n *= (uint32_t)q;
    for (uint32_t i = 0; i < n; ++i) {
        int32_t b[8];
        or_unpack_index(i, q, b);
        or_residual(b, q, legacy, strided, R + 8 * (size_t)i);
    }
}

void or_vlut_onesided_accumulate(const uint32_t* words, int64_t rows, int64_t kb_total, int M, int q,
                                 const float* R, const float* a, int64_t kb0, int64_t kb1, float* table,
                                 double* acc)
{
    uint32_t n = 1;
    for (int j = 0; j < 8; ++j) n *= (uint32_t)q;
    for (int64_t k = kb0; k < kb1; ++k) {
        const float* ak = a + 8 * k;
        for (uint32_t i = 0; i < n; ++i) {
            const float* r = R + 8 * (size_t)i;
            float s = 0.0f;
            for (int j = 0; j < 8; ++j) s += ak[j] * r[j];
            table[i] = s;
        }
        for (int64_t o = 0; o < rows; ++o) {
            const uint32_t* w = words + (o * kb_total + k) * M;
            double v = 0.0, qm = 1.0;
            for (int m = 0; m < M; ++m) {
                v += qm * (double)table[w[m]];
                qm *= q;
            }
            acc[o] += v;
        }
    }
}

void or_vlut_matmul(const uint32_t* words, const float* scale, int scale_mode,
                    const float* act, int64_t B, int64_t rows, int64_t K,
                    int q, int M, int legacy, float* out)
{
    int64_t kb = K / 8;
    for (int64_t o = 0; o < rows; ++o) {
        for (int64_t t = 0; t < B; ++t) {
            double acc = 0.0;
            for (int64_t k = 0; k < kb; ++k) {
                const float* a = act + t * K + 8 * k;
                double w = 1.0;
                for (int m = 0; m < M; ++m) {
                    int32_t b[8];
                    float r[8];
                    or_unpack_index(words[(o * kb + k) * M + m], q, b);
                    or_residual(b, q, legacy, !legacy, r);
                    double d = 0.0;
                    for (int j = 0; j < 8; ++j) d += (double)a[j] * (double)r[j];
                    acc += w * d;
                    w *= q;
                }
            }
            double s = scale_mode == 0 ? (double)scale[o] : 1.0 / (double)scale[o];
            out[t * rows + o] = (float)(acc * s);
        }
    }
}

/* ---------------------------------------------------------------- legacy
 * Hierarchical encode/decode of coset/legacy/quant/functional.py (the
 * paper's Algorithms 1 and 2), one 8-vector at a time as the reference. */

/* _encode_internal (functional.py:83-116): y = Q(x_l), b = coords(y),
 * x_l = y / q for M levels with the legacy Q; overload = Q(x_M) != 0
 * (allclose to 0 at atol 1e-8 on lattice points). */
static int legacy_chain(const float* xs, int q, int M, int32_t* codes)
{
    float xl[8], y[8];
    memcpy(xl, xs, sizeof xl);
    for (int m = 0; m < M; ++m) {
        project1(xl, 1, 0, y);
        encode_coords1(y, q, codes + 8 * m);
        for (int i = 0; i < 8; ++i) xl[i] = y[i] / (float)q;
    }
    project1(xl, 1, 0, y);
    for (int i = 0; i < 8; ++i)
        if (!(fabsf(y[i]) <= 1e-8f)) return 1;  /* NaN also fails allclose */
    return 0;
}

/* encode (functional.py:15-80): xs = x / beta (+ dither), then while
 * overload and t < max_iter (protect only): xs = xs / two_alpha, t += 1.
 * codes [n, M, 8]; T [n]; overload [n] = the final chain's flag. */
void or_legacy_encode(const float* x, int64_t n, float beta, float two_alpha, int max_iter, int protect,
                      const float* dither, int64_t dither_stride, int q, int M, int32_t* codes, int32_t* T,
                      uint8_t* overload)
{
    for (int64_t b = 0; b < n; ++b) {
        float xs[8];
        for (int i = 0; i < 8; ++i) {
            xs[i] = x[8 * b + i] / beta;
            if (dither) xs[i] = xs[i] + dither[dither_stride * b + i];
        }
        int t = 0;
        int ov = legacy_chain(xs, q, M, codes + (size_t)b * M * 8);
        while (protect && ov && t < max_iter) {
            ++t;
            for (int i = 0; i < 8; ++i) xs[i] = xs[i] / two_alpha;
            ov = legacy_chain(xs, q, M, codes + (size_t)b * M * 8);
        }
        T[b] = t;
        overload[b] = (uint8_t)ov;
    }
}

/* decode (functional.py:119-181): x_hat = sum_i q^i (G b_i - q Q(G b_i / q))
 * accumulated in fp32 from zero, minus dither, then (beta * x_hat) * s_T
 * with s_T = (float)2^(alpha T) (scale_T[T[b]]). */
void or_legacy_decode(const int32_t* codes, const int32_t* T, int64_t n, float beta, const float* scale_T,
                      const float* dither, int64_t dither_stride, int q, int M, float* out)
{
    for (int64_t b = 0; b < n; ++b) {
        float acc[8] = {0};
        float w = 1.f;
        for (int m = 0; m < M; ++m) {
            float r[8];
            or_residual(codes + ((size_t)b * M + m) * 8, q, 1, 0, r);
            for (int i = 0; i < 8; ++i) acc[i] = acc[i] + w * r[i];
            w = w * (float)q;
        }
        for (int i = 0; i < 8; ++i) {
            float v = acc[i];
            if (dither) v = v - dither[dither_stride * b + i];
            out[8 * b + i] = (beta * v) * scale_T[T[b]];
        }
    }
}

/* ------------------------------------------------------------------ D4 */

/* D4 g_x (coset/core/d4/lattice.py:62-111): the first coordinate farthest
 * from its rounding moves +1 when x_k >= 0 and f_k < x_k, -1 otherwise. */
void or_d4_g_x(const float* x, float* out)
{
    float f[4], delta[4];
    for (int i = 0; i < 4; ++i) {
        f[i] = or_custom_round(x[i]);
        delta[i] = fabsf(x[i] - f[i]);
    }
    int k = 0;
    for (int i = 1; i < 4; ++i)
        if (delta[i] > delta[k]) k = i;
    memcpy(out, f, sizeof f);
    out[k] = (x[k] >= 0.f && f[k] < x[k]) ? f[k] + 1.f : f[k] - 1.f;
}

/* D4 projection (lattice.py:113-146): custom_round(x) when torch.sum of it
 * % 2 == 0, else g_x(x). */
void or_d4_projection(const float* x, int64_t n, float* y)
{
    for (int64_t i = 0; i < n; ++i) {
        const float* xi = x + 4 * i;
        float f[4], s = 0.f;
        for (int j = 0; j < 4; ++j) {
            f[j] = or_custom_round(xi[j]);
            s += f[j];
        }
        float r = s - 2.f * floorf(s / 2.f); /* torch.remainder(s, 2) */
        if (r == 0.f)
            memcpy(y + 4 * i, f, sizeof f);
        else
            or_d4_g_x(xi, y + 4 * i);
    }
}

/* Exact inverse of the D4 generator (columns (-1,-1,0,0), (1,-1,0,0),
 * (0,1,-1,0), (0,0,1,-1)). */
static const double D4GINV[4][4] = {
    {-0.5, -0.5, -0.5, -0.5}, {0.5, -0.5, -0.5, -0.5}, {0., 0., -1., -1.}, {0., 0., 0., -1.}};

/* round(G^-1 y) mod q (coset/core/base.py:134-154) from the exact product. */
void or_d4_encode_coords(const float* y, int64_t n, int q, int32_t* b)
{
    for (int64_t i = 0; i < n; ++i)
        for (int r = 0; r < 4; ++r) {
            double c = 0.0;
            for (int j = 0; j < 4; ++j) c += D4GINV[r][j] * (double)y[4 * i + j];
            b[4 * i + r] = pymod_int(nearbyint(c), q);
        }
}

/* G b (coset/core/base.py:156-176). */
void or_d4_decode_coords(const int32_t* b, int64_t n, float* y)
{
    for (int64_t i = 0; i < n; ++i) {
        const int32_t* c = b + 4 * i;
        y[4 * i + 0] = (float)(-c[0] + c[1]);
        y[4 * i + 1] = (float)(-c[0] - c[1] + c[2]);
        y[4 * i + 2] = (float)(-c[2] + c[3]);
        y[4 * i + 3] = (float)(-c[3]);
    }
}

/* The D4 layer's weight quantization (layers.py:428-463 with d4_quantize):
 * Wq = clamp(P(W * beta_t) / beta_t, -clip, clip), beta_t per tile of
 * blocks_per_tile 4-wide blocks. */
void or_d4_layer_quant(const float* W, int64_t rows, int64_t cols, const float* beta, int64_t blocks_per_tile,
                       float clip, float* Wq)
{
    const int64_t n = rows * (cols / 4);
    for (int64_t blk = 0; blk < n; ++blk) {
        const float bt = beta[blk / blocks_per_tile];
        float x[4], p[4];
        for (int j = 0; j < 4; ++j) x[j] = W[4 * blk + j] * bt;
        or_d4_projection(x, 1, p);
        for (int j = 0; j < 4; ++j) {
            float v = p[j] / bt;
            if (v == v) v = v < -clip ? -clip : (v > clip ? clip : v);
            Wq[4 * blk + j] = v;
        }
    }
}
