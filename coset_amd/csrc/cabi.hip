// cabi.hip -- extern "C" entry points of libcoset_amd.so (declared in
// include/coset_amd.h).  Validates every request on the host before any
// launch, so that a kernel only ever sees shapes its grid was sized for.
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <mutex>
#include <string>

#include "../../include/coset_amd.h"
#include "codec_kernels.hpp"
#include "gemm.hpp"
#include "legacy.hpp"
#include "probes.hpp"
#include "tables.hpp"
#include "vlut.hpp"

// Scratch of coset_vlut_matmul_noalloc: the split-K partials of the vLUT
// matmul's launch plan live in this fixed per-device array instead of a
// caller workspace.  8 MiB per device (the whole 4096 x 4096 matmul at 64
// tokens and 8 K splits fits), held until the process ends.  Host code never
// uses the name itself (in host code it is a host-side stand-in, not a
// device address): coset_init looks up each device's copy once with
// hipGetSymbolAddress and the entry point passes that address to the kernels.
constexpr int64_t kNoallocScratchFloats = (int64_t)2 << 20;
static __device__ __align__(256) float scratch[kNoallocScratchFloats];

namespace {

thread_local std::string g_last_error;

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
float* g_scratch_ptr[kMaxDevices] = {};   // per device: address of its `scratch`, set by coset_init

int fail(int code, const char* fmt, ...)
{
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    g_last_error = buf;
    return code;
}

int check_hip(hipError_t e, const char* what)
{
    if (e == hipSuccess) return COSET_OK;
    return fail(COSET_EHIP, "%s: %s", what, hipGetErrorString(e));
}

bool aligned(const void* p, size_t a) { return ((uintptr_t)p % a) == 0; }

int check_qm(int q, int M)
{
    if (q < 2 || q > 16) return fail(COSET_EINVAL, "q=%d outside [2,16]", q);
    if (M < 1 || M > coset::kMaxM) return fail(COSET_EINVAL, "M=%d outside [1,%d]", M, coset::kMaxM);
    return COSET_OK;
}

int check_scale(int scale_mode, float beta, const float* beta_row, int64_t blocks_per_row,
                int64_t n)
{
    switch (scale_mode) {
    case COSET_SCALE_NONE: return COSET_OK;
    case COSET_SCALE_CODEC:
        if (!(beta > 0.f)) return fail(COSET_EINVAL, "beta must be positive (got %g)", (double)beta);
        return COSET_OK;
    case COSET_SCALE_LAYER:
        if (!beta_row) return fail(COSET_EINVAL, "layer scaling needs beta_row");
        if (blocks_per_row <= 0 || n % blocks_per_row != 0)
            return fail(COSET_EINVAL, "n_blocks=%lld is not a multiple of blocks_per_row=%lld",
                        (long long)n, (long long)blocks_per_row);
        return COSET_OK;
    default: return fail(COSET_EINVAL, "unknown scale_mode %d", scale_mode);
    }
}

int check_dtype(int dt, const char* what)
{
    if (dt != COSET_F32 && dt != COSET_BF16)
        return fail(COSET_EUNSUPPORTED, "%s dtype %d not supported (fp32, bf16)", what, dt);
    return COSET_OK;
}

}  // namespace

extern "C" {

int coset_abi_version(void) { return COSET_ABI_VERSION; }

const char* coset_last_error(void) { return g_last_error.c_str(); }

int coset_word_bytes(int q) { return coset::word_bytes(q); }

int coset_set_option(int key, int value)
{
    switch (key) {
    case COSET_OPT_CODEC_PATH:
        if (value < 0 || value > 2) return fail(COSET_EINVAL, "codec path %d not in {0,1,2}", value);
        coset::g_codec_path = value;
        return COSET_OK;
    case COSET_OPT_VLUT_DECODE:
        if (value < 0 || value > 1) return fail(COSET_EINVAL, "vLUT decode %d not in {0,1}", value);
        coset::g_vlut_swar = value;
        return COSET_OK;
    case COSET_OPT_FAST_PROJECTION:
        if (value < 0 || value > 1) return fail(COSET_EINVAL, "fast projection %d not in {0,1}", value);
        coset::g_fast_projection = value;
        return COSET_OK;
    case COSET_OPT_CODEC_PLAIN:
        if (value < 0 || value > 1) return fail(COSET_EINVAL, "codec plain %d not in {0,1}", value);
        coset::g_codec_plain = value;
        return COSET_OK;
    case COSET_OPT_CODEC_DYNAMIC:
        if (value < 0 || value > 1) return fail(COSET_EINVAL, "codec dynamic %d not in {0,1}", value);
        coset::g_codec_dynamic = value;
        return COSET_OK;
    case COSET_OPT_VLUT_SPLITS:
        if (value < 0) return fail(COSET_EINVAL, "vLUT splits %d < 0", value);
        coset::g_vlut_splits = value;
        return COSET_OK;
    case COSET_OPT_VLUT_DEEP:
        if (value < 0 || value > 1) return fail(COSET_EINVAL, "vLUT deep %d not in {0,1}", value);
        coset::g_vlut_deep = value;
        return COSET_OK;
    case COSET_OPT_GEMM_TN_TILE:
        if (value != 0 && value != 64 && value != 96) return fail(COSET_EINVAL, "gemm_tn tile %d not in {0,64,96}", value);
        coset::g_gemm_tn_tile = value;
        return COSET_OK;
    default: return fail(COSET_EINVAL, "unknown option %d", key);
    }
}

int coset_init(int device)
{
    int cur = 0;
    hipError_t e = hipGetDevice(&cur);
    if (e != hipSuccess) return check_hip(e, "hipGetDevice");
    if (device >= 0 && device != cur && (e = hipSetDevice(device)) != hipSuccess)
        return check_hip(e, "hipSetDevice");
    int rc = COSET_OK;
    for (int q : {2, 4})
        for (int legacy : {0, 1}) {
            const coset::DecodeTables* t = nullptr;
            if (rc == COSET_OK) rc = check_hip(coset::get_decode_tables(q, legacy, &t), "decode tables");
        }
    // this device's copy of the no-allocation scratch array (looked up with
    // the device current; each device holds its own copy at its own address)
    const int dev = device >= 0 ? device : cur;
    if (rc == COSET_OK && dev < kMaxDevices) {
        std::lock_guard<std::mutex> lk(g_scratch_mu);
        if (!g_scratch_ptr[dev]) {
            float* p = nullptr;
            rc = check_hip(hipGetSymbolAddress((void**)&p, HIP_SYMBOL(scratch)), "hipGetSymbolAddress(scratch)");
            if (rc == COSET_OK) g_scratch_ptr[dev] = p;
        }
    }
    if (device >= 0 && device != cur) (void)hipSetDevice(cur);
    return rc;
}

static int codec_common(int mode, const void* x, int x_dtype, int64_t n, int scale_mode,
                        float beta, const float* beta_row, int64_t bpr, float clip,
                        const float* dither, int64_t dither_stride, int q, int M, int strided,
                        const void* packed_in, const float* codes_in, void* packed,
                        float* codes_f32, void* out, int out_dtype, void* stream)
{
    int rc;
    if (n < 0) return fail(COSET_EINVAL, "n_blocks < 0");
    if (n > (int64_t)0x7fffffff * 256) return fail(COSET_EINVAL, "n_blocks too large");
    if ((rc = check_qm(q, M))) return rc;
    if ((rc = check_scale(scale_mode, beta, beta_row, bpr, n))) return rc;
    if (mode != coset::MODE_DECODE) {
        if (n > 0 && !x) return fail(COSET_EINVAL, "x is NULL");
        if ((rc = check_dtype(x_dtype, "input"))) return rc;
        if (!aligned(x, 16)) return fail(COSET_EINVAL, "x must be 16-byte aligned");
        if (dither && dither_stride != 0 && dither_stride != 8)
            return fail(COSET_EINVAL, "dither_stride must be 0 or 8");
    } else {
        if (n > 0 && !packed_in && !codes_in) return fail(COSET_EINVAL, "no codes to decode");
        if (codes_in && !aligned(codes_in, 16)) return fail(COSET_EINVAL, "codes must be 16-byte aligned");
    }
    if (mode != coset::MODE_ENCODE && out) {
        if ((rc = check_dtype(out_dtype, "output"))) return rc;
        if (!aligned(out, 16)) return fail(COSET_EINVAL, "out must be 16-byte aligned");
    }
    if (codes_f32 && !aligned(codes_f32, 16)) return fail(COSET_EINVAL, "codes_f32 must be 16-byte aligned");
    if (packed && !aligned(packed, 4)) return fail(COSET_EINVAL, "packed must be 4-byte aligned");
    if (scale_mode == COSET_SCALE_LAYER && !(clip >= 0.f)) return fail(COSET_EINVAL, "clip must be >= 0");

    coset::CodecArgs a{};
    a.n = n;
    a.q = q;
    a.M = M;
    a.scale_mode = scale_mode;
    a.beta = beta;
    {
        int ex = 0;
        float m = std::frexp(beta, &ex);
        a.beta_is_pow2 = (scale_mode == COSET_SCALE_CODEC && m == 0.5f) ? 1 : 0;
        a.beta_inv = a.beta_is_pow2 ? std::ldexp(1.0f, 1 - ex) : 1.0f;
    }
    a.beta_row = beta_row;
    a.blocks_per_row = bpr > 0 ? bpr : 1;
    a.clip = clip;
    a.strided = strided ? 1 : 0;
    a.x = x;
    a.x_dtype = x_dtype;
    a.dither = dither;
    a.dither_stride = dither_stride;
    a.packed = packed;
    a.codes_f32 = codes_f32;
    a.packed_in = packed_in;
    a.codes_in_f32 = packed_in ? nullptr : codes_in;
    a.out = out;
    a.out_dtype = out_dtype;
    return check_hip(coset::launch_codec(a, mode, (hipStream_t)stream), "codec launch");
}

static int legacy_common(coset::LegacyArgs& a, int64_t n, float beta, double alpha, int q, int M,
                         const float* dither, int64_t dither_stride)
{
    int rc;
    if (n < 0) return fail(COSET_EINVAL, "n_blocks < 0");
    if (n > (int64_t)0x7fffffff * 256) return fail(COSET_EINVAL, "n_blocks too large");
    if ((rc = check_qm(q, M))) return rc;
    if (!(beta > 0.f) || !std::isfinite(beta)) return fail(COSET_EINVAL, "beta must be positive (got %g)", (double)beta);
    if (!(alpha >= 0.0) || !std::isfinite(alpha)) return fail(COSET_EINVAL, "alpha must be >= 0 (got %g)", alpha);
    if (dither && dither_stride != 0 && dither_stride != 8) return fail(COSET_EINVAL, "dither_stride must be 0 or 8");
    a.n = n;
    a.q = q;
    a.M = M;
    a.beta = beta;
    int ex = 0;
    const float m = std::frexp(beta, &ex);
    a.beta_is_pow2 = m == 0.5f ? 1 : 0;
    a.beta_inv = a.beta_is_pow2 ? std::ldexp(1.0f, 1 - ex) : 1.0f;
    // Python's 2 ** alpha and 2 ** (alpha * T) are doubles, rounded to fp32
    // where they meet the fp32 tensor
    a.two_alpha = (float)std::pow(2.0, alpha);
    for (int t = 0; t <= coset::kLegacyMaxT; ++t) a.scale_T[t] = (float)std::pow(2.0, alpha * t);
    a.dither = dither;
    a.dither_stride = dither_stride;
    return COSET_OK;
}

int coset_e8_legacy_encode(const void* x, int x_dtype, int64_t n_blocks, float beta, double alpha, int max_iter,
                           int protect, const float* dither, int64_t dither_stride, int q, int M, void* packed,
                           float* codes_f32, int32_t* T, uint8_t* overload, float* decoded, void* stream)
{
    int rc;
    coset::LegacyArgs a{};
    if ((rc = legacy_common(a, n_blocks, beta, alpha, q, M, dither, dither_stride))) return rc;
    if (max_iter < 0 || max_iter > coset::kLegacyMaxT)
        return fail(COSET_EINVAL, "max_iter=%d outside [0,%d]", max_iter, coset::kLegacyMaxT);
    if (n_blocks > 0 && !x) return fail(COSET_EINVAL, "x is NULL");
    if ((rc = check_dtype(x_dtype, "input"))) return rc;
    if (!aligned(x, 16)) return fail(COSET_EINVAL, "x must be 16-byte aligned");
    if (codes_f32 && !aligned(codes_f32, 16)) return fail(COSET_EINVAL, "codes_f32 must be 16-byte aligned");
    if (decoded && !aligned(decoded, 16)) return fail(COSET_EINVAL, "decoded must be 16-byte aligned");
    if (packed && !aligned(packed, 4)) return fail(COSET_EINVAL, "packed must be 4-byte aligned");
    a.max_iter = max_iter;
    a.protect = protect ? 1 : 0;
    a.x = x;
    a.x_dtype = x_dtype;
    a.packed = packed;
    a.codes_f32 = codes_f32;
    a.T = T;
    a.overload = overload;
    a.out = decoded;
    return check_hip(coset::launch_legacy(a, false, (hipStream_t)stream), "legacy encode launch");
}

int coset_e8_legacy_decode(const void* packed, const float* codes_f32, const int32_t* T, int64_t n_blocks,
                           float beta, double alpha, const float* dither, int64_t dither_stride, int q, int M,
                           float* out, void* stream)
{
    int rc;
    coset::LegacyArgs a{};
    if ((rc = legacy_common(a, n_blocks, beta, alpha, q, M, dither, dither_stride))) return rc;
    if (n_blocks > 0 && ((!packed && !codes_f32) || !out)) return fail(COSET_EINVAL, "NULL buffer");
    if (codes_f32 && !aligned(codes_f32, 16)) return fail(COSET_EINVAL, "codes_f32 must be 16-byte aligned");
    if (!aligned(out, 16)) return fail(COSET_EINVAL, "out must be 16-byte aligned");
    a.packed_in = packed;
    a.codes_in_f32 = packed ? nullptr : codes_f32;
    a.T_in = T;
    a.out = out;
    return check_hip(coset::launch_legacy(a, true, (hipStream_t)stream), "legacy decode launch");
}

int coset_e8_hnlq_encode(const void* x, int x_dtype, int64_t n_blocks, int scale_mode,
                         float beta, const float* beta_row, int64_t blocks_per_row,
                         const float* dither, int64_t dither_stride, int q, int M,
                         void* packed, float* codes_f32, void* stream)
{
    return codec_common(coset::MODE_ENCODE, x, x_dtype, n_blocks, scale_mode, beta, beta_row,
                        blocks_per_row, 0.f, dither, dither_stride, q, M, 0, nullptr, nullptr,
                        packed, codes_f32, nullptr, COSET_F32, stream);
}

int coset_e8_hnlq_decode(const void* packed, const float* codes_f32, int64_t n_blocks,
                         int scale_mode, float beta, const float* beta_row,
                         int64_t blocks_per_row, float clip, int q, int M, int strided,
                         void* out, int out_dtype, void* stream)
{
    if (n_blocks > 0 && !out) return fail(COSET_EINVAL, "out is NULL");
    return codec_common(coset::MODE_DECODE, nullptr, COSET_F32, n_blocks, scale_mode, beta,
                        beta_row, blocks_per_row, clip, nullptr, 0, q, M, strided, packed,
                        codes_f32, nullptr, nullptr, out, out_dtype, stream);
}

int coset_e8_hnlq_roundtrip(const void* x, int x_dtype, int64_t n_blocks, int scale_mode,
                            float beta, const float* beta_row, int64_t blocks_per_row,
                            float clip, const float* dither, int64_t dither_stride, int q,
                            int M, int strided, void* packed, float* codes_f32, void* out,
                            int out_dtype, void* stream)
{
    return codec_common(coset::MODE_ROUNDTRIP, x, x_dtype, n_blocks, scale_mode, beta, beta_row,
                        blocks_per_row, clip, dither, dither_stride, q, M, strided, nullptr,
                        nullptr, packed, codes_f32, out, out_dtype, stream);
}

int coset_e8_qat_fwd(const float* W, int64_t rows, int64_t cols, const float* beta,
                     int64_t blocks_per_tile, float clip, int q, int M, void* Wq, int wq_dtype,
                     void* packed, void* stream)
{
    if (rows < 0 || cols < 0 || cols % 8) return fail(COSET_EINVAL, "W must be [rows, 8k] (got %lld x %lld)",
                                                      (long long)rows, (long long)cols);
    int64_t n = rows * (cols / 8);
    if (n > 0 && !Wq && !packed) return fail(COSET_EINVAL, "nothing to write");
    return codec_common(coset::MODE_ROUNDTRIP, W, COSET_F32, n, COSET_SCALE_LAYER, 1.f, beta,
                        blocks_per_tile, clip, nullptr, 0, q, M, n > 1, nullptr, nullptr, packed,
                        nullptr, Wq, wq_dtype, stream);
}

int coset_e8_qat_bwd(const void* gWq, int g_dtype, const float* W, const void* packed,
                     const float* beta, int64_t rows, int64_t cols, int64_t blocks_per_tile,
                     float clip, int q, int M, float* dW, float* dbeta, void* stream)
{
    int rc;
    if (rows < 0 || cols < 0 || cols % 8) return fail(COSET_EINVAL, "W must be [rows, 8k]");
    int64_t n = rows * (cols / 8);
    if ((rc = check_qm(q, M))) return rc;
    if ((rc = check_dtype(g_dtype, "gradient"))) return rc;
    if (blocks_per_tile <= 0 || n % blocks_per_tile) return fail(COSET_EINVAL, "blocks_per_tile must divide the block count");
    if (n > 0 && (!gWq || !W || !packed || !beta || !dW || !dbeta)) return fail(COSET_EINVAL, "NULL buffer");
    if (!aligned(gWq, 16) || !aligned(W, 16) || !aligned(dW, 16)) return fail(COSET_EINVAL, "g, W, dW must be 16-byte aligned");
    if (!(clip >= 0.f)) return fail(COSET_EINVAL, "clip must be >= 0");
    if (n / blocks_per_tile > 0x7fffffff) return fail(COSET_EINVAL, "too many tiles");
    return check_hip(coset::launch_qat_bwd(gWq, g_dtype, W, packed, beta, n, blocks_per_tile, clip, q, M,
                                           dW, dbeta, nullptr, nullptr, (hipStream_t)stream),
                     "qat backward launch");
}

static coset::ThetaBeta make_theta_beta(const float* theta, const float* sigma, const float* xmax, double delta0,
                                        double eta, double gamma_inv, int q, int M_bounds)
{
    // Python-double constants of HNLQLinearQAT._bounds (coset/core/layers.py:383-391),
    // rounded to fp32 the way torch applies a Python scalar to an fp32 tensor
    double qM = 1.0;
    for (int i = 0; i < M_bounds; ++i) qM *= q;
    coset::ThetaBeta tb{};
    tb.theta = theta;
    tb.sigma = sigma;
    tb.xmax = xmax;
    tb.c_min = (float)(delta0 / qM);
    tb.c_eta_ginv = (float)(eta * gamma_inv);
    tb.c_det = (float)(delta0 * (qM - 1));
    tb.c_2ginv = (float)(2 * gamma_inv);
    tb.c_2eta_ginv = (float)(2 * eta * gamma_inv);
    return tb;
}

int coset_e8_qat_fwd_theta(const float* W, int64_t rows, int64_t cols, int64_t blocks_per_tile,
                           const float* theta, const float* sigma_ema, const float* xmax_ema, double delta0,
                           double eta, double gamma_inv, int M_bounds, float clip, int q, int M, void* Wq,
                           int wq_dtype, void* packed, float* beta_out, float* dbeta_dtheta_out,
                           int64_t* step_counter, const float* bias, void* bias_out, void* stream)
{
    int rc;
    if (rows < 0 || cols < 0 || cols % 8) return fail(COSET_EINVAL, "W must be [rows, 8k]");
    if ((bias == nullptr) != (bias_out == nullptr)) return fail(COSET_EINVAL, "bias and bias_out go together");
    int64_t n = rows * (cols / 8);
    if ((rc = check_qm(q, M))) return rc;
    if (M_bounds < 1 || M_bounds > 16) return fail(COSET_EINVAL, "M_bounds=%d", M_bounds);
    if (blocks_per_tile <= 0 || n % blocks_per_tile) return fail(COSET_EINVAL, "blocks_per_tile must divide the block count");
    if (n > 0 && (!W || !theta || !sigma_ema || !xmax_ema)) return fail(COSET_EINVAL, "NULL buffer");
    if (n > 0 && !Wq && !packed) return fail(COSET_EINVAL, "nothing to write");
    if (!aligned(W, 16) || (Wq && !aligned(Wq, 16))) return fail(COSET_EINVAL, "W and Wq must be 16-byte aligned");
    if (packed && !aligned(packed, 4)) return fail(COSET_EINVAL, "packed must be 4-byte aligned");
    if ((rc = check_dtype(wq_dtype, "Wq"))) return rc;
    if (!(clip >= 0.f)) return fail(COSET_EINVAL, "clip must be >= 0");
    if (!(delta0 > 0) || !(eta > 0) || !(gamma_inv > 0)) return fail(COSET_EINVAL, "delta0, eta, gamma_inv must be positive");
    coset::CodecArgs a{};
    a.n = n;
    a.q = q;
    a.M = M;
    a.scale_mode = COSET_SCALE_LAYER;
    a.beta = 1.f;
    a.blocks_per_row = blocks_per_tile;
    a.clip = clip;
    a.strided = n > 1;
    a.x = W;
    a.x_dtype = COSET_F32;
    a.packed = packed;
    a.out = Wq;
    a.out_dtype = wq_dtype;
    a.use_theta = 1;
    a.tb = make_theta_beta(theta, sigma_ema, xmax_ema, delta0, eta, gamma_inv, q, M_bounds);
    a.beta_out = beta_out;
    a.dbdt_out = dbeta_dtheta_out;
    a.step_counter = step_counter;
    a.aux_in = bias;
    a.aux_out = bias_out;
    a.aux_n = bias ? rows : 0;
    return check_hip(coset::launch_codec(a, coset::MODE_ROUNDTRIP, (hipStream_t)stream), "qat forward launch");
}

int coset_e8_qat_head_fwd(const float* W, int64_t rows, int64_t cols, const float* theta, const float* sigma_ema,
                          const float* xmax_ema, double delta0, double eta, double gamma_inv, int M_bounds, float clip,
                          int q, const float* x, int64_t tokens, const float* bias, float* y, int64_t* step_counter,
                          void* stream)
{
    if (rows < 0 || tokens < 0) return fail(COSET_EINVAL, "negative size");
    if (q != 2 && q != 4) return fail(COSET_EUNSUPPORTED, "the fused layer forward takes q = 2, 4, got %d", q);
    if (cols <= 0 || cols % 8 || cols > 8192) return fail(COSET_EUNSUPPORTED, "cols=%lld: 8k <= 8192", (long long)cols);
    if (tokens > 64) return fail(COSET_EUNSUPPORTED, "tokens=%lld > 64", (long long)tokens);
    if (M_bounds < 1 || M_bounds > 16) return fail(COSET_EINVAL, "M_bounds=%d", M_bounds);
    if (rows == 0 || tokens == 0) return COSET_OK;
    if (!W || !theta || !sigma_ema || !xmax_ema || !x || !y) return fail(COSET_EINVAL, "NULL buffer");
    if (!aligned(W, 16) || !aligned(x, 16)) return fail(COSET_EINVAL, "W and x must be 16-byte aligned");
    if (!(clip >= 0.f)) return fail(COSET_EINVAL, "clip must be >= 0");
    if (!(delta0 > 0) || !(eta > 0) || !(gamma_inv > 0)) return fail(COSET_EINVAL, "delta0, eta, gamma_inv must be positive");
    const coset::ThetaBeta tb = make_theta_beta(theta, sigma_ema, xmax_ema, delta0, eta, gamma_inv, q, M_bounds);
    return check_hip(coset::launch_qat_head(W, rows, cols, tb, clip, q, x, (int)tokens, bias, y, step_counter,
                                            (hipStream_t)stream),
                     "qat head forward launch");
}

int coset_e8_qat_bwd_theta(const void* gWq, int g_dtype, const float* W, const void* packed, const float* beta,
                           const float* dbeta_dtheta, int64_t rows, int64_t cols, int64_t blocks_per_tile,
                           float clip, int q, int M, float* dW, float* dbeta, float* dtheta, void* stream)
{
    int rc;
    if (rows < 0 || cols < 0 || cols % 8) return fail(COSET_EINVAL, "W must be [rows, 8k]");
    int64_t n = rows * (cols / 8);
    if ((rc = check_qm(q, M))) return rc;
    if ((rc = check_dtype(g_dtype, "gradient"))) return rc;
    if (blocks_per_tile <= 0 || n % blocks_per_tile) return fail(COSET_EINVAL, "blocks_per_tile must divide the block count");
    if (n > 0 && (!gWq || !W || !packed || !beta || !dW || !dbeta || !dbeta_dtheta || !dtheta))
        return fail(COSET_EINVAL, "NULL buffer");
    if (!aligned(gWq, 16) || !aligned(W, 16) || !aligned(dW, 16)) return fail(COSET_EINVAL, "g, W, dW must be 16-byte aligned");
    if (!(clip >= 0.f)) return fail(COSET_EINVAL, "clip must be >= 0");
    if (n / blocks_per_tile > 0x7fffffff) return fail(COSET_EINVAL, "too many tiles");
    return check_hip(coset::launch_qat_bwd(gWq, g_dtype, W, packed, beta, n, blocks_per_tile, clip, q, M, dW,
                                           dbeta, dbeta_dtheta, dtheta, (hipStream_t)stream),
                     "qat backward launch");
}

int64_t coset_colsum_workspace_floats(int64_t rows, int64_t cols)
{
    if (rows < 0 || cols < 0) return 0;
    return coset::colsum_workspace_floats(rows, cols);
}

int coset_colsum(const void* g, int dtype, int64_t rows, int64_t cols, float* out, float* workspace,
                 int64_t workspace_floats, void* stream)
{
    if (rows < 0 || cols < 0) return fail(COSET_EINVAL, "rows, cols must be >= 0");
    if (dtype != COSET_F32 && dtype != COSET_BF16 && dtype != COSET_F16)
        return fail(COSET_EUNSUPPORTED, "gradient dtype %d not supported (fp32, bf16, fp16)", dtype);
    if (cols % 8) return fail(COSET_EINVAL, "cols must be a multiple of 8, got %lld", (long long)cols);
    if (cols > 0 && (!out || (rows > 0 && !g))) return fail(COSET_EINVAL, "NULL buffer");
    if (rows > 0 && !aligned(g, 16)) return fail(COSET_EINVAL, "g must be 16-byte aligned");
    int64_t need = coset::colsum_workspace_floats(rows, cols);
    if (cols > 0 && need > 0 && (!workspace || workspace_floats < need))
        return fail(COSET_EINVAL, "workspace too small: %lld floats needed", (long long)need);
    if ((rows + 63) / 64 > 65535) return fail(COSET_EINVAL, "too many rows");
    return check_hip(coset::launch_colsum(g, dtype, rows, cols, out, workspace, (hipStream_t)stream),
                     "column sum launch");
}

int coset_gemm_tn_supported(int64_t M, int64_t N, int64_t K)
{
    return coset::gemm_tn_plan(M, N, K).tile > 0 ? 1 : 0;
}

int64_t coset_gemm_tn_workspace_floats(int64_t M, int64_t N, int64_t K)
{
    return coset::gemm_tn_workspace_floats(coset::gemm_tn_plan(M, N, K), M, N);
}

int coset_gemm_tn(const void* A, int64_t lda, const void* B, int64_t ldb, void* C, int64_t ldc, int out_dtype,
                  int64_t M, int64_t N, int64_t K, float* colsum, float* workspace, int64_t workspace_floats,
                  void* stream)
{
    if (M < 0 || N < 0 || K < 0) return fail(COSET_EINVAL, "M, N, K must be >= 0");
    if (out_dtype != COSET_F32 && out_dtype != COSET_BF16)
        return fail(COSET_EUNSUPPORTED, "output dtype %d not supported (fp32, bf16)", out_dtype);
    const coset::GemmTnPlan plan = coset::gemm_tn_plan(M, N, K);
    if (plan.tile == 0)
        return fail(COSET_EUNSUPPORTED,
                    "shape M=%lld N=%lld K=%lld not taken: M, N multiples of 64, at most 256 tiles of 64 x 64, "
                    "K = 256 s m (s a power of two, m in 4, 8, 16, 32)",
                    (long long)M, (long long)N, (long long)K);
    if (!A || !B || !C) return fail(COSET_EINVAL, "NULL buffer");
    if (!aligned(A, 16) || !aligned(B, 16) || !aligned(C, 16)) return fail(COSET_EINVAL, "buffers must be 16-byte aligned");
    if (lda < M || ldb < N || ldc < N || lda % 8 || ldb % 8 || ldc % 8)
        return fail(COSET_EINVAL, "leading dimensions must cover the rows and be multiples of 8");
    const int64_t need = coset::gemm_tn_workspace_floats(plan, M, N);
    if (need > 0 && (!workspace || workspace_floats < need))
        return fail(COSET_EINVAL, "workspace too small: %lld floats needed", (long long)need);
    if (need > 0 && !aligned(workspace, 16)) return fail(COSET_EINVAL, "workspace must be 16-byte aligned");
    if (colsum && !aligned(colsum, 16)) return fail(COSET_EINVAL, "colsum must be 16-byte aligned");
    return check_hip(coset::gemm_tn_bf16(static_cast<const uint16_t*>(A), lda, static_cast<const uint16_t*>(B), ldb, C,
                                         ldc, out_dtype, M, N, K, plan, need > 0 ? workspace : nullptr, colsum,
                                         (hipStream_t)stream),
                     "gemm_tn launch");
}

int coset_qat_stats_update(const float* W, int64_t tiles, int64_t tile_size, double momentum, float* sigma_ema,
                           float* xmax_ema, void* stream)
{
    if (tiles < 0 || tile_size < 2) return fail(COSET_EINVAL, "tiles >= 0 and tile_size >= 2 required");
    if (tiles > 0x7fffffff) return fail(COSET_EINVAL, "too many tiles");
    if (tiles > 0 && (!W || !sigma_ema || !xmax_ema)) return fail(COSET_EINVAL, "NULL buffer");
    if (tile_size == 8 && !aligned(W, 16)) return fail(COSET_EINVAL, "W must be 16-byte aligned");
    return check_hip(coset::launch_qat_stats(W, tiles, tile_size, momentum, sigma_ema, xmax_ema, (hipStream_t)stream),
                     "statistics launch");
}

int coset_vlut_build_one_sided(const float* queries, int64_t n_queries, int q, int legacy, float* vlut,
                               void* stream)
{
    if (n_queries < 0) return fail(COSET_EINVAL, "n_queries < 0");
    if (q < 2 || q > 8) return fail(COSET_EINVAL, "one-sided vLUT needs q in [2,8] (q^8 entries), got %d", q);
    if (n_queries > 0 && (!queries || !vlut)) return fail(COSET_EINVAL, "NULL buffer");
    int64_t n = 1;
    for (int i = 0; i < 8; ++i) n *= q;
    if (n_queries * n > ((int64_t)1 << 40)) return fail(COSET_EINVAL, "table too large");
    return check_hip(coset::vlut_build(queries, n_queries, q, legacy ? 1 : 0, vlut, (hipStream_t)stream),
                     "vLUT build launch");
}

int coset_vlut_lookup_dot(const void* words, int64_t n_blocks, int q, int M, const float* vlut, float* out,
                          void* stream)
{
    int rc;
    if ((rc = check_qm(q, M))) return rc;
    if (q > 8) return fail(COSET_EINVAL, "one-sided vLUT needs q in [2,8]");
    if (n_blocks < 0) return fail(COSET_EINVAL, "n_blocks < 0");
    if (n_blocks > 0 && (!words || !vlut || !out)) return fail(COSET_EINVAL, "NULL buffer");
    return check_hip(coset::vlut_dot(words, n_blocks, M, q, vlut, out, (hipStream_t)stream), "vLUT dot launch");
}

static int vlut_method(int method, int act_dtype, int q, int M)
{
    // the MFMA path multiplies 2*x_hat held exactly in fp16 (|v| < 2048)
    // or bf16 (|v| < 256); max |2x_hat| <= 12 q^M at q <= 4.  fp32
    // activations run on it as three exact bf16 planes.
    int64_t qm = 1;
    for (int i = 0; i < M; ++i) qm *= q;
    bool exact = (act_dtype == COSET_F16 && 12 * qm < 2048) || (act_dtype == COSET_BF16 && 12 * qm < 256);
    bool split = act_dtype == COSET_F32 && 12 * qm < 256;
    if (method == coset::VLUT_METHOD_MFMA || method == coset::VLUT_METHOD_AUTO) {
        if (exact) return coset::VLUT_METHOD_MFMA;
        if (split) return coset::VLUT_METHOD_MFMA_SPLIT;
        return method == coset::VLUT_METHOD_MFMA ? -1 : coset::VLUT_METHOD_LDS;
    }
    return method;
}

// Workspace floats of a matmul under resolved method m.
static int64_t vlut_method_workspace(int m, int64_t B, int64_t rows, int64_t K, int q, int M)
{
    if (m == coset::VLUT_METHOD_MFMA_SPLIT) return coset::vlut_split_workspace_floats(B, rows, K, q, M);
    return coset::vlut_workspace_floats(coset::vlut_plan(rows, B, K, q, M, m), B, rows);
}

int64_t coset_vlut_workspace_floats(int64_t B, int64_t rows, int64_t K, int q, int M, int act_dtype, int method)
{
    int m = vlut_method(method, act_dtype, q, M);
    if (m < 0 || B < 0 || rows < 0 || K < 8) return 0;
    return vlut_method_workspace(m, B, rows, K, q, M);
}

int coset_d4_lattice_op(int op, const float* in, int64_t n_blocks, int q, float* out, void* stream)
{
    if (n_blocks < 0) return fail(COSET_EINVAL, "n_blocks < 0");
    if (op < COSET_OP_G_X || op > COSET_OP_DECODE_COORDS) return fail(COSET_EINVAL, "unknown D4 lattice op %d", op);
    if (n_blocks > 0 && (!in || !out)) return fail(COSET_EINVAL, "NULL buffer");
    if (!aligned(in, 16) || !aligned(out, 16)) return fail(COSET_EINVAL, "buffers must be 16-byte aligned");
    if (op == COSET_OP_ENCODE_COORDS && q < 1) return fail(COSET_EINVAL, "q must be positive");
    return check_hip(coset::launch_d4_lattice_op(op, in, n_blocks, q, out, (hipStream_t)stream), "D4 lattice op launch");
}

static int check_d4_qat(const float* W, int64_t rows, int64_t cols, int64_t blocks_per_tile, float clip,
                        int64_t* n_blocks)
{
    if (rows < 0 || cols < 0 || cols % 4) return fail(COSET_EINVAL, "W must be [rows, 4k]");
    const int64_t n = rows * (cols / 4);
    if (blocks_per_tile <= 0 || n % blocks_per_tile) return fail(COSET_EINVAL, "blocks_per_tile must divide the block count");
    if (n / blocks_per_tile > 0x7fffffff) return fail(COSET_EINVAL, "too many tiles");
    if (!(clip >= 0.f)) return fail(COSET_EINVAL, "clip must be >= 0");
    if (n > 0 && !W) return fail(COSET_EINVAL, "NULL buffer");
    if (!aligned(W, 16)) return fail(COSET_EINVAL, "W must be 16-byte aligned");
    *n_blocks = n;
    return COSET_OK;
}

int coset_d4_qat_fwd(const float* W, int64_t rows, int64_t cols, const float* beta, int64_t blocks_per_tile,
                     float clip, void* Wq, int wq_dtype, void* stream)
{
    int rc;
    int64_t n = 0;
    if ((rc = check_d4_qat(W, rows, cols, blocks_per_tile, clip, &n))) return rc;
    if ((rc = check_dtype(wq_dtype, "Wq"))) return rc;
    if (n > 0 && (!beta || !Wq)) return fail(COSET_EINVAL, "NULL buffer");
    if (!aligned(Wq, wq_dtype == COSET_F32 ? 16 : 8)) return fail(COSET_EINVAL, "Wq misaligned");
    if (n == 0) return COSET_OK;
    return check_hip(coset::launch_d4_qat_fwd(W, n, blocks_per_tile, beta, nullptr, clip, Wq, wq_dtype, nullptr,
                                              nullptr, nullptr, (hipStream_t)stream),
                     "D4 qat forward launch");
}

int coset_d4_qat_fwd_theta(const float* W, int64_t rows, int64_t cols, int64_t blocks_per_tile, const float* theta,
                           const float* sigma_ema, const float* xmax_ema, double delta0, double eta,
                           double gamma_inv, int q, int M_bounds, float clip, void* Wq, int wq_dtype,
                           float* beta_out, float* dbeta_dtheta_out, int64_t* step_counter, void* stream)
{
    int rc;
    int64_t n = 0;
    if ((rc = check_d4_qat(W, rows, cols, blocks_per_tile, clip, &n))) return rc;
    if ((rc = check_dtype(wq_dtype, "Wq"))) return rc;
    if (q < 2 || M_bounds < 1 || M_bounds > 16) return fail(COSET_EINVAL, "bad q=%d / M=%d for the bounds", q, M_bounds);
    if (n > 0 && (!theta || !sigma_ema || !xmax_ema || !Wq)) return fail(COSET_EINVAL, "NULL buffer");
    if (!aligned(Wq, wq_dtype == COSET_F32 ? 16 : 8)) return fail(COSET_EINVAL, "Wq misaligned");
    const coset::ThetaBeta tb = make_theta_beta(theta, sigma_ema, xmax_ema, delta0, eta, gamma_inv, q, M_bounds);
    return check_hip(coset::launch_d4_qat_fwd(W, n, blocks_per_tile, nullptr, &tb, clip, Wq, wq_dtype, beta_out,
                                              dbeta_dtheta_out, step_counter, (hipStream_t)stream),
                     "D4 qat forward launch");
}

int coset_d4_qat_bwd(const void* gWq, int g_dtype, const float* W, const float* beta, const float* dbeta_dtheta,
                     int64_t rows, int64_t cols, int64_t blocks_per_tile, float clip, float* dW, float* dbeta,
                     float* dtheta, void* stream)
{
    int rc;
    int64_t n = 0;
    if ((rc = check_d4_qat(W, rows, cols, blocks_per_tile, clip, &n))) return rc;
    if ((rc = check_dtype(g_dtype, "gradient"))) return rc;
    if (n > 0 && (!gWq || !beta || !dW || !dbeta)) return fail(COSET_EINVAL, "NULL buffer");
    if (dbeta_dtheta && !dtheta) return fail(COSET_EINVAL, "dtheta needed with dbeta_dtheta");
    if (!aligned(gWq, g_dtype == COSET_F32 ? 16 : 8) || !aligned(dW, 16)) return fail(COSET_EINVAL, "g or dW misaligned");
    return check_hip(coset::launch_d4_qat_bwd(gWq, g_dtype, W, beta, dbeta_dtheta, n, blocks_per_tile, clip, dW,
                                              dbeta, dtheta, (hipStream_t)stream),
                     "D4 qat backward launch");
}

int64_t coset_lsq_workspace_floats(int64_t n) { return n < 0 ? 0 : coset::lsq_workspace_floats(n); }

static int check_lsq(const void* x, int dtype, int64_t n, const float* alpha, int qmax)
{
    if (n < 0) return fail(COSET_EINVAL, "n must be >= 0");
    if (dtype != COSET_F32 && dtype != COSET_BF16 && dtype != COSET_F16)
        return fail(COSET_EUNSUPPORTED, "activation dtype %d not supported (fp32, bf16, fp16)", dtype);
    if (qmax < 1) return fail(COSET_EINVAL, "qmax must be >= 1 (bit_width >= 2)");
    if (!alpha) return fail(COSET_EINVAL, "NULL alpha");
    if (n > 0 && !x) return fail(COSET_EINVAL, "NULL buffer");
    return COSET_OK;
}

int coset_lsq_fwd(const void* x, int dtype, int64_t n, const float* alpha, int qmax, void* out, void* stream)
{
    int rc;
    if ((rc = check_lsq(x, dtype, n, alpha, qmax))) return rc;
    if (n > 0 && !out) return fail(COSET_EINVAL, "NULL buffer");
    return check_hip(coset::launch_lsq_fwd(x, dtype, n, alpha, qmax, out, (hipStream_t)stream), "lsq forward launch");
}

int coset_lsq_bwd(const void* x, const void* g, int dtype, int64_t n, const float* alpha, int qmax, void* dx,
                  float* d_alpha, float* workspace, int64_t workspace_floats, void* stream)
{
    int rc;
    if ((rc = check_lsq(x, dtype, n, alpha, qmax))) return rc;
    if ((n > 0 && (!g || !dx)) || !d_alpha || !workspace) return fail(COSET_EINVAL, "NULL buffer");
    if (workspace_floats < coset::lsq_workspace_floats(n))
        return fail(COSET_EINVAL, "workspace holds %lld floats, %lld needed", (long long)workspace_floats,
                    (long long)coset::lsq_workspace_floats(n));
    return check_hip(coset::launch_lsq_bwd(x, g, dtype, n, alpha, qmax, dx, d_alpha, workspace, (hipStream_t)stream),
                     "lsq backward launch");
}

int64_t coset_vlut_prepared_words(int64_t rows, int64_t kb, int M, int word_format)
{
    if (rows < 0 || kb < 0 || M < 1 || word_format < 0 || word_format > 5) return 0;
    return coset::vlut_prepared_words(rows, kb, M, word_format);
}

int coset_vlut_prepare(const void* words, int64_t rows, int64_t kb, int M, int q, int legacy, int word_format,
                       uint32_t* prepared, void* stream)
{
    if (q != 2 && q != 4) return fail(COSET_EUNSUPPORTED, "vLUT prepare supports q = 2 or 4 (got %d)", q);
    if (rows < 0 || kb < 0 || M < 1 || M > 4) return fail(COSET_EINVAL, "bad shape rows=%lld kb=%lld M=%d",
                                                         (long long)rows, (long long)kb, M);
    if (word_format < 1 || word_format > 5) return fail(COSET_EINVAL, "prepared word_format must be 1, 2, 3, 4 or 5");
    if (word_format == 3 && !((q == 4 && M <= 2) || (q == 2 && M <= 4)))
        return fail(COSET_EUNSUPPORTED, "decoded format needs |2 x_hat| <= 127: q = 4 with M <= 2 or q = 2 with M <= 4");
    if (word_format == 5) {
        const coset::DecodeTables* t = nullptr;
        int rc = check_hip(coset::get_decode_tables(q, legacy ? 1 : 0, &t), "decode tables");
        if (rc) return rc;
        if (coset::decoded6_offset(*t, M) < 0)
            return fail(COSET_EUNSUPPORTED, "the 6-byte decoded format does not hold 2 x_hat at q = %d, M = %d", q, M);
    }
    if (rows * kb > 0 && (!words || !prepared)) return fail(COSET_EINVAL, "NULL buffer");
    if (!aligned(prepared, 16)) return fail(COSET_EINVAL, "prepared must be 16-byte aligned");
    return check_hip(coset::vlut_prepare((const uint16_t*)words, rows, kb, M, q, legacy ? 1 : 0, word_format, prepared,
                                         (hipStream_t)stream), "vLUT prepare launch");
}

static int vlut_matmul_impl(const void* words, int word_format, const float* scale, int scale_mode, const void* act,
                            int act_dtype, int64_t B, int64_t rows, int64_t K, int q, int M, int legacy, int method,
                            const float* bias, const float* lsq_alpha, int lsq_qmax, float* workspace,
                            int64_t workspace_floats, float* out, void* stream, bool may_build = true)
{
    int rc;
    if (lsq_alpha && lsq_qmax < 1) return fail(COSET_EINVAL, "lsq_qmax must be >= 1 (bit_width >= 2)");
    if ((rc = check_qm(q, M))) return rc;
    if (q != 2 && q != 4) return fail(COSET_EUNSUPPORTED, "vLUT matmul supports q = 2 or 4 (got %d)", q);
    if (M > 4) return fail(COSET_EUNSUPPORTED, "vLUT matmul supports M <= 4");
    if (B < 0 || rows < 0 || K < 8 || K % 8) return fail(COSET_EINVAL, "bad shape B=%lld rows=%lld K=%lld",
                                                         (long long)B, (long long)rows, (long long)K);
    if (act_dtype != COSET_F32 && act_dtype != COSET_BF16 && act_dtype != COSET_F16)
        return fail(COSET_EINVAL, "activation dtype %d", act_dtype);
    if (scale_mode != 0 && scale_mode != 1) return fail(COSET_EINVAL, "scale_mode must be 0 or 1");
    if (word_format == coset::VLUT_PAIRS) {  // read by the LDS-table method only
        if (method == coset::VLUT_METHOD_MFMA)
            return fail(COSET_EUNSUPPORTED, "the pairs format is read by the LDS-table method (1) only");
        if (method == coset::VLUT_METHOD_AUTO) method = coset::VLUT_METHOD_LDS;
    }
    if (method < coset::VLUT_METHOD_AUTO || method > coset::VLUT_METHOD_MFMA)
        return fail(COSET_EINVAL, "unknown method %d", method);
    int m = vlut_method(method, act_dtype, q, M);
    if (m < 0) return fail(COSET_EUNSUPPORTED, "MFMA method needs activations holding 2*x_hat exactly (q^M too large)");
    if (B == 0 || rows == 0) return COSET_OK;
    if (!words || !act || !out) return fail(COSET_EINVAL, "NULL buffer");
    if (!aligned(act, 16) || !aligned(words, 4)) return fail(COSET_EINVAL, "act must be 16-byte aligned, words 4-byte");
    const bool split = m == coset::VLUT_METHOD_MFMA_SPLIT;
    // the split path's inner product: 3B bf16 tokens on the matrix cores
    const coset::VlutPlan plan = coset::vlut_plan(rows, split ? 3 * B : B, K, q, M, split ? coset::VLUT_METHOD_MFMA : m);
    const int64_t need = vlut_method_workspace(m, B, rows, K, q, M);
    if (workspace_floats < need)
        return fail(COSET_EINVAL, "workspace holds %lld floats, needs %lld", (long long)workspace_floats,
                    (long long)need);
    if (need > 0 && !workspace) return fail(COSET_EINVAL, "NULL workspace");
    if (word_format < 0 || word_format > 5) return fail(COSET_EINVAL, "word_format must be 0, 1, 2, 3, 4 or 5");
    if (word_format == 3 && plan.kernel != coset::VK_MFMA_ROWS && plan.kernel != coset::VK_MFMA_WIDE &&
        plan.kernel != coset::VK_MFMA_DEEP)
        return fail(COSET_EUNSUPPORTED, "the decoded format runs on the matrix-core rows kernel only (fp16/bf16 activations)");
    if (word_format == 5 && plan.kernel != coset::VK_MFMA_ROWS && plan.kernel != coset::VK_MFMA_DEEP)
        return fail(COSET_EUNSUPPORTED, "the 6-byte decoded format runs on the matrix-core rows and deep kernels only");
    if (word_format != 0 && !aligned(words, 16)) return fail(COSET_EINVAL, "prepared words must be 16-byte aligned");
    coset::VlutMatmulArgs p{};
    p.words = words;
    p.prepared = word_format;
    p.scale = scale;
    p.scale_mode = scale_mode;
    p.act = act;
    p.act_dtype = act_dtype;
    p.B = B;
    p.rows = rows;
    p.K = K;
    p.q = q;
    p.M = M;
    p.legacy = legacy ? 1 : 0;
    p.partial = workspace;
    p.out = out;
    p.bias = bias;
    p.lsq_alpha = lsq_alpha;
    p.lsq_qmax = lsq_qmax;
    const coset::DecodeTables* t = nullptr;
    if (may_build) {
        if ((rc = check_hip(coset::get_decode_tables(q, p.legacy, &t), "decode tables"))) return rc;
    } else if (coset::find_decode_tables(q, p.legacy, &t) != hipSuccess) {
        return fail(COSET_EINVAL, "decode tables not built on this device: call coset_init(device) first");
    }
    if (t->n_coarse > coset::kMaxCoarseVlut) return fail(COSET_EUNSUPPORTED, "too many coarse points");
    if (split) return check_hip(coset::vlut_matmul_split(p, workspace, (hipStream_t)stream), "vLUT matmul launch");
    return check_hip(coset::vlut_matmul(p, plan, (hipStream_t)stream), "vLUT matmul launch");
}

int coset_vlut_matmul(const void* words, int word_format, const float* scale, int scale_mode, const void* act,
                      int act_dtype, int64_t B, int64_t rows, int64_t K, int q, int M, int legacy, int method,
                      float* workspace, int64_t workspace_floats, float* out, void* stream)
{
    return vlut_matmul_impl(words, word_format, scale, scale_mode, act, act_dtype, B, rows, K, q, M, legacy, method,
                            nullptr, nullptr, 0, workspace, workspace_floats, out, stream);
}

int coset_vlut_matmul_noalloc(const void* words, int word_format, const float* scale, int scale_mode,
                              const void* act, int act_dtype, int64_t B, int64_t rows, int64_t K, int q, int M,
                              int legacy, int method, float* out, void* stream)
{
    int dev = 0;
    int rc = check_hip(hipGetDevice(&dev), "hipGetDevice");
    if (rc) return rc;
    float* ws = nullptr;
    if (dev < kMaxDevices) {
        std::lock_guard<std::mutex> lk(g_scratch_mu);
        ws = g_scratch_ptr[dev];
    }
    if (!ws) return fail(COSET_EINVAL, "coset_vlut_matmul_noalloc: call coset_init(%d) on this device first", dev);
    const bool pairs_auto = word_format == coset::VLUT_PAIRS && method == coset::VLUT_METHOD_AUTO;
    const int m = vlut_method(pairs_auto ? coset::VLUT_METHOD_LDS : method, act_dtype, q, M);
    if (m >= 0 && B > 0 && rows > 0 && K >= 8 && q >= 2 && q <= 4 && M >= 1 && M <= 4) {
        const int64_t need = vlut_method_workspace(m, B, rows, K, q, M);
        if (need > kNoallocScratchFloats)
            return fail(COSET_EINVAL,
                        "coset_vlut_matmul_noalloc: B=%lld rows=%lld K=%lld needs %lld floats of scratch, more than "
                        "the %lld (8 MiB) it holds; use coset_vlut_matmul with a workspace",
                        (long long)B, (long long)rows, (long long)K, (long long)need,
                        (long long)kNoallocScratchFloats);
    }
    return vlut_matmul_impl(words, word_format, scale, scale_mode, act, act_dtype, B, rows, K, q, M, legacy, method,
                            nullptr, nullptr, 0, ws, kNoallocScratchFloats, out, stream, false);
}

int64_t coset_vlut_noalloc_scratch_floats(void) { return kNoallocScratchFloats; }

int coset_vlut_linear(const void* words, int word_format, const float* scale, int scale_mode, const void* act,
                      int act_dtype, int64_t B, int64_t rows, int64_t K, int q, int M, int legacy, int method,
                      const float* bias, const float* lsq_alpha, int lsq_qmax, float* workspace,
                      int64_t workspace_floats, float* out, void* stream)
{
    return vlut_matmul_impl(words, word_format, scale, scale_mode, act, act_dtype, B, rows, K, q, M, legacy, method,
                            bias, lsq_alpha, lsq_qmax, workspace, workspace_floats, out, stream);
}

int coset_e8_lattice_op(int op, int legacy, const float* in, int64_t n_blocks, int q,
                        float* out, void* stream)
{
    if (n_blocks < 0) return fail(COSET_EINVAL, "n_blocks < 0");
    if (op < COSET_OP_CUSTOM_ROUND || op > COSET_OP_DECODE_COORDS)
        return fail(COSET_EINVAL, "unknown lattice op %d", op);
    if (n_blocks > 0 && (!in || !out)) return fail(COSET_EINVAL, "NULL buffer");
    if (!aligned(in, 16) || !aligned(out, 16)) return fail(COSET_EINVAL, "buffers must be 16-byte aligned");
    if (op == COSET_OP_ENCODE_COORDS && q < 1) return fail(COSET_EINVAL, "q must be positive");
    return check_hip(coset::launch_lattice_op(op, legacy, in, n_blocks, q, out, (hipStream_t)stream),
                     "lattice op launch");
}

// ---------------------------------------------------------------- measurement probes

int coset_probe_empty(int grid, int threads, int lds_bytes, uint32_t* out, void* stream)
{
    if (grid < 1 || grid > (1 << 24) || threads < 64 || threads > 1024 || threads % 64)
        return fail(COSET_EINVAL, "grid in [1, 2^24] and threads a multiple of 64 in [64, 1024] required");
    if (lds_bytes < 0 || lds_bytes > 160 * 1024) return fail(COSET_EINVAL, "lds_bytes outside [0, 160 KiB]");
    if (!out) return fail(COSET_EINVAL, "NULL buffer");
    return check_hip(coset::launch_probe_empty(grid, threads, lds_bytes, out, (hipStream_t)stream), "probe launch");
}

int coset_probe_read(const void* src, int64_t bytes, int grid, int threads, uint32_t* out, void* stream)
{
    if (grid < 1 || grid > (1 << 24) || threads < 64 || threads > 1024 || threads % 64)
        return fail(COSET_EINVAL, "grid in [1, 2^24] and threads a multiple of 64 in [64, 1024] required");
    if (bytes < 16 || bytes % 16) return fail(COSET_EINVAL, "bytes must be a positive multiple of 16");
    if (!src || !out) return fail(COSET_EINVAL, "NULL buffer");
    if (!aligned(src, 16)) return fail(COSET_EINVAL, "src must be 16-byte aligned");
    if (coset::probe_read_loads(bytes, grid, threads) < 0)
        return fail(COSET_EINVAL, "more than 32 loads per thread: use a larger grid");
    return check_hip(coset::launch_probe_read(src, bytes, grid, threads, out, (hipStream_t)stream), "probe launch");
}

int coset_probe_valu(int kind, int grid, int iters, float* out, void* stream)
{
    if (kind != 0 && kind != 1) return fail(COSET_EINVAL, "kind must be 0 (fp32 FMA) or 1 (compare + select)");
    if (grid < 1 || grid > (1 << 20) || iters < 1) return fail(COSET_EINVAL, "grid in [1, 2^20], iters >= 1 required");
    if (!out) return fail(COSET_EINVAL, "NULL buffer");
    return check_hip(coset::launch_probe_valu(kind, grid, iters, out, (hipStream_t)stream), "probe launch");
}

int coset_probe_c2_stream(const float* x, int64_t n_blocks, uint32_t* packed, float* out, int staged, void* stream)
{
    if (n_blocks < 1) return fail(COSET_EINVAL, "n_blocks must be positive");
    if (!x || !packed || !out) return fail(COSET_EINVAL, "NULL buffer");
    if (!aligned(x, 16) || !aligned(out, 16) || !aligned(packed, 4))
        return fail(COSET_EINVAL, "x and out must be 16-byte aligned, packed 4-byte aligned");
    return check_hip(coset::launch_c2_stream_probe(x, n_blocks, packed, out, staged, (hipStream_t)stream),
                     "probe launch");
}

}  // extern "C"
