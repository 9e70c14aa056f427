// vlut.hip -- value lookup tables (vLUTs) of the E8 HNLQ codes.
//
// Reference definition (coset/legacy/quant/vlut.py:72-117, 217-238;
// tests/legacy/test_one_sided_vlut_pytest.py:22-43): for a query a in R^8
//   vLUT_a[idx(b)] = <a, r(b)>,   r(b) = G b - q P(G b / q)
// over all b in [0,q)^8, idx(b) = sum_j b_j q^(7-j), and for an encoded block
//   <a, x_hat> = sum_m q^m vLUT_a[idx(b_m)].
// P is the legacy textbook rule for the legacy vLUT and the core rule for
// tables that match e8_decode.
//
// Kernels
//   vlut_build_kernel      full one-sided tables, one thread per entry
//   vlut_dot_kernel        sum_m q^m vLUT[idx_m] over encoded blocks
//   vlut_lds_kernel        matmul out[t,o] = s_o sum_k sum_m q^m vLUT_{a_tk}[idx]
//                          with per-(token, k-block) factorized tables in LDS:
//                            vLUT_a[idx(b)] = sum_j b_j <a, g_j> - q <a, c(b)>
//                          (8 + n_coarse floats instead of q^8 = 65536 at q = 4)
//   vlut_mfma_kernel       same product by decoding 2 x_hat (exact in fp16/bf16)
//                          into LDS and multiplying on the matrix cores
//   vlut_reduce_kernel     sums the split-K partials and applies s_o
#include <algorithm>

#include "codec_kernels.hpp"
#include "tables.hpp"
#include "vlut.hpp"

namespace coset {

// ---------------------------------------------------------------- helpers
__device__ __forceinline__ float load_act(const void* p, int dt, int64_t i)
{
    if (dt == DT_F32) return reinterpret_cast<const float*>(p)[i];
    uint16_t h = reinterpret_cast<const uint16_t*>(p)[i];
    if (dt == DT_BF16) return __uint_as_float((uint32_t)h << 16);
    return (float)__builtin_bit_cast(_Float16, h);
}

// 2 r(b) from the level word with the decode tables: U - q*(2c), U = 2Gb.
template <int Q>
__device__ __forceinline__ void two_r_lut(uint32_t w, const uint16_t* map, const uint64_t* coarse, int out[8])
{
    int b[8];
    unpack_word<Q>(w, Q, b);
    uint64_t c = coarse[map[w]];
    out[0] = 4 * b[0] - 2 * b[1] + b[7];
#pragma unroll
    for (int j = 1; j < 6; ++j) out[j] = 2 * (b[j] - b[j + 1]) + b[7];
    out[6] = 2 * b[6] + b[7];
    out[7] = b[7];
#pragma unroll
    for (int j = 0; j < 8; ++j) out[j] -= Q * (int)(int8_t)(uint8_t)(c >> (8 * j));
}

// ---------------------------------------------------------------- build
template <int Q>
__global__ void __launch_bounds__(256) vlut_build_kernel(const float* a, int64_t n_queries, uint32_t n_codes,
                                                        int q, int legacy, const uint16_t* map,
                                                        const uint64_t* coarse, float* vlut)
{
    int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (gid >= n_queries * (int64_t)n_codes) return;
    int64_t qi = gid / n_codes;
    uint32_t idx = (uint32_t)(gid - qi * n_codes);
    float r[8];
    if (Q == 2 || Q == 4) {
        int t[8];
        two_r_lut<Q>(idx, map, coarse, t);
#pragma unroll
        for (int j = 0; j < 8; ++j) r[j] = 0.5f * (float)t[j];
    } else {
        int b[8];
        float gb[8];
        unpack_word<0>(idx, q, b);
        lattice_point(b, gb);
        // the legacy vLUT projects one 8-vector at a time (contiguous rule)
        if (legacy)
            residual_from_point<true, false>(gb, (float)q, r);
        else
            residual_from_point<false, true>(gb, (float)q, r);
    }
    const float* av = a + 8 * qi;
    float acc = 0.f;
#pragma unroll
    for (int j = 0; j < 8; ++j) acc = __fmaf_rn(av[j], r[j], acc);
    vlut[gid] = acc;
}

// ---------------------------------------------------------------- lookup
__global__ void __launch_bounds__(256) vlut_dot_kernel(const void* words, int word_bytes_, int64_t n, int M,
                                                      int q, const float* vlut, float* out)
{
    int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    float acc = 0.f, w = 1.f;
    for (int m = 0; m < M; ++m) {
        uint32_t idx = word_bytes_ == 2 ? reinterpret_cast<const uint16_t*>(words)[i * M + m]
                                        : reinterpret_cast<const uint32_t*>(words)[i * M + m];
        acc = __fmaf_rn(w, vlut[idx], acc);
        w *= (float)q;
    }
    out[i] = acc;
}

// ---------------------------------------------------------------- LDS vLUT matmul
constexpr int kVlutThreads = 256;
constexpr int kVlutRowsPerThread = 2;
constexpr int kVlutTableFloats = 24 * (8 + kMaxCoarseVlut);  // TT * KBW <= 24

template <int Q, int M, int TT>
__global__ void __launch_bounds__(kVlutThreads) vlut_lds_kernel(VlutMatmulArgs p)
{
    // grid.x: row chunks of 512 rows; grid.y: k splits; grid.z: token tiles
    __shared__ float s_tab[kVlutTableFloats];
    const int nc = p.n_coarse;
    const int stride = 8 + nc;                    // floats per (token, k-block) table
    const int kbw = p.kb_per_chunk;               // k-blocks per LDS chunk
    const int t0 = blockIdx.z * TT;
    const int nt = min(TT, (int)(p.B - t0));
    const int64_t kb_total = p.K / 8;
    const int64_t ks_len = (kb_total + gridDim.y - 1) / gridDim.y;
    const int64_t k_begin = blockIdx.y * ks_len;
    const int64_t k_end = min(kb_total, k_begin + ks_len);
    const int64_t r0 = (int64_t)blockIdx.x * kVlutThreads * kVlutRowsPerThread;

    float acc[kVlutRowsPerThread][TT];
#pragma unroll
    for (int rr = 0; rr < kVlutRowsPerThread; ++rr)
#pragma unroll
        for (int t = 0; t < TT; ++t) acc[rr][t] = 0.f;

    for (int64_t kc = k_begin; kc < k_end; kc += kbw) {
        const int nk = (int)min((int64_t)kbw, k_end - kc);
        __syncthreads();
        // tables: T[t][k][j] = <a_tk, g_j> (j < 8), T[t][k][8 + c] = <a_tk, c>
        const int entries = nt * nk * stride;
        for (int e = threadIdx.x; e < entries; e += kVlutThreads) {
            int t = e / (nk * stride);
            int rem = e - t * nk * stride;
            int k = rem / stride;
            int j = rem - k * stride;
            int64_t base = (int64_t)(t0 + t) * p.K + (kc + k) * 8;
            float av[8];
#pragma unroll
            for (int i = 0; i < 8; ++i) av[i] = load_act(p.act, p.act_dtype, base + i);
            float v;
            if (j == 0) {
                v = 2.f * av[0];
            } else if (j < 7) {
                v = av[j] - av[j - 1];
            } else if (j == 7) {
                v = 0.f;
#pragma unroll
                for (int i = 0; i < 8; ++i) v += av[i];
                v *= 0.5f;
            } else {
                uint64_t c = p.coarse[j - 8];
                v = 0.f;
#pragma unroll
                for (int i = 0; i < 8; ++i) v = __fmaf_rn(av[i], (float)(int8_t)(uint8_t)(c >> (8 * i)), v);
                v *= 0.5f;
            }
            s_tab[(t * kbw + k) * stride + j] = v;
        }
        __syncthreads();
#pragma unroll
        for (int rr = 0; rr < kVlutRowsPerThread; ++rr) {
            int64_t row = r0 + threadIdx.x + rr * kVlutThreads;
            if (row >= p.rows) continue;
            const uint16_t* wrow = reinterpret_cast<const uint16_t*>(p.words) + (row * kb_total + kc) * M;
            for (int k = 0; k < nk; ++k) {
                float qm = 1.f;
#pragma unroll
                for (int m = 0; m < M; ++m) {
                    uint32_t w = wrow[k * M + m];
                    int cid = p.map[w];
                    int b[8];
                    unpack_word<Q>(w, Q, b);
#pragma unroll
                    for (int t = 0; t < TT; ++t) {
                        if (t >= nt) break;
                        const float* T = s_tab + (t * kbw + k) * stride;
                        float s = 0.f;
#pragma unroll
                        for (int j = 0; j < 8; ++j) s = __fmaf_rn((float)b[j], T[j], s);
                        s = __fmaf_rn(-(float)Q, T[8 + cid], s);
                        acc[rr][t] = __fmaf_rn(qm, s, acc[rr][t]);
                    }
                    qm *= (float)Q;
                }
            }
        }
    }
#pragma unroll
    for (int rr = 0; rr < kVlutRowsPerThread; ++rr) {
        int64_t row = r0 + threadIdx.x + rr * kVlutThreads;
        if (row >= p.rows) continue;
        for (int t = 0; t < nt; ++t)
            p.partial[((int64_t)blockIdx.y * p.B + t0 + t) * p.rows + row] = acc[rr][t];
    }
}

// ---------------------------------------------------------------- MFMA matmul
// Tile: 64 output rows x up to 64 tokens per workgroup (4 waves, one 16-row
// slice each), K split over grid.y.  Per step of 4 k-blocks (32 K values)
// each thread decodes one (row, k-block) pair to 8 halves of 2*x_hat in LDS;
// then each wave runs 16x16x16 MFMAs: A = activations (tokens x K) read
// straight from HBM/L2, B = the decoded slice (K x rows).
typedef _Float16 half4_t __attribute__((ext_vector_type(4)));
typedef short bf16x4_t __attribute__((ext_vector_type(4)));
typedef float float4_t __attribute__((ext_vector_type(4)));

constexpr int kMfmaRows = 64;
constexpr int kMfmaKStep = 32;  // K values per decode step (4 k-blocks)

template <int Q, int M, bool BF16>
__global__ void __launch_bounds__(256) vlut_mfma_kernel(VlutMatmulArgs p)
{
    __shared__ __align__(16) uint16_t s_b[kMfmaRows][kMfmaKStep + 4];  // +4 halves: bank skew
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int64_t kb_total = p.K / 8;
    const int64_t ks_len = ((kb_total + gridDim.y - 1) / gridDim.y + 3) / 4 * 4;
    const int64_t k_begin = blockIdx.y * ks_len;
    const int64_t k_end = min(kb_total, k_begin + ks_len);
    const int64_t r0 = (int64_t)blockIdx.x * kMfmaRows;
    const int64_t t_base = (int64_t)blockIdx.z * 64;  // token tile of up to 64
    const int n_tsub = (int)min((int64_t)4, (p.B - t_base + 15) / 16);

    float4_t acc[4];
#pragma unroll
    for (int s = 0; s < 4; ++s) acc[s] = (float4_t){0.f, 0.f, 0.f, 0.f};

    // this thread decodes row dr, k-block dk of each step
    const int dr = threadIdx.x >> 2;
    const int dk = threadIdx.x & 3;
    const int64_t drow = r0 + dr;

    for (int64_t kc = k_begin; kc < k_end; kc += 4) {
        int two_x[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) two_x[j] = 0;
        if (drow < p.rows && kc + dk < k_end) {
            const uint16_t* wp = reinterpret_cast<const uint16_t*>(p.words) + (drow * kb_total + kc + dk) * M;
            int wq = 1;
#pragma unroll
            for (int m = 0; m < M; ++m) {
                int tr[8];
                two_r_lut<Q>(wp[m], p.map, p.coarse, tr);
#pragma unroll
                for (int j = 0; j < 8; ++j) two_x[j] += wq * tr[j];
                wq *= Q;
            }
        }
        uint16_t hv[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            if (BF16) {
                hv[j] = (uint16_t)(__float_as_uint((float)two_x[j]) >> 16);  // exact: |2x| < 256
            } else {
                _Float16 h = (_Float16)two_x[j];                              // exact: |2x| < 2048
                hv[j] = *reinterpret_cast<uint16_t*>(&h);
            }
        }
        __syncthreads();  // previous step's MFMAs are done with s_b
        uint4 pk;
        pk.x = hv[0] | ((uint32_t)hv[1] << 16);
        pk.y = hv[2] | ((uint32_t)hv[3] << 16);
        pk.z = hv[4] | ((uint32_t)hv[5] << 16);
        pk.w = hv[6] | ((uint32_t)hv[7] << 16);
        *reinterpret_cast<uint2*>(&s_b[dr][dk * 8]) = make_uint2(pk.x, pk.y);
        *reinterpret_cast<uint2*>(&s_b[dr][dk * 8 + 4]) = make_uint2(pk.z, pk.w);
        __syncthreads();

#pragma unroll
        for (int kk = 0; kk < kMfmaKStep / 16; ++kk) {
            // B operand: K rows 4*(lane/16).. of this 16-K slice, column = row lane%16
            const int brow = wave * 16 + (lane & 15);
            const int kof = kk * 16 + 4 * (lane >> 4);
            uint2 bv = *reinterpret_cast<const uint2*>(&s_b[brow][kof]);
            const int64_t kglob = (kc * 8) + kof;
            for (int s = 0; s < n_tsub; ++s) {
                const int64_t tok = t_base + s * 16 + (lane & 15);
                uint2 av = make_uint2(0u, 0u);
                if (tok < p.B && kglob < k_end * 8)
                    av = *reinterpret_cast<const uint2*>(reinterpret_cast<const uint16_t*>(p.act) + tok * p.K + kglob);
                if (BF16) {
                    bf16x4_t A = *reinterpret_cast<bf16x4_t*>(&av);
                    bf16x4_t Bv = *reinterpret_cast<bf16x4_t*>(&bv);
                    acc[s] = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(A, Bv, acc[s], 0, 0, 0);
                } else {
                    half4_t A = *reinterpret_cast<half4_t*>(&av);
                    half4_t Bv = *reinterpret_cast<half4_t*>(&bv);
                    acc[s] = __builtin_amdgcn_mfma_f32_16x16x16f16(A, Bv, acc[s], 0, 0, 0);
                }
            }
        }
    }
    // D[token = 16 s + 4 (lane/16) + i][row = 16 wave + lane%16]
    const int64_t row = r0 + wave * 16 + (lane & 15);
    if (row < p.rows) {
        for (int s = 0; s < n_tsub; ++s) {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                int64_t tok = t_base + s * 16 + 4 * (lane >> 4) + i;
                if (tok < p.B) p.partial[((int64_t)blockIdx.y * p.B + tok) * p.rows + row] = acc[s][i];
            }
        }
    }
}

// ---------------------------------------------------------------- reduce
__global__ void __launch_bounds__(256) vlut_reduce_kernel(const float* partial, int splits, int64_t B,
                                                         int64_t rows, const float* scale, int scale_mode,
                                                         float mult, float* out)
{
    int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= B * rows) return;
    int64_t o = i % rows;
    float acc = 0.f;
    for (int s = 0; s < splits; ++s) acc += partial[(int64_t)s * B * rows + i];
    float sc = scale ? (scale_mode == 0 ? scale[o] : 1.f / scale[o]) : 1.f;
    out[i] = acc * mult * sc;
}

// ---------------------------------------------------------------- launchers
namespace {

template <int Q, int M>
hipError_t launch_lds(VlutMatmulArgs p, int splits, hipStream_t s)
{
    int TT = p.B >= 8 ? 8 : (p.B >= 4 ? 4 : (p.B >= 2 ? 2 : 1));
    p.kb_per_chunk = std::max(1, 24 / TT);
    dim3 grid((unsigned)((p.rows + kVlutThreads * kVlutRowsPerThread - 1) / (kVlutThreads * kVlutRowsPerThread)),
              (unsigned)splits, (unsigned)((p.B + TT - 1) / TT));
    switch (TT) {
    case 8: hipLaunchKernelGGL((vlut_lds_kernel<Q, M, 8>), grid, dim3(kVlutThreads), 0, s, p); break;
    case 4: hipLaunchKernelGGL((vlut_lds_kernel<Q, M, 4>), grid, dim3(kVlutThreads), 0, s, p); break;
    case 2: hipLaunchKernelGGL((vlut_lds_kernel<Q, M, 2>), grid, dim3(kVlutThreads), 0, s, p); break;
    default: hipLaunchKernelGGL((vlut_lds_kernel<Q, M, 1>), grid, dim3(kVlutThreads), 0, s, p); break;
    }
    return hipGetLastError();
}

template <int Q, int M>
hipError_t launch_mfma(const VlutMatmulArgs& p, int splits, hipStream_t s)
{
    dim3 grid((unsigned)((p.rows + kMfmaRows - 1) / kMfmaRows), (unsigned)splits, (unsigned)((p.B + 63) / 64));
    if (p.act_dtype == DT_BF16)
        hipLaunchKernelGGL((vlut_mfma_kernel<Q, M, true>), grid, dim3(256), 0, s, p);
    else
        hipLaunchKernelGGL((vlut_mfma_kernel<Q, M, false>), grid, dim3(256), 0, s, p);
    return hipGetLastError();
}

template <int Q>
hipError_t dispatch_m(const VlutMatmulArgs& p, int method, int splits, hipStream_t s)
{
    switch (p.M) {
#define COSET_M(MM) \
    case MM: return method == VLUT_METHOD_MFMA ? launch_mfma<Q, MM>(p, splits, s) : launch_lds<Q, MM>(p, splits, s);
    COSET_M(1) COSET_M(2) COSET_M(3) COSET_M(4)
#undef COSET_M
    default: return hipErrorInvalidValue;
    }
}

}  // namespace

hipError_t vlut_build(const float* a, int64_t n_queries, int q, int legacy, float* vlut, hipStream_t s)
{
    uint32_t n = 1;
    for (int i = 0; i < 8; ++i) n *= (uint32_t)q;
    int64_t total = n_queries * (int64_t)n;
    if (total == 0) return hipSuccess;
    dim3 grid((unsigned)((total + 255) / 256));
    if (q == 2 || q == 4) {
        const DecodeTables* t = nullptr;
        hipError_t e = get_decode_tables(q, legacy, &t);
        if (e != hipSuccess) return e;
        if (q == 4)
            hipLaunchKernelGGL(vlut_build_kernel<4>, grid, dim3(256), 0, s, a, n_queries, n, q, legacy, t->cid_map, t->coarse, vlut);
        else
            hipLaunchKernelGGL(vlut_build_kernel<2>, grid, dim3(256), 0, s, a, n_queries, n, q, legacy, t->cid_map, t->coarse, vlut);
    } else {
        hipLaunchKernelGGL(vlut_build_kernel<0>, grid, dim3(256), 0, s, a, n_queries, n, q, legacy,
                           (const uint16_t*)nullptr, (const uint64_t*)nullptr, vlut);
    }
    return hipGetLastError();
}

hipError_t vlut_dot(const void* words, int64_t n, int M, int q, const float* vlut, float* out, hipStream_t s)
{
    if (n == 0) return hipSuccess;
    hipLaunchKernelGGL(vlut_dot_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, words, word_bytes(q), n,
                       M, q, vlut, out);
    return hipGetLastError();
}

int vlut_default_splits(int64_t rows, int64_t B, int64_t K, int method)
{
    int64_t kb = K / 8;
    if (method == VLUT_METHOD_MFMA) {
        int64_t row_tiles = (rows + kMfmaRows - 1) / kMfmaRows;
        int64_t want = std::max<int64_t>(1, 512 / std::max<int64_t>(1, row_tiles));
        return (int)std::max<int64_t>(1, std::min<int64_t>(want, kb / 4));
    }
    int TT = B >= 8 ? 8 : (B >= 4 ? 4 : (B >= 2 ? 2 : 1));
    int64_t row_chunks = (rows + kVlutThreads * kVlutRowsPerThread - 1) / (kVlutThreads * kVlutRowsPerThread);
    int64_t tiles = (B + TT - 1) / TT;
    int64_t want = std::max<int64_t>(1, 256 / std::max<int64_t>(1, row_chunks * tiles));
    return (int)std::max<int64_t>(1, std::min<int64_t>(want, kb));
}

hipError_t vlut_matmul(VlutMatmulArgs p, int method, int splits, hipStream_t s)
{
    if (p.B == 0 || p.rows == 0) return hipSuccess;
    const DecodeTables* t = nullptr;
    hipError_t e = get_decode_tables(p.q, p.legacy, &t);
    if (e != hipSuccess) return e;
    p.map = t->cid_map;
    p.coarse = t->coarse;
    p.n_coarse = t->n_coarse;
    e = p.q == 4 ? dispatch_m<4>(p, method, splits, s) : dispatch_m<2>(p, method, splits, s);
    if (e != hipSuccess) return e;
    int64_t n = p.B * p.rows;
    float mult = method == VLUT_METHOD_MFMA ? 0.5f : 1.f;
    hipLaunchKernelGGL(vlut_reduce_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, p.partial, splits,
                       p.B, p.rows, p.scale, p.scale_mode, mult, p.out);
    return hipGetLastError();
}

}  // namespace coset
