// tables.hip -- per-device constant tables of the single-level decode.
//
// For q in {2, 4} every level word idx in [0, q^8) has the residual
//   r(b) = G b - q c(b),   c(b) = P(G b / q)          (codecs.py:164-166)
// and c(b) takes few distinct values (637 for the core rule at q = 4).  The
// tables store, per rule (core / legacy):
//   cid_map[idx]  uint16 id of c(b)
//   coarse[cid]   the 8 coordinates 2c as int8, packed in a uint64
// so 2r = 2Gb - q*(2c) needs two small lookups instead of a projection,
// plus the byte-lane form of the same sum (build_swar) and the coordinate
// pairs of r with their ids per word (build_pairs, the LDS vLUT's tables).  They
// are built once per device: a kernel evaluates c(b) for all q^8 words with
// the same device projection the codec uses, the host assigns dense ids in
// increasing key order, and the result is uploaded and kept for the life of
// the process.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <array>
#include <map>
#include <atomic>
#include <mutex>
#include <vector>

#include "codec_kernels.hpp"
#include "tables.hpp"

namespace coset {

template <bool LEGACY>
__global__ void __launch_bounds__(256) coarse_key_kernel(int q, uint32_t n, uint32_t* keys)
{
    uint32_t idx = blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= n) return;
    int b[8];
    unpack_word<0>(idx, q, b);
    float gb[8], z[8], c[8];
    lattice_point(b, gb);
    float qf = (float)q;
#pragma unroll
    for (int i = 0; i < 8; ++i) z[i] = __fdiv_rn(gb[i], qf);
    project<LEGACY, false>(z, c);
    uint32_t key = 0;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        int two_c = (int)__fmul_rn(2.f, c[i]);  // |2c| <= 7 for q <= 4
        key |= (uint32_t)((two_c + 8) & 15) << (4 * i);
    }
    keys[idx] = key;
}

namespace {

// U(b) = 2 G b for the digit vector of idx (same rows as lattice_point).
void two_gb(uint32_t idx, int q, int u[8])
{
    int b[8];
    for (int j = 7; j >= 0; --j) {
        b[j] = (int)(idx % (uint32_t)q);
        idx /= (uint32_t)q;
    }
    u[0] = 4 * b[0] - 2 * b[1] + b[7];
    for (int j = 1; j < 6; ++j) u[j] = 2 * (b[j] - b[j + 1]) + b[7];
    u[6] = 2 * b[6] + b[7];
    u[7] = b[7];
}

uint64_t pack_bytes(const int v[8], int bias)
{
    uint64_t w = 0;
    for (int j = 0; j < 8; ++j) w |= (uint64_t)(uint8_t)(v[j] + bias) << (8 * j);
    return w;
}

// Byte tables of the SWAR decode and the levels they can combine.
void build_swar(int q, uint32_t n, const std::vector<uint16_t>& map, const std::vector<uint64_t>& coarse,
                std::vector<uint64_t>& swar, int* max_m, int bias[5], int r2_min[8], int r2_max[8])
{
    int hi[256][8], lo[256][8];
    std::vector<std::array<int, 8>> cc(coarse.size());
    int min_hi = 0, max_hi = 0, min_lo = 0, max_lo = 0, min_c = 0, max_c = 0;
    for (int h = 0; h < 256; ++h) {
        if (q == 4)
            two_gb((uint32_t)h << 8, q, hi[h]);
        else
            for (int j = 0; j < 8; ++j) hi[h][j] = 0;  // q = 2 words fit in the low byte
        two_gb((uint32_t)h, q, lo[h]);
        for (int j = 0; j < 8; ++j) {
            min_hi = std::min(min_hi, hi[h][j]);
            max_hi = std::max(max_hi, hi[h][j]);
            min_lo = std::min(min_lo, lo[h][j]);
            max_lo = std::max(max_lo, lo[h][j]);
        }
    }
    for (size_t c = 0; c < coarse.size(); ++c)
        for (int j = 0; j < 8; ++j) {
            cc[c][j] = -q * (int)(int8_t)(uint8_t)(coarse[c] >> (8 * j));
            min_c = std::min(min_c, cc[c][j]);
            max_c = std::max(max_c, cc[c][j]);
        }
    int r_max = -1 << 20;  // largest coordinate of 2r over all words
    for (int j = 0; j < 8; ++j) {
        r2_min[j] = 1 << 20;
        r2_max[j] = -(1 << 20);
    }
    for (uint32_t i = 0; i < n; ++i) {
        int u[8];
        two_gb(i, q, u);
        for (int j = 0; j < 8; ++j) {
            const int v = u[j] + cc[map[i]][j];
            r_max = std::max(r_max, v);
            r2_min[j] = std::min(r2_min[j], v);
            r2_max[j] = std::max(r2_max[j], v);
        }
    }
    const int b_hi = -min_hi, b_lo = -min_lo, b_c = -min_c, b_l = b_hi + b_lo + b_c;
    swar.resize(512 + coarse.size());
    for (int h = 0; h < 256; ++h) {
        swar[h] = pack_bytes(hi[h], b_hi);
        swar[256 + h] = pack_bytes(lo[h], b_lo);
    }
    for (size_t c = 0; c < coarse.size(); ++c) swar[512 + c] = pack_bytes(cc[c].data(), b_c);
    // partial sums: T_hi + T_lo, then + C (= 2r + b_l)
    bool ok = max_hi + b_hi + max_lo + b_lo <= 255 && max_c + b_c <= 255 && r_max + b_l <= 255;
    const int l_max = r_max + b_l;
    int acc = l_max, off = b_l;
    *max_m = 0;
    for (int m = 1; m <= 4 && ok; ++m) {
        if (m > 1) {
            ok = acc * q <= 255 && acc * q + l_max <= 255;
            acc = acc * q + l_max;
            off = off * q + b_l;
        }
        if (ok) {
            *max_m = m;
            bias[m] = off;
        }
    }
}

// Dense ids of the four coordinate pairs of 2r = U(b) - q (2c) over all
// words, in increasing (2r_2p, 2r_2p+1) order per pair, and their values r.
bool build_pairs(int q, uint32_t n, const std::vector<uint16_t>& map, const std::vector<uint64_t>& coarse,
                 std::vector<uint32_t>& pair_map, std::vector<float2>& vals, int count[4])
{
    std::vector<std::array<int, 8>> r2(n);
    for (uint32_t i = 0; i < n; ++i) {
        int u[8];
        two_gb(i, q, u);
        for (int j = 0; j < 8; ++j) r2[i][j] = u[j] - q * (int)(int8_t)(uint8_t)(coarse[map[i]] >> (8 * j));
    }
    pair_map.assign(n, 0u);
    vals.assign(4 * kPairSlots, make_float2(0.f, 0.f));
    for (int p = 0; p < 4; ++p) {
        std::vector<std::pair<int, int>> keys(n);
        for (uint32_t i = 0; i < n; ++i) keys[i] = {r2[i][2 * p], r2[i][2 * p + 1]};
        std::vector<std::pair<int, int>> uniq(keys);
        std::sort(uniq.begin(), uniq.end());
        uniq.erase(std::unique(uniq.begin(), uniq.end()), uniq.end());
        if (uniq.size() > (size_t)kPairSlots) return false;
        count[p] = (int)uniq.size();
        for (size_t k = 0; k < uniq.size(); ++k)
            vals[kPairSlots * p + k] = make_float2(0.5f * (float)uniq[k].first, 0.5f * (float)uniq[k].second);
        for (uint32_t i = 0; i < n; ++i) {
            const uint32_t id = (uint32_t)(std::lower_bound(uniq.begin(), uniq.end(), keys[i]) - uniq.begin());
            pair_map[i] |= id << (8 * p);
        }
    }
    return true;
}

struct Slot {
    std::once_flag once;
    DecodeTables t{};
    hipError_t err = hipSuccess;
    std::atomic<bool> ready{false};   // set once the tables are built
};

std::mutex g_mu;
std::map<long, Slot*> g_slots;  // key: device * 64 + q * 2 + legacy

hipError_t build(int device, int q, int legacy, DecodeTables* out)
{
    hipError_t e;
    int cur = 0;
    if ((e = hipGetDevice(&cur)) != hipSuccess) return e;
    if (cur != device && (e = hipSetDevice(device)) != hipSuccess) return e;
    uint32_t n = 1;
    for (int i = 0; i < 8; ++i) n *= (uint32_t)q;
    uint32_t* d_keys = nullptr;
    std::vector<uint32_t> keys(n);
    std::vector<uint16_t> map(n);
    std::vector<uint64_t> coarse, swar;
    std::vector<uint32_t> pair_map;
    std::vector<float2> pair_vals;
    if ((e = hipMalloc(&d_keys, n * sizeof(uint32_t))) != hipSuccess) goto done;
    if (legacy)
        hipLaunchKernelGGL(coarse_key_kernel<true>, dim3((n + 255) / 256), dim3(256), 0, nullptr, q, n, d_keys);
    else
        hipLaunchKernelGGL(coarse_key_kernel<false>, dim3((n + 255) / 256), dim3(256), 0, nullptr, q, n, d_keys);
    if ((e = hipGetLastError()) != hipSuccess) goto done;
    if ((e = hipMemcpy(keys.data(), d_keys, n * sizeof(uint32_t), hipMemcpyDeviceToHost)) != hipSuccess) goto done;
    {
        std::vector<uint32_t> uniq(keys);
        std::sort(uniq.begin(), uniq.end());
        uniq.erase(std::unique(uniq.begin(), uniq.end()), uniq.end());
        if (uniq.size() > kMaxCoarse) {
            e = hipErrorInvalidValue;
            goto done;
        }
        for (uint32_t i = 0; i < n; ++i)
            map[i] = (uint16_t)(std::lower_bound(uniq.begin(), uniq.end(), keys[i]) - uniq.begin());
        coarse.resize(uniq.size());
        for (size_t c = 0; c < uniq.size(); ++c) {
            uint64_t packed = 0;
            for (int i = 0; i < 8; ++i) {
                int v = (int)((uniq[c] >> (4 * i)) & 15) - 8;
                packed |= (uint64_t)(uint8_t)(int8_t)v << (8 * i);
            }
            coarse[c] = packed;
        }
    }
    build_swar(q, n, map, coarse, swar, &out->swar_max_m, out->swar_bias, out->r2_min, out->r2_max);
    if (!build_pairs(q, n, map, coarse, pair_map, pair_vals, out->pair_count)) {
        e = hipErrorInvalidValue;
        goto done;
    }
    out->q = q;
    out->n_codes = n;
    out->n_coarse = (int)coarse.size();
    if ((e = hipMalloc((void**)&out->cid_map, n * sizeof(uint16_t))) != hipSuccess) goto done;
    if ((e = hipMalloc((void**)&out->coarse, coarse.size() * sizeof(uint64_t))) != hipSuccess) goto done;
    if ((e = hipMalloc((void**)&out->swar, swar.size() * sizeof(uint64_t))) != hipSuccess) goto done;
    if ((e = hipMemcpy((void*)out->cid_map, map.data(), n * sizeof(uint16_t), hipMemcpyHostToDevice)) != hipSuccess) goto done;
    if ((e = hipMemcpy((void*)out->swar, swar.data(), swar.size() * sizeof(uint64_t), hipMemcpyHostToDevice)) != hipSuccess)
        goto done;
    if ((e = hipMemcpy((void*)out->coarse, coarse.data(), coarse.size() * sizeof(uint64_t), hipMemcpyHostToDevice)) !=
        hipSuccess)
        goto done;
    if ((e = hipMalloc((void**)&out->pair_map, n * sizeof(uint32_t))) != hipSuccess) goto done;
    if ((e = hipMalloc((void**)&out->pair_vals, pair_vals.size() * sizeof(float2))) != hipSuccess) goto done;
    if ((e = hipMemcpy((void*)out->pair_map, pair_map.data(), n * sizeof(uint32_t), hipMemcpyHostToDevice)) !=
        hipSuccess)
        goto done;
    e = hipMemcpy((void*)out->pair_vals, pair_vals.data(), pair_vals.size() * sizeof(float2), hipMemcpyHostToDevice);
done:
    if (d_keys) (void)hipFree(d_keys);
    if (cur != device) (void)hipSetDevice(cur);
    return e;
}

}  // namespace

hipError_t get_decode_tables(int q, int legacy, const DecodeTables** out)
{
    int device = 0;
    hipError_t e = hipGetDevice(&device);
    if (e != hipSuccess) return e;
    if (q != 2 && q != 4) return hipErrorInvalidValue;
    Slot* s;
    {
        std::lock_guard<std::mutex> lk(g_mu);
        Slot*& ref = g_slots[(long)device * 64 + q * 2 + (legacy ? 1 : 0)];
        if (!ref) ref = new Slot();
        s = ref;
    }
    std::call_once(s->once, [&] {
        s->err = build(device, q, legacy, &s->t);
        if (s->err == hipSuccess) s->ready.store(true, std::memory_order_release);
    });
    if (s->err != hipSuccess) return s->err;
    *out = &s->t;
    return hipSuccess;
}

hipError_t find_decode_tables(int q, int legacy, const DecodeTables** out)
{
    int device = 0;
    hipError_t e = hipGetDevice(&device);
    if (e != hipSuccess) return e;
    if (q != 2 && q != 4) return hipErrorInvalidValue;
    std::lock_guard<std::mutex> lk(g_mu);
    auto it = g_slots.find((long)device * 64 + q * 2 + (legacy ? 1 : 0));
    if (it == g_slots.end() || !it->second->ready.load(std::memory_order_acquire)) return hipErrorNotReady;
    *out = &it->second->t;
    return hipSuccess;
}

}  // namespace coset
