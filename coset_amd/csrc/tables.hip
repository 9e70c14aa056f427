// tables.hip -- per-device constant tables of the single-level decode.
//
// For q in {2, 4} every level word idx in [0, q^8) has the residual
//   r(b) = G b - q c(b),   c(b) = P(G b / q)          (codecs.py:164-166)
// and c(b) takes few distinct values (637 for the core rule at q = 4).  The
// tables store, per rule (core / legacy):
//   cid_map[idx]  uint16 id of c(b)
//   coarse[cid]   the 8 coordinates 2c as int8, packed in a uint64
// so 2r = 2Gb - q*(2c) needs two small lookups instead of a projection.  They
// are built once per device: a kernel evaluates c(b) for all q^8 words with
// the same device projection the codec uses, the host assigns dense ids in
// increasing key order, and the result is uploaded and kept for the life of
// the process.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <map>
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

struct Slot {
    std::once_flag once;
    DecodeTables t{};
    hipError_t err = hipSuccess;
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
    std::vector<uint64_t> coarse;
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
    out->q = q;
    out->n_codes = n;
    out->n_coarse = (int)coarse.size();
    if ((e = hipMalloc((void**)&out->cid_map, n * sizeof(uint16_t))) != hipSuccess) goto done;
    if ((e = hipMalloc((void**)&out->coarse, coarse.size() * sizeof(uint64_t))) != hipSuccess) goto done;
    if ((e = hipMemcpy((void*)out->cid_map, map.data(), n * sizeof(uint16_t), hipMemcpyHostToDevice)) != hipSuccess) goto done;
    e = hipMemcpy((void*)out->coarse, coarse.data(), coarse.size() * sizeof(uint64_t), hipMemcpyHostToDevice);
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
    std::call_once(s->once, [&] { s->err = build(device, q, legacy, &s->t); });
    if (s->err != hipSuccess) return s->err;
    *out = &s->t;
    return hipSuccess;
}

}  // namespace coset
