// probes.hpp -- measurement kernels (probes.hip; the C2 streaming probe in
// hnlq_lut.hip).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace coset {

hipError_t launch_probe_empty(int grid, int threads, int lds_bytes, uint32_t* out, hipStream_t s);
// 16-byte loads per thread the read probe needs for `bytes` at this launch
// shape (1, 2, 4, ..., 32), or -1 when more would be needed
int probe_read_loads(int64_t bytes, int grid, int threads);
hipError_t launch_probe_read(const void* src, int64_t bytes, int grid, int threads, uint32_t* out, hipStream_t s);
// the C2 round trip's launch, schedule, loads and stores without its lattice
// arithmetic (staged: with its decode-table staging)
// VALU issue-rate probe: kind 0 fp32 FMA chains, 1 compare + select chains
hipError_t launch_probe_valu(int kind, int grid, int iters, float* out, hipStream_t s);
hipError_t launch_c2_stream_probe(const float* x, int64_t n, uint32_t* packed, float* out, int staged, hipStream_t s);

}  // namespace coset
