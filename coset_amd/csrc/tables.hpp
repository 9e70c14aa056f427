// tables.hpp -- per-device decode tables (see tables.hip).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace coset {

constexpr int kMaxCoarse = 1024;  // distinct coarse points c(b) per table (637 for q = 4)

struct DecodeTables {
    int q;
    uint32_t n_codes;        // q^8
    int n_coarse;
    const uint16_t* cid_map;  // [n_codes]
    const uint64_t* coarse;   // [n_coarse], 8 x int8 of 2c
};

// Tables of the core (legacy = 0) or legacy residual rule for q in {2, 4} on
// the current device; built on first use (blocking), then cached.
hipError_t get_decode_tables(int q, int legacy, const DecodeTables** out);

}  // namespace coset
