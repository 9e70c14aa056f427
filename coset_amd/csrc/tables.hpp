// tables.hpp -- per-device decode tables (see tables.hip).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace coset {

constexpr int kMaxCoarse = 1024;  // distinct coarse points c(b) per table (637 for q = 4)
constexpr int kPairSlots = 72;    // distinct values of one coordinate pair of r (<= 70 for q = 4)

struct DecodeTables {
    int q;
    uint32_t n_codes;        // q^8
    int n_coarse;
    const uint16_t* cid_map;  // [n_codes]
    const uint64_t* coarse;   // [n_coarse], 8 x int8 of 2c
    // Byte-lane (SWAR) form of 2r = U(b) - q (2c), U(b) = 2Gb split over the
    // two bytes of the level word (U is linear in the digits):
    //   swar[h]         U(digits of h << 8) + bias_hi   (q = 4; zero for q = 2)
    //   swar[256 + l]   U(digits of l) + bias_lo
    //   swar[512 + c]   -q (2c) + bias_c
    // as 8 unsigned bytes (byte j = coordinate j).  Every entry and every
    // partial sum stays in [0, 255], so the three are added as two 32-bit
    // words with no carry between bytes; M levels combine as acc = acc*q + L_m
    // while swar_max_m allows it, leaving 2 x_hat + swar_bias[M] per byte.
    const uint64_t* swar;     // [512 + n_coarse]
    int swar_max_m;           // largest M whose combined bytes stay < 256 (0: none)
    int swar_bias[5];         // byte offset of 2 x_hat after combining M levels
    // Coordinate-pair form of r: the pairs (r_2p, r_2p+1), p = 0..3, take few
    // distinct values (70, 68, 68, 55 for q = 4, core rule).
    //   pair_map[idx]            byte p = id of the word's pair p
    //   pair_vals[72 p + id]     that pair's two coordinates of r (zero past
    //                            pair_count[p])
    // so <a, r> = sum_p <(a_2p, a_2p+1), pair_vals[72 p + id_p]>.
    const uint32_t* pair_map;   // [n_codes]
    const float2* pair_vals;    // [4 * kPairSlots]
    int pair_count[4];
    // smallest and largest coordinate j of 2r over all words
    int r2_min[8], r2_max[8];
};

// Field offset of the 6-byte decoded weight format (vlut.hpp) for M levels of
// these tables: every coordinate of 2 x_hat = sum_m q^m 2r_m stored as
// floor(2 x_hat / 2) + off (6 bits; 5 bits for coordinate 7) with the common
// parity in one bit.  -1 when the range does not fit.
inline int decoded6_offset(const DecodeTables& t, int M)
{
    long lo[8], hi[8], qm = 1;
    for (int j = 0; j < 8; ++j) lo[j] = hi[j] = 0;
    for (int m = 0; m < M; ++m, qm *= t.q)
        for (int j = 0; j < 8; ++j) {
            lo[j] += qm * t.r2_min[j];
            hi[j] += qm * t.r2_max[j];
        }
    auto fl2 = [](long v) { return v >= 0 ? v / 2 : -((-v + 1) / 2); };  // floor(v / 2)
    long off = 0;
    for (int j = 0; j < 8; ++j) off = off > -fl2(lo[j]) ? off : -fl2(lo[j]);
    for (int j = 0; j < 8; ++j)
        if (fl2(hi[j]) + off > (j < 7 ? 63 : 31)) return -1;
    return (int)off;
}

// Tables of the core (legacy = 0) or legacy residual rule for q in {2, 4} on
// the current device; built on first use (blocking), then cached.
hipError_t get_decode_tables(int q, int legacy, const DecodeTables** out);

// The same tables only if they were already built on the current device
// (coset_init or an earlier call): never builds or allocates; returns
// hipErrorNotReady otherwise.
hipError_t find_decode_tables(int q, int legacy, const DecodeTables** out);

}  // namespace coset
