// counters.hpp -- host-side bookkeeping of the per-device counter ring.
//
// Kernels that hand out work dynamically (the codec's tile schedule) keep
// their counters in a device array of kCounterRing unsigned counters,
// zero-initialised when the code object is loaded.  Each launch takes the
// next run of n consecutive counters from a host-side cursor, and the
// launch's last workgroup puts them back to zero, so every launch starts
// from zero without a memset.  Consecutive launches use different counters,
// so launches on different streams never share counters unless both run at
// the same time and kCounterRing / n launches were issued between them (at
// n = 2: 8192 launches while one is still running).  Plain C++ (no HIP), so
// the bookkeeping is unit-tested on the CPU.
#pragma once

#include <atomic>
#include <stdint.h>

namespace coset {

constexpr uint32_t kCounterRing = 1u << 14;  // counters per device (64 KiB)

// Offset of a run of n consecutive counters (1 <= n <= ring) for one launch.
// A run never crosses the end of the ring: when it would, it starts over at
// offset 0 (the counters skipped stay zero).  Thread-safe.
inline uint32_t ring_take(std::atomic<uint64_t>& cursor, uint32_t n, uint32_t ring)
{
    uint64_t cur = cursor.load(std::memory_order_relaxed);
    for (;;) {
        const uint64_t start = cur % ring;
        const uint64_t skip = start + n > ring ? ring - start : 0;
        if (cursor.compare_exchange_weak(cur, cur + skip + n, std::memory_order_relaxed))
            return (uint32_t)((cur + skip) % ring);
    }
}

}  // namespace coset
