// counters.hpp -- host-side bookkeeping of the per-device counter ring.
//
// Kernels that hand out work dynamically (the codec's tile schedule) take a
// pair of counters per launch from a device array of kCounterSlots pairs,
// zero-initialised when the code object is loaded.  The launch's last
// workgroup puts its pair back to zero and then sets the slot's release flag
// to 1; the flags live in host-visible memory, so the host reads them.  A
// slot is handed to a launch only while its flag reads 1, i.e. once every
// earlier launch that held it has finished, whatever order streams and
// event waits give the launches: two launches never share a pair, however
// long one of them is held back.  When every slot is held (kCounterSlots
// launches in flight), the launch takes its static schedule instead.
// Plain C++ (no HIP), so the bookkeeping is unit-tested on the CPU.
#pragma once

#include <mutex>
#include <stdint.h>

namespace coset {

constexpr uint32_t kCounterSlots = 1u << 13;    // counter pairs per device
constexpr uint32_t kCounterRing = 2 * kCounterSlots;  // counters per device (64 KiB)

struct CounterRing {
    std::mutex mu;
    uint32_t cursor = 0;          // next slot to try
    uint32_t slots = kCounterSlots;
    uint32_t* release = nullptr;  // [slots]: 1 = free, 0 = held by a launch (written by the GPU)
};

// A free slot for one launch, its flag set to 0 (held), or -1 when every
// slot is held.  Slots are tried in ring order from the one after the last
// handed out, so a slot is reused as late as possible.  Thread-safe.
inline int64_t ring_acquire(CounterRing& r)
{
    std::lock_guard<std::mutex> lock(r.mu);
    for (uint32_t i = 0; i < r.slots; ++i) {
        const uint32_t s = (r.cursor + i) % r.slots;
        if (__atomic_load_n(&r.release[s], __ATOMIC_ACQUIRE) == 1u) {
            __atomic_store_n(&r.release[s], 0u, __ATOMIC_RELAXED);
            r.cursor = (s + 1) % r.slots;
            return s;
        }
    }
    return -1;
}

// Hands a slot back from the host: the launch that took it never ran (its
// launch call failed).  A kernel that ran releases its slot itself.
inline void ring_release(CounterRing& r, int64_t s)
{
    __atomic_store_n(&r.release[s], 1u, __ATOMIC_RELEASE);
}

}  // namespace coset
