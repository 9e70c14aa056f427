// CPU unit test of the counter-ring bookkeeping (coset_amd/csrc/counters.hpp).
// A "launch" takes a slot with ring_acquire and its kernel's last workgroup
// releases it; here the release is ring_release, called when the simulated
// launch finishes.
#include <atomic>
#include <cstdio>
#include <thread>
#include <vector>

#include "counters.hpp"

static int fails = 0;
#define CHECK(c) do { if (!(c)) { std::printf("FAIL %s:%d %s\n", __FILE__, __LINE__, #c); ++fails; } } while (0)

using coset::CounterRing;
using coset::ring_acquire;
using coset::ring_release;

struct Ring {
    std::vector<uint32_t> flags;
    CounterRing r;
    explicit Ring(uint32_t slots) : flags(slots, 1u)
    {
        r.slots = slots;
        r.release = flags.data();
    }
};

// The earlier scheme: slots handed out by a cursor alone, whether or not the
// previous holder has finished.  The held-back check below must catch it.
static int64_t acquire_by_cursor(CounterRing& r)
{
    const uint32_t s = r.cursor;
    r.cursor = (s + 1) % r.slots;
    r.release[s] = 0u;
    return s;
}

// One launch held back (never finishing) while `others` launches start and
// finish one after another; returns how many of them were handed its slot.
template <typename Acquire>
static int held_back_sharing(uint32_t slots, int others, Acquire acquire)
{
    Ring ring(slots);
    const int64_t held = acquire(ring.r);
    int shared = 0;
    for (int i = 0; i < others; ++i) {
        const int64_t s = acquire(ring.r);
        if (s == held) ++shared;
        if (s >= 0) ring_release(ring.r, s);
    }
    return shared;
}

int main()
{
    // launches that finish in order take the slots in ring order
    {
        Ring ring(5);
        for (int i = 0; i < 12; ++i) {
            const int64_t s = ring_acquire(ring.r);
            CHECK(s == i % 5);
            ring_release(ring.r, s);
        }
    }
    // a held-back launch keeps its slot through many laps of the ring, at the
    // real ring size and a tiny one; a cursor-only scheme hands it out again
    {
        CHECK(held_back_sharing(coset::kCounterSlots, 3 * (int)coset::kCounterSlots, ring_acquire) == 0);
        CHECK(held_back_sharing(3, 100, ring_acquire) == 0);
        CHECK(held_back_sharing(coset::kCounterSlots, 3 * (int)coset::kCounterSlots, acquire_by_cursor) == 3);
        CHECK(held_back_sharing(3, 100, acquire_by_cursor) == 33);
    }
    // released late, the slot is handed out again within one lap
    {
        Ring ring(4);
        const int64_t held = ring_acquire(ring.r);
        for (int i = 0; i < 10; ++i) ring_release(ring.r, ring_acquire(ring.r));
        ring_release(ring.r, held);
        bool back = false;
        for (int i = 0; i < 4 && !back; ++i) {
            const int64_t s = ring_acquire(ring.r);
            back = s == held;
            ring_release(ring.r, s);
        }
        CHECK(back);
    }
    // every slot held: no slot (the static schedule); one released: that one
    {
        Ring ring(6);
        std::vector<int> seen(6, 0);
        for (int i = 0; i < 6; ++i) {
            const int64_t s = ring_acquire(ring.r);
            CHECK(s >= 0 && s < 6);
            if (s >= 0 && s < 6) ++seen[s];
        }
        for (int c : seen) CHECK(c == 1);
        CHECK(ring_acquire(ring.r) == -1);
        ring_release(ring.r, 4);
        CHECK(ring_acquire(ring.r) == 4);
        CHECK(ring_acquire(ring.r) == -1);
    }
    // concurrent launches that finish out of order: no slot is ever held by
    // two launches at once
    {
        Ring ring(64);
        std::vector<std::atomic<int>> owner(64);
        for (auto& o : owner) o.store(0);
        std::atomic<int> doubles{0}, none{0};
        std::vector<std::thread> ts;
        for (int t = 0; t < 8; ++t)
            ts.emplace_back([&, t] {
                std::vector<int64_t> mine;
                for (int i = 0; i < 20000; ++i) {
                    const int64_t s = ring_acquire(ring.r);
                    if (s < 0) {
                        ++none;
                    } else {
                        if (owner[s].exchange(t + 1) != 0) ++doubles;
                        mine.push_back(s);
                    }
                    // finish a pseudo-random earlier launch of this thread, or hold on
                    const size_t k = (size_t)((i * 2654435761u + t) % 7);
                    if (!mine.empty() && k < 4) {
                        const size_t j = (size_t)((i * 40503u) % mine.size());
                        const int64_t f = mine[j];
                        mine.erase(mine.begin() + (long)j);
                        owner[f].store(0);
                        ring_release(ring.r, f);
                    }
                }
                for (int64_t f : mine) {
                    owner[f].store(0);
                    ring_release(ring.r, f);
                }
            });
        for (auto& th : ts) th.join();
        CHECK(doubles.load() == 0);
        int held = 0;
        for (uint32_t f : ring.flags) held += f != 1u;
        CHECK(held == 0);
        std::printf("concurrent: %d acquisitions found every slot held\n", none.load());
    }
    std::printf("%s (%d failures)\n", fails ? "FAILED" : "ok", fails);
    return fails ? 1 : 0;
}
