// CPU unit test of the counter-ring bookkeeping (coset_amd/csrc/counters.hpp).
#include <cstdio>
#include <thread>
#include <vector>

#include "counters.hpp"

static int fails = 0;
#define CHECK(c) do { if (!(c)) { std::printf("FAIL %s:%d %s\n", __FILE__, __LINE__, #c); ++fails; } } while (0)

int main()
{
    using coset::ring_take;
    // sequential runs are consecutive, wrap at the end and never cross it
    {
        std::atomic<uint64_t> cur{0};
        const uint32_t ring = 10;
        uint32_t want[] = {0, 3, 6, 0, 3, 6, 0};
        for (uint32_t w : want) CHECK(ring_take(cur, 3, ring) == w);
        std::atomic<uint64_t> c2{0};
        for (int i = 0; i < 100; ++i) {
            const uint32_t n = 1 + (uint32_t)(i * 7 % 10);
            const uint32_t o = ring_take(c2, n, ring);
            CHECK(o + n <= ring);
        }
        std::atomic<uint64_t> c3{0};
        for (int i = 0; i < 5; ++i) CHECK(ring_take(c3, ring, ring) == 0);   // the whole ring each time
    }
    // concurrent takers: within one lap of the ring no two runs overlap
    {
        const uint32_t ring = coset::kCounterRing, n = 2;
        const int threads = 8, per = 256;   // 8 * 256 * 2 = 4096 < ring: one lap
        std::atomic<uint64_t> cur{0};
        std::vector<std::vector<uint32_t>> got(threads);
        std::vector<std::thread> ts;
        for (int t = 0; t < threads; ++t)
            ts.emplace_back([&, t] {
                for (int i = 0; i < per; ++i) got[t].push_back(ring_take(cur, n, ring));
            });
        for (auto& th : ts) th.join();
        std::vector<int> use(ring, 0);
        for (auto& g : got)
            for (uint32_t o : g) {
                CHECK(o + n <= ring);
                for (uint32_t j = 0; j < n; ++j) ++use[o + j];
            }
        int twice = 0, once = 0;
        for (int u : use) {
            twice += u > 1;
            once += u == 1;
        }
        CHECK(twice == 0);
        CHECK(once == threads * per * (int)n);
    }
    // runs of different sizes over many laps stay inside the ring
    {
        std::atomic<uint64_t> cur{0};
        const uint32_t ring = coset::kCounterRing;
        for (int i = 0; i < 100000; ++i) {
            const uint32_t n = 1 + (uint32_t)((i * 2654435761u) % 300);
            const uint32_t o = ring_take(cur, n, ring);
            CHECK(o + n <= ring);
        }
    }
    std::printf("%s (%d failures)\n", fails ? "FAILED" : "ok", fails);
    return fails ? 1 : 0;
}
