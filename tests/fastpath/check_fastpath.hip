// CPU check of coset_amd/csrc/e8_fast.hpp against the C oracle (test
// infrastructure; built by tests/fastpath/Makefile, run by
// tests/test_fastpath.py).  The device header is compiled for the host here:
// every operation in project_fast is an IEEE fp32 operation on both.
//
//   check_fastpath lemma [limit]    every float |t| < 2^22: t - rint(t) is
//                                   exact, and |t - rint t| < 1/2 - 2^-20
//                                   implies custom_round(t) == rint(t)
//   check_fastpath blocks N seed    N blocks from each input family: where
//                                   project_fast succeeds its point equals
//                                   the oracle's projection bit for bit, and
//                                   fast_rows succeeds on the same blocks
//                                   with the exact rows of G^-1 y, and
//                                   fast_rows<true> (condition (5)) on a
//                                   superset of them, with the exact rows
//   check_fastpath dyadic q N       the decoders' residual G b - q P(G b / q)
//                                   through project_dyadic against the
//                                   oracle's (both distance rules): every
//                                   code for q^8 <= N, else N random codes
//                                   plus every code with digits in
//                                   {0, 1, q/2 - 1, q/2, q - 1}
//   check_fastpath fastres q N [T]  the same residual through
//                                   residual_dyadic<q> (q = 8, 16, 32) on T
//                                   threads: every code for q^8 <= N (all
//                                   2^32 at q = 16 with N = 4294967296),
//                                   else the structured codes and N random;
//                                   also that no residual coordinate
//                                   exceeds 3q/2 in magnitude
//   check_fastpath tabres q N [T]   the same residual through the integer
//                                   table form dyadic_level_acc<q> (q = 2,
//                                   4, 8, 16), codes as for fastres
//   check_fastpath divq S K [T]     div_by_recip<S>(a, b, RN(1/b)) against
//                                   the IEEE quotient a / b for every b
//                                   significand in [1, 2) and a = k / 2,
//                                   k = 0 .. K (signs of a and b varied),
//                                   plus, for S >= 2, random a of any
//                                   exponent in the helper's domain
//   check_fastpath u32div N         u32div against n / d: every d < 2^16 and
//                                   N random d, each with the n next to its
//                                   multiples, the ends of the range and
//                                   random n
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <atomic>
#include <random>
#include <thread>
#include <vector>

#include "e8_fast.hpp"
#include "fastdiv.hpp"

extern "C" {
float or_custom_round(float x);
void or_projection(const float* x, int64_t n, int legacy, float* y);
void or_residual(const int32_t* b, int q, int legacy, int strided, float* r);
}

static float from_bits(uint32_t u)
{
    float f;
    memcpy(&f, &u, 4);
    return f;
}

static uint32_t to_bits(float f)
{
    uint32_t u;
    memcpy(&u, &f, 4);
    return u;
}

static int lemma(float tie_limit)
{
    const uint32_t limit = to_bits(4194304.0f);  // 2^22: magnitudes below it
    const int n_threads = 8;
    std::atomic<uint64_t> bad_exact{0}, bad_round{0}, checked{0};
    std::vector<std::thread> pool;
    for (int th = 0; th < n_threads; ++th) {
        pool.emplace_back([&, th] {
            uint64_t be = 0, br = 0, ck = 0;
            for (uint32_t mag = th; mag < limit; mag += n_threads) {
                for (uint32_t sign = 0; sign < 2; ++sign) {
                    float t = from_bits(mag | (sign << 31));
                    float r = rintf(t);
                    float d = t - r;
                    if ((double)d != (double)t - (double)r) ++be;
                    if (fabsf(d) < tie_limit) {
                        ++ck;
                        if (or_custom_round(t) != r) ++br;
                    }
                }
            }
            bad_exact += be;
            bad_round += br;
            checked += ck;
        });
    }
    for (auto& t : pool) t.join();
    printf("lemma: %llu floats below the tie limit, %llu inexact t - rint(t), %llu custom_round != rint\n",
           (unsigned long long)checked.load(), (unsigned long long)bad_exact.load(),
           (unsigned long long)bad_round.load());
    return (bad_exact.load() || bad_round.load()) ? 1 : 0;
}

// Input families: each fills one block of 8.
static void family(int fam, std::mt19937_64& g, float x[8])
{
    std::normal_distribution<float> nd(0.f, 1.f);
    std::uniform_real_distribution<float> ud(0.f, 1.f);
    std::uniform_int_distribution<int> id(-8, 8);
    static const float scales[] = {1.f, 0.25f, 0.0625f, 3.f, 100.f, 1e4f, 1048576.f, 1e-20f};
    switch (fam) {
    case 0:  // Gaussian at several scales
    case 1: {
        float s = scales[g() % 8];
        for (int i = 0; i < 8; ++i) x[i] = nd(g) * s;
        break;
    }
    case 2:  // dyadic grid values (ties and exact lattice points)
        for (int i = 0; i < 8; ++i) x[i] = (float)id(g) / (float)(1 << (g() % 5));
        break;
    case 3:  // within a few ulp of half-integers and integers
        for (int i = 0; i < 8; ++i) {
            float base = 0.5f * (float)id(g);
            int k = (int)(g() % 9) - 4;
            float v = base;
            for (int s = 0; s < abs(k); ++s) v = nextafterf(v, k > 0 ? INFINITY : -INFINITY);
            x[i] = g() % 2 ? v : nd(g);
        }
        break;
    case 4: {  // near the boundary between a D8 point and a D8 + 1/2 point
        float p[8], q[8];
        int s = 0;
        for (int i = 0; i < 8; ++i) {
            p[i] = (float)id(g);
            s += (int)p[i];
        }
        if (s & 1) p[0] += 1.f;
        s = 0;
        for (int i = 0; i < 8; ++i) {
            q[i] = (float)id(g) + 0.5f;
            s += (int)floorf(q[i]);
        }
        if (s & 1) q[1] += 1.f;
        float lam = 0.5f + (ud(g) - 0.5f) * (g() % 2 ? 1e-3f : 1e-6f);
        for (int i = 0; i < 8; ++i) x[i] = p[i] + lam * (q[i] - p[i]) + nd(g) * 1e-7f;
        break;
    }
    case 5: {  // large, tiny, signed zeros, denormals, non-finite
        static const float sp[] = {0.f, -0.f, 1e-40f, -1e-40f, 2097151.f, -2097152.5f, 4194304.f,
                                   8388609.f, INFINITY, -INFINITY, NAN, 0.5f, -0.5f, 1.5f, -1.5f};
        for (int i = 0; i < 8; ++i) x[i] = g() % 3 ? sp[g() % 15] : nd(g);
        break;
    }
    case 6: {  // uniform in a box
        for (int i = 0; i < 8; ++i) x[i] = (ud(g) - 0.5f) * 16.f;
        break;
    }
    default: {  // tiny blocks (every level of them encodes to 0) and sparse ones (exact zeros among values)
        static const float tiny[] = {0.124f, 1e-2f, 1e-4f, 1e-6f, 9.5e-7f, 1e-9f, 1e-20f, 1e-38f, 1e-44f};
        const int kind = (int)(g() % 3);
        const float s = tiny[g() % 9];
        for (int i = 0; i < 8; ++i) {
            if (kind == 0)
                x[i] = fminf(fmaxf(nd(g) * s, -0.124f), 0.124f);
            else if (kind == 1)
                x[i] = g() % 2 ? (g() % 2 ? 0.f : -0.f) : nd(g) * s;
            else
                x[i] = g() % 3 ? (g() % 2 ? 0.f : -0.f) : nd(g) * (float)(1 << (g() % 4));
        }
        break;
    }
    }
}

static int blocks(long n, unsigned seed)
{
    const int n_fam = 8;
    int rc = 0;
    for (int fam = 0; fam < n_fam; ++fam) {
        std::mt19937_64 g(seed * 7919u + fam);
        long ok = 0, ok5 = 0, bad = 0, bad_rows = 0;
        float x[8], yf[8], yr[8];
        for (long it = 0; it < n; ++it) {
            family(fam, g, x);
            int rows[8], rows5[8];
            const bool fast_ok = coset::project_fast(x, yf);
            const bool rows_ok = coset::fast_rows(x, rows, coset::fast_in_range(x));
            // with condition (5): a superset of the blocks, the same rows where both decide
            const bool rows5_ok = coset::fast_rows<true>(x, rows5, coset::fast_in_range(x));
            if (fast_ok != rows_ok || (rows_ok && !rows5_ok)) {
                ++bad_rows;
                continue;
            }
            if (!rows5_ok) continue;
            ++ok5;
            or_projection(x, 1, 0, yr);
            // rows of G^-1 y_ref, exact in double
            double suf = 0.0, want[8];
            for (int r = 6; r >= 0; --r) {
                suf += (double)yr[r];
                if (r >= 1) want[r] = suf - (double)(7 - r) * yr[7];
            }
            want[0] = suf / 2.0 - 3.5 * (double)yr[7];
            want[7] = 2.0 * (double)yr[7];
            bool rows_match = true;
            for (int r = 0; r < 8; ++r) rows_match = rows_match && (double)rows5[r] == want[r];
            if (fast_ok) {
                ++ok;
                for (int r = 0; r < 8; ++r) rows_match = rows_match && (double)rows[r] == want[r];
            }
            if (!rows_match) {
                if (bad_rows < 5) {
                    printf("rows mismatch family %d:", fam);
                    for (int i = 0; i < 8; ++i) printf(" %.9g", x[i]);
                    printf("\n  fast rows:");
                    for (int i = 0; i < 8; ++i) printf(" %d", fast_ok ? rows[i] : rows5[i]);
                    printf("\n  ref rows: ");
                    for (int i = 0; i < 8; ++i) printf(" %.1f", want[i]);
                    printf("\n");
                }
                ++bad_rows;
            }
            if (fast_ok && memcmp(yf, yr, sizeof yf) != 0) {
                if (bad < 5) {
                    printf("mismatch family %d:", fam);
                    for (int i = 0; i < 8; ++i) printf(" %.9g", x[i]);
                    printf("\n  fast:");
                    for (int i = 0; i < 8; ++i) printf(" %g", yf[i]);
                    printf("\n  ref: ");
                    for (int i = 0; i < 8; ++i) printf(" %g", yr[i]);
                    printf("\n");
                }
                ++bad;
            }
        }
        printf("family %d: %ld blocks, fast path taken %ld (%.4f%%), with (5) %ld (%.4f%%), mismatches %ld, "
               "row mismatches %ld\n", fam, n, ok, 100.0 * ok / n, ok5, 100.0 * ok5 / n, bad, bad_rows);
        if (bad || bad_rows) rc = 1;
    }
    return rc;
}

static int residual_check(const int32_t b[8], int q, long* bad)
{
    float gb[8], z[8], c[8], r[8], ref0[8], ref1[8];
    const float h = 0.5f * (float)b[7];
    gb[0] = (float)(2 * b[0] - b[1]) + h;
    for (int i = 1; i < 6; ++i) gb[i] = (float)(b[i] - b[i + 1]) + h;
    gb[6] = (float)b[6] + h;
    gb[7] = h;
    for (int i = 0; i < 8; ++i) z[i] = gb[i] / (float)q;
    coset::project_dyadic(z, c);
    for (int i = 0; i < 8; ++i) r[i] = gb[i] - (float)q * c[i];
    or_residual(b, q, 0, 0, ref0);
    or_residual(b, q, 0, 1, ref1);
    if (memcmp(r, ref0, sizeof r) != 0 || memcmp(r, ref1, sizeof r) != 0) {
        if (*bad < 5) {
            printf("mismatch q=%d b=", q);
            for (int i = 0; i < 8; ++i) printf("%d ", b[i]);
            printf("\n");
        }
        ++*bad;
        return 1;
    }
    return 0;
}

// residual_dyadic<Q> (the decoders' fast residual straight from the digits)
// against the oracle under both distance rules, bit for bit
// TABLE: the residual from dyadic_level_acc (one level, shift 0) instead
template <int Q, bool TABLE = false>
static long fast_residual_check(const int32_t b[8], long* shown)
{
    float r[8], ref0[8], ref1[8];
    int bi[8];
    for (int i = 0; i < 8; ++i) bi[i] = b[i];
    if constexpr (TABLE) {
        static const std::vector<uint4> tab = [] {
            std::vector<uint4> t(7 * Q);
            for (int z = -2 * Q; z < 5 * Q; ++z) t[z + 2 * Q] = coset::dyadic_table_entry<Q>(z);
            return t;
        }();
        int acc2[8];
        coset::dyadic_level_acc<Q, true>(bi, tab.data(), 0, acc2);
        for (int i = 0; i < 8; ++i) r[i] = 0.5f * (float)(acc2[i] - Q);
    } else {
        coset::residual_dyadic<Q>(bi, r);
    }
    or_residual(b, Q, 0, 0, ref0);
    or_residual(b, Q, 0, 1, ref1);
    bool in_bound = true;  // |r_i| <= 3q/2 (div_by_recip's domain rests on it)
    for (int i = 0; i < 8; ++i) in_bound = in_bound && fabsf(r[i]) <= 1.5f * (float)Q;
    if (in_bound && memcmp(r, ref0, sizeof r) == 0 && memcmp(r, ref1, sizeof r) == 0) return 0;
    if (*shown < 5) {
        ++*shown;
        printf("mismatch q=%d b=", Q);
        for (int i = 0; i < 8; ++i) printf("%d ", b[i]);
        printf(" r=");
        for (int i = 0; i < 8; ++i) printf("%g ", r[i]);
        printf(" ref=");
        for (int i = 0; i < 8; ++i) printf("%g ", ref0[i]);
        printf("\n");
    }
    return 1;
}

// every code for q^8 <= n (threads over the leading digit pairs), else the
// 5^8 structured codes and n random ones
template <int Q, bool TABLE = false>
static int fast_residual(long n, int threads)
{
    long total = 1;
    for (int i = 0; i < 8; ++i) total *= Q;
    std::atomic<long> bad{0}, checked{0}, shown{0};
    if (total <= n) {
        std::atomic<int> next{0};
        auto work = [&]() {
            long my_bad = 0, my_checked = 0, my_shown = 0;
            for (;;) {
                const int hi = next.fetch_add(1);
                if (hi >= Q * Q) break;
                int32_t b[8];
                b[0] = hi / Q;
                b[1] = hi % Q;
                long rest = total / (Q * Q);
                for (long idx = 0; idx < rest; ++idx) {
                    long v = idx;
                    for (int j = 7; j >= 2; --j) {
                        b[j] = (int32_t)(v % Q);
                        v /= Q;
                    }
                    my_bad += fast_residual_check<Q, TABLE>(b, &my_shown);
                }
                my_checked += rest;
            }
            bad += my_bad;
            checked += my_checked;
            shown += my_shown;
        };
        std::vector<std::thread> pool;
        for (int t = 0; t < threads; ++t) pool.emplace_back(work);
        for (auto& t : pool) t.join();
    } else {
        long my_shown = 0, b_ = 0, c_ = 0;
        int32_t b[8];
        const int pick[5] = {0, 1, Q / 2 - 1, Q / 2, Q - 1};
        for (long idx = 0; idx < 390625; ++idx) {  // 5^8
            long v = idx;
            for (int j = 7; j >= 0; --j) {
                b[j] = pick[v % 5];
                v /= 5;
            }
            b_ += fast_residual_check<Q, TABLE>(b, &my_shown);
            ++c_;
        }
        std::mt19937_64 g(4321 + Q);
        for (long it = 0; it < n; ++it) {
            for (int j = 0; j < 8; ++j) b[j] = (int32_t)(g() % (uint64_t)Q);
            b_ += fast_residual_check<Q, TABLE>(b, &my_shown);
            ++c_;
        }
        bad += b_;
        checked += c_;
    }
    printf("%s residual q=%d: %ld codes, mismatches %ld\n", TABLE ? "table" : "fast", Q, checked.load(),
           bad.load());
    return bad ? 1 : 0;
}

// div_by_recip<S> against the IEEE quotient: every significand of b in
// [1, 2) (the quotient's rounding does not depend on b's exponent in the
// helper's domain), a = k / 2 for k = 0 .. K with the four sign pairs on
// every 16th b, and for S >= 2 eight random a per b with exponents from
// 2^-1 to 2^46 and b scaled by 2^-64 .. 2^64
template <int S>
static int divq(long K, int threads)
{
    std::atomic<long> bad{0}, checked{0}, shown{0};
    std::atomic<long> next{0};
    constexpr long kChunk = 1 << 12;
    auto work = [&]() {
        long my_bad = 0, my_checked = 0;
        std::mt19937_64 g;
        for (;;) {
            const long s0 = next.fetch_add(kChunk);
            if (s0 >= (1L << 23)) break;
            g.seed(977 + s0);
            for (long sig = s0; sig < s0 + kChunk; ++sig) {
                const float b = from_bits(0x3f800000u | (uint32_t)sig);
                volatile float one = 1.f;
                const float y = one / b;
                auto check = [&](float a, float bb, float yy) {
                    const float got = coset::div_by_recip<S>(a, bb, yy);
                    volatile float va = a, vb = bb;
                    const float want = va / vb;
                    ++my_checked;
                    if (to_bits(got) != to_bits(want)) {
                        ++my_bad;
                        if (shown.fetch_add(1) < 5)
                            printf("mismatch S=%d a=%a b=%a got=%a want=%a\n", S, a, bb, got, want);
                    }
                };
                for (long k = 0; k <= K; ++k) {
                    const float a = 0.5f * (float)k;
                    check(a, b, y);
                    if ((sig & 15) == 0 && k > 0) {
                        check(-a, b, y);
                        check(a, -b, -y);
                        check(-a, -b, -y);
                    }
                }
                if (S >= 2) {
                    for (int t = 0; t < 8; ++t) {
                        const uint64_t h = g();
                        const int ea = (int)(h % 48) - 1, eb = (int)((h >> 8) % 129) - 64;
                        const float a = ldexpf(from_bits(0x3f800000u | (uint32_t)(h >> 40 & 0x7fffff)), ea);
                        const float bb = ldexpf(b, eb), yy = ldexpf(y, -eb);
                        check((h >> 63) ? -a : a, bb, yy);
                    }
                }
            }
        }
        bad += my_bad;
        checked += my_checked;
    };
    std::vector<std::thread> pool;
    for (int t = 0; t < threads; ++t) pool.emplace_back(work);
    for (auto& t : pool) t.join();
    printf("divq S=%d K=%ld: %ld quotients, mismatches %ld\n", S, K, checked.load(), bad.load());
    return bad ? 1 : 0;
}

static int u32div_check(long n_random)
{
    std::mt19937_64 g(2024);
    long bad = 0, checked = 0;
    auto one = [&](uint32_t d) {
        const coset::U32Div dv = coset::u32div_of(d);
        auto at = [&](uint32_t n) {
            ++checked;
            if (coset::u32div(n, dv) != n / d) {
                if (++bad <= 5) printf("mismatch n=%u d=%u got=%u\n", n, d, coset::u32div(n, dv));
            }
        };
        at(0u);
        at(0xffffffffu);
        at(0xffffffffu - 1u);
        for (int t = 0; t < 16; ++t) {
            const uint64_t k = g() % (0xffffffffull / d + 1);
            const uint64_t m = k * d;
            if (m > 0) at((uint32_t)(m - 1));
            if (m <= 0xffffffffull) at((uint32_t)m);
            if (m + 1 <= 0xffffffffull) at((uint32_t)(m + 1));
            at((uint32_t)g());
        }
    };
    for (uint32_t d = 1; d < (1u << 16); ++d) one(d);
    for (int k = 16; k < 32; ++k) {
        one(1u << k);
        one((1u << k) - 1u);
        one((1u << k) + 1u);
    }
    one(0xffffffffu);
    for (long t = 0; t < n_random; ++t) one(((uint32_t)g() >> (g() % 32)) | 1u);
    printf("u32div: %ld quotients, mismatches %ld\n", checked, bad);
    return bad ? 1 : 0;
}

static int dyadic(int q, long n)
{
    long total = 1, bad = 0, checked = 0;
    for (int i = 0; i < 8; ++i) total *= q;
    int32_t b[8];
    if (total <= n) {
        for (long idx = 0; idx < total; ++idx) {
            long v = idx;
            for (int j = 7; j >= 0; --j) {
                b[j] = (int32_t)(v % q);
                v /= q;
            }
            residual_check(b, q, &bad);
            ++checked;
        }
    } else {
        const int pick[5] = {0, 1, q / 2 - 1, q / 2, q - 1};
        for (long idx = 0; idx < 390625; ++idx) {  // 5^8
            long v = idx;
            for (int j = 7; j >= 0; --j) {
                b[j] = pick[v % 5];
                v /= 5;
            }
            residual_check(b, q, &bad);
            ++checked;
        }
        std::mt19937_64 g(1234 + q);
        for (long it = 0; it < n; ++it) {
            for (int j = 0; j < 8; ++j) b[j] = (int32_t)(g() % (uint64_t)q);
            residual_check(b, q, &bad);
            ++checked;
        }
    }
    printf("dyadic q=%d: %ld codes, mismatches %ld\n", q, checked, bad);
    return bad ? 1 : 0;
}

int main(int argc, char** argv)
{
    if (argc >= 4 && !strcmp(argv[1], "dyadic")) return dyadic(atoi(argv[2]), atol(argv[3]));
    if (argc >= 4 && !strcmp(argv[1], "tabres")) {
        const int q = atoi(argv[2]);
        const long n = atol(argv[3]);
        const int th = argc >= 5 ? atoi(argv[4]) : 1;
        if (q == 2) return fast_residual<2, true>(n, th);
        if (q == 4) return fast_residual<4, true>(n, th);
        if (q == 8) return fast_residual<8, true>(n, th);
        if (q == 16) return fast_residual<16, true>(n, th);
        fprintf(stderr, "tabres: q must be 2, 4, 8 or 16\n");
        return 2;
    }
    if (argc >= 4 && !strcmp(argv[1], "fastres")) {
        const int q = atoi(argv[2]);
        const long n = atol(argv[3]);
        const int th = argc >= 5 ? atoi(argv[4]) : 1;
        if (q == 8) return fast_residual<8>(n, th);
        if (q == 16) return fast_residual<16>(n, th);
        if (q == 32) return fast_residual<32>(n, th);
        fprintf(stderr, "fastres: q must be 8, 16 or 32\n");
        return 2;
    }
    if (argc >= 3 && !strcmp(argv[1], "u32div")) return u32div_check(atol(argv[2]));
    if (argc >= 4 && !strcmp(argv[1], "divq")) {
        const int steps = atoi(argv[2]);
        const long k = atol(argv[3]);
        const int th = argc >= 5 ? atoi(argv[4]) : 1;
        if (steps == 0) return divq<0>(k, th);
        if (steps == 1) return divq<1>(k, th);
        if (steps == 2) return divq<2>(k, th);
        fprintf(stderr, "divq: steps must be 0, 1 or 2\n");
        return 2;
    }
    // an optional second argument replaces the tie limit (a looser one must fail)
    if (argc >= 2 && !strcmp(argv[1], "lemma")) return lemma(argc >= 3 ? strtof(argv[2], nullptr) : coset::kFastTieLimit);
    if (argc >= 4 && !strcmp(argv[1], "blocks")) return blocks(atol(argv[2]), (unsigned)atoi(argv[3]));
    fprintf(stderr, "usage: %s lemma [limit] | blocks N seed | dyadic q N | fastres q N [threads] | tabres q N [threads] | divq steps K [threads] | u32div N\n", argv[0]);
    return 2;
}
