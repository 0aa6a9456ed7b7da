// Host check of the device requantization fast paths: qa_mbqm_fast must
// equal the plain 128-bit form qa_mbqm (round(x * m * 2^-(31+shift)) with an
// __int128 product, qa_kernels.cpp:196-205) on edge values and on seeded
// random inputs covering every magnitude of x and m. Exit status 0 = equal.
#include <cstdio>
#include <random>

#include "qa_common.h"

int main(int argc, char** argv) {
    const long trials = argc > 1 ? atol(argv[1]) : 2000000;
    std::mt19937_64 r(12345);
    long bad = 0, n = 0;
    auto check = [&](int64_t x, int64_t m, int64_t s) {
        ++n;
        if (qa_mbqm(x, m, s) != qa_mbqm_fast(x, m, s)) {
            if (bad < 5)
                printf("mismatch x=%lld m=%lld shift=%lld\n", (long long)x,
                       (long long)m, (long long)s);
            ++bad;
        }
    };
    const int64_t xs[] = {0, 1, -1, (1LL << 32) - 1, 1LL << 32,
                          -(1LL << 32), 1LL << 53, -(1LL << 53),
                          (1LL << 62) - 1, -(1LL << 62) + 1, 1LL << 62,
                          -(1LL << 62), INT64_MAX, INT64_MIN + 1,
                          12345678901LL, -98765432109LL};
    const int64_t ms[] = {0, 1, -1, (1LL << 31) - 1, -(1LL << 31) + 1,
                          1LL << 30, -(1LL << 30), 1LL << 31, -(1LL << 31),
                          1518500250, -1518500250, 3};
    for (int64_t x : xs)
        for (int64_t m : ms)
            for (int s = -40; s <= 100; ++s) check(x, m, s);
    for (long i = 0; i < trials; ++i) {
        const int bits = (int)(r() % 63);
        const int64_t x =
            (int64_t)(r() >> (63 - bits)) * ((r() & 1) ? 1 : -1);
        int64_t m = (int64_t)(r() >> 33) * ((r() & 1) ? 1 : -1);
        if (r() % 8 == 0) m = (int64_t)(r() >> 31) * ((r() & 1) ? 1 : -1);
        check(x, m, (int64_t)(r() % 140) - 40);
    }
    printf("checked %ld, mismatches %ld\n", n, bad);
    return bad != 0;
}
