// Host check of the invariant-divisor division (flash-attention-npu_amd/csrc/
// fa_udiv.h, host and device code alike) against the plain division: every
// divisor up to 4096 on every numerator below 70000, on random 32-bit
// numerators and on the edge values around multiples of the divisor and the
// 32-bit ends; a few large divisors (2^31 - 1, 2^31, 2^31 + 1, 2^32 - 1 ...) on
// random numerators.
#include <cstdint>
#include <cstdio>
#include <random>

#include "fa_udiv.h"

static long failures = 0;

static void check(const fa::UDiv& u, uint32_t n) {
    const uint32_t got = fa::udiv(u, n), want = n / u.d;
    if (got != want && ++failures <= 20) std::printf("FAIL d=%u n=%u: got %u want %u\n", u.d, n, got, want);
}

int main() {
    std::mt19937_64 rng(7);
    long checked = 0;
    for (uint32_t d = 1; d <= 4096; ++d) {
        const fa::UDiv u = fa::udiv_make(d);
        for (uint32_t n = 0; n < 70000; ++n) check(u, n);
        for (int k = 0; k < 2000; ++k) check(u, (uint32_t)rng());
        const uint32_t edges[] = {0u, 1u, d - 1, d, d + 1, 2 * d - 1, 2 * d, 0x7fffffffu, 0x80000000u,
                                  0xfffffffeu, 0xffffffffu, 0xffffffffu - d, (0xffffffffu / d) * d,
                                  (0xffffffffu / d) * d - 1};
        for (uint32_t n : edges) check(u, n);
        checked += 70000 + 2000 + 14;
    }
    const uint32_t big[] = {65537u, 1000003u, 0x7fffffffu, 0x80000000u, 0x80000001u, 0xfffffffeu, 0xffffffffu};
    for (uint32_t d : big) {
        const fa::UDiv u = fa::udiv_make(d);
        for (int k = 0; k < 100000; ++k) check(u, (uint32_t)rng());
        check(u, d - 1);
        check(u, d);
        check(u, 0xffffffffu);
        checked += 100003;
    }
    std::printf("%ld divisions checked, %ld failures\n", checked, failures);
    return failures != 0;
}
