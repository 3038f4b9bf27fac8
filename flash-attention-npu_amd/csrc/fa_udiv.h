// fa_udiv.h -- exact unsigned division by a run-time invariant divisor with a
// multiply-high, for index arithmetic in kernel loops (a 32-bit division is a
// ~20-instruction sequence on the GPU, scalar or vector). Callable from host
// and device; checked against the plain division by
// tests/host/fa_udiv_check.cpp.
//
// The method of Granlund and Montgomery, "Division by invariant integers using
// multiplication" (PLDI 1994), figure 4.1: for a divisor d >= 1 let
// l = ceil(log2 d) and m = floor(2^32 (2^l - d) / d) + 1 (fits 32 bits); then for
// every 32-bit n, with t = floor(m n / 2^32),
//   n / d = (t + ((n - t) >> min(l, 1))) >> max(l - 1, 0).
#pragma once
#include <stdint.h>

#if defined(__HIPCC__) || defined(__HIP__)
#define FA_UDIV_FN __host__ __device__ inline
#else
#define FA_UDIV_FN inline
#endif

namespace fa {

struct UDiv {
    uint32_t m;    // the multiplier
    uint32_t s1;   // min(l, 1)
    uint32_t s2;   // max(l - 1, 0)
    uint32_t d;    // the divisor
};

FA_UDIV_FN UDiv udiv_make(uint32_t d) {
    uint32_t l = 0;
    while (l < 32 && (1ull << l) < d) ++l;  // ceil(log2 d)
    UDiv u;
    u.m = (uint32_t)((((1ull << l) - d) << 32) / d + 1);
    u.s1 = l < 1 ? l : 1;
    u.s2 = l > 1 ? l - 1 : 0;
    u.d = d;
    return u;
}

FA_UDIV_FN uint32_t udiv_mulhi(uint32_t a, uint32_t b) { return (uint32_t)(((uint64_t)a * b) >> 32); }

// n / d
FA_UDIV_FN uint32_t udiv(const UDiv& u, uint32_t n) {
    const uint32_t t = udiv_mulhi(u.m, n);
    return (t + ((n - t) >> u.s1)) >> u.s2;
}

}  // namespace fa
