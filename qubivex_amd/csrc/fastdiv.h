// Division of 32-bit unsigned integers by a divisor fixed for a launch, as a multiply-high,
// an add, a subtract and two shifts (Granlund and Montgomery, "Division by Invariant
// Integers using Multiplication", PLDI 1994, Figure 4.1): for a divisor d >= 1 with
// l = ceil(log2 d) and m = floor(2^32 (2^l - d) / d) + 1,
//   t = mulhi(m, n);  n / d = (t + ((n - t) >> min(l, 1))) >> max(l - 1, 0)
// for every 32-bit n, with no intermediate overflow.  Plain C++ (usable on the host and
// in kernels) so the host tests can check it against `/`.
#pragma once
#include <stdint.h>

#if defined(__HIPCC__)
#define QV_HD __host__ __device__
#else
#define QV_HD
#endif

namespace qvkv {

struct FastDiv {
    uint32_t d, m, s1, s2;

    FastDiv() : d(1), m(1), s1(0), s2(0) {}
    explicit FastDiv(uint32_t divisor) : d(divisor ? divisor : 1) {
        uint32_t l = 0;
        while (l < 32 && (1ull << l) < d) l++;
        m = (uint32_t)(((1ull << 32) * ((1ull << l) - d)) / d + 1);
        s1 = l < 1 ? l : 1;
        s2 = l > 1 ? l - 1 : 0;
    }
    QV_HD uint32_t div(uint32_t n) const {
        const uint32_t t = (uint32_t)(((uint64_t)m * n) >> 32);
        return (t + ((n - t) >> s1)) >> s2;
    }
};

}  // namespace qvkv
