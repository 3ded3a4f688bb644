// cc1d_fastdiv.hpp -- division of 32-bit unsigned values below 2^31 by a
// divisor fixed at launch, as a multiply-high, an add and a shift
// (T. Granlund, P. Montgomery, "Division by invariant integers using
// multiplication", PLDI 1994, section 4): with l = ceil(log2 d) and
// m = floor(2^32 (2^l - d) / d) + 1, floor(n / d) = (mulhi(m, n) + n) >> l
// for 0 <= n < 2^32; the sum needs 33 bits in general and fits in 32 when
// n < 2^31, which every caller guarantees. Host code builds the constants,
// kernels divide in scalar registers. No HIP header is needed, so host-only
// tests compile it with a plain C++ compiler.
#pragma once

#include <stdint.h>

#if defined(__HIPCC__)
#define CC1D_HD __host__ __device__
#else
#define CC1D_HD
#endif

namespace cc1d {

struct FastDiv {
    uint32_t d = 1, m = 1, l = 0;

    FastDiv() = default;
    // divisor in [1, 2^31]
    explicit FastDiv(uint32_t divisor) : d(divisor) {
        l = 0;
        while (l < 32 && ((uint64_t)1 << l) < divisor) ++l;
        m = (uint32_t)((((uint64_t)1 << 32) * (((uint64_t)1 << l) - divisor)) / divisor + 1);
    }
    // floor(n / d) for n < 2^31
    CC1D_HD uint32_t div(uint32_t n) const {
        const uint32_t hi = (uint32_t)(((uint64_t)m * n) >> 32);
        return (hi + n) >> l;
    }
};

}  // namespace cc1d
