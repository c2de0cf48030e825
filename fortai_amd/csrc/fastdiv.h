// Division by a divisor that is fixed for a launch, as a multiply-high, an
// add and a shift instead of the ~25-instruction integer division sequence.
//
// Method: T. Granlund and P. L. Montgomery, "Division by Invariant Integers
// using Multiplication" (PLDI 1994), the round-up variant with a 33-bit
// multiplier 2^32 + mul:  l = ceil(log2 d),  mul = floor(2^32 (2^l - d) / d) + 1,
// n / d = (umulhi(n, mul) + n) >> l  for every 0 <= n < 2^31 (the sum stays
// below 2^32).  Built on the host (fast_div), applied on the device (div / mod).
// This header includes nothing: the HIP sources include it after the HIP
// runtime (which defines __host__ / __device__); a host-only checker defines
// them itself.
#pragma once
#include <stdint.h>

namespace fortai_hip {

struct FastDiv {
    uint32_t d = 1;      // the divisor (>= 1)
    uint32_t mul = 0;    // low 32 bits of the multiplier 2^32 + mul
    uint32_t shift = 0;  // l = ceil(log2 d)
};

inline FastDiv fast_div(uint32_t d) {
    FastDiv f;
    f.d = d < 1 ? 1 : d;
    uint32_t l = 0;
    while (l < 32 && (uint64_t(1) << l) < f.d) ++l;
    f.shift = l;
    f.mul = static_cast<uint32_t>(((uint64_t(1) << 32) * ((uint64_t(1) << l) - f.d)) / f.d + 1);
    return f;
}

__host__ __device__ inline uint32_t umulhi32(uint32_t a, uint32_t b) {
    return static_cast<uint32_t>((static_cast<uint64_t>(a) * b) >> 32);
}

// n / f.d and n % f.d for 0 <= n < 2^31
__host__ __device__ inline int div(int n, const FastDiv &f) {
    const uint32_t u = static_cast<uint32_t>(n);
    return static_cast<int>((umulhi32(u, f.mul) + u) >> f.shift);
}
__host__ __device__ inline int mod(int n, const FastDiv &f) { return n - div(n, f) * static_cast<int>(f.d); }

}  // namespace fortai_hip
