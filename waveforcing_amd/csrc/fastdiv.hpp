// Division by a launch-invariant divisor with a multiply-high and a shift
// (Granlund-Montgomery round-up method), for the 32-bit index arithmetic of
// the page-table kernels.  Valid for numerators n < 2^31 and divisors >= 1.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace wf {

struct FastDiv {
  uint32_t d;
  uint32_t mul;
  uint32_t shift;

  FastDiv() = default;
  explicit FastDiv(uint32_t divisor) : d(divisor), mul(0), shift(0) {
    // Smallest s with 2^s >= d; then mul = ceil(2^(32+s) / d) - 2^32 fits in
    // 32 bits and n / d == (mulhi(n, mul) + n) >> s for n < 2^31.
    uint32_t s = 0;
    while ((1ull << s) < divisor) ++s;
    shift = s;
    const uint64_t one = 1;
    mul = static_cast<uint32_t>(((one << 32) * ((one << s) - divisor)) / divisor + 1);
  }

  __host__ __device__ inline uint32_t div(uint32_t n) const {
#if defined(__HIP_DEVICE_COMPILE__)
    const uint32_t hi = __umulhi(n, mul);
#else
    const uint32_t hi = static_cast<uint32_t>((static_cast<uint64_t>(n) * mul) >> 32);
#endif
    return (hi + n) >> shift;
  }
  __host__ __device__ inline void divmod(uint32_t n, uint32_t& q, uint32_t& r) const {
    q = div(n);
    r = n - q * d;
  }
};

}  // namespace wf
