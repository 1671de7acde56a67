// Index arithmetic shared by the kernels and their host-side launch code.
// Plain C++ (no HIP headers), so host tests can compile it with g++.
#pragma once

#if defined(__HIPCC__)
#define MI_HD __host__ __device__
#else
#define MI_HD
#endif

namespace mi {

// Number of trips of a loop that visits first, first + step, first + 2*step,
// ... while below n, for 0 <= first, 0 <= n < 2^31 and 1 <= step <= 2^31.
// In that domain n - first + step - 1 < 2^32, so unsigned 32-bit arithmetic
// is exact, where the int form (n - first + step - 1 > INT_MAX once n is
// within one step of INT_MAX) overflows.
MI_HD inline unsigned strided_trips(unsigned first, unsigned n, unsigned step) {
    return first < n ? (n - first + step - 1u) / step : 0u;
}

}  // namespace mi
