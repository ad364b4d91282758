// Division of non-negative 31-bit integers by a launch-invariant divisor with one multiply-high
// (Granlund & Montgomery, "Division by Invariant Integers using Multiplication", 1994): the
// rank-generic index decodes of unfold/select_axis would otherwise spend most of their time in
// the GPU's multi-instruction integer divide.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

struct FastDiv {
    uint32_t d = 1;
    uint32_t m = 1;
    uint32_t s = 0;

    FastDiv() = default;
    __host__ explicit FastDiv(uint32_t divisor) : d(divisor ? divisor : 1) {
        s = 0;
        while ((uint64_t(1) << s) < d) ++s;
        m = static_cast<uint32_t>(((uint64_t(1) << 32) * ((uint64_t(1) << s) - d)) / d + 1);
    }
    // n < 2^31.
    __device__ __forceinline__ uint32_t div(uint32_t n) const {
        uint32_t t = __umulhi(n, m);
        return (t + n) >> s;
    }
    __device__ __forceinline__ uint32_t mod(uint32_t n) const { return n - div(n) * d; }
};
