// fp32 -> bf16 -> fp32 rounding (round to nearest, ties to even; NaN stays a quiet NaN): the
// operand conversion of the reference's bf16 matrix products (convert_tile in matmul_bf16 and its
// backward kernels, runtime/backend.rs:2209-2312).  The result is a float whose low 16 bits are 0,
// so a product of two such values is exact in fp32 and an fp32 MFMA accumulates bf16 products.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

__device__ __forceinline__ float bf16_round(float x) {
    uint32_t bits = __builtin_bit_cast(uint32_t, x);
    if ((bits & 0x7fffffffu) > 0x7f800000u) return __builtin_bit_cast(float, (bits | 0x00400000u) & 0xffff0000u);
    bits += 0x7fffu + ((bits >> 16) & 1u);
    return __builtin_bit_cast(float, bits & 0xffff0000u);
}
