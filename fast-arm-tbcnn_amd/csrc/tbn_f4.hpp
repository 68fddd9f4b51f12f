// fp4 (E2M1) building blocks of TBN mode, shared by the TBN GEMM
// (tbn_mode.hip) and the TBN convolution (tbn_conv.hip).
//
// -1, 0 and +1 are exact E2M1 values: codes 0xA, 0x0 and 0x2.  With ternary
// activations and +-1 weights both in fp4, every product of
// v_mfma_scale_f32_32x32x64_f8f6f4 (unit scales) is exact and every partial
// sum is an integer of magnitude at most K, exact in the fp32 accumulators
// while K <= 2^24.  Operand lane layout (32 x 32 x 64): lane l holds row (or
// column) l % 32, the 32 values k = 32 (l / 32) .. +31 in four dwords, value
// k at nibble k % 8 of dword (k % 32) / 8 (low nibble first).
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

#include "mfma_core.hpp"

namespace tbnk {

typedef int i32x4_t __attribute__((ext_vector_type(4)));
typedef int i32x8_t __attribute__((ext_vector_type(8)));

constexpr uint32_t kF4Plus = 0x2u, kF4Minus = 0xAu;

// One 32 x 32 x 64 fp4 product-accumulate (formats 4 / 4, scales 2^0).
__device__ __forceinline__ f32x16_t mfma_f4(i32x4_t a, i32x4_t b, f32x16_t c) {
    const i32x8_t a8 = {a[0], a[1], a[2], a[3], 0, 0, 0, 0};
    const i32x8_t b8 = {b[0], b[1], b[2], b[3], 0, 0, 0, 0};
    return __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(a8, b8, c, 4, 4, 0, 127, 0, 127);
}

// The ternarization of TBN mode as an fp4 code: v < lo -> -1, v > hi -> +1,
// else 0 (NaN gives 0).  tbn-runtime/src/operators/quantized_gemm_neon.cpp:
// 93-113 and tbn-runtime/src/operators/conv2d.cpp:561-566,583-588.
__device__ __forceinline__ uint32_t ternary_f4(float v, float lo, float hi) {
    return v < lo ? kF4Minus : (v > hi ? kF4Plus : 0u);
}

// 8 BinaryMatrix bits (bit 1 = -1) -> 8 fp4 codes: bit e moved to bit 4 e + 3
// over the +1 code (0x2 | 0x8 = 0xA is -1).
__device__ __forceinline__ uint32_t bits_word(uint32_t b) {
    uint32_t x = b & 0xFFu;
    x = (x | (x << 12)) & 0x000F000Fu;
    x = (x | (x << 6)) & 0x03030303u;
    x = (x | (x << 3)) & 0x11111111u;
    return 0x22222222u | (x << 3);
}

}  // namespace tbnk
