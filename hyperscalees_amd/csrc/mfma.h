// mfma.h -- CDNA4 matrix-core helpers shared by the GEMM kernels.
//
// 16x16 MFMA output layout (all variants used here): lane l holds
// D[4*(l/16) + v][l % 16] in accumulator element v.  For the operands, lane l
// supplies row (A) / column (B) l % 16 and a k-group selected by l / 16; A and
// B fragments are always loaded with the same k mapping, so the product does
// not depend on the instruction's internal k order.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace hses {

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef uint16_t u16x8 __attribute__((ext_vector_type(8)));

typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef float f32x2 __attribute__((ext_vector_type(2)));

// Two f32 -> packed bf16 bits (lo in bits 0..15), round to nearest even:
// one v_cvt_pk_bf16_f32.
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
    return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2){lo, hi}, bf16x2));
}

// Round-to-nearest-even f32 -> bf16 bits.
__device__ __forceinline__ uint16_t f2bf(float f) { return (uint16_t)pack_bf16x2(f, 0.0f); }
__device__ __forceinline__ float bf2f(uint16_t h) { return __uint_as_float((uint32_t)h << 16); }

__device__ __forceinline__ f32x4 mfma_f32(float a, float b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ f32x4 mfma_bf16(const u16x8& a, const u16x8& b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a),
                                                   __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
}

__device__ __forceinline__ u16x8 lds_u16x8(const uint16_t* p) {
    return *reinterpret_cast<const u16x8*>(p);
}

}  // namespace hses
