// CDNA4 matrix-core helpers: v_mfma_f32_32x32x16_{f16,bf16} on 16-byte
// fragments. Lane layout (checked on gfx950 against an exact integer
// product), for C[32 x 32] += A[32 x 16] . B[16 x 32]:
//   A fragment: lane l holds A[l % 32][(l / 32) * 8 + i], i < 8
//   B fragment: lane l holds B[(l / 32) * 8 + i][l % 32]
//   C (16 floats): lane l, element i is C[(i / 4) * 8 + (l / 32) * 4 + i % 4][l % 32]
#pragma once

#include "common.hpp"

namespace pk {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf168 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

template <typename T>
struct Mma;
template <>
struct Mma<F16> {
    __device__ static inline f32x16 run(u32x4 a, u32x4 b, f32x16 c) {
        return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(half8, a), __builtin_bit_cast(half8, b), c, 0,
                                                      0, 0);
    }
};
template <>
struct Mma<BF16> {
    __device__ static inline f32x16 run(u32x4 a, u32x4 b, f32x16 c) {
        return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf168, a), __builtin_bit_cast(bf168, b), c,
                                                       0, 0, 0);
    }
};

// v_mfma_f32_16x16x32_{f16,bf16}, for C[16 x 16] += A[16 x 32] . B[32 x 16]:
//   A fragment: lane l holds A[l % 16][(l / 16) * 8 + i], i < 8
//   B fragment: lane l holds B[(l / 16) * 8 + i][l % 16]
//   C (4 floats): lane l, element i is C[(l / 16) * 4 + i][l % 16]
typedef float f32x4 __attribute__((ext_vector_type(4)));
template <typename T>
struct Mma16;
template <>
struct Mma16<F16> {
    __device__ static inline f32x4 run(u32x4 a, u32x4 b, f32x4 c) {
        return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(half8, a), __builtin_bit_cast(half8, b), c, 0,
                                                      0, 0);
    }
};
template <>
struct Mma16<BF16> {
    __device__ static inline f32x4 run(u32x4 a, u32x4 b, f32x4 c) {
        return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf168, a), __builtin_bit_cast(bf168, b), c,
                                                       0, 0, 0);
    }
};

// 16-bit storage bits of x in T (f16 IEEE RNE; bf16 the reference's formula).
template <typename T>
__device__ inline uint32_t bits16(float x);
template <>
__device__ inline uint32_t bits16<F16>(float x) {
    return (uint32_t)__builtin_bit_cast(uint16_t, F16::store(x));
}
template <>
__device__ inline uint32_t bits16<BF16>(float x) {
    return (uint32_t)BF16::store(x);
}

// Two f32 values rounded to nearest-even in T and packed (a in the low half):
// one v_cvt_pk_f16_f32 / v_cvt_pk_bf16_f32 on gfx950. For finite values the
// bf16 result equals BF16::store's.
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
template <typename T>
__device__ inline uint32_t pack2(float a, float b);
template <>
__device__ inline uint32_t pack2<F16>(float a, float b) {
    const f16x2 v = {(_Float16)a, (_Float16)b};
    return __builtin_bit_cast(uint32_t, v);
}
template <>
__device__ inline uint32_t pack2<BF16>(float a, float b) {
    const bf16x2 v = {(__bf16)a, (__bf16)b};
    return __builtin_bit_cast(uint32_t, v);
}

// f32 value of 16-bit storage bits in T.
template <typename T>
__device__ inline float from_bits16(uint32_t b);
template <>
__device__ inline float from_bits16<F16>(uint32_t b) {
    return (float)__builtin_bit_cast(_Float16, (uint16_t)b);
}
template <>
__device__ inline float from_bits16<BF16>(uint32_t b) {
    return BF16::load((uint16_t)b);
}

}  // namespace pk
