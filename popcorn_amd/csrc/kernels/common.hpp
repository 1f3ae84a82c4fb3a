// Device helpers shared by the gfx950 kernels: element load/store with the
// reference's conversion rules, 16-byte vector access, wave64 reductions.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <type_traits>

#include "popcorn_kernel_types.h"

#define POPCORN_KERNEL extern "C" __global__

namespace pk {

// ---- element types -------------------------------------------------------
// Storage types: f32 = float, f16 = _Float16, bf16 = raw uint16_t bits.
// Loads widen to f32; stores round from f32:
//   bf16 load  = bits << 16                  (PopcornDTypes.h:11)
//   bf16 store = (bits + 0x7fff + lsb) >> 16 (PopcornDTypes.h:29-34)
//   f16 store  = IEEE round-to-nearest-even   (PopcornDTypes.h:37)

struct F32 {
    using storage = float;
    static constexpr int kTag = 8;
    __device__ static inline float load(storage v) { return v; }
    __device__ static inline storage store(float x) { return x; }
};

struct F16 {
    using storage = _Float16;
    static constexpr int kTag = 9;
    __device__ static inline float load(storage v) { return (float)v; }
    __device__ static inline storage store(float x) { return (_Float16)x; }
};

struct BF16 {
    using storage = uint16_t;
    static constexpr int kTag = 10;
    __device__ static inline float load(storage v) { return __uint_as_float((uint32_t)v << 16); }
    __device__ static inline storage store(float x) {
        uint32_t bits = __float_as_uint(x);
        uint32_t lsb = (bits >> 16) & 1u;
        return (uint16_t)((bits + 0x7fffu + lsb) >> 16);
    }
};

// Value after a store/load round trip in dtype `tag` (POPCORN_DTYPE_*).
__device__ inline float round_through(uint32_t tag, float x) {
    if (tag == 10u) return BF16::load(BF16::store(x));
    if (tag == 9u) return F16::load(F16::store(x));
    return x;
}

// The same with the dtype fixed at compile time: straight-line code, for
// bodies that branch on the tag once (with_round_tag) instead of per element.
template <uint32_t TAG>
__device__ inline float round_as(float x) {
    if constexpr (TAG == 10u) return BF16::load(BF16::store(x));
    else if constexpr (TAG == 9u) return F16::load(F16::store(x));
    else return x;
}

// Calls f(std::integral_constant<uint32_t, TAG>) for the tag's rounding:
// 10 (bf16), 9 (f16) or 0 (f32, no rounding).
template <typename Fn>
__device__ inline void with_round_tag(uint32_t tag, Fn &&f) {
    if (tag == 10u) f(std::integral_constant<uint32_t, 10u>{});
    else if (tag == 9u) f(std::integral_constant<uint32_t, 9u>{});
    else f(std::integral_constant<uint32_t, 0u>{});
}

// ---- 16-byte vectors -------------------------------------------------------
// One 16B load/store per lane; kVec elements per vector.

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

template <typename T>
struct Vec {
    static constexpr int kVec = 16 / sizeof(typename T::storage);
    u32x4 raw;

    __device__ inline void load(const typename T::storage *p) { raw = *reinterpret_cast<const u32x4 *>(p); }
    // Streaming load: data read once (weights, KV) should not evict reused lines.
    __device__ inline void load_nt(const typename T::storage *p) {
        raw = __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(p));
    }
    __device__ inline float get(int i) const;
    __device__ inline void to_float(float *out) const {
#pragma unroll
        for (int i = 0; i < kVec; ++i) out[i] = get(i);
    }
};

template <>
__device__ inline float Vec<F32>::get(int i) const {
    uint32_t w = i == 0 ? raw.x : i == 1 ? raw.y : i == 2 ? raw.z : raw.w;
    return __uint_as_float(w);
}

template <>
__device__ inline float Vec<BF16>::get(int i) const {
    uint32_t w = (i >> 1) == 0 ? raw.x : (i >> 1) == 1 ? raw.y : (i >> 1) == 2 ? raw.z : raw.w;
    return (i & 1) ? __uint_as_float(w & 0xffff0000u) : __uint_as_float(w << 16);
}

template <>
__device__ inline float Vec<F16>::get(int i) const {
    uint32_t w = (i >> 1) == 0 ? raw.x : (i >> 1) == 1 ? raw.y : (i >> 1) == 2 ? raw.z : raw.w;
    uint16_t h = (i & 1) ? (uint16_t)(w >> 16) : (uint16_t)(w & 0xffffu);
    return (float)__builtin_bit_cast(_Float16, h);
}

// ---- wave64 reductions --------------------------------------------------
// DPP moves within 16-lane rows, then the gfx950 lane swaps across rows
// (v_permlane16_swap) and across the wave's halves (v_permlane32_swap), all
// in registers. Each swap step adds (or maxes) a lane's value and its
// partner's; addition is commutative, so every lane ends with the same bits.

template <int kCtrl>
__device__ inline float dpp(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), kCtrl, 0xf, 0xf, false));
}

// Sum over each 16-lane row, result in every lane of the row.
__device__ inline float row16_sum(float v) {
    v += dpp<0xB1>(v);   // quad_perm [1,0,3,2]
    v += dpp<0x4E>(v);   // quad_perm [2,3,0,1]
    v += dpp<0x141>(v);  // row_half_mirror
    v += dpp<0x140>(v);  // row_mirror
    return v;
}

__device__ inline float row16_max(float v) {
    v = fmaxf(v, dpp<0xB1>(v));
    v = fmaxf(v, dpp<0x4E>(v));
    v = fmaxf(v, dpp<0x141>(v));
    v = fmaxf(v, dpp<0x140>(v));
    return v;
}

// max and sum of v over lanes l and l ^ 32 in registers: v_permlane32_swap
// trades lanes 0-31 of its first operand with lanes 32-63 of its second, so
// with v in both, lane l holds v[l | 32] in the first result and
// v[l & 31] in the second (both halves add in the same order)
__device__ inline float pair32_max(float v) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
// max and sum over lanes l and l ^ 16 (v_permlane16_swap: odd 16-lane rows of
// the first operand trade places with even rows of the second)
__device__ inline float pair16_max(float v) {
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ inline float pair16_sum(float v) {
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ inline float pair32_sum(float v) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// Sum over each 32-lane half, result in every lane of the half.
__device__ inline float half32_sum(float v) { return pair16_sum(row16_sum(v)); }
__device__ inline float half32_max(float v) { return pair16_max(row16_max(v)); }

// Sum over the wave, result in every lane.
__device__ inline float wave_sum(float v) { return pair32_sum(half32_sum(v)); }
__device__ inline float wave_max(float v) { return pair32_max(half32_max(v)); }

// Sum over groups of `kLanes` consecutive lanes (power of two, 1..64),
// result in every lane of the group.
template <int kLanes>
__device__ inline float group_sum(float v) {
    if constexpr (kLanes >= 2) v += dpp<0xB1>(v);
    if constexpr (kLanes >= 4) v += dpp<0x4E>(v);
    if constexpr (kLanes >= 8) v += dpp<0x141>(v);
    if constexpr (kLanes >= 16) v += dpp<0x140>(v);
    if constexpr (kLanes >= 32) v = pair16_sum(v);
    if constexpr (kLanes >= 64) v = pair32_sum(v);
    return v;
}

template <int kLanes>
__device__ inline float group_max(float v) {
    if constexpr (kLanes >= 2) v = fmaxf(v, dpp<0xB1>(v));
    if constexpr (kLanes >= 4) v = fmaxf(v, dpp<0x4E>(v));
    if constexpr (kLanes >= 8) v = fmaxf(v, dpp<0x141>(v));
    if constexpr (kLanes >= 16) v = fmaxf(v, dpp<0x140>(v));
    if constexpr (kLanes >= 32) v = pair16_max(v);
    if constexpr (kLanes >= 64) v = pair32_max(v);
    return v;
}

// exp(x) through the hardware exp2 (v_exp_f32) with a log2(e) prescale.
__device__ inline float fast_exp(float x) { return __builtin_amdgcn_exp2f(x * 1.4426950408889634f); }

// GELU with tanh, GeluTanh.metal:6-11: 0.5*v*(1+tanh(clamp(k0*(v+k1*v^3),
// +-20))). tanh(t) = 1 - 2/(exp(2t)+1) for the clamped t; the absolute error
// of that form is a few ulp of 1, and the result adds tanh to 1.
__device__ inline float gelu_tanh(float v) {
    const float k0 = 0.7978845608028654f;
    const float k1 = 0.044715f;
    float inner = k0 * (v + k1 * v * v * v);
    inner = fminf(fmaxf(inner, -20.0f), 20.0f);
    float e = __builtin_amdgcn_exp2f(inner * (2.0f * 1.4426950408889634f));
    float t = 1.0f - 2.0f / (e + 1.0f);
    return 0.5f * v * (1.0f + t);
}

}  // namespace pk
