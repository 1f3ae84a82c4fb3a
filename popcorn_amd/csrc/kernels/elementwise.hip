// Elementwise kernels of the gated-MLP composition and the decode glue:
// GeluTanh (GeluTanh.metal:6-39), Mul (Mul.metal:6-29), Add (Add.metal:6-29),
// ScalarMul (ScalarMul.metal). Grid-stride over 16-byte vectors with a scalar
// tail; every element is widened to f32, computed, and stored with the
// dtype's rounding.
#include "common.hpp"

namespace {

template <typename T, typename Op>
__device__ void map2(const typename T::storage *__restrict__ a, const typename T::storage *__restrict__ b,
                     typename T::storage *__restrict__ out, uint32_t count, Op op) {
    constexpr int kV = pk::Vec<T>::kVec;
    const uint64_t stride = (uint64_t)gridDim.x * blockDim.x;
    const uint64_t tid = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    const bool aligned = ((reinterpret_cast<uintptr_t>(a) | reinterpret_cast<uintptr_t>(b) |
                           reinterpret_cast<uintptr_t>(out)) % 16) == 0;
    uint64_t nvec = aligned ? count / kV : 0;
    for (uint64_t i = tid; i < nvec; i += stride) {
        pk::Vec<T> va, vb;
        va.load(a + i * kV);
        vb.load(b + i * kV);
        typename T::storage r[kV];
#pragma unroll
        for (int e = 0; e < kV; ++e) r[e] = T::store(op(va.get(e), vb.get(e)));
        *reinterpret_cast<pk::u32x4 *>(out + i * kV) = *reinterpret_cast<const pk::u32x4 *>(r);
    }
    for (uint64_t i = nvec * kV + tid; i < count; i += stride) out[i] = T::store(op(T::load(a[i]), T::load(b[i])));
}

}  // namespace

#define UNARY(name, T, EXPR, CONSTS)                                                              \
    POPCORN_KERNEL void __launch_bounds__(256) name(const T::storage *x, T::storage *out, CONSTS p) { \
        map2<T>(x, x, out, p.count, [&](float v, float) { return EXPR; });                        \
    }
#define BINARY(name, T, EXPR, CONSTS)                                                           \
    POPCORN_KERNEL void __launch_bounds__(256)                                                 \
        name(const T::storage *a, const T::storage *b, T::storage *out, CONSTS p) {            \
        map2<T>(a, b, out, p.count, [&](float u, float v) { return EXPR; });                   \
    }

using pk::BF16;
using pk::F16;
using pk::F32;

UNARY(gelu_tanh, F32, pk::gelu_tanh(v), GeluTanhConstants)
UNARY(gelu_tanh_bf16, BF16, pk::gelu_tanh(v), GeluTanhConstants)
UNARY(gelu_tanh_f16, F16, pk::gelu_tanh(v), GeluTanhConstants)

BINARY(mul, F32, u *v, MulConstants)
BINARY(mul_bf16, BF16, u *v, MulConstants)
BINARY(mul_f16, F16, u *v, MulConstants)

BINARY(add, F32, u + v, AddConstants)
BINARY(add_bf16, BF16, u + v, AddConstants)
BINARY(add_f16, F16, u + v, AddConstants)

UNARY(scalar_mul, F32, v *p.scalar, ScalarMulConstants)
UNARY(scalar_mul_bf16, BF16, v *p.scalar, ScalarMulConstants)
UNARY(scalar_mul_f16, F16, v *p.scalar, ScalarMulConstants)
