// RMSNorm over the last axis: y = (x * rsqrt(mean(x^2) + eps)) * w', with
// w' = (addOneToWeight ? 1 + w : w) when a weight is bound, else 1.
// Semantics of Sources/Popcorn/Kernels/RMSNorm.metal:6-41; the weight is f32
// for every x dtype (RMSNorm.metal:42-46), indexed by the column only.
//
// One block per row. Rows whose length is a multiple of the 16B vector width
// are read with 16B loads and kept in registers between the two passes when
// they fit (H <= kCache * vector width * block size), otherwise re-read.
#include "common.hpp"

namespace {

template <typename X, typename O>
__device__ void rmsnorm_row(const typename X::storage *__restrict__ x, const float *__restrict__ weight,
                            typename O::storage *__restrict__ out, const RMSNormConstants &p) {
    __shared__ float partial[16];
    constexpr int kV = pk::Vec<X>::kVec;
    constexpr int kCache = 4;
    const uint32_t H = p.H;
    const uint64_t base = (uint64_t)blockIdx.x * H;
    const typename X::storage *xr = x + base;
    typename O::storage *yr = out + base;
    const uint32_t tid = threadIdx.x, bs = blockDim.x;
    const bool vec = (H % kV) == 0 && (reinterpret_cast<uintptr_t>(x) % 16) == 0;
    const uint32_t nvec = H / kV;

    float acc = 0.0f;
    pk::Vec<X> cache[kCache];
    const bool cached = vec && nvec <= kCache * bs;
    if (vec) {
        if (cached) {
#pragma unroll
            for (int c = 0; c < kCache; ++c) {
                uint32_t i = tid + c * bs;
                if (i < nvec) {
                    cache[c].load(xr + (uint64_t)i * kV);
#pragma unroll
                    for (int e = 0; e < kV; ++e) {
                        float v = cache[c].get(e);
                        acc += v * v;
                    }
                }
            }
        } else {
            for (uint32_t i = tid; i < nvec; i += bs) {
                pk::Vec<X> v;
                v.load(xr + (uint64_t)i * kV);
#pragma unroll
                for (int e = 0; e < kV; ++e) {
                    float f = v.get(e);
                    acc += f * f;
                }
            }
        }
    } else {
        for (uint32_t i = tid; i < H; i += bs) {
            float v = X::load(xr[i]);
            acc += v * v;
        }
    }
    acc = pk::wave_sum(acc);
    const uint32_t wave = tid >> 6, nwaves = (bs + 63) >> 6;
    if ((tid & 63) == 0) partial[wave] = acc;
    __syncthreads();
    float total = 0.0f;
    for (uint32_t w = 0; w < nwaves; ++w) total += partial[w];
    const float scale = 1.0f / sqrtf(total / (float)H + p.eps);

    auto finish = [&](uint32_t col, float v) {
        float y = v * scale;
        if (p.hasWeight) {
            float w = weight[col];
            if (p.addOneToWeight) w = 1.0f + w;
            y *= w;
        }
        return y;
    };
    if (vec) {
        auto emit = [&](const pk::Vec<X> &v, uint32_t i) {
#pragma unroll
            for (int e = 0; e < kV; ++e) {
                uint32_t col = i * kV + e;
                yr[col] = O::store(finish(col, v.get(e)));
            }
        };
        if (cached) {
#pragma unroll
            for (int c = 0; c < kCache; ++c) {
                uint32_t i = tid + c * bs;
                if (i < nvec) emit(cache[c], i);
            }
        } else {
            for (uint32_t i = tid; i < nvec; i += bs) {
                pk::Vec<X> v;
                v.load(xr + (uint64_t)i * kV);
                emit(v, i);
            }
        }
    } else {
        for (uint32_t i = tid; i < H; i += bs) yr[i] = O::store(finish(i, X::load(xr[i])));
    }
}

}  // namespace

#define RMSNORM(name, X, O)                                                                      \
    POPCORN_KERNEL void __launch_bounds__(1024)                                                 \
        name(const X::storage *x, const float *weight, O::storage *out, RMSNormConstants p) { \
        rmsnorm_row<X, O>(x, weight, out, p);                                                   \
    }

using pk::BF16;
using pk::F16;
using pk::F32;

RMSNORM(rmsnorm, F32, F32)
RMSNORM(rmsnorm_bf16, BF16, BF16)
RMSNORM(rmsnorm_f16, F16, F16)
