// Matrix-vector products for decode (m == 1 of Kernels.Matmul).
//
// matvec_nk_*: y[n] = sum_k x[k] * W[n, k] with W row-major [N, K] (the
// transposeB layout of Sources/Popcorn/Kernels/Matvec.metal:55-126; host names
// keep the reference's matvec_nk_simd_<x>_<w>_<out> pattern, with an _r1/_r2
// suffix for fewer rows per wave).
//
// The kernel is HBM-bound: W is read once, x is reused. A block of 4 waves
// stages x in LDS as f32, then each wave streams R rows of W with 16-byte
// non-temporal loads (U chunks per row in flight per lane), accumulates one
// f32 partial per row per lane, and reduces across the wave with DPP. Rows
// whose length is not a multiple of the 16-byte vector use a scalar loop
// (the reference's K % 4 != 0 tail, Matvec.metal:103-115).
//
// matvec*: y[n] = sum_k x[k] * W[k, n] (transposeW == 0, Matvec.metal:6-30),
// one thread per output column; not on the decode path.
#include "common.hpp"

namespace {

constexpr int kWaves = 4;
constexpr int kUnroll = 4;

template <typename X>
__device__ inline void stage_x(const typename X::storage *__restrict__ x, float *xs, uint32_t K) {
    for (uint32_t i = threadIdx.x; i < K; i += blockDim.x) xs[i] = X::load(x[i]);
    __syncthreads();
}

template <typename X, typename W, typename O, int R>
__device__ void matvec_nk(const typename X::storage *__restrict__ x, const typename W::storage *__restrict__ w,
                          typename O::storage *__restrict__ out, const MatvecConstants &p, float *xs) {
    constexpr int kV = pk::Vec<W>::kVec;
    const uint32_t K = p.K, N = p.N;
    stage_x<X>(x, xs, K);
    const uint32_t lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const uint32_t row0 = (blockIdx.x * kWaves + wave) * R;
    if (row0 >= N) return;

    float acc[R];
#pragma unroll
    for (int r = 0; r < R; ++r) acc[r] = 0.0f;

    const bool vec = (K % kV) == 0 && (reinterpret_cast<uintptr_t>(w) % 16) == 0;
    if (vec) {
        const uint32_t nchunks = K / kV;
        const typename W::storage *wr[R];
#pragma unroll
        for (int r = 0; r < R; ++r) wr[r] = w + (uint64_t)min(row0 + r, N - 1) * K;
        for (uint32_t c0 = lane; c0 < nchunks; c0 += 64 * kUnroll) {
            pk::Vec<W> wv[kUnroll][R];
#pragma unroll
            for (int u = 0; u < kUnroll; ++u) {
                uint32_t c = c0 + 64 * u;
                if (c < nchunks) {
#pragma unroll
                    for (int r = 0; r < R; ++r) wv[u][r].load_nt(wr[r] + (uint64_t)c * kV);
                }
            }
#pragma unroll
            for (int u = 0; u < kUnroll; ++u) {
                uint32_t c = c0 + 64 * u;
                if (c < nchunks) {
                    float xv[kV];
#pragma unroll
                    for (int e = 0; e < kV; ++e) xv[e] = xs[c * kV + e];
#pragma unroll
                    for (int r = 0; r < R; ++r) {
#pragma unroll
                        for (int e = 0; e < kV; ++e) acc[r] += xv[e] * wv[u][r].get(e);
                    }
                }
            }
        }
    } else {
        for (uint32_t k = lane; k < K; k += 64) {
            float xv = xs[k];
#pragma unroll
            for (int r = 0; r < R; ++r) {
                uint32_t row = min(row0 + r, N - 1);
                acc[r] += xv * W::load(w[(uint64_t)row * K + k]);
            }
        }
    }
#pragma unroll
    for (int r = 0; r < R; ++r) {
        float s = pk::wave_sum(acc[r]);
        if (lane == 0 && row0 + r < N) out[row0 + r] = O::store(s);
    }
}

template <typename X, typename W, typename O>
__device__ void matvec_kn(const typename X::storage *__restrict__ x, const typename W::storage *__restrict__ w,
                          typename O::storage *__restrict__ out, const MatvecConstants &p) {
    const uint32_t n = blockIdx.x * blockDim.x + threadIdx.x;
    if (n >= p.N) return;
    float acc = 0.0f;
    for (uint32_t k = 0; k < p.K; ++k) acc += X::load(x[k]) * W::load(w[(uint64_t)k * p.N + n]);
    out[n] = O::store(acc);
}

}  // namespace

// x is staged in dynamic LDS (K floats).
#define MATVEC_NK(name, X, W, O, R)                                                                   \
    POPCORN_KERNEL void __launch_bounds__(256)                                                        \
        name(const X::storage *x, const W::storage *w, O::storage *out, MatvecConstants p) {          \
        extern __shared__ float xs[];                                                                 \
        matvec_nk<X, W, O, R>(x, w, out, p, xs);                                                      \
    }
#define MATVEC_NK_ALL(base, X, W, O) \
    MATVEC_NK(base, X, W, O, 4)      \
    MATVEC_NK(base##_r2, X, W, O, 2) \
    MATVEC_NK(base##_r1, X, W, O, 1)

#define MATVEC_KN(name, X, W, O)                                                                    \
    POPCORN_KERNEL void __launch_bounds__(256)                                                      \
        name(const X::storage *x, const W::storage *w, O::storage *out, MatvecConstants p) {        \
        matvec_kn<X, W, O>(x, w, out, p);                                                           \
    }

using pk::BF16;
using pk::F16;
using pk::F32;

MATVEC_NK_ALL(matvec_nk_simd_f32_f32_f32, F32, F32, F32)
MATVEC_NK_ALL(matvec_nk_simd_f32_bf16_f32, F32, BF16, F32)
MATVEC_NK_ALL(matvec_nk_simd_bf16_bf16_f32, BF16, BF16, F32)
MATVEC_NK_ALL(matvec_nk_simd_bf16_bf16_bf16, BF16, BF16, BF16)
MATVEC_NK_ALL(matvec_nk_simd_f32_f16_f32, F32, F16, F32)
MATVEC_NK_ALL(matvec_nk_simd_f16_f16_f32, F16, F16, F32)
MATVEC_NK_ALL(matvec_nk_simd_f16_f16_f16, F16, F16, F16)

MATVEC_KN(matvec, F32, F32, F32)
MATVEC_KN(matvec_f16, F32, F16, F32)
MATVEC_KN(matvec_bf16, F32, BF16, F32)
MATVEC_KN(matvec_bf16_bf16_f32, BF16, BF16, F32)
MATVEC_KN(matvec_bf16_bf16_bf16, BF16, BF16, BF16)
MATVEC_KN(matvec_f16_f16_f32, F16, F16, F32)
MATVEC_KN(matvec_f16_f16_f16, F16, F16, F16)
