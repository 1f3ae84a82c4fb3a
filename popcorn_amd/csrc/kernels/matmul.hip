// General matmul C[m, n] = sum_k A[m, k] * B(^T)[k, n] with f32 accumulation:
// the semantics of Sources/Popcorn/Kernels/Matmul.metal:6-26 (dtype triples
// of Matmul.swift:222-229, plus f16 triples).
// matmul_tiled*: the SIMT fallback the Matmul descriptor runs for shapes and
// dtypes the MFMA GEMM does not take: 64x64 output tiles per 256-thread
// block, 4x4 outputs per thread, K staged through LDS in steps of 16.
// matmul*: the reference's host names, parameter list and launch geometry
// (one thread per output, thread x = row m, y = column n; Matmul.swift:63-64),
// for raw launches built like the reference's.
#include "common.hpp"

namespace {

constexpr int kTile = 64, kK = 16;

template <typename A, typename B, typename C>
__device__ void matmul_tiled(const typename A::storage *__restrict__ a, const typename B::storage *__restrict__ b,
                             typename C::storage *__restrict__ c, const MatmulConstants &p) {
    __shared__ float as[kK][kTile + 1];
    __shared__ float bs[kK][kTile + 1];
    const uint32_t M = p.M, N = p.N, K = p.K;
    const uint32_t m0 = blockIdx.y * kTile, n0 = blockIdx.x * kTile;
    const uint32_t tid = threadIdx.x;
    const uint32_t tm = (tid / 16) * 4, tn = (tid % 16) * 4;
    float acc[4][4] = {};
    for (uint32_t k0 = 0; k0 < K; k0 += kK) {
        for (uint32_t i = tid; i < kK * kTile; i += blockDim.x) {
            const uint32_t kk = i % kK, mm = i / kK;
            const uint32_t gm = m0 + mm, gk = k0 + kk;
            as[kk][mm] = (gm < M && gk < K) ? A::load(a[(uint64_t)gm * K + gk]) : 0.0f;
        }
        for (uint32_t i = tid; i < kK * kTile; i += blockDim.x) {
            uint32_t kk, nn;
            if (p.transposeB) {
                kk = i % kK;
                nn = i / kK;
            } else {
                nn = i % kTile;
                kk = i / kTile;
            }
            const uint32_t gn = n0 + nn, gk = k0 + kk;
            float v = 0.0f;
            if (gn < N && gk < K) v = B::load(p.transposeB ? b[(uint64_t)gn * K + gk] : b[(uint64_t)gk * N + gn]);
            bs[kk][nn] = v;
        }
        __syncthreads();
#pragma unroll
        for (int kk = 0; kk < kK; ++kk) {
            float av[4], bv[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                av[i] = as[kk][tm + i];
                bv[i] = bs[kk][tn + i];
            }
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int j = 0; j < 4; ++j) acc[i][j] += av[i] * bv[j];
        }
        __syncthreads();
    }
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const uint32_t gm = m0 + tm + i, gn = n0 + tn + j;
            if (gm < M && gn < N) c[(uint64_t)gm * N + gn] = C::store(acc[i][j]);
        }
}

// The reference's launch: the thread at (x, y) of the grid computes C[x, y];
// the grid strides in both dimensions, so any launch shape covers C.
template <typename A, typename B, typename C>
__device__ void matmul_ref(const typename A::storage *__restrict__ a, const typename B::storage *__restrict__ b,
                           typename C::storage *__restrict__ c, const MatmulConstants &p) {
    const uint32_t sx = gridDim.x * blockDim.x, sy = gridDim.y * blockDim.y;
    for (uint32_t m = blockIdx.x * blockDim.x + threadIdx.x; m < p.M; m += sx) {
        for (uint32_t n = blockIdx.y * blockDim.y + threadIdx.y; n < p.N; n += sy) {
            float acc = 0.0f;
            const uint64_t arow = (uint64_t)m * p.K;
            for (uint32_t k = 0; k < p.K; ++k) {
                const uint64_t bi = p.transposeB ? (uint64_t)n * p.K + k : (uint64_t)k * p.N + n;
                acc += A::load(a[arow + k]) * B::load(b[bi]);
            }
            c[(uint64_t)m * p.N + n] = C::store(acc);
        }
    }
}

}  // namespace

#define MATMUL(sfx, A, B, C)                                                                        \
    POPCORN_KERNEL void __launch_bounds__(256)                                                      \
        matmul_tiled##sfx(const A::storage *a, const B::storage *b, C::storage *c, MatmulConstants p) { \
        matmul_tiled<A, B, C>(a, b, c, p);                                                          \
    }                                                                                               \
    POPCORN_KERNEL void __launch_bounds__(1024)                                                     \
        matmul##sfx(const A::storage *a, const B::storage *b, C::storage *c, MatmulConstants p) {   \
        matmul_ref<A, B, C>(a, b, c, p);                                                            \
    }

using pk::BF16;
using pk::F16;
using pk::F32;

MATMUL(, F32, F32, F32)
MATMUL(_f16, F32, F16, F32)
MATMUL(_bf16, F32, BF16, F32)
MATMUL(_bf16_bf16_f32, BF16, BF16, F32)
MATMUL(_bf16_bf16_bf16, BF16, BF16, BF16)
MATMUL(_f16_f16_f32, F16, F16, F32)
MATMUL(_f16_f16_f16, F16, F16, F16)
