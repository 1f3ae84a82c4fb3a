// Matmul with f32 output and at least one f32 operand on the matrix cores:
// C[M, N] = A[M, K] . B, B as [N, K] (transposeB) or [K, N], in the
// reference's MPP combinations f32 x f32, f32 x bf16 and bf16 x f32
// (Matmul.swift:203-214, mpp_matmul_*_f32[_tb]). bf16 operands widen to f32
// exactly as they are staged, so every product is an f32 product and the
// sums are f32 (v_mfma_f32_16x16x4_f32; lane layout: A[l % 16][l / 16],
// B[l / 16][l % 16], C rows 4 (l / 16) + i of column l % 16).
//
// A block of 4 waves takes a 128 x 128 tile of C, each wave 64 x 64 (4 x 4
// MFMA tiles); a step stages 16 values of K for the tile's rows of A and of
// B^T in LDS (double-buffered, the next step's loads in registers). Product
// 4 s' + s of a step takes k = 4 (l / 16) + s from every lane, so one
// 16-byte read of a row gives a lane its operands for the step's four
// products. Rows past M and N read row M - 1 / N - 1 and are not stored;
// values past K read as zeros.
#include <type_traits>

#include "mfma.hpp"

namespace {

using pk::f32x4;

constexpr int BM = 128, BN = 128, BK = 16;
constexpr int LDK = BK + 4;  // LDS row pitch (floats): 16 rows a quarter-wave reads fall in distinct banks

template <typename T>
struct Src;
template <>
struct Src<pk::F32> {
    using storage = float;
};
template <>
struct Src<pk::BF16> {
    using storage = uint16_t;
};

// 4 values of row `row` at k .. k + 3 (zeros past K) as f32.
template <typename T>
__device__ inline f32x4 load4(const typename Src<T>::storage *base, uint64_t row, uint32_t ld, uint32_t k, uint32_t K) {
    f32x4 v = {0.0f, 0.0f, 0.0f, 0.0f};
    if constexpr (std::is_same<T, pk::F32>::value) {
        if (k + 4 <= K) {
            const float4 f = *reinterpret_cast<const float4 *>(base + row * ld + k);
            v = f32x4{f.x, f.y, f.z, f.w};
        } else {
#pragma unroll
            for (int e = 0; e < 4; ++e)
                if (k + e < K) v[e] = base[row * ld + k + e];
        }
    } else {
        if (k + 4 <= K) {
            const uint2 w = *reinterpret_cast<const uint2 *>(base + row * ld + k);
            v = f32x4{__uint_as_float(w.x << 16), __uint_as_float(w.x & 0xffff0000u), __uint_as_float(w.y << 16),
                      __uint_as_float(w.y & 0xffff0000u)};
        } else {
#pragma unroll
            for (int e = 0; e < 4; ++e)
                if (k + e < K) v[e] = __uint_as_float((uint32_t)base[row * ld + k + e] << 16);
        }
    }
    return v;
}

template <typename TA, typename TB, bool TRANSB>
__device__ void gemm_f32(const typename Src<TA>::storage *__restrict__ A, const typename Src<TB>::storage *__restrict__ B,
                         float *__restrict__ C, const MatmulConstants &p) {
    __shared__ __attribute__((aligned(16))) float sA[2][BM * LDK];
    __shared__ __attribute__((aligned(16))) float sB[2][BN * LDK];  // B^T: a row per column of C

    const uint32_t M = p.M, N = p.N, K = p.K;
    const uint32_t nM = (M + BM - 1) / BM;
    const uint32_t pm = blockIdx.x % nM, pn = blockIdx.x / nM;
    const uint32_t bm = pm * BM, bn = pn * BN;
    const uint32_t t = threadIdx.x, lane = t & 63, wave = t >> 6;
    const uint32_t g = lane >> 4, c16 = lane & 15;
    const uint32_t wm = (wave >> 1) * 64, wn = (wave & 1) * 64;

    // staging: runs of 4 values; A (and B^T) runs c = t + 256 j: row c / 4,
    // k 4 (c % 4); a [K, N] B: k row c / 32, columns 4 (c % 32) .. + 3
    f32x4 ra[2], rb[2];
    auto gload = [&](uint32_t k0) {
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const uint32_t c = t + 256 * j;
            ra[j] = load4<TA>(A, min(bm + (c >> 2), M - 1), K, k0 + 4 * (c & 3), K);
            if constexpr (TRANSB) {
                rb[j] = load4<TB>(B, min(bn + (c >> 2), N - 1), K, k0 + 4 * (c & 3), K);
            } else {
                const uint32_t kr = k0 + (c >> 5), n = bn + 4 * (c & 31);
                f32x4 v = {0.0f, 0.0f, 0.0f, 0.0f};
                if (kr < K) {
                    if (n + 4 <= N) {
                        v = load4<TB>(B, kr, N, n, N);
                    } else {
#pragma unroll
                        for (int e = 0; e < 4; ++e) {
                            const uint32_t ne = min(n + e, N - 1);
                            if constexpr (std::is_same<TB, pk::F32>::value) v[e] = B[(uint64_t)kr * N + ne];
                            else v[e] = __uint_as_float((uint32_t)B[(uint64_t)kr * N + ne] << 16);
                        }
                    }
                }
                rb[j] = v;
            }
        }
    };
    auto lstore = [&](int st) {
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const uint32_t c = t + 256 * j;
            *reinterpret_cast<f32x4 *>(&sA[st][(c >> 2) * LDK + 4 * (c & 3)]) = ra[j];
            if constexpr (TRANSB) {
                *reinterpret_cast<f32x4 *>(&sB[st][(c >> 2) * LDK + 4 * (c & 3)]) = rb[j];
            } else {
#pragma unroll
                for (int e = 0; e < 4; ++e) sB[st][(4 * (c & 31) + e) * LDK + (c >> 5)] = rb[j][e];
            }
        }
    };

    f32x4 acc[4][4];
#pragma unroll
    for (int mi = 0; mi < 4; ++mi)
#pragma unroll
        for (int ni = 0; ni < 4; ++ni) acc[mi][ni] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};

    auto compute = [&](int st) {
        f32x4 a[4], b[4];
#pragma unroll
        for (int mi = 0; mi < 4; ++mi) a[mi] = *reinterpret_cast<const f32x4 *>(&sA[st][(wm + mi * 16 + c16) * LDK + 4 * g]);
#pragma unroll
        for (int ni = 0; ni < 4; ++ni) b[ni] = *reinterpret_cast<const f32x4 *>(&sB[st][(wn + ni * 16 + c16) * LDK + 4 * g]);
#pragma unroll
        for (int s = 0; s < 4; ++s)
#pragma unroll
            for (int mi = 0; mi < 4; ++mi)
#pragma unroll
                for (int ni = 0; ni < 4; ++ni)
                    acc[mi][ni] = __builtin_amdgcn_mfma_f32_16x16x4f32(a[mi][s], b[ni][s], acc[mi][ni], 0, 0, 0);
    };

    const uint32_t steps = (K + BK - 1) / BK;
    if (steps > 0) {
        gload(0);
        lstore(0);
        __syncthreads();
    }
    for (uint32_t it = 0; it < steps; ++it) {
        const int st = (int)(it & 1);
        if (it + 1 < steps) gload((it + 1) * BK);
        compute(st);
        if (it + 1 < steps) lstore(st ^ 1);
        __syncthreads();
    }

    // C element i of lane l in tile (mi, ni): row 4 (l / 16) + i, column l % 16
#pragma unroll
    for (int ni = 0; ni < 4; ++ni) {
        const uint32_t n = bn + wn + ni * 16 + c16;
        if (n >= N) continue;
#pragma unroll
        for (int mi = 0; mi < 4; ++mi)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const uint32_t m = bm + wm + mi * 16 + 4 * g + i;
                if (m < M) C[(uint64_t)m * N + n] = acc[mi][ni][i];
            }
    }
}

}  // namespace

#define GEMM_F32(name, TA, TB, TRANSB)                                                                   \
    POPCORN_KERNEL void __launch_bounds__(256)                                                           \
        name(const Src<TA>::storage *a, const Src<TB>::storage *b, float *c, MatmulConstants p) {        \
        gemm_f32<TA, TB, TRANSB>(a, b, c, p);                                                            \
    }

using pk::BF16;
using pk::F32;

GEMM_F32(matmul_mfma_f32_f32_f32_tb, F32, F32, true)
GEMM_F32(matmul_mfma_f32_f32_f32, F32, F32, false)
GEMM_F32(matmul_mfma_f32_bf16_f32_tb, F32, BF16, true)
GEMM_F32(matmul_mfma_f32_bf16_f32, F32, BF16, false)
GEMM_F32(matmul_mfma_bf16_f32_f32_tb, BF16, F32, true)
GEMM_F32(matmul_mfma_bf16_f32_f32, BF16, F32, false)
