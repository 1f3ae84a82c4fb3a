// Block-affine 4-bit Matmul on the matrix cores for M > 1 rows of bf16
// activations (a prompt): C[M, N] = X[M, K] . W[N, K]^T with
// W[n, k] = q[n, k] * s[n, g] + b[n, g], g = k / 64 (AffineQuantizedMatmul.metal,
// whose aq_matvec_simd4 runs one matvec per row of X, Matmul.swift:279-332).
//
// Per group g and output element: sum_k x_k (q_k s + b) = s * sum_k x_k q_k +
// b * X_g, X_g = sum_k x_k (the identity aq_qmv_fast uses,
// AffineQuantizedMatmul.metal:75-82). The nibbles enter the products as the
// bf16 values 128 + q (0x4300 | q, exact), so a group's product D on
// v_mfma_f32_32x32x16_bf16 (exact bf16 products, f32 sums) is
// sum x (128 + q) and the element gains s * D + (b - 128 s) * X_g, with no
// rounding of the weights to bf16: s * D is one FMA per element and group;
// the (b - 128 s) * X_g terms, an outer product per group, go on
// v_mfma_f32_32x32x2_f32 two groups at a time (the per-element FMAs for
// them made the kernel bound by its vector ALU work).
//
// aq_gemm_prep writes, per row of X and group, X_g (f32) and a copy of the
// row with each run of 8 values in the order (0, 4, 1, 5, 2, 6, 3, 7): a
// packed word w then gives its values in that order as the 4 bf16 pairs
// ((w >> 4p) & 0x000F000F) | 0x43004300, p < 4, one shift and one and-or
// each, matching the copy's order (the products' order within a group is
// free).
//
// aq_gemm: a block of 4 waves takes a 128 x 128 tile of C, each wave 64 x 64
// (2 x 2 MFMA tiles); per group the block stages the X' tile (128 x 64 bf16),
// the unpacked weights (128 x 64 bf16), the columns' (s, b - 128 s) and the
// rows' X_g in LDS, double-buffered with the next group's loads in
// registers. Rows past M and columns past N read row M - 1 / N - 1 and are
// not stored. A block walks its groups one after another, so with few tiles
// the groups are split over gridDim.y blocks per tile (SPLIT): each writes
// its f32 partial tile to P [gridDim.y][M][N] and matmul_splitk_reduce_*
// sums them and rounds once.
#include "mfma.hpp"

namespace {

using pk::f32x16;
using pk::u32x4;

constexpr int BM = 128, BN = 128;
constexpr int kGroup = 64;
constexpr int LDT = kGroup + 8;  // LDS row pitch (bf16): 144 bytes, so 16 rows fall in 16 distinct 4-bank groups
constexpr uint32_t kPairBase = 0x43004300u;

// One thread per (row, group): X_g, and the row's 64 values in pair order.
__device__ void aq_gemm_prep(const uint16_t *__restrict__ X, uint16_t *__restrict__ Xp, float *__restrict__ Xs,
                             const AffineQMatmulConstants &p) {
    const uint32_t G = p.kGroups;
    const uint64_t t = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (t >= (uint64_t)p.M * G) return;
    const uint64_t m = t / G, g = t % G;
    const u32x4 *src = reinterpret_cast<const u32x4 *>(X + m * p.K + g * kGroup);
    u32x4 *dst = reinterpret_cast<u32x4 *>(Xp + m * p.K + g * kGroup);
    float sum = 0.0f;
#pragma unroll
    for (int c = 0; c < kGroup / 8; ++c) {
        const u32x4 v = src[c];  // (x0, x1), (x2, x3), (x4, x5), (x6, x7)
        sum += __uint_as_float(v.x << 16) + __uint_as_float(v.x & 0xffff0000u) + __uint_as_float(v.y << 16) +
               __uint_as_float(v.y & 0xffff0000u) + __uint_as_float(v.z << 16) + __uint_as_float(v.z & 0xffff0000u) +
               __uint_as_float(v.w << 16) + __uint_as_float(v.w & 0xffff0000u);
        u32x4 o;  // (x0, x4), (x1, x5), (x2, x6), (x3, x7)
        o.x = __builtin_amdgcn_perm(v.z, v.x, 0x05040100u);
        o.y = __builtin_amdgcn_perm(v.z, v.x, 0x07060302u);
        o.z = __builtin_amdgcn_perm(v.w, v.y, 0x05040100u);
        o.w = __builtin_amdgcn_perm(v.w, v.y, 0x07060302u);
        dst[c] = o;
    }
    Xs[t] = sum;
}

template <typename O, bool SPLIT>
__device__ void aq_gemm(const uint32_t *__restrict__ Wp, const uint16_t *__restrict__ S, const uint16_t *__restrict__ Bi,
                        const uint16_t *__restrict__ Xp, const float *__restrict__ Xs, typename O::storage *__restrict__ C,
                        float *__restrict__ P, const AffineQMatmulConstants &p) {
    __shared__ __attribute__((aligned(16))) uint16_t sX[2][BM * LDT];
    __shared__ __attribute__((aligned(16))) uint16_t sW[2][BN * LDT];
    __shared__ __attribute__((aligned(16))) float2 sSC[2][BN];  // (s, b - 128 s) per column
    __shared__ __attribute__((aligned(16))) float sXs[2][BM];   // X_g per row

    const uint32_t M = p.M, N = p.N, K = p.K, G = p.kGroups, WPR = p.wordsPerRow;
    const uint32_t nM = (M + BM - 1) / BM;
    const uint32_t pm = blockIdx.x % nM, pn = blockIdx.x / nM;  // blocks sharing weights run together
    const uint32_t bm = pm * BM, bn = pn * BN;
    const uint32_t t = threadIdx.x, lane = t & 63, wave = t >> 6;
    const uint32_t wm = (wave >> 1) * 64, wn = (wave & 1) * 64;

    // this thread's staging: 4 16-byte runs of X' (row c / 8, run c % 8 for
    // c = t + 256 j), 4 packed words (row t / 2, words 4 (t % 2) ..), and
    // for t < 128 the column's scale and bias and the row's X_g
    const uint32_t wrow = t >> 1, wh = t & 1;
    const uint64_t wbase = (uint64_t)min(bn + wrow, N - 1) * WPR + 4 * wh;
    const uint32_t srow = min(bn + (t & 127), N - 1), xrow = min(bm + (t & 127), M - 1);
    u32x4 xr[4], wr;
    uint32_t sr = 0, br = 0;
    float xsr = 0.0f;
    auto gload = [&](uint32_t g) {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const uint32_t c = t + 256 * j, row = c >> 3, run = c & 7;
            xr[j] = *reinterpret_cast<const u32x4 *>(Xp + (uint64_t)min(bm + row, M - 1) * K + g * kGroup + run * 8);
        }
        wr = *reinterpret_cast<const u32x4 *>(Wp + wbase + g * 8);
        if (t < 128) {
            sr = S[(uint64_t)srow * G + g];
            br = p.hasBias ? Bi[(uint64_t)srow * G + g] : 0u;
            xsr = Xs[(uint64_t)xrow * G + g];
        }
    };
    auto lstore = [&](int st) {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const uint32_t c = t + 256 * j, row = c >> 3, run = c & 7;
            *reinterpret_cast<u32x4 *>(&sX[st][row * LDT + run * 8]) = xr[j];
        }
        // word i holds values 8 i .. 8 i + 7 of this half-group; in pair order
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const uint32_t w = wr[i];
            u32x4 q;
            q.x = (w & 0x000F000Fu) | kPairBase;
            q.y = ((w >> 4) & 0x000F000Fu) | kPairBase;
            q.z = ((w >> 8) & 0x000F000Fu) | kPairBase;
            q.w = ((w >> 12) & 0x000F000Fu) | kPairBase;
            *reinterpret_cast<u32x4 *>(&sW[st][wrow * LDT + wh * 32 + i * 8]) = q;
        }
        if (t < 128) {
            const float s = __uint_as_float(sr << 16), b = __uint_as_float(br << 16);
            sSC[st][t] = float2{s, b - 128.0f * s};
            sXs[st][t] = xsr;
        }
    };

    f32x16 acc[2][2];
#pragma unroll
    for (int mi = 0; mi < 2; ++mi)
#pragma unroll
        for (int ni = 0; ni < 2; ++ni)
#pragma unroll
            for (int i = 0; i < 16; ++i) acc[mi][ni][i] = 0.0f;

    // j: the group's index in this block's range; the bias terms of groups
    // j - 1 and j go in one product at odd j, a last even j's alone
    float px[2] = {0.0f, 0.0f}, pb[2] = {0.0f, 0.0f};  // group j - 1's X_g and b - 128 s
    auto compute = [&](int st, uint32_t j, bool last) {
        // group product per tile, then its scale; the bias terms on the
        // matrix cores
        const uint32_t r = lane & 31, h = lane >> 5;
        f32x16 d[2][2];
#pragma unroll
        for (int mi = 0; mi < 2; ++mi)
#pragma unroll
            for (int ni = 0; ni < 2; ++ni)
#pragma unroll
                for (int i = 0; i < 16; ++i) d[mi][ni][i] = 0.0f;
#pragma unroll
        for (int kk = 0; kk < kGroup / 16; ++kk) {
            u32x4 a[2], b[2];
#pragma unroll
            for (int mi = 0; mi < 2; ++mi)
                a[mi] = *reinterpret_cast<const u32x4 *>(&sX[st][(wm + mi * 32 + r) * LDT + kk * 16 + h * 8]);
#pragma unroll
            for (int ni = 0; ni < 2; ++ni)
                b[ni] = *reinterpret_cast<const u32x4 *>(&sW[st][(wn + ni * 32 + r) * LDT + kk * 16 + h * 8]);
#pragma unroll
            for (int mi = 0; mi < 2; ++mi)
#pragma unroll
                for (int ni = 0; ni < 2; ++ni) d[mi][ni] = pk::Mma<pk::BF16>::run(a[mi], b[ni], d[mi][ni]);
        }
#pragma unroll
        for (int ni = 0; ni < 2; ++ni) {
            const float sc = sSC[st][wn + ni * 32 + r].x;
#pragma unroll
            for (int mi = 0; mi < 2; ++mi)
#pragma unroll
                for (int i = 0; i < 16; ++i) acc[mi][ni][i] = fmaf(sc, d[mi][ni][i], acc[mi][ni][i]);
        }
        // acc += X_g (rows) x (b - 128 s)_g (columns) for two groups at a
        // time on v_mfma_f32_32x32x2_f32 (A lane l: row l % 32, k l / 32; B
        // lane l: k l / 32, column l % 32; C in the layout of acc): k 0 is
        // group j - 1, whose terms this lane kept in registers at even j
        // (the other LDS buffer may already hold group j + 1), k 1 group j;
        // an unpaired last group takes k 0 with k 1 zero
        float cx[2], cb[2];
#pragma unroll
        for (int mi = 0; mi < 2; ++mi) cx[mi] = sXs[st][wm + mi * 32 + r];
#pragma unroll
        for (int ni = 0; ni < 2; ++ni) cb[ni] = sSC[st][wn + ni * 32 + r].y;
        if (!(j & 1)) {
#pragma unroll
            for (int e = 0; e < 2; ++e) {
                px[e] = cx[e];
                pb[e] = cb[e];
            }
        }
        if ((j & 1) || last) {
            const bool pair = (j & 1) != 0;
            float xa[2], bb[2];
#pragma unroll
            for (int e = 0; e < 2; ++e) {
                xa[e] = pair ? (h ? cx[e] : px[e]) : (h ? 0.0f : cx[e]);
                bb[e] = pair ? (h ? cb[e] : pb[e]) : (h ? 0.0f : cb[e]);
            }
#pragma unroll
            for (int mi = 0; mi < 2; ++mi)
#pragma unroll
                for (int ni = 0; ni < 2; ++ni)
                    acc[mi][ni] = __builtin_amdgcn_mfma_f32_32x32x2f32(xa[mi], bb[ni], acc[mi][ni], 0, 0, 0);
        }
    };

    // this block's groups: all, or split y of gridDim.y
    const uint32_t g0 = SPLIT ? (uint32_t)((uint64_t)G * blockIdx.y / gridDim.y) : 0u;
    const uint32_t g1 = SPLIT ? (uint32_t)((uint64_t)G * (blockIdx.y + 1) / gridDim.y) : G;
    if (g0 < g1) {
        gload(g0);
        lstore(0);
        __syncthreads();
    }
    for (uint32_t g = g0; g < g1; ++g) {
        const int st = (int)((g - g0) & 1);
        if (g + 1 < g1) gload(g + 1);
        compute(st, g - g0, g + 1 == g1);
        if (g + 1 < g1) lstore(st ^ 1);
        __syncthreads();
    }

    // C element i of lane l in tile (mi, ni): row (i / 4) * 8 + (l / 32) * 4 + i % 4, column l % 32
    const uint32_t r = lane & 31, h = lane >> 5;
#pragma unroll
    for (int mi = 0; mi < 2; ++mi)
#pragma unroll
        for (int ni = 0; ni < 2; ++ni) {
            const uint32_t n = bn + wn + ni * 32 + r;
            if (n >= N) continue;
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                const uint32_t m = bm + wm + mi * 32 + (i / 4) * 8 + h * 4 + (i % 4);
                if (m >= M) continue;
                if constexpr (SPLIT) {
                    P[((uint64_t)blockIdx.y * M + m) * N + n] = acc[mi][ni][i];
                } else {
                    C[(uint64_t)m * N + n] = O::store(acc[mi][ni][i]);
                }
            }
        }
}

}  // namespace

POPCORN_KERNEL void __launch_bounds__(256)
    aq_gemm_prep_bf16(const uint16_t *x, uint16_t *xp, float *xs, AffineQMatmulConstants p) {
    aq_gemm_prep(x, xp, xs, p);
}

#define AQ_GEMM(name, O)                                                                                  \
    POPCORN_KERNEL void __launch_bounds__(256)                                                            \
        name(const uint32_t *w, const uint16_t *s, const uint16_t *b, const uint16_t *xp, const float *xs, \
             O::storage *c, AffineQMatmulConstants p) {                                                   \
        aq_gemm<O, false>(w, s, b, xp, xs, c, nullptr, p);                                                \
    }

// f32 partial tiles of a K split (gridDim.y splits), for matmul_splitk_reduce_*
POPCORN_KERNEL void __launch_bounds__(256)
    aq_gemm_mfma_bf16_bf16_splitk_b4_g64(const uint32_t *w, const uint16_t *s, const uint16_t *b, const uint16_t *xp,
                                         const float *xs, float *partial, AffineQMatmulConstants p) {
    aq_gemm<pk::F32, true>(w, s, b, xp, xs, nullptr, partial, p);
}

using pk::BF16;
using pk::F32;

AQ_GEMM(aq_gemm_mfma_bf16_bf16_bf16_b4_g64, BF16)
AQ_GEMM(aq_gemm_mfma_bf16_bf16_f32_b4_g64, F32)
