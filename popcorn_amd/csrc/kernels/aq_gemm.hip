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
// (2 x 2 MFMA tiles); per group the block copies the X' tile (128 x 64
// bf16), the packed words, the columns' scale and bias words and the rows'
// X_g into LDS, three groups in flight (below). Rows past M and columns
// past N read zeros and are not stored. A block walks its groups one after
// another, so with few tiles the groups are split over gridDim.y blocks per
// tile (SPLIT): each writes its f32 partial tile to P [gridDim.y][M][N] and
// matmul_splitk_reduce_* sums them and rounds once.
#include "mfma.hpp"

namespace {

using pk::f32x16;
using pk::u32x4;

constexpr int BM = 128, BN = 128;
constexpr int kGroup = 64;
constexpr uint32_t kPairBase = 0x43004300u;

// The bf16 of group g in the 32-bit word that holds groups g & ~1 and g | 1.
__device__ inline float bf16_half(uint32_t v, uint32_t g) { return __uint_as_float((g & 1u) ? (v & 0xffff0000u) : (v << 16)); }

// One thread per run of 8 values (16 bytes): consecutive threads take
// consecutive runs of a row, so a wave's loads and stores are 1 KB
// contiguous; a group's 8 runs are 8 consecutive lanes (K % 64 == 0), whose
// sums meet by lane swaps and whose first lane writes X_g. Runs are written
// in pair order.
__device__ void aq_gemm_prep(const uint16_t *__restrict__ X, uint16_t *__restrict__ Xp, float *__restrict__ Xs,
                             const AffineQMatmulConstants &p) {
    const uint64_t runs = (uint64_t)p.M * (p.K / 8);
    const uint64_t t = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    const bool live = t < runs;  // every lane takes part in the swaps
    u32x4 v = {0u, 0u, 0u, 0u};  // (x0, x1), (x2, x3), (x4, x5), (x6, x7)
    if (live) v = reinterpret_cast<const u32x4 *>(X)[t];
    float sum = __uint_as_float(v.x << 16) + __uint_as_float(v.x & 0xffff0000u) + __uint_as_float(v.y << 16) +
                __uint_as_float(v.y & 0xffff0000u) + __uint_as_float(v.z << 16) + __uint_as_float(v.z & 0xffff0000u) +
                __uint_as_float(v.w << 16) + __uint_as_float(v.w & 0xffff0000u);
    u32x4 o;  // (x0, x4), (x1, x5), (x2, x6), (x3, x7)
    o.x = __builtin_amdgcn_perm(v.z, v.x, 0x05040100u);
    o.y = __builtin_amdgcn_perm(v.z, v.x, 0x07060302u);
    o.z = __builtin_amdgcn_perm(v.w, v.y, 0x05040100u);
    o.w = __builtin_amdgcn_perm(v.w, v.y, 0x07060302u);
    if (live) reinterpret_cast<u32x4 *>(Xp)[t] = o;
    // the group's 8 lanes (a group starts at a multiple of 8 runs, and
    // blocks hold whole groups)
    sum += __shfl_xor(sum, 1);
    sum += __shfl_xor(sum, 2);
    sum += __shfl_xor(sum, 4);
    if (live && (t & 7) == 0) Xs[t / 8] = sum;
}

// One stage per group, NS stages in flight, every tile copied buffer -> LDS
// directly (no staging registers), one barrier per group:
//  * x': 128 rows x 128 bytes, chunk c of row r in slot c ^ ((r >> 1) & 7)
//    (whole 128-byte lines per copy; a fragment read's 16 rows per
//    quarter-wave cover all banks);
//  * the packed words: 128 columns x 32 bytes, 16-byte half h of column n
//    in slot h ^ ((n >> 3) & 1), unpacked to bf16 pairs as the fragments
//    are read;
//  * the 32-bit words of the scales and biases that hold the group (and
//    its even/odd neighbour), and the rows' X_g.
// Wave w's copies per stage: x' instructions w, w + 4, w + 8, w + 12, the
// words' instruction w, one of the scale/bias words, and one of X_g (waves
// 2 and 3 copy the X_g of waves 0 and 1 again, identical bytes), so every
// wave issues kCopies per stage and the waits count them exactly. In a
// group's products lane half h takes chunk 4 h + kk of the group in step
// kk, in x' and in the words alike.
constexpr int NS = 3;                       // stages in flight
constexpr int kXB = BM * 128;               // x' bytes per stage
constexpr int kWB = BN * 32;                // packed-word bytes per stage
constexpr int kStageB = kXB + kWB + 3 * 512;  // + scale words, bias words, X_g
constexpr int kCopies = 7;
constexpr uint32_t kOOR = 0x80000000u;      // a buffer offset past every operand: zeros, no memory read
typedef __attribute__((address_space(3))) void lds_void;

template <int N>
__device__ inline void wait_vm() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}

template <typename O, bool SPLIT>
__device__ void aq_gemm(const uint32_t *__restrict__ Wp, const uint16_t *__restrict__ S, const uint16_t *__restrict__ Bi,
                        const uint16_t *__restrict__ Xp, const float *__restrict__ Xs, typename O::storage *__restrict__ C,
                        float *__restrict__ P, const AffineQMatmulConstants &p) {
    __shared__ __attribute__((aligned(16))) uint8_t smem[NS * kStageB];

    const uint32_t M = p.M, N = p.N, K = p.K, G = p.kGroups, WPR = p.wordsPerRow;
    const uint32_t nM = (M + BM - 1) / BM;
    const uint32_t pm = blockIdx.x % nM, pn = blockIdx.x / nM;  // blocks sharing weights run together
    const uint32_t bm = pm * BM, bn = pn * BN;
    const uint32_t lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const uint32_t wm = (wave >> 1) * 64, wn = (wave & 1) * 64;
    const uint32_t r = lane & 31, h = lane >> 5;

    // buffer resources over whole operands (the host keeps each under 2^31 bytes)
    const __amdgpu_buffer_rsrc_t rsX = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t *>(Xp), 0, (int)(M * K * 2u), 0x00020000);
    const __amdgpu_buffer_rsrc_t rsW = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint32_t *>(Wp), 0, (int)(N * WPR * 4u), 0x00020000);
    const __amdgpu_buffer_rsrc_t rsS = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t *>(S), 0, (int)(N * G * 2u), 0x00020000);
    const __amdgpu_buffer_rsrc_t rsB = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t *>(Bi), 0, (int)(N * G * 2u), 0x00020000);
    const __amdgpu_buffer_rsrc_t rsG = __builtin_amdgcn_make_buffer_rsrc(const_cast<float *>(Xs), 0, (int)(M * G * 4u), 0x00020000);

    auto stageOf = [&](uint32_t j) { return smem + (j % NS) * kStageB; };
    auto issue = [&](uint32_t g, uint8_t *stage) {
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int t = 0; t < 4; ++t) {  // x': rows 8 i .. 8 i + 7
            const uint32_t i = 4 * t + wave, row = 8 * i + (lane >> 3), c = (lane & 7) ^ ((row >> 1) & 7);
            const uint32_t off = bm + row < M ? ((bm + row) * K + g * kGroup + 8 * c) * 2u : kOOR;
            __builtin_amdgcn_raw_ptr_buffer_load_lds(rsX, (lds_void *)(stage + i * 1024), 16, off, 0, 0, 0);
        }
        {  // words: columns 32 w .. 32 w + 31
            const uint32_t col = 32 * wave + (lane >> 1), hh = (lane & 1) ^ ((col >> 3) & 1);
            const uint32_t off = bn + col < N ? ((bn + col) * WPR + g * 8 + 4 * hh) * 4u : kOOR;
            __builtin_amdgcn_raw_ptr_buffer_load_lds(rsW, (lds_void *)(stage + kXB + wave * 1024), 16, off, 0, 0, 0);
        }
        {  // scale words (waves 0, 1) or bias words (waves 2, 3) of columns 64 (w & 1) + l
            const uint32_t col = 64 * (wave & 1) + lane;
            const uint32_t off = bn + col < N ? ((bn + col) * G + (g & ~1u)) * 2u : kOOR;
            __builtin_amdgcn_raw_ptr_buffer_load_lds(wave < 2 ? rsS : rsB, (lds_void *)(stage + kXB + kWB + (wave >> 1) * 512 + (wave & 1) * 256),
                                                     4, off, 0, 0, 0);
        }
        {  // X_g of rows 64 (w & 1) + l
            const uint32_t row = 64 * (wave & 1) + lane;
            const uint32_t off = bm + row < M ? ((bm + row) * G + g) * 4u : kOOR;
            __builtin_amdgcn_raw_ptr_buffer_load_lds(rsG, (lds_void *)(stage + kXB + kWB + 1024 + (wave & 1) * 256), 4, off, 0, 0, 0);
        }
        __builtin_amdgcn_sched_barrier(0);
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
    auto compute = [&](const uint8_t *stage, uint32_t g, uint32_t j, bool last) {
        const uint8_t *sX = stage, *sW = stage + kXB;
        const uint32_t *sS = reinterpret_cast<const uint32_t *>(stage + kXB + kWB);
        const uint32_t *sB = sS + 128;
        const float *sG = reinterpret_cast<const float *>(stage + kXB + kWB + 1024);
        // this lane's 4 packed words of each of its two columns: chunks 4 h .. 4 h + 3
        u32x4 wr[2];
#pragma unroll
        for (int ni = 0; ni < 2; ++ni) {
            const uint32_t col = wn + ni * 32 + r;
            wr[ni] = *reinterpret_cast<const u32x4 *>(sW + col * 32 + ((h ^ ((col >> 3) & 1)) << 4));
        }
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
            for (int mi = 0; mi < 2; ++mi) {
                const uint32_t row = wm + mi * 32 + r, c = 4 * h + kk;
                a[mi] = *reinterpret_cast<const u32x4 *>(sX + row * 128 + ((c ^ ((row >> 1) & 7)) << 4));
            }
#pragma unroll
            for (int ni = 0; ni < 2; ++ni) {
                // a packed word gives its values in pair order as 4 bf16 pairs
                const uint32_t w = wr[ni][kk];
                b[ni].x = (w & 0x000F000Fu) | kPairBase;
                b[ni].y = ((w >> 4) & 0x000F000Fu) | kPairBase;
                b[ni].z = ((w >> 8) & 0x000F000Fu) | kPairBase;
                b[ni].w = ((w >> 12) & 0x000F000Fu) | kPairBase;
            }
#pragma unroll
            for (int mi = 0; mi < 2; ++mi)
#pragma unroll
                for (int ni = 0; ni < 2; ++ni) d[mi][ni] = pk::Mma<pk::BF16>::run(a[mi], b[ni], d[mi][ni]);
        }
        float cs[2], cb[2], cx[2];
#pragma unroll
        for (int ni = 0; ni < 2; ++ni) {
            const uint32_t col = wn + ni * 32 + r;
            cs[ni] = bf16_half(sS[col], g);
            const float bias = p.hasBias ? bf16_half(sB[col], g) : 0.0f;
            cb[ni] = bias - 128.0f * cs[ni];
        }
#pragma unroll
        for (int mi = 0; mi < 2; ++mi) cx[mi] = sG[wm + mi * 32 + r];
#pragma unroll
        for (int ni = 0; ni < 2; ++ni)
#pragma unroll
            for (int mi = 0; mi < 2; ++mi)
#pragma unroll
                for (int i = 0; i < 16; ++i) acc[mi][ni][i] = fmaf(cs[ni], d[mi][ni][i], acc[mi][ni][i]);
        // acc += X_g (rows) x (b - 128 s)_g (columns) for two groups at a
        // time on v_mfma_f32_32x32x2_f32 (A lane l: row l % 32, k l / 32; B
        // lane l: k l / 32, column l % 32; C in the layout of acc): k 0 is
        // group j - 1, whose terms this lane kept in registers at even j
        // (its stage may already be refilled), k 1 group j; an unpaired
        // last group takes k 0 with k 1 zero
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
    const uint32_t n = g1 > g0 ? g1 - g0 : 0u;
    // Group j: wait for this wave's copies of stage j (those of stage j + 1,
    // if issued, may stay in flight), barrier (every wave's copies of stage j
    // have landed, and every wave is done with stage j - 1), refill stage
    // j - 1's buffer with group j + NS - 1, then the products.
    static_assert(NS == 3, "the waits below count one stage in flight behind the awaited one");
    if (n > 0) issue(g0, stageOf(0));
    if (n > 1) issue(g0 + 1, stageOf(1));
    for (uint32_t j = 0; j < n; ++j) {
        if (j + 1 < n) wait_vm<kCopies>();
        else wait_vm<0>();
        __builtin_amdgcn_s_barrier();
        if (j + NS - 1 < n) issue(g0 + j + NS - 1, stageOf(j + NS - 1));
        compute(stageOf(j), g0 + j, j, j + 1 == n);
    }

    // C element i of lane l in tile (mi, ni): row (i / 4) * 8 + (l / 32) * 4 + i % 4, column l % 32
#pragma unroll
    for (int mi = 0; mi < 2; ++mi)
#pragma unroll
        for (int ni = 0; ni < 2; ++ni) {
            const uint32_t col = bn + wn + ni * 32 + r;
            if (col >= N) continue;
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                const uint32_t m = bm + wm + mi * 32 + (i / 4) * 8 + h * 4 + (i % 4);
                if (m >= M) continue;
                if constexpr (SPLIT) {
                    P[((uint64_t)blockIdx.y * M + m) * N + col] = acc[mi][ni][i];
                } else {
                    C[(uint64_t)m * N + col] = O::store(acc[mi][ni][i]);
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
