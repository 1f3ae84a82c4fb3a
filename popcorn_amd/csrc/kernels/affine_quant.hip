// Block-affine 4-bit matmul and embedding gather (AffineQuantizedMatmul.metal,
// AffineQuantizedEmbeddingGather.metal): y[m, n] = sum_k x[m, k] (q[n, k] s[n, g]
// + b[n, g]), g = k / 64; out[t, h] = q[ids[t], h] s + b. Kernel names follow
// the reference's (Matmul.swift:301-302, EmbeddingGather.swift:80), with the
// launch shape appended: _l<LPR> lanes per row, _j<J> x octets per thread.
//
// A block of 4 waves streams units of 64 / LPR rows per wave (q4.hpp) while
// the block stages its row of x in LDS; one block row of the grid (blockIdx.y)
// per row m of x (M == 1 is the decode matvec).
#include "q4.hpp"

namespace {

using pk::BF16;
using pk::F32;
using pk::kQ4Group;
using pk::Q4Staging;
using pk::Q4Stream;
using pk::u32x4;

// J octets per thread stage K <= 2048 J values: LDS holds K/2 pair words
// (bf16 x) or K floats (f32 x), plus K/64 group sums.
template <int J>
constexpr uint32_t maxK() { return 2048u * J; }

// The J octets (8 values) of x this thread stages, loaded into registers
// before the weight stream starts (loads retire in issue order); octets past
// the row load nothing and are not used.
template <typename X, int J>
struct XOctets {
    static constexpr int kPieces = sizeof(typename X::storage) * 8 / 16;  // 16-byte loads per octet
    u32x4 v[J][kPieces];
    __device__ void issue(const typename X::storage *x, uint32_t K) {
        const uint32_t octets = K / 8;
#pragma unroll
        for (int j = 0; j < J; ++j) {
            const uint32_t o = threadIdx.x + pk::kStreamThreads * (uint32_t)j;
            if (o >= octets) continue;
#pragma unroll
            for (int h = 0; h < kPieces; ++h) v[j][h] = *reinterpret_cast<const u32x4 *>(x + (uint64_t)o * 8 + h * (8 / kPieces));
        }
    }
    __device__ void get(int j, float *out) const {
        if constexpr (kPieces == 1) {
            pk::Vec<X> t;
            t.raw = v[j][0];
            t.to_float(out);
        } else {
#pragma unroll
            for (int h = 0; h < kPieces; ++h) {
                pk::Vec<X> t;
                t.raw = v[j][h];
                t.to_float(out + h * 4);
            }
        }
    }
};

template <typename X, typename O, int LPR, int J>
__device__ void aq_matvec(const uint32_t *__restrict__ W, const uint16_t *__restrict__ Sc, const uint16_t *__restrict__ Bi,
                          const typename X::storage *__restrict__ x, typename O::storage *__restrict__ y,
                          const AffineQMatmulConstants &p) {
    constexpr bool XF32 = sizeof(typename X::storage) == 4;
    constexpr int kRows = 64 / LPR;
    __shared__ uint32_t xw[XF32 ? 1 : maxK<J>() / kQ4Group * pk::kQ4GroupStride];
    __shared__ float xf[XF32 ? maxK<J>() : 1];
    __shared__ float gsum[maxK<J>() / kQ4Group];

    const uint32_t m = blockIdx.y;
    const uint32_t lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const uint32_t units = (p.N + kRows - 1) / kRows;
    const uint16_t *B = p.hasBias ? Bi : Sc;
    auto rowOf = [&](uint32_t unit) { return min(unit * kRows + lane / LPR, p.N - 1); };
    const pk::Q4Mat mats[1] = {{W, Sc, B}};
    XOctets<X, J> xo;
    xo.issue(x + (uint64_t)m * p.K, p.K);
    Q4Stream<LPR, 1, pk::kStreamSteps, XF32> st;
    st.init(rowOf, mats, p.N, p.K, units, blockIdx.x * pk::kStreamWaves + wave, gridDim.x * pk::kStreamWaves,
            p.hasBias != 0);
    st.template start<0, 1>(rowOf);  // one step before the staging barrier (see q4_gate_up)
    Q4Staging<XF32>::build(p.K, xw, xf, gsum, [&](uint32_t j, uint32_t, float *v) { xo.get(min(j, (uint32_t)J - 1), v); });
    st.template start<1>(rowOf);
    auto store = [&](uint32_t unit, const float *sums) {
        const uint32_t r = unit * kRows + lane / LPR;
        if (lane % LPR == 0 && lane / LPR < kRows && r < p.N) y[(uint64_t)m * p.N + r] = O::store(sums[0]);
    };
    st.run(xw, xf, gsum, rowOf, store);
}

// AffineQuantizedEmbeddingGather.metal:16-26, one thread per packed word (8
// values of one group) of one token (aq_embedding_gather_*_ext).
template <typename O>
__device__ void aq_gather(const int32_t *__restrict__ ids, const uint32_t *__restrict__ W, const uint16_t *__restrict__ Sc,
                          const uint16_t *__restrict__ Bi, typename O::storage *__restrict__ out,
                          const AffineQEmbeddingGatherExtConstants &p) {
    const uint64_t words = (uint64_t)p.T * p.wordsPerRow;
    for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < words; i += (uint64_t)gridDim.x * blockDim.x) {
        const uint32_t t = (uint32_t)(i / p.wordsPerRow), wi = (uint32_t)(i % p.wordsPerRow);
        const uint64_t row = (uint32_t)ids[t];
        typename O::storage *dst = out + (uint64_t)t * p.H + (uint64_t)wi * 8;
        if (p.V && row >= p.V) {
#pragma unroll
            for (int e = 0; e < 8; ++e) dst[e] = O::store(0.0f);
            continue;
        }
        const uint32_t g = wi / pk::kQ4GroupWords;
        const uint32_t w = W[row * p.wordsPerRow + wi];
        const float s = pk::bf16_lo(Sc[row * p.kGroups + g]);
        const float b = p.hasBias ? pk::bf16_lo(Bi[row * p.kGroups + g]) : 0.0f;
#pragma unroll
        for (int e = 0; e < 8; ++e) dst[e] = O::store((float)((w >> (4 * e)) & 15u) * s + b);
    }
}

// The reference's launch of the gather (EmbeddingGather.swift:90, :117-118):
// the thread at (x, y) writes value y of token x's row; the grid strides in
// both dimensions.
template <typename O>
__device__ void aq_gather_ref(const int32_t *__restrict__ ids, const uint32_t *__restrict__ W,
                              const uint16_t *__restrict__ Sc, const uint16_t *__restrict__ Bi,
                              typename O::storage *__restrict__ out, const AffineQEmbeddingGatherConstants &p) {
    const uint32_t sx = gridDim.x * blockDim.x, sy = gridDim.y * blockDim.y;
    for (uint32_t n = blockIdx.x * blockDim.x + threadIdx.x; n < p.T; n += sx) {
        const uint64_t row = (uint32_t)ids[n];
        for (uint32_t h = blockIdx.y * blockDim.y + threadIdx.y; h < p.H; h += sy) {
            const uint32_t g = h / kQ4Group;
            const float s = pk::bf16_lo(Sc[row * p.kGroups + g]);
            const float b = p.hasBias ? pk::bf16_lo(Bi[row * p.kGroups + g]) : 0.0f;
            const uint32_t q = (W[row * p.wordsPerRow + h / 8] >> (4 * (h % 8))) & 15u;
            out[(uint64_t)n * p.H + h] = O::store((float)q * s + b);
        }
    }
}

// Any alignment and any M: the reference's aq_matvec_simd4 launch
// (Matmul.swift:321-331: threads ceil(N / 4) * 32 by M): the 32-lane
// half-wave u of grid row m computes rows 4u .. 4u + 3 of x row m, its lanes
// strided over K (AffineQuantizedMatmul.metal:34-58). The Matmul descriptor
// takes it for shapes the fast kernels do not; the block size must be a
// multiple of 32.
template <typename X, typename O>
__device__ void aq_matvec_any(const uint32_t *__restrict__ W, const uint16_t *__restrict__ Sc,
                              const uint16_t *__restrict__ Bi, const typename X::storage *__restrict__ x,
                              typename O::storage *__restrict__ y, const AffineQMatmulConstants &p) {
    constexpr uint32_t kR = 4;
    const uint32_t lane = threadIdx.x & 31;
    const uint64_t row0 = (((uint64_t)blockIdx.x * blockDim.x + threadIdx.x) >> 5) * kR;
    if (row0 >= p.N) return;  // uniform over the half-wave
    for (uint32_t m = blockIdx.y * blockDim.y + threadIdx.y; m < p.M; m += gridDim.y * blockDim.y) {
        const typename X::storage *xr = x + (uint64_t)m * p.K;
        float acc[kR] = {0.0f, 0.0f, 0.0f, 0.0f};
        for (uint32_t k = lane; k < p.K; k += 32) {
            const float xv = X::load(xr[k]);
            const uint32_t g = k / kQ4Group;
#pragma unroll
            for (uint32_t r = 0; r < kR; ++r) {
                const uint64_t row = min(row0 + r, (uint64_t)p.N - 1);
                const float s = pk::bf16_lo(Sc[row * p.kGroups + g]);
                const float b = p.hasBias ? pk::bf16_lo(Bi[row * p.kGroups + g]) : 0.0f;
                const uint32_t q = (W[row * p.wordsPerRow + k / 8] >> (4 * (k % 8))) & 15u;
                acc[r] += xv * ((float)q * s + b);
            }
        }
#pragma unroll
        for (uint32_t r = 0; r < kR; ++r) {
            const float sum = pk::half32_sum(acc[r]);
            if (lane == 0 && row0 + r < p.N) y[(uint64_t)m * p.N + row0 + r] = O::store(sum);
        }
    }
}

// The reference's aq_qmv_fast launch (Matmul.swift:311-320: threadgroups of
// 64 threads, grid M by ceil(N / 8)): threadgroup (m, t), half-wave h < 2
// computes rows 8t + 4h .. + 3 of x row m; each lane takes 16 consecutive
// values of every 512 and sums s * sum(x q) + b * sum(x) per group
// (AffineQuantizedMatmul.metal:84-160). K is a multiple of 64.
template <typename X, typename O>
__device__ void aq_qmv_ref(const uint32_t *__restrict__ W, const uint16_t *__restrict__ Sc, const uint16_t *__restrict__ Bi,
                           const typename X::storage *__restrict__ x, typename O::storage *__restrict__ y,
                           const AffineQMatmulConstants &p) {
    constexpr uint32_t kR = 4, kPerLane = 16;
    const uint32_t half = threadIdx.x >> 5, lane = threadIdx.x & 31;
    const uint32_t m = blockIdx.x;
    const uint64_t row0 = (uint64_t)blockIdx.y * 8 + half * kR;
    if (half >= 2 || m >= p.M || row0 >= p.N) return;  // uniform over the half-wave
    float acc[kR] = {0.0f, 0.0f, 0.0f, 0.0f};
    for (uint32_t k0 = lane * kPerLane; k0 < p.K; k0 += 32 * kPerLane) {
        float xv[kPerLane], sx = 0.0f;
#pragma unroll
        for (uint32_t j = 0; j < kPerLane; ++j) {
            xv[j] = X::load(x[(uint64_t)m * p.K + k0 + j]);
            sx += xv[j];
        }
        const uint32_t g = k0 / kQ4Group;
#pragma unroll
        for (uint32_t r = 0; r < kR; ++r) {
            const uint64_t row = min(row0 + r, (uint64_t)p.N - 1);
            const float s = pk::bf16_lo(Sc[row * p.kGroups + g]);
            const float b = p.hasBias ? pk::bf16_lo(Bi[row * p.kGroups + g]) : 0.0f;
            float qdot = 0.0f;
#pragma unroll
            for (uint32_t j = 0; j < kPerLane; ++j) {
                const uint32_t w = W[row * p.wordsPerRow + (k0 + j) / 8];
                qdot += xv[j] * (float)((w >> (4 * ((k0 + j) % 8))) & 15u);
            }
            acc[r] += s * qdot + b * sx;
        }
    }
#pragma unroll
    for (uint32_t r = 0; r < kR; ++r) {
        const float sum = pk::half32_sum(acc[r]);
        if (lane == 0 && row0 + r < p.N) y[(uint64_t)m * p.N + row0 + r] = O::store(sum);
    }
}

// ---- decode forms with the layer glue (bf16 activations) ---------------------
// The decoder layer's glue is built by Stage (stream.hpp) into xs (f32, LDS),
// then turned into the 4-bit staging (pair words + group sums) behind it:
// dynamic LDS = K floats + K / 64 groups x 36 words + K / 64 floats. Every stored
// intermediate is rounded to bf16 (interDataType must be bf16, which is what
// makes the xs values exact bf16 pairs).

template <int LPR, int NS>
struct Q4Lds {
    float *xs;
    uint32_t *xw;
    float *gsum;
    __device__ Q4Lds(float *lds, uint32_t K)
        : xs(lds), xw(reinterpret_cast<uint32_t *>(lds + K)), gsum(lds + K + K / kQ4Group * pk::kQ4GroupStride) {}
    __device__ void stage_from_xs(uint32_t K) const {
        const float *x = xs;
        Q4Staging<false>::build(K, xw, nullptr, gsum, [&](uint32_t, uint32_t o, float *v) {
            const float4 a = *reinterpret_cast<const float4 *>(x + 8 * o);
            const float4 b = *reinterpret_cast<const float4 *>(x + 8 * o + 4);
            v[0] = a.x, v[1] = a.y, v[2] = a.z, v[3] = a.w, v[4] = b.x, v[5] = b.y, v[6] = b.z, v[7] = b.w;
        });
    }
};

// DecodeMatvecConstants semantics (flags bits 0-1 compiled in as RES / PRE,
// bit 2 the KV scatter) with W block-affine 4-bit.
template <typename O, int LPR, bool RES, bool PRE>
__device__ void q4_decode_matvec(const uint16_t *__restrict__ x_in, const uint16_t *__restrict__ delta,
                                 const float *__restrict__ w_post, const float *__restrict__ w_pre,
                                 const uint32_t *__restrict__ W, const uint16_t *__restrict__ Sc,
                                 const uint16_t *__restrict__ Bi, typename O::storage *__restrict__ out,
                                 uint16_t *__restrict__ x_out, typename O::storage *__restrict__ kcache,
                                 typename O::storage *__restrict__ vcache, const int32_t *__restrict__ position,
                                 const DecodeMatvecConstants &p, const AffineQMatmulConstants &q) {
    extern __shared__ float lds[];
    __shared__ float red[pk::kStreamWaves];
    constexpr int kRows = 64 / LPR;
    const uint32_t K = p.K, N = p.N;
    const Q4Lds<LPR, 1> L(lds, K);
    const uint32_t lane = threadIdx.x & 63, wave = pk::uniform(threadIdx.x >> 6);
    const uint32_t units = (N + kRows - 1) / kRows;
    const uint32_t first = blockIdx.x * pk::kStreamWaves + wave, stride = gridDim.x * pk::kStreamWaves;
    const uint16_t *B = q.hasBias ? Bi : Sc;
    auto rowOf = [&](uint32_t unit) { return min(unit * kRows + lane / LPR, N - 1); };
    const pk::Q4Mat mats[1] = {{W, Sc, B}};
    const bool scatter = (p.flags & pk::kKVScatter) != 0;
    const int32_t posLoaded = pk::load_position(position, scatter);
    auto store = [&](uint32_t unit, const float *sums) {
        const uint32_t row = unit * kRows + lane / LPR;
        if (lane % LPR != 0 || lane / LPR >= kRows || row >= N) return;
        if (scatter && row >= p.qRows) {
            uint32_t j = row - p.qRows;
            const bool isV = j >= p.kvRows;
            if (isV) j -= p.kvRows;
            const int32_t pos = pk::position_value(posLoaded);
            if (pos >= 0 && (uint32_t)pos < p.kvStride) {
                const uint64_t at = ((uint64_t)(j / p.headDim) * p.kvStride + (uint32_t)pos) * p.headDim + j % p.headDim;
                (isV ? vcache : kcache)[at] = O::store(sums[0]);
            }
        } else {
            out[row] = O::store(sums[0]);
        }
    };
    using Stage = pk::Stage<BF16, RES, PRE, 2>;
    Q4Stream<LPR, 1, pk::kStreamSteps, false> st;
    if (!Stage::fast_ok(x_in, delta, w_post, w_pre, x_out, K, 1u)) {
        Stage::finish_scalar(L.xs, red, x_in, delta, w_post, w_pre, x_out, K, 1u, p.eps, p.interDataType);
        L.stage_from_xs(K);
        st.init(rowOf, mats, N, K, units, first, stride, q.hasBias != 0);
        st.start(rowOf);
        st.run(L.xw, nullptr, L.gsum, rowOf, store);
        return;
    }
    Stage stage;
    stage.issue(x_in, delta, w_post, w_pre, K);
    st.init(rowOf, mats, N, K, units, first, stride, q.hasBias != 0);
    st.start(rowOf);
    stage.finish(L.xs, red, x_out, K, 1u, p.eps, p.interDataType);
    L.stage_from_xs(K);
    st.run(L.xw, nullptr, L.gsum, rowOf, store);
}

// The gated-MLP front half (GatedMLPConstants; gated_mlp.hip's semantics)
// with Wg and Wu block-affine 4-bit: each lane streams the same row of both.
// Each wave issues one step of its weight loads before the vector is built
// and the rest after: the block's barriers wait for every wave's issued
// loads, and under a full memory pipeline a wave's issue stalls (with all
// steps issued first, the vector was ready only once nearly all of the
// block's stream had arrived, and the dot products could not start before).
template <int LPR, bool RES>
__device__ void q4_gate_up(const uint16_t *__restrict__ x, const float *__restrict__ norm_w,
                           const uint32_t *__restrict__ Wg, const uint16_t *__restrict__ Sg, const uint16_t *__restrict__ Bg,
                           const uint32_t *__restrict__ Wu, const uint16_t *__restrict__ Su, const uint16_t *__restrict__ Bu,
                           uint16_t *__restrict__ h, const uint16_t *__restrict__ delta, const float *__restrict__ w_post,
                           uint16_t *__restrict__ x_out, const GatedMLPConstants &p, const AffineQMatmulConstants &q) {
    extern __shared__ float lds[];
    __shared__ float red[pk::kStreamWaves];
    constexpr int kRows = 64 / LPR;
    const uint32_t H = p.H, F = p.F;
    const Q4Lds<LPR, 2> L(lds, H);
    const uint32_t lane = threadIdx.x & 63, wave = pk::uniform(threadIdx.x >> 6);
    const uint32_t units = (F + kRows - 1) / kRows;
    const uint32_t first = blockIdx.x * pk::kStreamWaves + wave, stride = gridDim.x * pk::kStreamWaves;
    const uint32_t preMode = p.hasWeight ? (p.addOneToWeight ? 2u : 1u) : 0u;
    const uint32_t inter = p.interDataType;
    const uint16_t *BgB = q.hasBias ? Bg : Sg, *BuB = q.hasBias ? Bu : Su;
    auto rowOf = [&](uint32_t unit) { return min(unit * kRows + lane / LPR, F - 1); };
    const pk::Q4Mat mats[2] = {{Wg, Sg, BgB}, {Wu, Su, BuB}};
    auto store = [&](uint32_t unit, const float *sums) {
        const uint32_t row = unit * kRows + lane / LPR;
        if (lane % LPR != 0 || lane / LPR >= kRows || row >= F) return;
        const float g = pk::round_through(inter, sums[0]);
        const float u = pk::round_through(inter, sums[1]);
        const float a = pk::round_through(inter, pk::gelu_tanh(g));
        h[row] = BF16::store(a * u);
    };
    using Stage = pk::Stage<BF16, RES, true, 2>;
    Q4Stream<LPR, 2, pk::kStreamSteps, false> st;
    if (!Stage::fast_ok(x, delta, w_post, norm_w, x_out, H, preMode)) {
        Stage::finish_scalar(L.xs, red, x, delta, w_post, norm_w, x_out, H, preMode, p.eps, inter);
        L.stage_from_xs(H);
        st.init(rowOf, mats, F, H, units, first, stride, q.hasBias != 0);
        st.start(rowOf);
        st.run(L.xw, nullptr, L.gsum, rowOf, store);
        return;
    }
    Stage stage;
    stage.issue(x, delta, w_post, norm_w, H);
    st.init(rowOf, mats, F, H, units, first, stride, q.hasBias != 0);
    st.template start<0, 1>(rowOf);
    stage.finish(L.xs, red, x_out, H, preMode, p.eps, inter);
    L.stage_from_xs(H);
    st.template start<1>(rowOf);
    st.run(L.xw, nullptr, L.gsum, rowOf, store);
}

}  // namespace

#define Q4_DMV(ot, O, LPR, F, RES, PRE)                                                                            \
    POPCORN_KERNEL void __launch_bounds__(256) q4_decode_matvec_bf16_##ot##_l##LPR##_f##F(                          \
        const uint16_t *x_in, const uint16_t *delta, const float *w_post, const float *w_pre, const uint32_t *W,    \
        const uint16_t *S, const uint16_t *B, O::storage *out, uint16_t *x_out, O::storage *kcache,               \
        O::storage *vcache, const int32_t *position, DecodeMatvecConstants p, AffineQMatmulConstants q) {        \
        q4_decode_matvec<O, LPR, RES, PRE>(x_in, delta, w_post, w_pre, W, S, B, out, x_out, kcache, vcache,       \
                                           position, p, q);                                                       \
    }
#define Q4_DMV_F(ot, O, LPR)                                                                     \
    Q4_DMV(ot, O, LPR, 0, false, false) Q4_DMV(ot, O, LPR, 1, true, false) Q4_DMV(ot, O, LPR, 2, false, true) \
    Q4_DMV(ot, O, LPR, 3, true, true)
#define Q4_GU(LPR, SUFFIX, RES)                                                                                       \
    POPCORN_KERNEL void __launch_bounds__(256) q4_gate_up_bf16_l##LPR##SUFFIX(                                        \
        const uint16_t *x, const float *norm_w, const uint32_t *Wg, const uint16_t *Sg, const uint16_t *Bg,           \
        const uint32_t *Wu, const uint16_t *Su, const uint16_t *Bu, uint16_t *h, const uint16_t *delta,               \
        const float *w_post, uint16_t *x_out, GatedMLPConstants p, AffineQMatmulConstants q) {                       \
        q4_gate_up<LPR, RES>(x, norm_w, Wg, Sg, Bg, Wu, Su, Bu, h, delta, w_post, x_out, p, q);                     \
    }
#define Q4_ALL(LPR) Q4_DMV_F(bf16, BF16, LPR) Q4_DMV_F(f32, F32, LPR) Q4_GU(LPR, , false) Q4_GU(LPR, _res, true)
Q4_ALL(8)
Q4_ALL(12)
Q4_ALL(16)
Q4_ALL(32)

#define AQ_MV(prefix, xt, ot, X, O, LPR, J)                                                                         \
    POPCORN_KERNEL void __launch_bounds__(256) prefix##_##xt##_bf16_##ot##_b4_g64_l##LPR##_j##J(                      \
        const uint32_t *W, const uint16_t *S, const uint16_t *B, const X::storage *x, O::storage *y,                    \
        AffineQMatmulConstants p) {                                                                                    \
        aq_matvec<X, O, LPR, J>(W, S, B, x, y, p);                                                                     \
    }
// bf16 x: J 2 (K <= 4096) and 8 (K <= 16384); f32 x: J 2 (K <= 4096, 16 KB
// of LDS; larger K takes the any-shape kernel)
#define AQ_MV_L(prefix, xt, ot, X, O, J)                                                                 \
    AQ_MV(prefix, xt, ot, X, O, 8, J) AQ_MV(prefix, xt, ot, X, O, 12, J) AQ_MV(prefix, xt, ot, X, O, 16, J) \
        AQ_MV(prefix, xt, ot, X, O, 32, J)
#define AQ_MV_ALL(prefix)                                                                  \
    AQ_MV_L(prefix, bf16, bf16, BF16, BF16, 2) AQ_MV_L(prefix, bf16, bf16, BF16, BF16, 8) \
    AQ_MV_L(prefix, bf16, f32, BF16, F32, 2) AQ_MV_L(prefix, bf16, f32, BF16, F32, 8)     \
    AQ_MV_L(prefix, f32, f32, F32, F32, 2)

// Matmul.swift:301 (m == 1 -> aq_qmv_fast, else aq_matvec_simd4) and the
// dtype triples of Matmul.swift:343-347
AQ_MV_ALL(aq_qmv_fast)
AQ_MV_ALL(aq_matvec_simd4)

// The reference's host names on the reference's launch geometry.
#define AQ_ANY(xt, ot, X, O)                                                                                  \
    POPCORN_KERNEL void __launch_bounds__(1024) aq_matvec_simd4_##xt##_bf16_##ot##_b4_g64(                         \
        const uint32_t *W, const uint16_t *S, const uint16_t *B, const X::storage *x, O::storage *y,            \
        AffineQMatmulConstants p) {                                                                            \
        aq_matvec_any<X, O>(W, S, B, x, y, p);                                                                 \
    }                                                                                                          \
    POPCORN_KERNEL void __launch_bounds__(1024) aq_qmv_fast_##xt##_bf16_##ot##_b4_g64(                             \
        const uint32_t *W, const uint16_t *S, const uint16_t *B, const X::storage *x, O::storage *y,            \
        AffineQMatmulConstants p) {                                                                            \
        aq_qmv_ref<X, O>(W, S, B, x, y, p);                                                                    \
    }
AQ_ANY(bf16, bf16, BF16, BF16)
AQ_ANY(bf16, f32, BF16, F32)
AQ_ANY(f32, f32, F32, F32)

// EmbeddingGather.swift:80 (AffineQuantizedEmbeddingGather.metal:29-30): the
// reference's names on its parameter list and launch, and the _ext forms
// the descriptor runs.
#define AQ_GATHER(ot, O)                                                                                          \
    POPCORN_KERNEL void __launch_bounds__(1024) aq_embedding_gather_bf16_##ot##_b4_g64(                          \
        const int32_t *ids, const uint32_t *W, const uint16_t *S, const uint16_t *B, O::storage *out,           \
        AffineQEmbeddingGatherConstants p) {                                                                    \
        aq_gather_ref<O>(ids, W, S, B, out, p);                                                                 \
    }                                                                                                           \
    POPCORN_KERNEL void __launch_bounds__(256) aq_embedding_gather_bf16_##ot##_b4_g64_ext(                       \
        const int32_t *ids, const uint32_t *W, const uint16_t *S, const uint16_t *B, O::storage *out,           \
        AffineQEmbeddingGatherExtConstants p) {                                                                 \
        aq_gather<O>(ids, W, S, B, out, p);                                                                     \
    }
AQ_GATHER(bf16, BF16)
AQ_GATHER(f32, F32)
