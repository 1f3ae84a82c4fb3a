// Matrix-vector products of the decode step (the reference's Matmul with
// m == 1):
// matvec_nk_stream_<x>_<w>_<out>_r<R>: y[n] = sum_k x[k] * W[n, k] with W
// row-major [N, K] (the transposeB layout of
// Sources/Popcorn/Kernels/Matvec.metal:55-126, the reference's
// MatvecConstants), R = 4 or 1 rows per streamed unit; what the Matmul
// descriptor runs for m == 1.
// matvec_nk_simd_<x>_<w>_<out>: the reference's host name, parameter list
// and launch geometry (Matmul.swift:248-251: threads ceil(N / 4) * 32 in
// blocks of 128): each 32-lane half-wave takes 4 rows, its lanes strided
// over K, for raw launches built like the reference's.
// decode_matvec_<t>_<o>_r<R>_f<F>: the same product with the decoder-layer
// glue folded in (DecodeMatvecConstants): F bit 0 = residual + post-norm in
// front, bit 1 = pre-norm, compiled in; the KV-cache scatter of the output
// rows (flags bit 2) is a runtime choice.
//
// The kernel is HBM-bound: W is read once, x is reused from LDS. A block of
// 4 waves stages x (Stage), then every wave streams its units of R rows
// (RowStream, 4 loads of 16 bytes per row and lane in flight). The host
// sizes the grid so that each wave gets the same number of units, give or
// take one. Rows whose length is not a multiple of the vector width, or an
// unaligned W, take a scalar loop (the reference's K % 4 != 0 tail,
// Matvec.metal:103-115).
//
// matvec*: y[n] = sum_k x[k] * W[k, n] (transposeW == 0, Matvec.metal:6-30),
// one thread per output column; not on the decode path.
#include "stream.hpp"

namespace {

using pk::kStreamSteps;
using pk::kStreamWaves;

template <typename X, typename W, typename O, int R, bool RES, bool PRE, int J>
__device__ void matvec_nk(const typename X::storage *__restrict__ x_in, const typename X::storage *__restrict__ delta,
                          const float *__restrict__ w_post, const float *__restrict__ w_pre,
                          const typename W::storage *__restrict__ w, typename O::storage *__restrict__ out,
                          typename X::storage *__restrict__ x_out, typename O::storage *__restrict__ kcache,
                          typename O::storage *__restrict__ vcache, const int32_t *__restrict__ position,
                          const DecodeMatvecConstants &p, float *xs) {
    constexpr int U = kStreamSteps;
    constexpr int kV = pk::Vec<W>::kVec;
    __shared__ float red[kStreamWaves];
    const uint32_t K = p.K, N = p.N;
    const uint32_t units = (N + R - 1) / R;
    const uint32_t wave = pk::uniform(threadIdx.x >> 6);
    const uint32_t first = blockIdx.x * kStreamWaves + wave, stride = gridDim.x * kStreamWaves;
    const uint64_t wbytes = (uint64_t)N * K * sizeof(typename W::storage);
    const bool vec = (K % kV) == 0 && (reinterpret_cast<uintptr_t>(w) % 16) == 0 && wbytes < (1ull << 31);
    const bool scatter = (p.flags & pk::kKVScatter) != 0;
    const int32_t posLoaded = pk::load_position(position, scatter);
    auto rows = [&](uint32_t unit, int s) { return w + (uint64_t)min(unit * R + s, N - 1) * K; };

    using Stage = pk::Stage<X, RES, PRE, J>;
    auto store = [&](uint32_t unit, const float *sums) {
        if ((threadIdx.x & 63) != 0) return;
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const uint32_t row = unit * R + r;
            if (row >= N) break;
            if (scatter && row >= p.qRows) {
                // K rows then V rows, head-major: cache[(h * kvStride + pos) * headDim + d]
                uint32_t j = row - p.qRows;
                const bool isV = j >= p.kvRows;
                if (isV) j -= p.kvRows;
                const int32_t pos = pk::position_value(posLoaded);
                if (pos >= 0 && (uint32_t)pos < p.kvStride) {
                    const uint64_t at = ((uint64_t)(j / p.headDim) * p.kvStride + (uint32_t)pos) * p.headDim + j % p.headDim;
                    (isV ? vcache : kcache)[at] = O::store(sums[r]);
                }
            } else {
                out[row] = O::store(sums[r]);
            }
        }
    };
    if (!(vec && K >= (uint32_t)kV && Stage::fast_ok(x_in, delta, w_post, w_pre, x_out, K, 1u))) {
        Stage::finish_scalar(xs, red, x_in, delta, w_post, w_pre, x_out, K, 1u, p.eps, p.interDataType);
        pk::stream_rows_scalar<W, R>(xs, K, units, first, stride, rows, store);
        return;
    }
    Stage stage;
    stage.issue(x_in, delta, w_post, w_pre, K);
    pk::RowStream<W, R, U> rs;
    typename pk::RowStream<W, R, U>::Ptr base[R];
    uint64_t bytes[R];
#pragma unroll
    for (int r = 0; r < R; ++r) base[r] = w, bytes[r] = wbytes;
    rs.init(rows, base, bytes, K, units, first, stride);
    rs.start(rows);
    stage.finish(xs, red, x_out, K, 1u, p.eps, p.interDataType);
    rs.run(xs, rows, store);
}

// The reference's launch: half-wave u = global thread / 32 computes rows
// 4u .. 4u + 3, lanes strided over K (4 elements per step when K % 4 == 0,
// Matvec.metal:82-97, else 1), summed over the half-wave. The block size
// must be a multiple of 32 (the reference's is 128).
template <typename X, typename W, typename O>
__device__ void matvec_nk_ref(const typename X::storage *__restrict__ x, const typename W::storage *__restrict__ w,
                              typename O::storage *__restrict__ out, const MatvecConstants &p) {
    const uint64_t gid = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    const uint32_t lane = threadIdx.x & 31;
    const uint64_t row0 = (gid >> 5) * 4;
    if (row0 >= p.N) return;  // uniform over the half-wave
    const uint32_t K = p.K, step = (K % 4 == 0) ? 4u : 1u;
    float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    for (uint32_t k0 = lane * step; k0 < K; k0 += 32 * step) {
#pragma unroll
        for (uint32_t e = 0; e < 4; ++e) {
            if (e >= step) break;
            const float xv = X::load(x[k0 + e]);
#pragma unroll
            for (int r = 0; r < 4; ++r)
                if (row0 + r < p.N) acc[r] += xv * W::load(w[(row0 + r) * K + k0 + e]);
        }
    }
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        const float sum = pk::half32_sum(acc[r]);
        if (lane == 0 && row0 + r < p.N) out[row0 + r] = O::store(sum);
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

// Streaming matvec: plain product, x staged in dynamic LDS (K floats).
#define MATVEC_NK(name, X, W, O, R)                                                                   \
    POPCORN_KERNEL void __launch_bounds__(256)                                                        \
        name(const X::storage *x, const W::storage *w, O::storage *out, MatvecConstants p) {          \
        extern __shared__ float xs[];                                                                 \
        DecodeMatvecConstants d{p.K, p.N, 0.0f, 0u, 8u, 0u, 0u, 1u, 1u};                              \
        matvec_nk<X, W, O, R, false, false, 8>(x, nullptr, nullptr, nullptr, w, out, nullptr, nullptr, \
                                               nullptr, nullptr, d, xs);                              \
    }
#define MATVEC_NK_ALL(xt, wt, ot, X, W, O)                                                   \
    MATVEC_NK(matvec_nk_stream_##xt##_##wt##_##ot##_r4, X, W, O, 4)                          \
    MATVEC_NK(matvec_nk_stream_##xt##_##wt##_##ot##_r1, X, W, O, 1)                          \
    POPCORN_KERNEL void __launch_bounds__(1024) matvec_nk_simd_##xt##_##wt##_##ot(            \
        const X::storage *x, const W::storage *w, O::storage *out, MatvecConstants p) {      \
        matvec_nk_ref<X, W, O>(x, w, out, p);                                                \
    }

// Decode matvec with the layer glue; the plain form stages up to 8 runs of
// x per thread in registers, the glued forms 2 (K <= 4096 for 16-bit types).
#define DECODE_MATVEC(name, T, O, R, RES, PRE, J)                                                           \
    POPCORN_KERNEL void __launch_bounds__(256)                                                              \
        name(const T::storage *x_in, const T::storage *delta, const float *w_post, const float *w_pre,      \
             const T::storage *w, O::storage *out, T::storage *x_out, O::storage *kcache, O::storage *vcache, \
             const int32_t *position, DecodeMatvecConstants p) {                                            \
        extern __shared__ float xs[];                                                                       \
        matvec_nk<T, T, O, R, RES, PRE, J>(x_in, delta, w_post, w_pre, w, out, x_out, kcache, vcache,      \
                                           position, p, xs);                                                \
    }
#define DECODE_MATVEC_F(base, T, O, R)                         \
    DECODE_MATVEC(base##_f0, T, O, R, false, false, 8)         \
    DECODE_MATVEC(base##_f1, T, O, R, true, false, 2)          \
    DECODE_MATVEC(base##_f2, T, O, R, false, true, 2)          \
    DECODE_MATVEC(base##_f3, T, O, R, true, true, 2)
#define DECODE_MATVEC_R(base, T, O)       \
    DECODE_MATVEC_F(base##_r4, T, O, 4) \
    DECODE_MATVEC_F(base##_r1, T, O, 1)

#define MATVEC_KN(name, X, W, O)                                                                    \
    POPCORN_KERNEL void __launch_bounds__(256)                                                      \
        name(const X::storage *x, const W::storage *w, O::storage *out, MatvecConstants p) {        \
        matvec_kn<X, W, O>(x, w, out, p);                                                           \
    }

using pk::BF16;
using pk::F16;
using pk::F32;

MATVEC_NK_ALL(f32, f32, f32, F32, F32, F32)
MATVEC_NK_ALL(f32, bf16, f32, F32, BF16, F32)
MATVEC_NK_ALL(bf16, bf16, f32, BF16, BF16, F32)
MATVEC_NK_ALL(bf16, bf16, bf16, BF16, BF16, BF16)
MATVEC_NK_ALL(f32, f16, f32, F32, F16, F32)
MATVEC_NK_ALL(f16, f16, f32, F16, F16, F32)
MATVEC_NK_ALL(f16, f16, f16, F16, F16, F16)

DECODE_MATVEC_R(decode_matvec_bf16_bf16, BF16, BF16)
DECODE_MATVEC_R(decode_matvec_bf16_f32, BF16, F32)
DECODE_MATVEC_R(decode_matvec_f16_f16, F16, F16)
DECODE_MATVEC_R(decode_matvec_f16_f32, F16, F32)
DECODE_MATVEC_R(decode_matvec_f32_f32, F32, F32)

MATVEC_KN(matvec, F32, F32, F32)
MATVEC_KN(matvec_f16, F32, F16, F32)
MATVEC_KN(matvec_bf16, F32, BF16, F32)
MATVEC_KN(matvec_bf16_bf16_f32, BF16, BF16, F32)
MATVEC_KN(matvec_bf16_bf16_bf16, BF16, BF16, BF16)
MATVEC_KN(matvec_f16_f16_f32, F16, F16, F32)
MATVEC_KN(matvec_f16_f16_f16, F16, F16, F16)
