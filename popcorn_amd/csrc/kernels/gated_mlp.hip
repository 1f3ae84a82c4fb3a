// Fused front half of the gated MLP at decode (one token):
//   [x = round(x_in + round(RMSNorm(delta) * w_post))]   residual (optional)
//   n = RMSNorm(x; w_norm, eps)              stored as T
//   g = n . Wg[j], u = n . Wu[j]             stored as T
//   a = GeluTanh(g)                          stored as T
//   h[j] = a * u                             stored as T
// which the reference runs as RMSNorm, two Matmul dispatches, GeluTanh and
// Mul with a T-typed tensor between each (Examples/GemmaCLI/Sources/GemmaCLI/
// Gemma4TextInference.swift:416-428, Gemma4Workspace.swift:37-42), preceded
// in a decoder layer by the attention block's post-norm and residual Add
// (:400-404). Each intermediate is rounded through T exactly where the
// reference stores it (interDataType), so h matches the composition; the
// down projection then runs as a matvec over h.
//
// A unit is R rows of Wg and the same R rows of Wu (2R rows streamed
// together, RowStream); the block stages the normalised x (Stage, with the
// residual in front when p.residual) while the first weight loads are in
// flight. The host sizes the grid so every wave gets the same number of
// units, give or take one.
#include "stream.hpp"

namespace {

using pk::kStreamSteps;
using pk::kStreamWaves;

template <typename T, int R, bool RES>
__device__ void gate_up(const typename T::storage *__restrict__ x, const float *__restrict__ norm_w,
                        const typename T::storage *__restrict__ wg, const typename T::storage *__restrict__ wu,
                        typename T::storage *__restrict__ h, const typename T::storage *__restrict__ delta,
                        const float *__restrict__ w_post, typename T::storage *__restrict__ x_out,
                        const GatedMLPConstants &p, float *xs) {
    constexpr int S = 2 * R, U = kStreamSteps;
    constexpr int kV = pk::Vec<T>::kVec;
    __shared__ float red[kStreamWaves];
    const uint32_t H = p.H, F = p.F;
    const uint32_t units = (F + R - 1) / R;
    const uint32_t wave = pk::uniform(threadIdx.x >> 6);
    const uint32_t first = blockIdx.x * kStreamWaves + wave, stride = gridDim.x * kStreamWaves;
    const uint64_t wbytes = (uint64_t)F * H * sizeof(typename T::storage);
    const bool vec = (H % kV) == 0 && ((reinterpret_cast<uintptr_t>(wg) | reinterpret_cast<uintptr_t>(wu)) % 16) == 0 &&
                     wbytes < (1ull << 31);
    const uint32_t preMode = p.hasWeight ? (p.addOneToWeight ? 2u : 1u) : 0u;
    const uint32_t inter = p.interDataType;
    auto rows = [&](uint32_t unit, int s) {
        const uint64_t row = min(unit * R + (uint32_t)(s % R), F - 1);
        return (s < R ? wg : wu) + row * H;
    };
    auto store = [&](uint32_t unit, const float *sums) {
        if ((threadIdx.x & 63) != 0) return;
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const uint32_t row = unit * R + r;
            if (row >= F) break;
            const float g = pk::round_through(inter, sums[r]);
            const float u = pk::round_through(inter, sums[R + r]);
            const float a = pk::round_through(inter, pk::gelu_tanh(g));
            h[row] = T::store(a * u);
        }
    };
    using Stage = pk::Stage<T, RES, true, 2>;
    if (!(vec && H >= (uint32_t)kV && Stage::fast_ok(x, delta, w_post, norm_w, x_out, H, preMode))) {
        Stage::finish_scalar(xs, red, x, delta, w_post, norm_w, x_out, H, preMode, p.eps, inter);
        pk::stream_rows_scalar<T, S>(xs, H, units, first, stride, rows, store);
        return;
    }
    Stage stage;
    stage.issue(x, delta, w_post, norm_w, H);
    pk::RowStream<T, S, U> rs;
    typename pk::RowStream<T, S, U>::Ptr base[S];
    uint64_t bytes[S];
#pragma unroll
    for (int s = 0; s < S; ++s) base[s] = s < R ? wg : wu, bytes[s] = wbytes;
    rs.init(rows, base, bytes, H, units, first, stride);
    rs.start(rows);
    stage.finish(xs, red, x_out, H, preMode, p.eps, inter);
    rs.run(xs, rows, store);
}

}  // namespace

// x is normalised into dynamic LDS (H floats). delta, w_post and x_out are
// read / written only by the _res forms (p.residual set).
#define GATE_UP(name, T, R, RES)                                                                        \
    POPCORN_KERNEL void __launch_bounds__(256)                                                          \
        name(const T::storage *x, const float *norm_w, const T::storage *wg, const T::storage *wu,      \
             T::storage *h, const T::storage *delta, const float *w_post, T::storage *x_out,            \
             GatedMLPConstants p) {                                                                     \
        extern __shared__ float xs[];                                                                   \
        gate_up<T, R, RES>(x, norm_w, wg, wu, h, delta, w_post, x_out, p, xs);                          \
    }
#define GATE_UP_ALL(base, T)                  \
    GATE_UP(base, T, 2, false)                \
    GATE_UP(base##_r1, T, 1, false)           \
    GATE_UP(base##_res, T, 2, true)           \
    GATE_UP(base##_r1_res, T, 1, true)

using pk::BF16;
using pk::F16;
using pk::F32;

GATE_UP_ALL(gated_mlp_gate_up_f32, F32)
GATE_UP_ALL(gated_mlp_gate_up_bf16, BF16)
GATE_UP_ALL(gated_mlp_gate_up_f16, F16)
