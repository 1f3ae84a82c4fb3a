// Fused front half of the gated MLP at decode (one token):
//   n = RMSNorm(x; w_norm, eps)              stored as T
//   g = n . Wg[j], u = n . Wu[j]             stored as T
//   a = GeluTanh(g)                          stored as T
//   h[j] = a * u                             stored as T
// which the reference runs as RMSNorm, two Matmul dispatches, GeluTanh and
// Mul with a T-typed tensor between each (Examples/GemmaCLI/Sources/GemmaCLI/
// Gemma4TextInference.swift:416-428, Gemma4Workspace.swift:37-42). Each
// intermediate is rounded through T exactly where the reference stores it
// (interDataType), so h matches the composition; the down projection then
// runs as a matvec over h.
//
// Every block recomputes the normalisation of x (H values from L2) into LDS;
// each of its 4 waves then streams R rows of Wg and the same R rows of Wu
// with 16-byte non-temporal loads, so 2R row streams are in flight per wave.
#include "common.hpp"

namespace {

constexpr int kWaves = 4;
constexpr int kUnroll = 4;

template <typename T, int R>
__device__ void gate_up(const typename T::storage *__restrict__ x, const float *__restrict__ norm_w,
                        const typename T::storage *__restrict__ wg, const typename T::storage *__restrict__ wu,
                        typename T::storage *__restrict__ h, const GatedMLPConstants &p, float *xs) {
    __shared__ float partial[kWaves];
    constexpr int kV = pk::Vec<T>::kVec;
    const uint32_t H = p.H, F = p.F;
    const uint32_t tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;

    // RMSNorm prologue (RMSNorm.metal:16-41), result rounded through T.
    float ss = 0.0f;
    for (uint32_t i = tid; i < H; i += blockDim.x) {
        float v = T::load(x[i]);
        xs[i] = v;
        ss += v * v;
    }
    ss = pk::wave_sum(ss);
    if (lane == 0) partial[wave] = ss;
    __syncthreads();
    const float total = partial[0] + partial[1] + partial[2] + partial[3];
    const float scale = 1.0f / sqrtf(total / (float)H + p.eps);
    for (uint32_t i = tid; i < H; i += blockDim.x) {
        float v = xs[i] * scale;
        if (p.hasWeight) {
            float w = norm_w[i];
            if (p.addOneToWeight) w = 1.0f + w;
            v *= w;
        }
        xs[i] = pk::round_through(p.interDataType, v);
    }
    __syncthreads();

    const uint32_t row0 = (blockIdx.x * kWaves + wave) * R;
    if (row0 >= F) return;
    float ag[R], au[R];
#pragma unroll
    for (int r = 0; r < R; ++r) ag[r] = au[r] = 0.0f;

    const bool vec = (H % kV) == 0 && ((reinterpret_cast<uintptr_t>(wg) | reinterpret_cast<uintptr_t>(wu)) % 16) == 0;
    if (vec) {
        const uint32_t nchunks = H / kV;
        const typename T::storage *rg[R], *ru[R];
#pragma unroll
        for (int r = 0; r < R; ++r) {
            uint64_t row = min(row0 + r, F - 1);
            rg[r] = wg + row * H;
            ru[r] = wu + row * H;
        }
        for (uint32_t c0 = lane; c0 < nchunks; c0 += 64 * kUnroll) {
            pk::Vec<T> vg[kUnroll][R], vu[kUnroll][R];
#pragma unroll
            for (int u = 0; u < kUnroll; ++u) {
                uint32_t c = c0 + 64 * u;
                if (c < nchunks) {
#pragma unroll
                    for (int r = 0; r < R; ++r) {
                        vg[u][r].load_nt(rg[r] + (uint64_t)c * kV);
                        vu[u][r].load_nt(ru[r] + (uint64_t)c * kV);
                    }
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
                        for (int e = 0; e < kV; ++e) {
                            ag[r] += xv[e] * vg[u][r].get(e);
                            au[r] += xv[e] * vu[u][r].get(e);
                        }
                    }
                }
            }
        }
    } else {
        for (uint32_t k = lane; k < H; k += 64) {
            float xv = xs[k];
#pragma unroll
            for (int r = 0; r < R; ++r) {
                uint64_t row = min(row0 + r, F - 1);
                ag[r] += xv * T::load(wg[row * H + k]);
                au[r] += xv * T::load(wu[row * H + k]);
            }
        }
    }
#pragma unroll
    for (int r = 0; r < R; ++r) {
        float g = pk::round_through(p.interDataType, pk::wave_sum(ag[r]));
        float u = pk::round_through(p.interDataType, pk::wave_sum(au[r]));
        if (lane == 0 && row0 + r < F) {
            float a = pk::round_through(p.interDataType, pk::gelu_tanh(g));
            h[row0 + r] = T::store(a * u);
        }
    }
}

}  // namespace

// x is normalised into dynamic LDS (H floats).
#define GATE_UP(name, T, R)                                                                             \
    POPCORN_KERNEL void __launch_bounds__(256)                                                          \
        name(const T::storage *x, const float *norm_w, const T::storage *wg, const T::storage *wu,      \
             T::storage *h, GatedMLPConstants p) {                                                      \
        extern __shared__ float xs[];                                                                   \
        gate_up<T, R>(x, norm_w, wg, wu, h, p, xs);                                                     \
    }

using pk::BF16;
using pk::F16;
using pk::F32;

GATE_UP(gated_mlp_gate_up_f32, F32, 2)
GATE_UP(gated_mlp_gate_up_bf16, BF16, 2)
GATE_UP(gated_mlp_gate_up_f16, F16, 2)
GATE_UP(gated_mlp_gate_up_f32_r1, F32, 1)
GATE_UP(gated_mlp_gate_up_bf16_r1, BF16, 1)
GATE_UP(gated_mlp_gate_up_f16_r1, F16, 1)
