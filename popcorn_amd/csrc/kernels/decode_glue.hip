// Decode-loop glue: token in (embedding gather), token out (argmax), the
// position update that closes a captured step, and a device-side normal
// generator for synthetic benchmark inputs.
#include "common.hpp"
#include "q4.hpp"

namespace {

// EmbeddingGather.metal:6-23: out[n, :] = table[ids[n], :].
// embedding_gather*_ext (the descriptor's): one thread per 16-byte run of a
// row; an id outside [0, V) (when V is given) gives zeros.
// embedding_gather* keep the reference's host names, parameter list and
// launch geometry (EmbeddingGather.swift:26, :117-118): the thread at (x, y)
// copies elements 4y .. 4y + 3 of token x's row; the grid strides in both
// dimensions, so any launch shape covers the rows.
template <typename T, typename O>
__device__ void gather_ref(const int32_t *__restrict__ ids, const typename T::storage *__restrict__ table,
                           typename O::storage *__restrict__ out, const EmbeddingGatherConstants &p) {
    const uint32_t chunks = (p.H + 3) / 4;
    const uint32_t sx = gridDim.x * blockDim.x, sy = gridDim.y * blockDim.y;
    for (uint32_t n = blockIdx.x * blockDim.x + threadIdx.x; n < p.N; n += sx) {
        const uint64_t row = (uint32_t)ids[n];
        for (uint32_t c = blockIdx.y * blockDim.y + threadIdx.y; c < chunks; c += sy) {
            for (uint32_t h = 4 * c; h < 4 * c + 4 && h < p.H; ++h)
                out[(uint64_t)n * p.H + h] = O::store(T::load(table[row * p.H + h]));
        }
    }
}

template <typename T, typename O>
__device__ void gather(const int32_t *__restrict__ ids, const typename T::storage *__restrict__ table,
                       typename O::storage *__restrict__ out, const EmbeddingGatherExtConstants &p) {
    constexpr uint32_t kRun = 16 / sizeof(typename T::storage);
    const uint32_t runs = (p.H + kRun - 1) / kRun;
    const uint64_t total = (uint64_t)p.N * runs;
    for (uint64_t r = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; r < total; r += (uint64_t)gridDim.x * blockDim.x) {
        const uint32_t n = (uint32_t)(r / runs), h0 = (uint32_t)(r % runs) * kRun;
        const int32_t id = ids[n];
        const bool ok = id >= 0 && (p.V == 0 || (uint32_t)id < p.V);
        for (uint32_t h = h0; h < h0 + kRun && h < p.H; ++h) {
            float v = ok ? T::load(table[(uint64_t)(uint32_t)id * p.H + h]) : 0.0f;
            out[(uint64_t)n * p.H + h] = O::store(v);
        }
    }
}

// Argmax.metal:7-9: a candidate wins on a larger value, or an equal value at
// a smaller index.
__device__ inline bool better(float v, int32_t i, float bv, int32_t bi) { return v > bv || (v == bv && i < bi); }

__device__ inline void wave_best(float &bv, int32_t &bi) {
    for (int s = 32; s > 0; s >>= 1) {
        float ov = __shfl_xor(bv, s, 64);
        int32_t oi = __shfl_xor(bi, s, 64);
        if (better(ov, oi, bv, bi)) {
            bv = ov;
            bi = oi;
        }
    }
}

__device__ void block_best(float &bv, int32_t &bi) {
    __shared__ float sv[16];
    __shared__ int32_t si[16];
    wave_best(bv, bi);
    const uint32_t lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nw = (blockDim.x + 63) >> 6;
    if (lane == 0) {
        sv[wave] = bv;
        si[wave] = bi;
    }
    __syncthreads();
    bv = -INFINITY;
    bi = 0x7fffffff;
    for (uint32_t w = 0; w < nw; ++w)
        if (better(sv[w], si[w], bv, bi)) {
            bv = sv[w];
            bi = si[w];
        }
}

}  // namespace

#define GATHER(name, T, O)                                                                                   \
    POPCORN_KERNEL void __launch_bounds__(1024)                                                              \
        name(const int32_t *ids, const T::storage *table, O::storage *out, EmbeddingGatherConstants p) {     \
        gather_ref<T, O>(ids, table, out, p);                                                                \
    }                                                                                                        \
    POPCORN_KERNEL void __launch_bounds__(256)                                                               \
        name##_ext(const int32_t *ids, const T::storage *table, O::storage *out, EmbeddingGatherExtConstants p) { \
        gather<T, O>(ids, table, out, p);                                                                    \
    }

using pk::BF16;
using pk::F16;
using pk::F32;

GATHER(embedding_gather, F32, F32)
GATHER(embedding_gather_f16, F16, F16)
GATHER(embedding_gather_bf16, BF16, BF16)
GATHER(embedding_gather_bf16_to_f32, BF16, F32)

// Stage 1: block (slice, row) reduces its slice of the row to one candidate.
// Grid: x = slices, y = rows. A NaN never wins (v > best is false for NaN),
// as in the reference's sequential loop when the first element is not NaN.
POPCORN_KERNEL void __launch_bounds__(256)
    argmax_partial(const float *x, float *pv, int32_t *pi, ArgmaxSliceConstants p) {
    const uint32_t row = blockIdx.y, slices = gridDim.x;
    const uint64_t per = ((uint64_t)p.N + slices - 1) / slices;
    const uint64_t lo = (uint64_t)blockIdx.x * per, hi = min(lo + per, (uint64_t)p.N);
    const float *xr = x + (uint64_t)row * p.N;
    float bv = -INFINITY;
    int32_t bi = 0x7fffffff;
    // kArgmaxBatch loads per thread in flight together (a decode-sized slice
    // of 4096 is one memory round trip); entries past the slice re-read its
    // last element and are masked. better() is a total order on (value,
    // index), so the visiting order does not change the result.
    constexpr int kArgmaxBatch = 16;
    if (lo < hi) {
        for (uint64_t i0 = lo + threadIdx.x; i0 < hi; i0 += (uint64_t)blockDim.x * kArgmaxBatch) {
            float v[kArgmaxBatch];
#pragma unroll
            for (int b = 0; b < kArgmaxBatch; ++b) v[b] = xr[min(i0 + (uint64_t)b * blockDim.x, hi - 1)];
#pragma unroll
            for (int b = 0; b < kArgmaxBatch; ++b) {
                const uint64_t i = i0 + (uint64_t)b * blockDim.x;
                if (i < hi && better(v[b], (int32_t)i, bv, bi)) {
                    bv = v[b];
                    bi = (int32_t)i;
                }
            }
        }
    }
    block_best(bv, bi);
    if (threadIdx.x == 0) {
        pv[(uint64_t)row * slices + blockIdx.x] = bv;
        pi[(uint64_t)row * slices + blockIdx.x] = bi;
    }
}

// Stage 2: one block per row merges the p.slices candidates. The reference's
// loop starts from x[0] (Argmax.metal:20-21), so a NaN at x[0] keeps index 0;
// a row with no candidate (all NaN) also yields 0.
POPCORN_KERNEL void __launch_bounds__(256)
    argmax_finish(const float *x, const float *pv, const int32_t *pi, int32_t *indices, ArgmaxSliceConstants p) {
    const uint32_t row = blockIdx.x, slices = p.slices;
    float bv = -INFINITY;
    int32_t bi = 0x7fffffff;
    for (uint32_t s = threadIdx.x; s < slices; s += blockDim.x) {
        float v = pv[(uint64_t)row * slices + s];
        int32_t i = pi[(uint64_t)row * slices + s];
        if (better(v, i, bv, bi)) {
            bv = v;
            bi = i;
        }
    }
    block_best(bv, bi);
    if (threadIdx.x == 0) {
        if (bi == 0x7fffffff || __builtin_isnan(x[(uint64_t)row * p.N])) bi = 0;
        indices[row] = bi;
    }
}

namespace {

// The tail of a greedy decode step (DecodeNextTokenConstants): stage 2 of the
// argmax over the candidates of argmax_partial; the token is stored in
// history[position % historyLen] and the position advances by delta (a
// kernel, so graph replays need no host write); then the next step's input
// row as the gather and scalar multiply at the head of a step compute it.
// One block.
template <bool Q4>
__device__ void next_token(const float *logits, const float *pv, const int32_t *pi, int32_t *token, int32_t *pos,
                           int32_t *history, const uint16_t *table, const uint32_t *W, const uint16_t *Sc,
                           const uint16_t *Bi, uint16_t *x, const DecodeNextTokenConstants &c) {
    float bv = -INFINITY;
    int32_t bi = 0x7fffffff;
    for (uint32_t s = threadIdx.x; s < c.slices; s += blockDim.x) {
        if (better(pv[s], pi[s], bv, bi)) {
            bv = pv[s];
            bi = pi[s];
        }
    }
    block_best(bv, bi);  // every thread holds the winner
    if (bi == 0x7fffffff || __builtin_isnan(logits[0])) bi = 0;
    if (threadIdx.x == 0) {
        token[0] = bi;
        const int32_t at = pos[0];
        if (c.historyLen && at >= 0) history[(uint32_t)at % c.historyLen] = bi;
        pos[0] = at + c.delta;
    }
    const uint64_t row = (uint32_t)bi;
    if constexpr (!Q4) {
        for (uint32_t h = threadIdx.x; h < c.H; h += blockDim.x)
            x[h] = BF16::store(BF16::load(table[row * c.H + h]) * c.scale);
    } else {
        const uint32_t wordsPerRow = c.H / 8, groups = c.H / 64;
        for (uint32_t wi = threadIdx.x; wi < wordsPerRow; wi += blockDim.x) {
            const uint32_t g = wi / pk::kQ4GroupWords;
            const uint32_t w = W[row * wordsPerRow + wi];
            const float s = pk::bf16_lo(Sc[row * groups + g]);
            const float b = c.hasBias ? pk::bf16_lo(Bi[row * groups + g]) : 0.0f;
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                const uint16_t te = BF16::store((float)((w >> (4 * e)) & 15u) * s + b);
                x[wi * 8 + e] = BF16::store(BF16::load(te) * c.scale);
            }
        }
    }
}

}  // namespace

POPCORN_KERNEL void __launch_bounds__(256)
    decode_next_token_bf16(const float *logits, const float *pv, const int32_t *pi, int32_t *token, int32_t *pos,
                           int32_t *history, const uint16_t *table, uint16_t *x, DecodeNextTokenConstants c) {
    next_token<false>(logits, pv, pi, token, pos, history, table, nullptr, nullptr, nullptr, x, c);
}

POPCORN_KERNEL void __launch_bounds__(256)
    decode_next_token_q4_bf16(const float *logits, const float *pv, const int32_t *pi, int32_t *token, int32_t *pos,
                              int32_t *history, const uint32_t *W, const uint16_t *Sc, const uint16_t *Bi, uint16_t *x,
                              DecodeNextTokenConstants c) {
    next_token<true>(logits, pv, pi, token, pos, history, nullptr, W, Sc, Bi, x, c);
}


namespace {

__device__ inline uint64_t splitmix64(uint64_t z) {
    z += 0x9E3779B97F4A7C15ull;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

// Element i takes the pair (i / 2): two uniforms from splitmix64 of the
// pair index, Box-Muller, cos for even i and sin for odd i.
template <typename T>
__device__ void fill_normal(typename T::storage *out, const FillNormalConstants &p) {
    const float two_pi = 6.283185307179586f;
    for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < p.count; i += (uint64_t)gridDim.x * blockDim.x) {
        const uint64_t pair = i >> 1;
        const uint64_t h1 = splitmix64(p.seed * 0xD1B54A32D192ED03ull + 2 * pair);
        const uint64_t h2 = splitmix64(p.seed * 0xD1B54A32D192ED03ull + 2 * pair + 1);
        const float u1 = ((float)(h1 >> 40) + 1.0f) * (1.0f / 16777216.0f);  // (0, 1]
        const float u2 = (float)(h2 >> 40) * (1.0f / 16777216.0f);           // [0, 1)
        const float r = sqrtf(-2.0f * __logf(u1));
        const float z = (i & 1) ? r * __sinf(two_pi * u2) : r * __cosf(two_pi * u2);
        out[i] = T::store(p.mean + p.stddev * z);
    }
}

}  // namespace

POPCORN_KERNEL void __launch_bounds__(256) fill_normal_f32(float *out, FillNormalConstants p) { fill_normal<F32>(out, p); }
POPCORN_KERNEL void __launch_bounds__(256) fill_normal_bf16(uint16_t *out, FillNormalConstants p) { fill_normal<BF16>(out, p); }
POPCORN_KERNEL void __launch_bounds__(256) fill_normal_f16(_Float16 *out, FillNormalConstants p) { fill_normal<F16>(out, p); }

// Holds its stream for `ticks` of the 100 MHz constant clock (at most 0.1 s)
// and touches no memory: launched ahead of timed dispatches, so that the host
// has enqueued them before the GPU reaches them and they run back to back, as
// a graph replay runs them.
POPCORN_KERNEL void __launch_bounds__(64) hold_stream(uint64_t ticks) {
    const uint64_t limit = ticks < 10000000ull ? ticks : 10000000ull;
    const uint64_t t0 = __builtin_amdgcn_s_memrealtime();
    while (__builtin_amdgcn_s_memrealtime() - t0 < limit) __builtin_amdgcn_s_sleep(32);
}
