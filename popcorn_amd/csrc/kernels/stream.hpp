// Building blocks of the decode matvecs (matvec.hip, gated_mlp.hip): a block
// stages the vector it multiplies in LDS as f32 (Stage), then each wave
// streams the weight rows of its row groups against it (RowStream).
//
// Both are shaped by one property of the vector memory pipeline: a wave's
// loads complete in issue order (vmcnt counts them in order), so waiting
// for a load also waits for every load issued before it. Stage therefore
// issues the vector's loads (L2-resident, short latency) before the first
// weight loads, and computes the layer glue while those weight loads are in
// flight; RowStream keeps U weight loads per row in flight and refills each
// slot as soon as it is consumed, so a wave never drains its queue.
#pragma once

#include "common.hpp"

namespace pk {

// Steps in flight in a RowStream (U): each step is one 16-byte load per
// row of a unit, so a lane has U x S loads in flight. 4, at 12 waves per CU
// (the host's grid), measured best on MI355X for every decode matvec shape
// (depth 2..24 x 4..24 waves per CU swept).
#ifndef POPCORN_STREAM_STEPS
#define POPCORN_STREAM_STEPS 4
#endif
constexpr int kStreamSteps = POPCORN_STREAM_STEPS;
static_assert(kStreamSteps >= 1, "a RowStream needs at least one step in flight");
constexpr int kStreamThreads = 256;
constexpr int kStreamWaves = kStreamThreads / 64;
constexpr uint32_t kKVScatter = 4u;  // DecodeMatvecConstants.flags bit 2 (runtime)

__device__ inline uint32_t uniform(uint32_t v) { return __builtin_amdgcn_readfirstlane(v); }

// The device position read by a vector (buffer) load, issued where it is
// called: a plain read of a uniform address becomes a scalar load, and
// scalar loads are waited for all together, so the kernel's first use of an
// argument would wait for this memory round trip before a weight load could
// go out. With `valid` false the load reads nothing (an empty buffer) and
// returns 0, so every path issues the same loads. Read the value through
// position_value() where it is used: the compiler would otherwise move the
// value to a scalar register, and wait for the load, right after issuing it.
__device__ inline int32_t load_position(const int32_t *position, bool valid) {
    const __amdgpu_buffer_rsrc_t r = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<int32_t *>(valid ? position : nullptr), 0, valid ? 4 : 0, 0x00020000);
    return (int32_t)__builtin_amdgcn_raw_buffer_load_b32(r, 0, 0, 0);
}
__device__ inline int32_t position_value(int32_t loaded) {
    asm volatile("" : "+v"(loaded));
    return loaded;
}

// Sum over the block (every thread gets it); `red` holds one float per wave.
__device__ inline float block_sum(float v, float *red) {
    const uint32_t lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    v = wave_sum(v);
    if (lane == 0) red[wave] = v;
    __syncthreads();
    float t = 0.0f;
#pragma unroll
    for (int w = 0; w < kStreamWaves; ++w) t += red[w];
    __syncthreads();
    return t;
}

// E floats -> one 16-byte vector of T storage (E = Vec<T>::kVec).
template <typename T>
__device__ inline u32x4 pack16(const float *v);

template <>
__device__ inline u32x4 pack16<F32>(const float *v) {
    return u32x4{__float_as_uint(v[0]), __float_as_uint(v[1]), __float_as_uint(v[2]), __float_as_uint(v[3])};
}

template <>
__device__ inline u32x4 pack16<BF16>(const float *v) {
    u32x4 r;
    r.x = (uint32_t)BF16::store(v[0]) | ((uint32_t)BF16::store(v[1]) << 16);
    r.y = (uint32_t)BF16::store(v[2]) | ((uint32_t)BF16::store(v[3]) << 16);
    r.z = (uint32_t)BF16::store(v[4]) | ((uint32_t)BF16::store(v[5]) << 16);
    r.w = (uint32_t)BF16::store(v[6]) | ((uint32_t)BF16::store(v[7]) << 16);
    return r;
}

__device__ inline uint32_t f16bits(float x) { return (uint32_t)__builtin_bit_cast(uint16_t, F16::store(x)); }

template <>
__device__ inline u32x4 pack16<F16>(const float *v) {
    return u32x4{f16bits(v[0]) | (f16bits(v[1]) << 16), f16bits(v[2]) | (f16bits(v[3]) << 16),
                 f16bits(v[4]) | (f16bits(v[5]) << 16), f16bits(v[6]) | (f16bits(v[7]) << 16)};
}

// ---- Stage -------------------------------------------------------------------
// Builds xs[0..K) (f32, LDS) with the decoder-layer glue chosen at compile
// time, in the operation order of RMSNorm.metal:32-40 and Add.metal:
//   RES: x = round(x_in + round((delta * s_d) * w_post)),
//        s_d = 1 / sqrt(mean(delta^2) + eps); block 0 also stores x to x_out
//        (the next residual stream);
//   PRE: v = round((x * s_x) * w'), s_x = 1 / sqrt(mean(x^2) + eps), with
//        w' = 1 (preMode 0), w_pre (1) or 1 + w_pre (2);
// round() being the store to the intermediate dtype `inter`. Each thread
// owns runs of E = 16 / sizeof(X) consecutive elements, run q = tid + 256 j.
// issue() loads them into registers (J runs per thread); finish() computes,
// writes LDS and ends with a barrier. Inputs that do not fit (fast_ok())
// take finish_scalar(), element by element, instead.
template <typename X, bool RES, bool PRE, int J>
struct Stage {
    static constexpr int E = Vec<X>::kVec;
    static constexpr int EW = E / 4;  // f32 vectors per run of norm weights
    using S = typename X::storage;
    Vec<X> xv[J];
    Vec<X> dv[RES ? J : 1];
    Vec<F32> wpo[RES ? J : 1][EW];
    Vec<F32> wpr[PRE ? J : 1][EW];

    // The register path needs whole 16-byte runs, aligned pointers, at most
    // J runs per thread and, with PRE, a norm weight (preMode != 0).
    __device__ static bool fast_ok(const S *x_in, const S *delta, const float *w_post, const float *w_pre,
                                   const S *x_out, uint32_t K, uint32_t preMode) {
        uintptr_t al = reinterpret_cast<uintptr_t>(x_in);
        if (RES) al |= reinterpret_cast<uintptr_t>(delta) | reinterpret_cast<uintptr_t>(w_post) |
                       reinterpret_cast<uintptr_t>(x_out);
        if (PRE) al |= reinterpret_cast<uintptr_t>(w_pre);
        return (K % E) == 0 && K / E <= (uint32_t)(kStreamThreads * J) && (al % 16) == 0 && (!PRE || preMode != 0u);
    }

    // Each thread loads its runs q < K / E; a run past the end loads nothing
    // (its registers are not read): a re-read of a valid run instead would
    // cost the memory pipeline as much as a real load (at K 2304, 288 runs
    // over 2 x 256 threads, 44% of the loads would be such re-reads).
    __device__ void issue(const S *x_in, const S *delta, const float *w_post, const float *w_pre, uint32_t K) {
        const uint32_t runs = K / E, tid = threadIdx.x;
#pragma unroll
        for (int j = 0; j < J; ++j) {
            const uint32_t q = tid + (uint32_t)(kStreamThreads * j);
            if (q >= runs) continue;
            const uint64_t at = (uint64_t)q * E;
            xv[j].load(x_in + at);
            if constexpr (RES) {
                dv[j].load(delta + at);
#pragma unroll
                for (int h = 0; h < EW; ++h) wpo[j][h].load(w_post + at + 4 * h);
            }
            if constexpr (PRE) {
#pragma unroll
                for (int h = 0; h < EW; ++h) wpr[j][h].load(w_pre + at + 4 * h);
            }
        }
    }

    // One straight-line body per rounding dtype: this code runs once per
    // launch from a cold instruction cache, and a branch on `inter` at every
    // element made it several times longer (and slower) than the arithmetic.
    __device__ void finish(float *xs, float *red, S *x_out, uint32_t K, uint32_t preMode, float eps, uint32_t inter) {
        with_round_tag(inter, [&](auto tag) { this->template finish_as<decltype(tag)::value>(xs, red, x_out, K, preMode, eps); });
    }

    template <uint32_t TAG>
    __device__ void finish_as(float *xs, float *red, S *x_out, uint32_t K, uint32_t preMode, float eps) {
        const uint32_t runs = K / E, tid = threadIdx.x;
        float ss = 0.0f;
        if constexpr (RES) {
            float sd = 0.0f;
#pragma unroll
            for (int j = 0; j < J; ++j) {
                if (tid + (uint32_t)(kStreamThreads * j) < runs) {
#pragma unroll
                    for (int e = 0; e < E; ++e) sd += dv[j].get(e) * dv[j].get(e);
                }
            }
            const float s = 1.0f / sqrtf(block_sum(sd, red) / (float)K + eps);
#pragma unroll
            for (int j = 0; j < J; ++j) {
                const uint32_t q = tid + (uint32_t)(kStreamThreads * j);
                if (q < runs) {
                    float r[E];
#pragma unroll
                    for (int e = 0; e < E; ++e) {
                        const float t = round_as<TAG>((dv[j].get(e) * s) * wpo[j][e / 4].get(e % 4));
                        r[e] = round_as<TAG>(xv[j].get(e) + t);
                        ss += r[e] * r[e];
                    }
                    store_lds(xs + (uint64_t)q * E, r);
                    if (blockIdx.x == 0) *reinterpret_cast<u32x4 *>(x_out + (uint64_t)q * E) = pack16<X>(r);
                }
            }
        } else {
#pragma unroll
            for (int j = 0; j < J; ++j) {
                const uint32_t q = tid + (uint32_t)(kStreamThreads * j);
                if (q < runs) {
                    float r[E];
#pragma unroll
                    for (int e = 0; e < E; ++e) {
                        r[e] = xv[j].get(e);
                        ss += r[e] * r[e];
                    }
                    store_lds(xs + (uint64_t)q * E, r);
                }
            }
        }
        if constexpr (PRE) {
            const float s = 1.0f / sqrtf(block_sum(ss, red) / (float)K + eps);
#pragma unroll
            for (int j = 0; j < J; ++j) {
                const uint32_t q = tid + (uint32_t)(kStreamThreads * j);
                if (q < runs) {
                    float r[E];
                    load_lds(xs + (uint64_t)q * E, r);  // this thread's own writes
#pragma unroll
                    for (int e = 0; e < E; ++e) {
                        float v = r[e] * s;
                        const float w = wpr[j][e / 4].get(e % 4);
                        v *= preMode == 2u ? 1.0f + w : w;
                        r[e] = round_as<TAG>(v);
                    }
                    store_lds(xs + (uint64_t)q * E, r);
                }
            }
        }
        __syncthreads();
    }

    __device__ static void store_lds(float *p, const float *r) {
#pragma unroll
        for (int h = 0; h < EW; ++h) *reinterpret_cast<float4 *>(p + 4 * h) = float4{r[4 * h], r[4 * h + 1], r[4 * h + 2], r[4 * h + 3]};
    }
    __device__ static void load_lds(const float *p, float *r) {
#pragma unroll
        for (int h = 0; h < EW; ++h) {
            const float4 v = *reinterpret_cast<const float4 *>(p + 4 * h);
            r[4 * h] = v.x;
            r[4 * h + 1] = v.y;
            r[4 * h + 2] = v.z;
            r[4 * h + 3] = v.w;
        }
    }

    // Element-wise form of the same computation, any K and alignment.
    __device__ static void finish_scalar(float *xs, float *red, const S *x_in, const S *delta, const float *w_post,
                                         const float *w_pre, S *x_out, uint32_t K, uint32_t preMode, float eps,
                                         uint32_t inter) {
        const uint32_t tid = threadIdx.x;
        if constexpr (RES) {
            float sd = 0.0f;
            for (uint32_t i = tid; i < K; i += kStreamThreads) {
                const float d = X::load(delta[i]);
                xs[i] = d;
                sd += d * d;
            }
            const float s = 1.0f / sqrtf(block_sum(sd, red) / (float)K + eps);
            for (uint32_t i = tid; i < K; i += kStreamThreads) {
                const float t = round_through(inter, (xs[i] * s) * w_post[i]);
                const float r = round_through(inter, X::load(x_in[i]) + t);
                xs[i] = r;
                if (blockIdx.x == 0) x_out[i] = X::store(r);
            }
        } else {
            for (uint32_t i = tid; i < K; i += kStreamThreads) xs[i] = X::load(x_in[i]);
        }
        if constexpr (PRE) {
            float ss = 0.0f;
            for (uint32_t i = tid; i < K; i += kStreamThreads) ss += xs[i] * xs[i];
            const float s = 1.0f / sqrtf(block_sum(ss, red) / (float)K + eps);
            for (uint32_t i = tid; i < K; i += kStreamThreads) {
                float v = xs[i] * s;
                if (preMode) v *= preMode == 2u ? 1.0f + w_pre[i] : w_pre[i];
                xs[i] = round_through(inter, v);
            }
        }
        __syncthreads();
    }
};

// ---- RowStream -----------------------------------------------------------------
// Rows are read through buffer resources, one per row stream s over the
// matrix that holds its rows (`base[s]`, `bytes[s]` long, under 2 GB: the
// kernels check), with 32-bit byte offsets.
constexpr uint32_t kOutOfRange = 0x80000000u;  // a buffer load there returns zeros and reads no memory

template <typename W, int S, int U>
struct RowStream {
    static constexpr int kV = Vec<W>::kVec;
    using Ptr = const typename W::storage *;
    Vec<W> buf[U][S];
    __amdgpu_buffer_rsrc_t rsrc[S];
    Ptr bases[S];
    uint32_t ioff[S];  // byte offsets of the rows of the unit being issued
    uint32_t nchunks, cpl, steps, first, stride;
    uint32_t is, ii, iu;  // issue cursor: steps issued, step within unit, unit

    template <class Rows>
    __device__ void init(const Rows &rows, const Ptr (&base)[S], const uint64_t (&bytes)[S], uint32_t K, uint32_t units,
                         uint32_t first_, uint32_t stride_) {
        nchunks = K / kV;
        cpl = (nchunks + 63) / 64;
        first = first_;
        stride = stride_;
        const uint32_t nu = first < units ? (units - first + stride - 1) / stride : 0u;
        steps = nu * cpl;
        is = 0;
        ii = 0;
        iu = first;
#pragma unroll
        for (int s = 0; s < S; ++s) {
            bases[s] = base[s];
            rsrc[s] = __builtin_amdgcn_make_buffer_rsrc(const_cast<typename W::storage *>(base[s]), 0, (int)bytes[s],
                                                        0x00020000);
        }
        set_unit(rows, iu);
    }

    template <class Rows>
    __device__ inline void set_unit(const Rows &rows, uint32_t unit) {
#pragma unroll
        for (int s = 0; s < S; ++s)
            ioff[s] = (uint32_t)(reinterpret_cast<const char *>(rows(unit, s)) - reinterpret_cast<const char *>(bases[s]));
    }

    // Loads step `is` into `slot`. Once every step is issued, a slot is
    // filled from out-of-range offsets instead (zeros, no memory read), so
    // that every path through the kernel issues the same loads and the
    // compiler's wait counts stay exact.
    template <class Rows>
    __device__ inline void issue(int slot, const Rows &rows) {
        const bool real = is < steps;
        const uint32_t c = min((threadIdx.x & 63) + 64 * ii, nchunks - 1) * 16u;
#pragma unroll
        for (int s = 0; s < S; ++s)
            buf[slot][s].raw = __builtin_bit_cast(
                u32x4, __builtin_amdgcn_raw_buffer_load_b128(rsrc[s], real ? ioff[s] + c : kOutOfRange, 0, 2));
        if (real) {
            ++is;
            if (++ii == cpl) {
                ii = 0;
                iu += stride;
                if (is < steps) set_unit(rows, iu);
            }
        }
    }

    template <class Rows>
    __device__ void start(const Rows &rows) {
#pragma unroll
        for (int u = 0; u < U; ++u) issue(u, rows);
    }

    template <class Store>
    __device__ inline void consume(int slot, const float *xs, float (&acc)[S], uint32_t &ci, uint32_t &cu,
                                   Store &store) {
        const uint32_t c = (threadIdx.x & 63) + 64 * ci;
        if (c < nchunks) {
            float xv[kV];
#pragma unroll
            for (int h = 0; h < kV / 4; ++h) {
                const float4 v = *reinterpret_cast<const float4 *>(xs + (uint64_t)c * kV + 4 * h);
                xv[4 * h] = v.x;
                xv[4 * h + 1] = v.y;
                xv[4 * h + 2] = v.z;
                xv[4 * h + 3] = v.w;
            }
#pragma unroll
            for (int s = 0; s < S; ++s) {
#pragma unroll
                for (int e = 0; e < kV; ++e) acc[s] += xv[e] * buf[slot][s].get(e);
            }
        }
        if (++ci == cpl) {
            float sums[S];
#pragma unroll
            for (int s = 0; s < S; ++s) {
                sums[s] = wave_sum(acc[s]);
                acc[s] = 0.0f;
            }
            store(cu, sums);
            ci = 0;
            cu += stride;
        }
    }

    template <class Rows, class Store>
    __device__ void run(const float *xs, const Rows &rows, Store &store) {
        float acc[S];
#pragma unroll
        for (int s = 0; s < S; ++s) acc[s] = 0.0f;
        uint32_t cs = 0, ci = 0, cu = first;
        // steady state: every refill is a real step
        while (cs + 2 * U <= steps) {
#pragma unroll
            for (int u = 0; u < U; ++u) {
                consume(u, xs, acc, ci, cu, store);
                issue(u, rows);
            }
            cs += U;
        }
        while (cs < steps) {
#pragma unroll
            for (int u = 0; u < U; ++u) {
                if (cs + u < steps) consume(u, xs, acc, ci, cu, store);
                issue(u, rows);
            }
            cs += U;
        }
    }
};

// The same product with scalar loads, for rows whose length is not a
// multiple of the vector width or whose base is not 16-byte aligned.
template <typename W, int S, class Rows, class Store>
__device__ void stream_rows_scalar(const float *xs, uint32_t K, uint32_t units, uint32_t first, uint32_t stride,
                                   const Rows &rows, Store &store) {
    const uint32_t lane = threadIdx.x & 63;
    for (uint32_t unit = first; unit < units; unit += stride) {
        float acc[S];
#pragma unroll
        for (int s = 0; s < S; ++s) acc[s] = 0.0f;
        for (uint32_t k = lane; k < K; k += 64) {
            const float x = xs[k];
#pragma unroll
            for (int s = 0; s < S; ++s) acc[s] += x * W::load(rows(unit, s)[k]);
        }
        float sums[S];
#pragma unroll
        for (int s = 0; s < S; ++s) sums[s] = wave_sum(acc[s]);
        store(unit, sums);
    }
}

}  // namespace pk
