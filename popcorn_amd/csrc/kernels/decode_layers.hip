// The decoder layers of one batch-1 decode step as one persistent kernel
// (DecodeLayersConstants): per layer, the op sequence of
// Examples/GemmaCLI/Sources/GemmaCLI/Gemma4TextInference.swift:312-436
// (input RMSNorm, QKV matvec, KV-cache write, split-KV attention with its
// log-sum-exp combine, O projection, post-attention norm + residual, pre-FFN
// norm, gate/up matvecs with GELU-tanh gating, down matvec, post-FFN norm +
// residual), with the rounding points of the per-kernel decode path
// (matvec.hip, gated_mlp.hip, flash_decoding.hip): every intermediate the
// reference stores is rounded to bf16 where it stores it.
//
// Why one kernel: each decode matvec or attention launch pays a fixed cost of
// a few microseconds (launch, the first memory round trip, the tail), and a
// kernel boundary is a point where nothing streams. Here the grid is one
// block per CU, and nothing waits for the whole grid:
//  * every activation a phase produces (q/k/v, attention partials, attn, o,
//    hidden, mlp) is stored element by element together with a tag naming
//    the launch, layer and phase (agent-coherent sc1 stores of single-copy
//    atomic words), so a consumer knows a value is ready by reading it; a
//    block's last producing wave then bumps one of 8 arrival counters, which
//    consumers poll (8 lines) before they fetch a vector, so the polling
//    itself moves almost no data;
//  * each block has one staging wave that polls the next phase's input vector
//    until every element carries the expected tag, computes the residual and
//    norm glue on it and leaves it in LDS (double-buffered), while the
//    block's streaming waves still work on the current phase;
//  * the streaming waves run the matvecs from per-wave LDS rings filled by
//    direct global -> LDS copies, and issue the first copies of their next
//    phase (and the next layer's cached K/V rows) before they wait at the
//    block barrier, so HBM keeps streaming while the inputs settle.
// The staging wave's polls are its only global memory operations, so they
// never queue behind the streaming waves' copies. Every poll is bounded
// (spinTicks of the 100 MHz clock): one that runs out sets the abort word
// and the block's abort flag, after which no poll of the block waits, so the
// grid always drains. Tags are 16 bits, (epoch * layers * 8 + layer * 8 +
// phase) mod 2^16, with the epoch advanced by the last block to finish: a
// buffer word is rewritten every layer, so a stale word's tag is 8 behind.
#include "decode_layers_geometry.hpp"
#include "stream.hpp"

namespace {

using pk::BF16;
using pk::u32x4;
namespace LY = pk::layers;
using LY::kThreads;
using LY::kWaves;
using LY::kWork;

constexpr int kKvLoads = 3;  // K (and V) loads per worker wave prefetched for the attention phase
// Ring depths (steps of 1 KB per row): QKV and down over the whole region,
// gate/up (two rows per unit) in ring 0, O in ring 1.
constexpr int kDepthQKV = 12, kDepthGU = 4, kDepthO = 4, kDepthDown = 12;
static_assert(kDepthQKV * 1024 <= (int)LY::kRegion && kDepthDown * 1024 <= (int)LY::kRegion, "region");
static_assert(kDepthGU * 2048 <= (int)LY::kRing0 && kDepthO * 1024 <= (int)LY::kRing1, "rings");

// phases (the tag's low 3 bits)
constexpr uint32_t kPhQKV = 0, kPhPart = 1, kPhAttn = 2, kPhO = 3, kPhHidden = 4, kPhMlp = 5;

// ---- agent-coherent access (sc1) -----------------------------------------------
__device__ inline uint32_t ld32(const void *p) {
    return __hip_atomic_load(reinterpret_cast<uint32_t *>(const_cast<void *>(p)), __ATOMIC_RELAXED,
                             __HIP_MEMORY_SCOPE_AGENT);
}
__device__ inline uint64_t ld64(const void *p) {
    return __hip_atomic_load(reinterpret_cast<uint64_t *>(const_cast<void *>(p)), __ATOMIC_RELAXED,
                             __HIP_MEMORY_SCOPE_AGENT);
}
__device__ inline void st64(void *p, uint64_t v) {
    __hip_atomic_store(reinterpret_cast<uint64_t *>(p), v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ inline void st32(void *p, uint32_t v) {
    __hip_atomic_store(reinterpret_cast<uint32_t *>(p), v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// 16-byte coherent load through a buffer resource (cache policy sc1): four
// 32-bit words, each single-copy atomic. Offsets in bytes.
__device__ inline __amdgpu_buffer_rsrc_t rsrc(const void *base, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), 0, bytes, 0x00020000);
}
constexpr int kSc1 = 16;
__device__ inline u32x4 ldc16(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    return __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, kSc1);
}

__device__ inline float bf(uint32_t bits16) { return __uint_as_float(bits16 << 16); }
__device__ inline uint32_t bfbits(float x) { return (uint32_t)BF16::store(x); }
__device__ inline float rnd(float x) { return pk::round_as<10u>(x); }

// 1 when every active lane's v is non-zero (uniform)
__device__ inline uint32_t wave_all(uint32_t v) { return __ballot(v == 0u) == 0ull ? 1u : 0u; }

// ---- polls (the staging wave, or a worker wave for its share) ------------------
// Block-local abort flag in LDS, set when a poll times out (the global abort
// word tells the host).
struct Poll {
    uint32_t *abortWord;
    volatile uint32_t *blockAbort;  // LDS
    uint64_t limit;

    __device__ bool aborted() const { return *blockAbort != 0u; }
    __device__ bool expired(uint64_t t0, uint32_t lane) {
        if (__builtin_amdgcn_s_memrealtime() - t0 <= limit) return false;
        if (lane == 0) {
            st32(abortWord, 1u);
            *blockAbort = 1u;
        }
        return true;
    }
};

// Loads n tagged bf16 words (n % 4 == 0, n <= 4 * 64 * N) from `src` until
// every word carries `tag`, lane-interleaved in 16-byte groups: v[g][e] is
// element 4 (lane + 64 g) + e.
template <int N>
__device__ inline void poll_vector(const uint32_t *src, uint32_t n, uint32_t tag, Poll &pl, float (&v)[N][4],
                                   uint32_t lane) {
    const uint32_t groups = n / 4u;
    const __amdgpu_buffer_rsrc_t r = rsrc(src, n * 4u);
    const uint64_t t0 = __builtin_amdgcn_s_memrealtime();
    for (;;) {
        u32x4 w[N];
#pragma unroll
        for (int g = 0; g < N; ++g) {
            const uint32_t gi = lane + 64u * g;
            w[g] = ldc16(r, (gi < groups ? gi : 0u) * 16u);
        }
        uint32_t ok = 1u;
#pragma unroll
        for (int g = 0; g < N; ++g) {
            if (lane + 64u * g < groups)
                ok &= (w[g].x >> 16) == tag && (w[g].y >> 16) == tag && (w[g].z >> 16) == tag && (w[g].w >> 16) == tag;
            v[g][0] = bf(w[g].x & 0xffffu);
            v[g][1] = bf(w[g].y & 0xffffu);
            v[g][2] = bf(w[g].z & 0xffffu);
            v[g][3] = bf(w[g].w & 0xffffu);
        }
        if (wave_all(ok) || pl.aborted() || pl.expired(t0, lane)) return;
        __builtin_amdgcn_s_sleep(1);
    }
}

__device__ inline uint32_t wave_sum_u32(uint32_t v) {
#pragma unroll
    for (int s = 1; s < 64; s <<= 1) v += (uint32_t)__shfl_xor((int)v, s, 64);
    return v;
}

// ---- readiness: arrival counters --------------------------------------------------
// Every block arrives once per phase of every layer, when its producing waves
// have issued their stores of the phase (without waiting for them to land:
// the tags say when each word has), on counter blockIdx % 8. A consumer
// first waits until the 8 counters sum to the arrivals of that phase (a
// poll of 8 lines), then fetches the vector and checks its tags, retrying
// words whose stores are still on their way.
__device__ inline void arrive_global(uint32_t *sync) {
    __hip_atomic_fetch_add(sync + (blockIdx.x % LY::kCounters) * LY::kLine, 1u, __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_AGENT);
}

// The streaming waves of a block: the last one to finish the phase arrives.
__device__ inline void arrive_workers(uint32_t *sync, uint32_t *ldsCount, uint32_t lane) {
    asm volatile("" ::: "memory");
    uint32_t n = 0;
    if (lane == 0) n = atomicAdd(ldsCount, 1u);
    n = __shfl(n, 0, 64);
    if (n == (uint32_t)kWork - 1u && lane == 0) {
        *ldsCount = 0;  // every worker has arrived; the next phase starts after a block barrier
        arrive_global(sync);
    }
}

__device__ inline void wait_arrivals(const uint32_t *sync, uint32_t target, Poll &pl, uint32_t lane) {
    if (pl.aborted()) return;
    const uint64_t t0 = __builtin_amdgcn_s_memrealtime();
    for (;;) {
        uint32_t v = lane < (uint32_t)LY::kCounters ? ld32(sync + lane * LY::kLine) : 0u;
        v = wave_sum_u32(v);
        if (v >= target || pl.aborted() || pl.expired(t0, lane)) return;
        __builtin_amdgcn_s_sleep(1);
    }
}

// ---- the staging wave's glue (RMSNorm.metal:32-40 and Add.metal, in the
// order of the decode matvecs' Stage) ---------------------------------------------
//   first layer: x = x_in;
//   else:        x = round(xres + round((delta * s_d) * w_post)),
//                s_d = 1 / sqrt(mean(delta^2) + eps);
//   xres = x;   xs = round((x * s_x) * w_pre), s_x = 1 / sqrt(mean(x^2) + eps).
// v holds delta (or x_in), elements 4 (lane + 64 g) + e. x_out (optional)
// receives x as bf16.
// The glue's norm weights (f32): copied into LDS by direct global -> LDS
// loads (1 KB per instruction, H % 256 == 0) before the staging wave starts
// waiting for its input, so their round trip overlaps the wait; they land
// before anything the wave loads later (issue order).
typedef __attribute__((address_space(3))) void lds_void;
__device__ inline void load_norms(float *dst, const float *w_post, const float *w_pre, uint32_t n, uint32_t lane) {
    const uint32_t chunks = n / 256u;  // 1 KB of f32 each
    for (uint32_t k = 0; k < chunks; ++k) {
        if (w_post)
            __builtin_amdgcn_global_load_lds(w_post + 256u * k + 4u * lane, (lds_void *)(dst + 256u * k), 16, 0, 0);
        __builtin_amdgcn_global_load_lds(w_pre + 256u * k + 4u * lane, (lds_void *)(dst + n + 256u * k), 16, 0, 0);
    }
}

template <int N>
__device__ inline void glue(float (&v)[N][4], uint32_t n, bool first, uint16_t *xres, uint16_t *xs, const float *nw,
                            float eps, uint16_t *x_out, uint32_t lane) {
    const uint32_t groups = n / 4u;
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // the norm weights' copies have landed
    if (!first) {
        float sd = 0.0f;
#pragma unroll
        for (int g = 0; g < N; ++g)
            if (lane + 64u * g < groups)
#pragma unroll
                for (int e = 0; e < 4; ++e) sd += v[g][e] * v[g][e];
        const float s = 1.0f / sqrtf(pk::wave_sum(sd) / (float)n + eps);
#pragma unroll
        for (int g = 0; g < N; ++g) {
            const uint32_t gi = lane + 64u * g;
            if (gi < groups) {
                const float4 w = *reinterpret_cast<const float4 *>(nw + 4u * gi);
                const uint2 xb = *reinterpret_cast<const uint2 *>(xres + 4u * gi);
                const float4 x = float4{bf(xb.x & 0xffffu), bf(xb.x >> 16), bf(xb.y & 0xffffu), bf(xb.y >> 16)};
                v[g][0] = rnd(x.x + rnd((v[g][0] * s) * w.x));
                v[g][1] = rnd(x.y + rnd((v[g][1] * s) * w.y));
                v[g][2] = rnd(x.z + rnd((v[g][2] * s) * w.z));
                v[g][3] = rnd(x.w + rnd((v[g][3] * s) * w.w));
            }
        }
    }
    float ss = 0.0f;
#pragma unroll
    for (int g = 0; g < N; ++g) {
        const uint32_t gi = lane + 64u * g;
        if (gi < groups) {
            *reinterpret_cast<uint2 *>(xres + 4u * gi) =
                uint2{bfbits(v[g][0]) | (bfbits(v[g][1]) << 16), bfbits(v[g][2]) | (bfbits(v[g][3]) << 16)};
#pragma unroll
            for (int e = 0; e < 4; ++e) ss += v[g][e] * v[g][e];
            if (x_out) {
                const uint32_t lo = bfbits(v[g][0]) | (bfbits(v[g][1]) << 16), hi = bfbits(v[g][2]) | (bfbits(v[g][3]) << 16);
                *reinterpret_cast<uint2 *>(x_out + 4u * gi) = uint2{lo, hi};
            }
        }
    }
    const float s2 = 1.0f / sqrtf(pk::wave_sum(ss) / (float)n + eps);
#pragma unroll
    for (int g = 0; g < N; ++g) {
        const uint32_t gi = lane + 64u * g;
        if (gi < groups) {
            const float4 w = *reinterpret_cast<const float4 *>(nw + n + 4u * gi);
            const uint32_t lo = bfbits((v[g][0] * s2) * w.x) | (bfbits((v[g][1] * s2) * w.y) << 16);
            const uint32_t hi = bfbits((v[g][2] * s2) * w.z) | (bfbits((v[g][3] * s2) * w.w) << 16);
            *reinterpret_cast<uint2 *>(xs + 4u * gi) = uint2{lo, hi};
        }
    }
}

template <int N>
__device__ inline void to_lds_bf16(const float (&v)[N][4], uint32_t n, uint16_t *xs, uint32_t lane) {
    const uint32_t groups = n / 4u;
#pragma unroll
    for (int g = 0; g < N; ++g) {
        const uint32_t gi = lane + 64u * g;
        if (gi < groups) {
            const uint32_t lo = bfbits(v[g][0]) | (bfbits(v[g][1]) << 16), hi = bfbits(v[g][2]) | (bfbits(v[g][3]) << 16);
            *reinterpret_cast<uint2 *>(xs + 4u * gi) = uint2{lo, hi};
        }
    }
}

// ---- weight streams through LDS ---------------------------------------------------
// A worker wave streams its units (S rows each; unit u = rows u of S
// matrices, units first, first + stride, ...) through a ring of D steps in
// its own LDS region: a step is one 16-byte chunk per lane of each of the S
// rows, copied global -> LDS by global_load_lds_dwordx4 (lane l writes 16
// bytes at the slot + 16 l), so the loads in flight hold no registers and
// the ring can be filled before the wave waits for its inputs. Consuming a
// step waits until only the steps issued after it are outstanding (vector
// memory operations complete in issue order; a store issued in between only
// makes the wait longer), reads the lane's chunks back with ds_read_b128,
// multiplies them by x (bf16 in LDS) and refills the slot with the step D
// ahead.
constexpr int kNonTemporal = 2;  // cache policy of the weight copies: nt

template <int N>
__device__ inline void wait_vm() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

__device__ inline float dot8_bf16(u32x4 w, u32x4 x) {
    float acc = 0.0f;
#pragma unroll
    for (int h = 0; h < 4; ++h) {
        const uint32_t a = h == 0 ? w.x : h == 1 ? w.y : h == 2 ? w.z : w.w;
        const uint32_t b = h == 0 ? x.x : h == 1 ? x.y : h == 2 ? x.z : x.w;
        acc += __uint_as_float(b << 16) * __uint_as_float(a << 16);
        acc += __uint_as_float(b & 0xffff0000u) * __uint_as_float(a & 0xffff0000u);
    }
    return acc;
}

template <int S, int D>
struct LdsStream {
    uint8_t *ring;  // this wave's D * S KB
    uint32_t lane, nchunks, cpl, steps, first, stride;
    uint32_t is, ii, iu;  // issue cursor: steps issued, step within the unit, unit
    const uint16_t *rp[S];

    template <class Rows>
    __device__ void init(uint8_t *ring_, const Rows &rows, uint32_t K, uint32_t units, uint32_t first_,
                         uint32_t stride_, uint32_t lane_) {
        ring = ring_;
        lane = lane_;
        nchunks = K / 8u;
        cpl = (nchunks + 63u) / 64u;
        first = first_;
        stride = stride_;
        const uint32_t nu = first < units ? (units - first + stride - 1u) / stride : 0u;
        steps = nu * cpl;
        is = 0;
        ii = 0;
        iu = first;
#pragma unroll
        for (int s = 0; s < S; ++s) rp[s] = rows(iu, s);
    }

    template <class Rows>
    __device__ inline void issue(const Rows &rows) {
        if (is >= steps) return;
        const uint32_t c = min(lane + 64u * ii, nchunks - 1u);
        uint8_t *slot = ring + (is % (uint32_t)D) * (uint32_t)(S * 1024);
#pragma unroll
        for (int s = 0; s < S; ++s)
            __builtin_amdgcn_global_load_lds(rp[s] + (uint64_t)c * 8u, (lds_void *)(slot + s * 1024), 16, 0,
                                             kNonTemporal);
        ++is;
        if (++ii == cpl) {
            ii = 0;
            iu += stride;
#pragma unroll
            for (int s = 0; s < S; ++s) rp[s] = rows(iu, s);
        }
    }

    template <class Rows>
    __device__ void start(const Rows &rows) {
#pragma unroll
        for (int d = 0; d < D; ++d) issue(rows);
    }

    template <class Rows, class Store>
    __device__ void run(const uint16_t *xs, const Rows &rows, Store &store) {
        float acc[S];
#pragma unroll
        for (int s = 0; s < S; ++s) acc[s] = 0.0f;
        uint32_t ci = 0, cu = first;
        for (uint32_t t = 0; t < steps; ++t) {
            if (steps - 1u - t >= (uint32_t)(D - 1)) wait_vm<(D - 1) * S>();
            else wait_vm<0>();
            const uint8_t *slot = ring + (t % (uint32_t)D) * (uint32_t)(S * 1024) + lane * 16u;
            u32x4 w[S];
#pragma unroll
            for (int s = 0; s < S; ++s) w[s] = *reinterpret_cast<const u32x4 *>(slot + s * 1024);
            const uint32_t c = lane + 64u * ci;
            if (c < nchunks) {
                const u32x4 x = *reinterpret_cast<const u32x4 *>(xs + c * 8u);
#pragma unroll
                for (int s = 0; s < S; ++s) acc[s] += dot8_bf16(w[s], x);
            }
            issue(rows);
            if (++ci == cpl) {
                float sums[S];
#pragma unroll
                for (int s = 0; s < S; ++s) {
                    sums[s] = pk::wave_sum(acc[s]);
                    acc[s] = 0.0f;
                }
                store(cu, sums);
                ci = 0;
                cu += stride;
            }
        }
    }
};

// ---- attention ----------------------------------------------------------------
// One block per (KV head, partition): the G query heads of the KV head
// (GQA) against the partition's keys. A key row (HD bf16) spans LPK lanes of
// one 16-byte chunk each, so one wave-wide load covers KPW key rows; worker
// wave w takes loads t*kWork + w of the partition. The first kKvLoads loads
// of each wave (keys written by earlier steps) are issued at the end of the
// QKV phase; the key at the step's own position, produced by this launch's
// QKV phase, comes from the staged rows.
template <int HD>
struct KvGeom {
    static constexpr int LPK = HD / 8, KPW = 64 / LPK;
    uint32_t hkv, part, lo, hi, cachedHi;
    bool active, owner;

    __device__ void init(const DecodeLayersConstants &c, int32_t pos) {
        const uint32_t P = c.partitions;
        const uint32_t item = blockIdx.x;
        active = item < c.Nkv * P;
        hkv = item % c.Nkv;
        part = item / c.Nkv;
        uint32_t Sk = pos < 0 ? 0u : (uint32_t)pos + 1u;
        if (Sk > c.kvStride) Sk = c.kvStride;
        const uint32_t per = (Sk + P - 1u) / P;
        lo = min(part * per, Sk);
        hi = min(lo + per, Sk);
        // rows below the position were written by earlier steps, the row at
        // the position (when it lies in the cache) by this launch; a
        // partition past the last key has lo == hi == Sk > pos: its cached
        // range stays empty, never negative
        const bool fresh = pos >= 0 && (uint32_t)pos < c.kvStride;
        cachedHi = fresh ? max(lo, min(hi, (uint32_t)pos)) : hi;
        owner = active && fresh && lo <= (uint32_t)pos && (uint32_t)pos < hi;
        if (!active) lo = hi = cachedHi = 0;
    }
};

template <int HD>
struct KvSlots {
    pk::Vec<BF16> k[kKvLoads], v[kKvLoads];

    // The loads of round `round` for worker wave `w` (rows past the cached
    // range read row 0 of the head and are masked later).
    __device__ void issue(const KvGeom<HD> &g, const uint16_t *kc, const uint16_t *vc, uint32_t kvStride,
                          uint32_t w, uint32_t round, uint32_t lane) {
        const uint32_t kg = lane / KvGeom<HD>::LPK, dl = lane % KvGeom<HD>::LPK;
        const uint64_t base = (uint64_t)g.hkv * kvStride * HD + dl * 8u;
#pragma unroll
        for (int t = 0; t < kKvLoads; ++t) {
            const uint32_t j = g.lo + ((round * kKvLoads + t) * kWork + w) * KvGeom<HD>::KPW + kg;
            const uint64_t at = base + (uint64_t)(j < g.cachedHi ? j : 0u) * HD;
            k[t].load_nt(kc + at);
            v[t].load_nt(vc + at);
        }
    }
};

// Running softmax state of one wave for its G query heads: every lane holds
// 8 dims of each head's output (its key group's keys); m is wave-uniform.
template <int HD, int G>
struct FdState {
    static constexpr int LPK = HD / 8;
    float q[G][8], o[G][8], m[G], l[G];

    template <int N>
    __device__ void tile(const pk::Vec<BF16> (&k)[N], const pk::Vec<BF16> (&v)[N], const bool (&valid)[N]) {
        float s[G][N];
#pragma unroll
        for (int t = 0; t < N; ++t) {
            float kf[8];
            k[t].to_float(kf);
#pragma unroll
            for (int g = 0; g < G; ++g) {
                float acc = 0.0f;
#pragma unroll
                for (int e = 0; e < 8; ++e) acc += q[g][e] * kf[e];
                s[g][t] = valid[t] ? pk::group_sum<LPK>(acc) : -INFINITY;
            }
        }
#pragma unroll
        for (int g = 0; g < G; ++g) {
            float mx = -INFINITY;
#pragma unroll
            for (int t = 0; t < N; ++t) mx = fmaxf(mx, s[g][t]);
            if constexpr (LPK < 64) mx = pk::wave_max(mx);
            const float mNew = fmaxf(m[g], mx);
            if (mNew == -INFINITY) continue;  // no allowed key yet (uniform)
            const float alpha = pk::fast_exp(m[g] - mNew);
            float pt[N], psum = 0.0f;
#pragma unroll
            for (int t = 0; t < N; ++t) {
                pt[t] = pk::fast_exp(s[g][t] - mNew);
                psum += pt[t];
            }
            l[g] = alpha * l[g] + psum;
            m[g] = mNew;
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                float acc = o[g][e] * alpha;
#pragma unroll
                for (int t = 0; t < N; ++t) acc += pt[t] * v[t].get(e);
                o[g][e] = acc;
            }
        }
    }
};

struct Args {
    const uint16_t *x_in;
    const uint16_t *wqkv, *wo, *wg, *wu, *wd;
    const float *norms;
    uint16_t *kc, *vc;
    const int32_t *position;
    uint16_t *q, *attn, *o, *hidden, *mlp, *x2;  // plain bf16 copies of the last layer's vectors
    uint8_t *tagged;                              // pk::layers::taggedLayout
    uint32_t *sync;
    uint64_t *stamps;
};

// The block-wide barrier at a phase boundary: a bare s_barrier, so the
// streaming waves' copies stay in flight; LDS writes before it are complete.
__device__ inline void block_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

// Keeps the compiler from moving the next phase's copies above this phase's
// stores (their order in the queue decides how long a later wait lasts).
__device__ inline void after_stores() {
    asm volatile("" ::: "memory");
    __builtin_amdgcn_sched_barrier(0);
}

template <int HD, int G>
__device__ void decode_layers(const Args &a, const DecodeLayersConstants &c) {
    static_assert(HD % 8 == 0 && HD / 8 <= 64, "a key row spans at most one wave");
    constexpr int NS = LY::kStagedGroups;  // 16-byte groups per lane of a staged small vector
    constexpr int NQ = ((G + 2) * HD / 4 + 63) / 64;  // groups per lane of the attention rows
    constexpr int NH = 4;  // groups per lane and pass of a worker's share of the hidden vector
    extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
    __shared__ float fd_m[kWork][G], fd_l[kWork][G];
    __shared__ uint32_t fd_count, arrive_count, block_abort;

    const uint32_t H = c.H, F = c.F, QW = c.Nq * HD, KW = c.Nkv * HD, QKV = QW + 2u * KW;
    const uint32_t L = c.layers, P = c.partitions, S = c.kvStride;
    const uint32_t lane0 = threadIdx.x & 63;
    const uint32_t wave = pk::uniform(threadIdx.x >> 6);
    const bool worker = wave < (uint32_t)kWork, stager = !worker;
    const uint32_t wslot = worker ? wave : 0u;
    const uint32_t blocks = gridDim.x;
    const uint32_t first = wslot * blocks + blockIdx.x, stride = blocks * kWork;

    const LY::Lds ll = LY::ldsLayout(H, QW, F, G, HD);
    uint16_t *xres = reinterpret_cast<uint16_t *>(lds + ll.xres);
    float *normw = reinterpret_cast<float *>(lds + ll.normw);  // [2][H]: the next glue's w_post, w_pre
    uint16_t *small0 = reinterpret_cast<uint16_t *>(lds + ll.small0);
    uint16_t *small1 = reinterpret_cast<uint16_t *>(lds + ll.small1);
    uint16_t *big = reinterpret_cast<uint16_t *>(lds + ll.big);
    float *fd_o = reinterpret_cast<float *>(lds + ll.big);  // [kWork][G][HD], attention phase only
    uint16_t *qbuf = reinterpret_cast<uint16_t *>(lds + ll.qbuf);  // [G + 2][HD]
    uint8_t *region = lds + ll.rings + wslot * LY::kRegion;
    uint8_t *ring0 = region, *ring1 = region + LY::kRing0;

    const LY::Tagged tl = LY::taggedLayout(H, c.Nq, c.Nkv, HD, F, P);
    uint32_t *qkv_t = reinterpret_cast<uint32_t *>(a.tagged + tl.qkv);
    uint32_t *attn_t = reinterpret_cast<uint32_t *>(a.tagged + tl.attn);
    uint32_t *o_t = reinterpret_cast<uint32_t *>(a.tagged + tl.o);
    uint32_t *hidden_t = reinterpret_cast<uint32_t *>(a.tagged + tl.hidden);
    uint32_t *mlp_t = reinterpret_cast<uint32_t *>(a.tagged + tl.mlp);
    uint64_t *pO_t = reinterpret_cast<uint64_t *>(a.tagged + tl.pO);    // [Nq][P][HD]
    uint64_t *pML_t = reinterpret_cast<uint64_t *>(a.tagged + tl.pML);  // [Nq][P][2]: m, l

    const int32_t pos = a.position[0];
    const bool scatter = pos >= 0 && (uint32_t)pos < S;
    const uint32_t epoch = ld32(a.sync + LY::kEpochWord);
    const uint32_t tagBase = epoch * L * 8u;
    auto tag16 = [&](uint32_t l, uint32_t ph) { return (tagBase + l * 8u + ph) & 0xffffu; };
    auto tag32 = [&](uint32_t l, uint32_t ph) { return tagBase + l * 8u + ph; };
    // arrivals that complete phase ph of layer l (every block arrives once per phase)
    auto arrivals = [&](uint32_t l, uint32_t ph) { return (l * 6u + ph + 1u) * gridDim.x; };

    if (threadIdx.x == 0) {
        fd_count = 0;
        arrive_count = 0;
        block_abort = 0;
    }
    __syncthreads();
    Poll pl{a.sync + LY::kAbortWord, &block_abort, c.spinTicks ? (uint64_t)c.spinTicks : 50000000ull};
    uint32_t nbar = 0;
    auto barrier = [&]() {
        block_barrier();
        if (a.stamps && stager && lane0 == 0 && nbar < LY::kStampsPerBlock)
            a.stamps[(uint64_t)blockIdx.x * LY::kStampsPerBlock + nbar] = __builtin_amdgcn_s_memrealtime();
        ++nbar;
    };

    KvGeom<HD> kv;
    kv.init(c, pos);

    uint32_t layer = 0;  // the layer the row functions address
    auto rowsA = [&](uint32_t unit, int) { return a.wqkv + ((uint64_t)layer * QKV + min(unit, QKV - 1u)) * H; };
    auto rowsO = [&](uint32_t unit, int) { return a.wo + ((uint64_t)layer * H + min(unit, H - 1u)) * QW; };
    auto rowsGU = [&](uint32_t unit, int s) {
        return (s == 0 ? a.wg : a.wu) + ((uint64_t)layer * F + min(unit, F - 1u)) * H;
    };
    auto rowsF = [&](uint32_t unit, int) { return a.wd + ((uint64_t)layer * H + min(unit, H - 1u)) * F; };
    auto normL = [&](uint32_t l, uint32_t slot) { return a.norms + ((uint64_t)l * 4u + slot) * H; };
    auto kcL = [&](uint32_t l) { return a.kc + (uint64_t)l * c.Nkv * S * HD; };
    auto vcL = [&](uint32_t l) { return a.vc + (uint64_t)l * c.Nkv * S * HD; };

    LdsStream<1, kDepthQKV> rsA;
    rsA.init(region, rowsA, H, QKV, first, stride, lane0);
    if (worker) rsA.start(rowsA);

    for (uint32_t l = 0; l < L; ++l) {
        layer = l;
        const bool last = l + 1u == L;
        // per-lane addresses are recomputed in every layer instead of being
        // hoisted out of the loop and held (spilled) across all of it
        uint32_t lane = lane0;
        asm volatile("" : "+v"(lane));
        // ---- A's input: [post-FFN norm + residual], input norm -> small0 (staging wave)
        if (stager) {
            float v[NS][4];
            load_norms(normw, l == 0 ? nullptr : normL(l - 1u, 3), normL(l, 0), H, lane);
            if (l == 0) {
                // the step's input row, written before the launch
#pragma unroll
                for (int g = 0; g < NS; ++g) {
                    const uint32_t gi = min(lane + 64u * g, H / 4u - 1u);
                    const uint2 w = *reinterpret_cast<const uint2 *>(a.x_in + 4u * gi);
                    v[g][0] = bf(w.x & 0xffffu);
                    v[g][1] = bf(w.x >> 16);
                    v[g][2] = bf(w.y & 0xffffu);
                    v[g][3] = bf(w.y >> 16);
                }
            } else {
                wait_arrivals(a.sync, arrivals(l - 1u, kPhMlp), pl, lane);
                poll_vector<NS>(mlp_t, H, tag16(l - 1u, kPhMlp), pl, v, lane);
            }
            glue<NS>(v, H, l == 0, xres, small0, normw, c.eps, nullptr, lane);
        }
        barrier();  // A

        // ---- A: QKV rows (workers): q -> tagged; k, v -> tagged and into the caches
        if (worker) {
            uint16_t *kcl = kcL(l), *vcl = vcL(l);
            const uint32_t t = tag16(l, kPhQKV) << 16;
            auto storeA = [&](uint32_t unit, const float *sums) {
                if (lane != 0 || unit >= QKV) return;
                const uint32_t v = bfbits(sums[0]);
                st32(qkv_t + unit, t | v);
                if (unit < QW) {
                    if (last) a.q[unit] = (uint16_t)v;
                } else if (scatter) {
                    uint32_t j = unit - QW;
                    const bool isV = j >= KW;
                    if (isV) j -= KW;
                    (isV ? vcl : kcl)[((uint64_t)(j / HD) * S + (uint32_t)pos) * HD + j % HD] = (uint16_t)v;
                }
            };
            rsA.run(small0, rowsA, storeA);
            arrive_workers(a.sync, &arrive_count, lane);
        }
        LdsStream<1, kDepthO> rsO;
        KvSlots<HD> slots;
        rsO.init(ring1, rowsO, QW, H, first, stride, lane);
        after_stores();
        if (worker) {
            slots.issue(kv, kcL(l), vcL(l), S, wave, 0, lane);
            rsO.start(rowsO);
        }
        // ---- B's input: the block's query heads and the new K/V rows -> qbuf (staging wave)
        if (stager && kv.active) {
            wait_arrivals(a.sync, arrivals(l, kPhQKV), pl, lane);
            const uint32_t tq = tag16(l, kPhQKV);
            const __amdgpu_buffer_rsrc_t r = rsrc(qkv_t, QKV * 4u);
            const uint64_t t0 = __builtin_amdgcn_s_memrealtime();
            for (;;) {
                // 16-byte groups: G query heads, then the key and value head rows
                uint32_t ok = 1u;
#pragma unroll
                for (int g = 0; g < NQ; ++g) {
                    const uint32_t gi = lane + 64u * g;
                    if (gi < (uint32_t)((G + 2) * HD / 4)) {
                        const uint32_t row = gi / (HD / 4), d4 = gi % (HD / 4);
                        const bool need = row < (uint32_t)G || kv.owner;
                        const uint32_t src = row < (uint32_t)G ? (kv.hkv * G + row) * HD
                                           : row == (uint32_t)G ? QW + kv.hkv * HD : QW + KW + kv.hkv * HD;
                        const u32x4 w = ldc16(r, (src + 4u * d4) * 4u);
                        if (need)
                            ok &= (w.x >> 16) == tq && (w.y >> 16) == tq && (w.z >> 16) == tq && (w.w >> 16) == tq;
                        *reinterpret_cast<uint2 *>(qbuf + row * HD + 4u * d4) =
                            uint2{(w.x & 0xffffu) | (w.y << 16), (w.z & 0xffffu) | (w.w << 16)};
                    }
                }
                if (wave_all(ok) || pl.aborted() || pl.expired(t0, lane)) break;
                __builtin_amdgcn_s_sleep(1);
            }
        }
        barrier();  // B

        // ---- B: split-KV attention partials (workers); the last worker to
        // finish merges the block's states into the partition's
        if (worker && kv.active) {
            const uint32_t kg = lane / KvGeom<HD>::LPK, dl = lane % KvGeom<HD>::LPK;
            FdState<HD, G> st;
#pragma unroll
            for (int g = 0; g < G; ++g) {
                pk::Vec<BF16> qv;
                qv.raw = *reinterpret_cast<const u32x4 *>(qbuf + g * HD + dl * 8u);
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    st.q[g][e] = qv.get(e) * c.scale;
                    st.o[g][e] = 0.0f;
                }
                st.m[g] = -INFINITY;
                st.l[g] = 0.0f;
            }
            const uint32_t span = kv.cachedHi - kv.lo;  // cachedHi >= lo
            constexpr uint32_t kPerRound = (uint32_t)(kKvLoads * kWork * KvGeom<HD>::KPW);
            const uint32_t rounds = (span + kPerRound - 1u) / kPerRound;  // <= kvStride / kPerRound + 1
            for (uint32_t round = 0; round < max(rounds, 1u); ++round) {
                if (round > 0) {
                    if ((round * kKvLoads * kWork + wave) * KvGeom<HD>::KPW >= span) break;
                    slots.issue(kv, kcL(l), vcL(l), S, wave, round, lane);
                }
                bool valid[kKvLoads];
#pragma unroll
                for (int t = 0; t < kKvLoads; ++t)
                    valid[t] = kv.lo + ((round * kKvLoads + t) * kWork + wave) * KvGeom<HD>::KPW + kg < kv.cachedHi;
                st.tile(slots.k, slots.v, valid);
            }
            if (kv.owner && wave == 0) {
                // the key at the position, from the staged rows
                pk::Vec<BF16> fk[1], fv[1];
                fk[0].raw = *reinterpret_cast<const u32x4 *>(qbuf + G * HD + dl * 8u);
                fv[0].raw = *reinterpret_cast<const u32x4 *>(qbuf + (G + 1) * HD + dl * 8u);
                const bool fvalid[1] = {kg == 0};
                st.tile(fk, fv, fvalid);
            }
            // merge the key groups of the wave (lanes dl, dl + LPK, ...)
#pragma unroll
            for (int g = 0; g < G; ++g) {
                for (int sft = KvGeom<HD>::LPK; sft < 64; sft <<= 1) {
                    st.l[g] += __shfl_xor(st.l[g], sft, 64);
#pragma unroll
                    for (int e = 0; e < 8; ++e) st.o[g][e] += __shfl_xor(st.o[g][e], sft, 64);
                }
                if (kg == 0) {
                    float *dst = fd_o + ((uint32_t)wave * G + g) * HD + dl * 8u;
                    *reinterpret_cast<float4 *>(dst) = float4{st.o[g][0], st.o[g][1], st.o[g][2], st.o[g][3]};
                    *reinterpret_cast<float4 *>(dst + 4) = float4{st.o[g][4], st.o[g][5], st.o[g][6], st.o[g][7]};
                    if (dl == 0) {
                        fd_m[wave][g] = st.m[g];
                        fd_l[wave][g] = st.l[g];
                    }
                }
            }
            asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
            uint32_t arrived = 0;
            if (lane == 0) arrived = atomicAdd(&fd_count, 1u);
            arrived = __shfl(arrived, 0, 64);
            if (arrived == (uint32_t)kWork - 1u) {
                // every worker's state is in LDS: merge them into the partition's
                const uint32_t t = tag32(l, kPhPart);
                for (uint32_t idx = lane; idx < (uint32_t)(G * HD); idx += 64u) {
                    const uint32_t g = idx / HD, d = idx % HD;
                    float mstar = -INFINITY;
#pragma unroll
                    for (int w = 0; w < kWork; ++w) mstar = fmaxf(mstar, fd_m[w][g]);
                    float o = 0.0f, lsum = 0.0f;
                    if (mstar != -INFINITY) {
#pragma unroll
                        for (int w = 0; w < kWork; ++w) {
                            const float e = pk::fast_exp(fd_m[w][g] - mstar);
                            o += e * fd_o[((uint32_t)w * G + g) * HD + d];
                            lsum += e * fd_l[w][g];
                        }
                    }
                    const uint64_t slot = (uint64_t)(kv.hkv * G + g) * P + kv.part;
                    st64(pO_t + slot * HD + d, ((uint64_t)t << 32) | __float_as_uint(o));
                    if (d == 0) {
                        st64(pML_t + 2u * slot, ((uint64_t)t << 32) | __float_as_uint(mstar));
                        st64(pML_t + 2u * slot + 1u, ((uint64_t)t << 32) | __float_as_uint(lsum));
                    }
                }
                if (lane == 0) {
                    fd_count = 0;
                    arrive_global(a.sync);
                }
            }
        }
        LdsStream<2, kDepthGU> rsGU;
        rsGU.init(ring0, rowsGU, H, F, first, stride, lane);
        after_stores();
        if (worker) rsGU.start(rowsGU);

        // ---- C: log-sum-exp combine (staging wave), attn = sum_p exp(m_p - m*) O_p /
        // sum_p exp(m_p - m*) l_p; then D's input: attn -> small1
        if (stager) {
            if (!kv.active && lane == 0) arrive_global(a.sync);  // no partition: nothing to store
            const uint32_t items = c.Nq * (HD / 8);
            if (blockIdx.x < items) wait_arrivals(a.sync, arrivals(l, kPhPart), pl, lane);
            const uint32_t tp = tag32(l, kPhPart), ta = tag16(l, kPhAttn) << 16;
            for (uint32_t it = blockIdx.x; it < items; it += blocks) {
                const uint32_t hq = it / (HD / 8), d0 = 8u * (it % (HD / 8));
                const bool has = lane < P;
                const uint64_t slot = (uint64_t)hq * P + (has ? lane : 0u);
                uint64_t ml[2], ov[8];
                const uint64_t t0 = __builtin_amdgcn_s_memrealtime();
                for (;;) {
                    uint32_t ok = 1u;
#pragma unroll
                    for (int h = 0; h < 2; ++h) {
                        ml[h] = ld64(pML_t + 2u * slot + h);
                        ok &= !has || (uint32_t)(ml[h] >> 32) == tp;
                    }
#pragma unroll
                    for (int h = 0; h < 8; ++h) {
                        ov[h] = ld64(pO_t + slot * HD + d0 + h);
                        ok &= !has || (uint32_t)(ov[h] >> 32) == tp;
                    }
                    if (wave_all(ok) || pl.aborted() || pl.expired(t0, lane)) break;
                    __builtin_amdgcn_s_sleep(1);
                }
                const float m = has ? __uint_as_float((uint32_t)ml[0]) : -INFINITY;
                const float lp = __uint_as_float((uint32_t)ml[1]);
                const float mstar = pk::wave_max(m);
                float out[8];
                if (mstar == -INFINITY) {
#pragma unroll
                    for (int e = 0; e < 8; ++e) out[e] = 0.0f;
                } else {
                    const float w = has ? pk::fast_exp(m - mstar) : 0.0f;
                    const float lstar = pk::wave_sum(w * lp);
#pragma unroll
                    for (int e = 0; e < 8; ++e) out[e] = pk::wave_sum(w * __uint_as_float((uint32_t)ov[e])) / lstar;
                }
                if (lane < 8u) {
                    float mine = out[0];
#pragma unroll
                    for (int e = 1; e < 8; ++e)
                        if (lane == (uint32_t)e) mine = out[e];
                    const uint32_t v = bfbits(mine);
                    st32(attn_t + (uint64_t)hq * HD + d0 + lane, ta | v);
                    if (last) a.attn[(uint64_t)hq * HD + d0 + lane] = (uint16_t)v;
                }
            }
            after_stores();
            if (lane == 0) arrive_global(a.sync);
            float v[NS][4];
            wait_arrivals(a.sync, arrivals(l, kPhAttn), pl, lane);
            poll_vector<NS>(attn_t, QW, tag16(l, kPhAttn), pl, v, lane);
            to_lds_bf16<NS>(v, QW, small1, lane);
        }
        barrier();  // D

        // ---- D: O projection (workers) -> tagged o
        if (worker) {
            const uint32_t t = tag16(l, kPhO) << 16;
            auto storeO = [&](uint32_t unit, const float *sums) {
                if (lane != 0 || unit >= H) return;
                const uint32_t v = bfbits(sums[0]);
                st32(o_t + unit, t | v);
                if (last) a.o[unit] = (uint16_t)v;
            };
            rsO.run(small1, rowsO, storeO);
            arrive_workers(a.sync, &arrive_count, lane);
        }
        // ---- E's input: post-attention norm + residual, pre-FFN norm -> small0 (staging wave)
        if (stager) {
            float v[NS][4];
            load_norms(normw, normL(l, 1), normL(l, 2), H, lane);
            wait_arrivals(a.sync, arrivals(l, kPhO), pl, lane);
            poll_vector<NS>(o_t, H, tag16(l, kPhO), pl, v, lane);
            glue<NS>(v, H, false, xres, small0, normw, c.eps, (last && blockIdx.x == 0) ? a.x2 : nullptr, lane);
        }
        barrier();  // E

        // ---- E: gate/up, GELU-tanh * up (workers) -> tagged hidden
        if (worker) {
            const uint32_t t = tag16(l, kPhHidden) << 16;
            auto storeGU = [&](uint32_t unit, const float *sums) {
                if (lane != 0 || unit >= F) return;
                const float g = rnd(sums[0]), u = rnd(sums[1]);
                const float act = rnd(pk::gelu_tanh(g));
                const uint32_t v = bfbits(act * u);
                st32(hidden_t + unit, t | v);
                if (last) a.hidden[unit] = (uint16_t)v;
            };
            rsGU.run(small0, rowsGU, storeGU);
            arrive_workers(a.sync, &arrive_count, lane);
        }
        LdsStream<1, kDepthDown> rsF;
        rsF.init(region, rowsF, F, H, first, stride, lane);
        after_stores();
        if (worker) rsF.start(rowsF);
        // the staging wave waits for every block's hidden rows; the workers
        // then fetch a share each
        if (stager) wait_arrivals(a.sync, arrivals(l, kPhHidden), pl, lane);
        barrier();  // F1

        // ---- F's input: hidden -> big (workers, a share each)
        if (worker) {
            float v[NH][4];
            const uint32_t share = (F / 4u + kWork - 1u) / kWork;  // 16-byte groups per worker
            const uint32_t g0 = min(wave * share, F / 4u), g1 = min(g0 + share, F / 4u);
            for (uint32_t base = g0; base < g1; base += 64u * NH) {
                const uint32_t n = min(64u * NH, g1 - base) * 4u;
                poll_vector<NH>(hidden_t + 4u * base, n, tag16(l, kPhHidden), pl, v, lane);
                to_lds_bf16<NH>(v, n, big + 4u * base, lane);
            }
        }
        barrier();  // F2

        // ---- F: down projection (workers) -> tagged mlp; then the next layer's QKV copies
        if (worker) {
            const uint32_t t = tag16(l, kPhMlp) << 16;
            auto storeF = [&](uint32_t unit, const float *sums) {
                if (lane != 0 || unit >= H) return;
                const uint32_t v = bfbits(sums[0]);
                st32(mlp_t + unit, t | v);
                if (last) a.mlp[unit] = (uint16_t)v;
            };
            rsF.run(big, rowsF, storeF);
            arrive_workers(a.sync, &arrive_count, lane);
            if (!last) {
                layer = l + 1u;
                rsA.init(region, rowsA, H, QKV, first, stride, lane);
                after_stores();
                rsA.start(rowsA);
            }
        }
    }

    // The last block to finish advances the epoch for the next launch: every
    // block read it at its start.
    asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)" ::: "memory");
    __syncthreads();
    if (threadIdx.x == 0) {
        const uint32_t done = __hip_atomic_fetch_add(a.sync + LY::kDoneWord, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (done + 1u == blocks) {
            for (int i = 0; i < LY::kCounters; ++i) st32(a.sync + i * LY::kLine, 0u);
            st32(a.sync + LY::kDoneWord, 0u);
            st32(a.sync + LY::kEpochWord, epoch + 1u);
        }
    }
}

}  // namespace

#define DECODE_LAYERS(HD, G)                                                                                      \
    POPCORN_KERNEL void __launch_bounds__(kThreads)                                                               \
        decode_layers_bf16_h##HD##_g##G(const uint16_t *x_in, const uint16_t *wqkv, const uint16_t *wo,           \
                                        const uint16_t *wg, const uint16_t *wu, const uint16_t *wd,               \
                                        const float *norms, uint16_t *kc, uint16_t *vc, const int32_t *position,  \
                                        uint16_t *q, uint16_t *attn, uint16_t *o, uint16_t *hidden,               \
                                        uint16_t *mlp, uint16_t *x2, uint8_t *tagged, uint32_t *sync,             \
                                        uint64_t *stamps, DecodeLayersConstants c) {                              \
        const Args a{x_in, wqkv, wo, wg, wu, wd, norms, kc, vc, position, q, attn, o, hidden, mlp, x2,           \
                     tagged, sync, stamps};                                                                       \
        decode_layers<HD, G>(a, c);                                                                               \
    }

DECODE_LAYERS(256, 2)
DECODE_LAYERS(256, 1)
DECODE_LAYERS(128, 2)
DECODE_LAYERS(64, 2)
DECODE_LAYERS(64, 4)
