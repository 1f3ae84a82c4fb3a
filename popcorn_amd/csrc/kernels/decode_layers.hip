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
// Why one kernel: each decode matvec or attention launch pays a fixed cost
// of a few microseconds (launch, the first memory round trip, the tail), and
// a kernel boundary is a point where nothing streams. Here the grid is one
// block per CU (kWork streaming waves + one sync wave) and a phase boundary
// is a grid-wide wait on arrival counters; before it waits, every wave
// issues the first weight loads of its next phase (and, at the end of a
// layer, the next layer's cached K/V rows), so HBM keeps streaming while the
// counters settle.
//
// Memory model: data that one block writes and another reads inside the
// launch (q, the new K/V rows, attention partials, attn, o, hidden, mlp) is
// stored and loaded with agent-scope relaxed atomics (sc1: coherent across
// the XCDs' L2s). A wave waits for its own stores to complete before its
// block arrives; the sync wave then adds one to its block's counter (16
// counters on separate 256-byte lines, block b on counter b % 16, so each
// counter takes the blocks of one XCD) and polls the 16 counters until they
// sum to the arrivals this wait expects. Weights and the KV rows written in
// earlier steps are read with non-temporal loads. Every wait is bounded
// (spinTicks of the 100 MHz clock): a wait that runs out sets the abort word,
// and from then on no wait of the launch blocks, so the grid always drains.
// The counters are zeroed by the last block to finish, for the next launch.
#include "decode_layers_geometry.hpp"
#include "stream.hpp"

namespace {

using pk::BF16;
using pk::u32x4;
using pk::layers::kAbortWord;
using pk::layers::kCounters;
using pk::layers::kDoneWord;
using pk::layers::kLine;
using pk::layers::kRing0;
using pk::layers::kRing1;
using pk::layers::kThreads;
using pk::layers::kWaves;
using pk::layers::kWork;
constexpr int kKvLoads = 3;
#ifndef POPCORN_LAYER_POLL_SLEEP
#define POPCORN_LAYER_POLL_SLEEP 1
#endif  // K (and V) loads per wave prefetched for the attention phase

// ---- agent-coherent access (sc1) -----------------------------------------------
__device__ inline uint64_t ld64(const void *p) {
    return __hip_atomic_load(reinterpret_cast<uint64_t *>(const_cast<void *>(p)), __ATOMIC_RELAXED,
                             __HIP_MEMORY_SCOPE_AGENT);
}
__device__ inline uint32_t ld32(const void *p) {
    return __hip_atomic_load(reinterpret_cast<uint32_t *>(const_cast<void *>(p)), __ATOMIC_RELAXED,
                             __HIP_MEMORY_SCOPE_AGENT);
}
__device__ inline void st64(void *p, uint64_t v) {
    __hip_atomic_store(reinterpret_cast<uint64_t *>(p), v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ inline void st32(void *p, uint32_t v) {
    __hip_atomic_store(reinterpret_cast<uint32_t *>(p), v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ inline void st16(void *p, uint16_t v) {
    __hip_atomic_store(reinterpret_cast<uint16_t *>(p), v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// four bf16 in a 64-bit word <-> f32
__device__ inline void bf4(uint64_t v, float *r) {
    const uint32_t lo = (uint32_t)v, hi = (uint32_t)(v >> 32);
    r[0] = __uint_as_float(lo << 16);
    r[1] = __uint_as_float(lo & 0xffff0000u);
    r[2] = __uint_as_float(hi << 16);
    r[3] = __uint_as_float(hi & 0xffff0000u);
}
__device__ inline uint64_t pack_bf4(const float *r) {
    const uint32_t lo = (uint32_t)BF16::store(r[0]) | ((uint32_t)BF16::store(r[1]) << 16);
    const uint32_t hi = (uint32_t)BF16::store(r[2]) | ((uint32_t)BF16::store(r[3]) << 16);
    return (uint64_t)lo | ((uint64_t)hi << 32);
}
__device__ inline float rnd(float x) { return pk::round_as<10u>(x); }

__device__ inline uint32_t wave_sum_u32(uint32_t v) {
#pragma unroll
    for (int s = 1; s < 64; s <<= 1) v += (uint32_t)__shfl_xor((int)v, s, 64);
    return v;
}

// Sum over the block (every thread gets it); `red` holds one float per wave.
__device__ inline float block_sum(float v, float *red) {
    const uint32_t lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    v = pk::wave_sum(v);
    if (lane == 0) red[wave] = v;
    __syncthreads();
    float t = 0.0f;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) t += red[w];
    __syncthreads();
    return t;
}

// ---- grid-wide waits --------------------------------------------------------
struct GridSync {
    uint32_t *words;
    uint64_t *stamps;  // optional: [block][2 * wait]: arrival, release (100 MHz ticks)
    uint64_t limit;
    uint32_t blocks, waits;
    bool aborted;
};

// The end of a phase. Each worker wave's stores of the phase are complete
// once its queue holds only the `pending` loads issued after them (the next
// phase's prefetch; vector memory operations complete in issue order), and
// the block's LDS writes are done; the sync wave then arrives and waits for
// every block's arrival. The barriers are bare s_barrier: a __syncthreads()
// would also wait for the prefetch.
template <int PENDING>
__device__ inline void grid_wait(GridSync &s, bool syncWave) {
    if (syncWave) asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)" ::: "memory");
    else asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)" ::"n"(PENDING) : "memory");
    asm volatile("s_barrier" ::: "memory");
    const uint32_t k = s.waits++;
    if (syncWave) {
        const uint32_t lane = threadIdx.x & 63;
        if (s.stamps && lane == 0 && 2u * k + 1u < pk::layers::kStampsPerBlock) s.stamps[(uint64_t)blockIdx.x * pk::layers::kStampsPerBlock + 2u * k] = __builtin_amdgcn_s_memrealtime();
        if (lane == 0)
            __hip_atomic_fetch_add(s.words + (blockIdx.x % kCounters) * kLine, 1u, __ATOMIC_RELAXED,
                                   __HIP_MEMORY_SCOPE_AGENT);
        const uint32_t target = (k + 1u) * s.blocks;
        if (!s.aborted) {
            const uint64_t t0 = __builtin_amdgcn_s_memrealtime();
            for (;;) {
                uint32_t v = lane < (uint32_t)kCounters ? ld32(s.words + lane * kLine) : 0u;  // 16 arrival counters
                uint32_t a = lane == (uint32_t)kCounters ? ld32(s.words + kAbortWord) : 0u;
                v = wave_sum_u32(v);
                a = wave_sum_u32(a);
                if (v >= target) break;
                if (a != 0u) {
                    s.aborted = true;
                    break;
                }
                if (__builtin_amdgcn_s_memrealtime() - t0 > s.limit) {
                    if (lane == 0) st32(s.words + kAbortWord, 1u);
                    s.aborted = true;
                    break;
                }
#if POPCORN_LAYER_POLL_SLEEP
                __builtin_amdgcn_s_sleep(POPCORN_LAYER_POLL_SLEEP);
#endif
            }
        }
        if (s.stamps && lane == 0 && 2u * k + 1u < pk::layers::kStampsPerBlock)
            s.stamps[(uint64_t)blockIdx.x * pk::layers::kStampsPerBlock + 2u * k + 1u] = __builtin_amdgcn_s_memrealtime();
    }
    asm volatile("s_barrier" ::: "memory");
}

// Keeps the compiler from moving the next phase's prefetch loads above this
// phase's stores: grid_wait counts on the stores being older in the queue.
__device__ inline void issue_after_stores() {
    asm volatile("" ::: "memory");
    __builtin_amdgcn_sched_barrier(0);
}

// ---- staging (every thread of the block) ----------------------------------------
// The vector a matvec multiplies sits in LDS as bf16 (xs): every staged
// vector is bf16-valued (attn, hidden, or the glue's output rounded to bf16).
// xs[0..n) = bf16 vector (coherent loads). n % 4 == 0.
__device__ inline void stage_vector(uint16_t *xs, const uint16_t *src, uint32_t n) {
    for (uint32_t c = threadIdx.x; c < n / 4u; c += kThreads)
        *reinterpret_cast<uint64_t *>(xs + 4u * c) = ld64(src + 4u * c);
    __syncthreads();
}

// The residual glue in front of a matvec, the order of RMSNorm.metal:32-40
// and Add.metal as the decode matvecs' Stage computes it:
//   first layer: x = x_in;
//   else:        x = round(xres + round((delta * s_d) * w_post)),
//                s_d = 1 / sqrt(mean(delta^2) + eps);
//   xres = x (the residual stream stays in LDS, f32, between phases);
//   xs = round((x * s_x) * w_pre), s_x = 1 / sqrt(mean(x^2) + eps).
// x_out (optional) receives x as bf16. Before the residual add, delta is
// parked in xs.
__device__ inline void stage_glue(uint16_t *xs, float *xres, float *red, const uint16_t *delta, const float *w_post,
                                  const float *w_pre, uint32_t n, float eps, bool first, uint16_t *x_out) {
    const uint32_t nc = n / 4u;
    float ss = 0.0f;
    if (first) {
        for (uint32_t c = threadIdx.x; c < nc; c += kThreads) {
            float r[4];
            bf4(ld64(delta + 4u * c), r);
            *reinterpret_cast<float4 *>(xres + 4u * c) = float4{r[0], r[1], r[2], r[3]};
#pragma unroll
            for (int e = 0; e < 4; ++e) ss += r[e] * r[e];
        }
    } else {
        float sd = 0.0f;
        for (uint32_t c = threadIdx.x; c < nc; c += kThreads) {
            const uint64_t raw = ld64(delta + 4u * c);
            *reinterpret_cast<uint64_t *>(xs + 4u * c) = raw;
            float d[4];
            bf4(raw, d);
#pragma unroll
            for (int e = 0; e < 4; ++e) sd += d[e] * d[e];
        }
        const float s = 1.0f / sqrtf(block_sum(sd, red) / (float)n + eps);
        for (uint32_t c = threadIdx.x; c < nc; c += kThreads) {
            float d[4];
            bf4(*reinterpret_cast<const uint64_t *>(xs + 4u * c), d);  // this thread's own writes
            const float4 w = *reinterpret_cast<const float4 *>(w_post + 4u * c);
            const float4 x = *reinterpret_cast<const float4 *>(xres + 4u * c);
            float r[4];
            r[0] = rnd(x.x + rnd((d[0] * s) * w.x));
            r[1] = rnd(x.y + rnd((d[1] * s) * w.y));
            r[2] = rnd(x.z + rnd((d[2] * s) * w.z));
            r[3] = rnd(x.w + rnd((d[3] * s) * w.w));
            *reinterpret_cast<float4 *>(xres + 4u * c) = float4{r[0], r[1], r[2], r[3]};
#pragma unroll
            for (int e = 0; e < 4; ++e) ss += r[e] * r[e];
            if (x_out) st64(x_out + 4u * c, pack_bf4(r));
        }
    }
    const float s2 = 1.0f / sqrtf(block_sum(ss, red) / (float)n + eps);
    for (uint32_t c = threadIdx.x; c < nc; c += kThreads) {
        const float4 x = *reinterpret_cast<const float4 *>(xres + 4u * c);  // this thread's own writes
        const float4 w = *reinterpret_cast<const float4 *>(w_pre + 4u * c);
        const float r[4] = {(x.x * s2) * w.x, (x.y * s2) * w.y, (x.z * s2) * w.z, (x.w * s2) * w.w};
        *reinterpret_cast<uint64_t *>(xs + 4u * c) = pack_bf4(r);
    }
    __syncthreads();
}

// ---- weight streams through LDS ---------------------------------------------------
// A worker wave streams its units (S rows each; unit u = rows u of S
// matrices, units first, first + stride, ...) through a ring of D steps in
// its own LDS region: a step is one 16-byte chunk per lane of each of the S
// rows, copied global -> LDS by global_load_lds_dwordx4 (lane l writes 16
// bytes at the slot + 16 l), so the loads in flight hold no registers and
// the ring can be filled before a grid wait. Consuming a step waits until
// only the steps issued after it are outstanding (vector memory operations
// complete in issue order; a store issued in between only makes the wait
// longer), reads the lane's chunks back with ds_read_b128, multiplies them
// by x (bf16 in LDS) and refills the slot with the step D ahead.
typedef __attribute__((address_space(3))) void lds_void;
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
    uint32_t nchunks, cpl, steps, first, stride;
    uint32_t is, ii, iu;  // issue cursor: steps issued, step within the unit, unit
    const uint16_t *rp[S];

    template <class Rows>
    __device__ void init(uint8_t *ring_, const Rows &rows, uint32_t K, uint32_t units, uint32_t first_,
                         uint32_t stride_) {
        ring = ring_;
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
        const uint32_t c = min((threadIdx.x & 63u) + 64u * ii, nchunks - 1u);
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
        const uint32_t lane = threadIdx.x & 63u;
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
// of each wave (keys written by earlier steps) are issued before the grid
// wait ahead of the phase; the key at the step's own position, written by
// this launch's QKV phase, is read afterwards with coherent loads.
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
        // rows below the position were written by earlier steps; the row at
        // the position (when it lies in the cache) by this launch
        // (a partition past the last key has lo == hi == Sk > pos: its cached
        // range stays empty, never negative)
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
                          uint32_t w, uint32_t round) {
        const uint32_t lane = threadIdx.x & 63, kg = lane / KvGeom<HD>::LPK, dl = lane % KvGeom<HD>::LPK;
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
    uint16_t *q, *attn, *o, *hidden, *mlp, *x2;
    float *partials;
    uint32_t *sync;
    uint64_t *stamps;
};

// Ring depths (steps) of the four streams. Two ring sets alternate, so a
// phase's prefetch never lands in a ring still in use: ring 0 serves the QKV
// and gate/up streams, ring 1 the O and down streams.
constexpr int kDepthQKV = 8, kDepthGU = 4, kDepthO = 4, kDepthDown = 4;
static_assert(kDepthQKV * 1024 <= (int)kRing0 && kDepthGU * 2048 <= (int)kRing0, "ring 0");
static_assert(kDepthO * 1024 <= (int)kRing1 && kDepthDown * 1024 <= (int)kRing1, "ring 1");

template <int HD, int G>
__device__ void decode_layers(const Args &a, const DecodeLayersConstants &c) {
    static_assert((kWork * G * HD + 2 * kWork * G) * 4 <= kWork * (int)kRing0,
                  "the attention merge area must fit in ring 0");
    static_assert(HD % 8 == 0 && HD / 8 <= 64, "a key row spans at most one wave");
    extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
    __shared__ float red[kWaves];
    const uint32_t H = c.H, F = c.F, QW = c.Nq * HD, KW = c.Nkv * HD, QKV = QW + 2u * KW;
    const uint32_t L = c.layers, P = c.partitions, S = c.kvStride;
    const uint32_t maxK = max(max(H, QW), F);
    const uint32_t lane = threadIdx.x & 63;
    const uint32_t wave = pk::uniform(threadIdx.x >> 6);
    const bool worker = wave < (uint32_t)kWork, syncWave = !worker;
    const uint32_t wslot = worker ? wave : 0u;

    float *xres = reinterpret_cast<float *>(lds);                              // [H] f32
    uint16_t *xs = reinterpret_cast<uint16_t *>(lds + ((H * 4u + 15u) & ~15u)); // [maxK] bf16
    uint8_t *rings = lds + ((H * 4u + 15u) & ~15u) + ((maxK * 2u + 15u) & ~15u);
    uint8_t *ring0 = rings + wslot * kRing0;
    uint8_t *ring1 = rings + (uint32_t)kWork * kRing0 + wslot * kRing1;
    // attention merge area (phase B only, while ring 0 is idle)
    float *sm_o = reinterpret_cast<float *>(rings);                        // [kWork][G][HD]
    float *sm_m = sm_o + (uint32_t)(kWork * G * HD);                       // [kWork][G]
    float *sm_l = sm_m + (uint32_t)(kWork * G);                            // [kWork][G]

    const uint32_t blocks = gridDim.x;
    const uint32_t first = wslot * blocks + blockIdx.x, stride = blocks * kWork;
    const int32_t pos = a.position[0];
    const bool scatter = pos >= 0 && (uint32_t)pos < S;

    GridSync gs;
    gs.words = a.sync;
    gs.stamps = a.stamps;
    gs.limit = c.spinTicks ? c.spinTicks : 50000000u;
    gs.blocks = blocks;
    gs.waits = 0;
    gs.aborted = false;

    KvGeom<HD> kv;
    kv.init(c, pos);
    float *pO = a.partials;                               // [Nq][P][HD]
    float *pML = a.partials + (uint64_t)c.Nq * P * HD;    // [Nq][P][2]: m, l

    uint32_t layer = 0;  // the layer the row functions address
    auto rowsA = [&](uint32_t unit, int) {
        return a.wqkv + ((uint64_t)layer * QKV + min(unit, QKV - 1u)) * H;
    };
    auto rowsO = [&](uint32_t unit, int) { return a.wo + ((uint64_t)layer * H + min(unit, H - 1u)) * QW; };
    auto rowsGU = [&](uint32_t unit, int s) {
        return (s == 0 ? a.wg : a.wu) + ((uint64_t)layer * F + min(unit, F - 1u)) * H;
    };
    auto rowsF = [&](uint32_t unit, int) { return a.wd + ((uint64_t)layer * H + min(unit, H - 1u)) * F; };
    auto normL = [&](uint32_t l, uint32_t slot) { return a.norms + ((uint64_t)l * 4u + slot) * H; };
    auto kcL = [&](uint32_t l) { return a.kc + (uint64_t)l * c.Nkv * S * HD; };
    auto vcL = [&](uint32_t l) { return a.vc + (uint64_t)l * c.Nkv * S * HD; };

    LdsStream<1, kDepthQKV> rsA;
    rsA.init(ring0, rowsA, H, QKV, first, stride);
    if (worker) rsA.start(rowsA);

    for (uint32_t l = 0; l < L; ++l) {
        layer = l;
        // ---- A: [post-FFN norm + residual], input norm, QKV, KV-cache rows
        stage_glue(xs, xres, red, l == 0 ? a.x_in : a.mlp, l == 0 ? nullptr : normL(l - 1u, 3), normL(l, 0), H, c.eps,
                   l == 0, nullptr);
        if (worker) {
            uint16_t *kcl = kcL(l), *vcl = vcL(l);
            auto storeA = [&](uint32_t unit, const float *sums) {
                if (lane != 0 || unit >= QKV) return;
                const uint16_t v = BF16::store(sums[0]);
                if (unit < QW) {
                    st16(a.q + unit, v);
                } else if (scatter) {
                    uint32_t j = unit - QW;
                    const bool isV = j >= KW;
                    if (isV) j -= KW;
                    st16((isV ? vcl : kcl) + ((uint64_t)(j / HD) * S + (uint32_t)pos) * HD + j % HD, v);
                }
            };
            rsA.run(xs, rowsA, storeA);
        }
        LdsStream<1, kDepthO> rsO;
        KvSlots<HD> slots;
        rsO.init(ring1, rowsO, QW, H, first, stride);
        issue_after_stores();
        if (worker) {
            slots.issue(kv, kcL(l), vcL(l), S, wave, 0);
            rsO.start(rowsO);
        }
        grid_wait<kDepthO + 2 * kKvLoads>(gs, syncWave);

        // ---- B: split-KV attention partials
        if (worker && kv.active) {
            const uint32_t kg = lane / KvGeom<HD>::LPK, dl = lane % KvGeom<HD>::LPK;
            FdState<HD, G> st;
#pragma unroll
            for (int g = 0; g < G; ++g) {
                const uint16_t *qrow = a.q + (uint64_t)(kv.hkv * G + g) * HD + dl * 8u;
                float lo4[4], hi4[4];
                bf4(ld64(qrow), lo4);
                bf4(ld64(qrow + 4), hi4);
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    st.q[g][e] = lo4[e] * c.scale;
                    st.q[g][4 + e] = hi4[e] * c.scale;
                }
#pragma unroll
                for (int e = 0; e < 8; ++e) st.o[g][e] = 0.0f;
                st.m[g] = -INFINITY;
                st.l[g] = 0.0f;
            }
            const uint32_t span = kv.cachedHi - kv.lo;  // cachedHi >= lo
            constexpr uint32_t kPerRound = (uint32_t)(kKvLoads * kWork * KvGeom<HD>::KPW);
            const uint32_t rounds = (span + kPerRound - 1u) / kPerRound;  // <= kvStride / kPerRound + 1
            for (uint32_t round = 0; round < max(rounds, 1u); ++round) {
                if (round > 0) {
                    if ((round * kKvLoads * kWork + wave) * KvGeom<HD>::KPW >= span) break;
                    slots.issue(kv, kcL(l), vcL(l), S, wave, round);
                }
                bool valid[kKvLoads];
#pragma unroll
                for (int t = 0; t < kKvLoads; ++t)
                    valid[t] = kv.lo + ((round * kKvLoads + t) * kWork + wave) * KvGeom<HD>::KPW + kg < kv.cachedHi;
                st.tile(slots.k, slots.v, valid);
            }
            if (kv.owner && wave == 0) {
                // the key at the position, written by phase A of this launch
                const uint64_t at = ((uint64_t)kv.hkv * S + (uint32_t)pos) * HD + dl * 8u;
                pk::Vec<BF16> fk[1], fv[1];
                const uint64_t k0 = ld64(kcL(l) + at), k1 = ld64(kcL(l) + at + 4);
                const uint64_t v0 = ld64(vcL(l) + at), v1 = ld64(vcL(l) + at + 4);
                fk[0].raw = u32x4{(uint32_t)k0, (uint32_t)(k0 >> 32), (uint32_t)k1, (uint32_t)(k1 >> 32)};
                fv[0].raw = u32x4{(uint32_t)v0, (uint32_t)(v0 >> 32), (uint32_t)v1, (uint32_t)(v1 >> 32)};
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
                    float *dst = sm_o + ((uint32_t)wave * G + g) * HD + dl * 8u;
                    *reinterpret_cast<float4 *>(dst) = float4{st.o[g][0], st.o[g][1], st.o[g][2], st.o[g][3]};
                    *reinterpret_cast<float4 *>(dst + 4) = float4{st.o[g][4], st.o[g][5], st.o[g][6], st.o[g][7]};
                    if (dl == 0) {
                        sm_m[wave * G + g] = st.m[g];
                        sm_l[wave * G + g] = st.l[g];
                    }
                }
            }
        }
        __syncthreads();
        if (kv.active) {
            // the partition's state: the worker waves' states merged
            for (uint32_t idx = threadIdx.x; idx < (uint32_t)(G * HD / 2); idx += kThreads) {
                const uint32_t g = idx / (HD / 2), d = 2u * (idx % (HD / 2));
                float mstar = -INFINITY;
#pragma unroll
                for (int w = 0; w < kWork; ++w) mstar = fmaxf(mstar, sm_m[w * G + g]);
                float o0 = 0.0f, o1 = 0.0f, lsum = 0.0f;
                if (mstar != -INFINITY) {
#pragma unroll
                    for (int w = 0; w < kWork; ++w) {
                        const float e = pk::fast_exp(sm_m[w * G + g] - mstar);
                        o0 += e * sm_o[((uint32_t)w * G + g) * HD + d];
                        o1 += e * sm_o[((uint32_t)w * G + g) * HD + d + 1];
                        lsum += e * sm_l[w * G + g];
                    }
                }
                const uint64_t slot = (uint64_t)(kv.hkv * G + g) * P + kv.part;
                st64(pO + slot * HD + d, (uint64_t)__float_as_uint(o0) | ((uint64_t)__float_as_uint(o1) << 32));
                if (d == 0) st64(pML + 2u * slot, (uint64_t)__float_as_uint(mstar) | ((uint64_t)__float_as_uint(lsum) << 32));
            }
        }
        __syncthreads();  // the merge area (ring 0) is read; the gate/up copies may overwrite it
        LdsStream<2, kDepthGU> rsGU;
        rsGU.init(ring0, rowsGU, H, F, first, stride);
        issue_after_stores();
        if (worker) rsGU.start(rowsGU);
        grid_wait<2 * kDepthGU>(gs, syncWave);

        // ---- C: log-sum-exp combine, attn = sum_p exp(m_p - m*) O_p / sum_p exp(m_p - m*) l_p
        if (worker) {
            const uint32_t items = c.Nq * (HD / 8);
            for (uint32_t it = blockIdx.x + wave * blocks; it < items; it += stride) {
                const uint32_t hq = it / (HD / 8), d0 = 8u * (it % (HD / 8));
                const bool has = lane < P;
                const uint64_t slot = (uint64_t)hq * P + (has ? lane : 0u);
                const uint64_t ml = ld64(pML + 2u * slot);
                uint64_t ov[4];
#pragma unroll
                for (int h = 0; h < 4; ++h) ov[h] = ld64(pO + slot * HD + d0 + 2u * h);
                const float m = has ? __uint_as_float((uint32_t)ml) : -INFINITY;
                const float lp = __uint_as_float((uint32_t)(ml >> 32));
                const float mstar = pk::wave_max(m);
                float out[8];
                if (mstar == -INFINITY) {
#pragma unroll
                    for (int e = 0; e < 8; ++e) out[e] = 0.0f;
                } else {
                    const float w = has ? pk::fast_exp(m - mstar) : 0.0f;
                    const float lstar = pk::wave_sum(w * lp);
#pragma unroll
                    for (int h = 0; h < 4; ++h) {
                        out[2 * h] = pk::wave_sum(w * __uint_as_float((uint32_t)ov[h])) / lstar;
                        out[2 * h + 1] = pk::wave_sum(w * __uint_as_float((uint32_t)(ov[h] >> 32))) / lstar;
                    }
                }
                if (lane == 0) {
                    st64(a.attn + (uint64_t)hq * HD + d0, pack_bf4(out));
                    st64(a.attn + (uint64_t)hq * HD + d0 + 4, pack_bf4(out + 4));
                }
            }
        }
        grid_wait<0>(gs, syncWave);

        // ---- D: O projection
        stage_vector(xs, a.attn, QW);
        if (worker) {
            auto storeO = [&](uint32_t unit, const float *sums) {
                if (lane == 0 && unit < H) st16(a.o + unit, BF16::store(sums[0]));
            };
            rsO.run(xs, rowsO, storeO);
        }
        grid_wait<0>(gs, syncWave);

        // ---- E: post-attention norm + residual, pre-FFN norm, gate/up, GELU-tanh * up
        stage_glue(xs, xres, red, a.o, normL(l, 1), normL(l, 2), H, c.eps, false,
                   (l + 1u == L && blockIdx.x == 0) ? a.x2 : nullptr);
        if (worker) {
            auto storeGU = [&](uint32_t unit, const float *sums) {
                if (lane != 0 || unit >= F) return;
                const float g = rnd(sums[0]), u = rnd(sums[1]);
                const float act = rnd(pk::gelu_tanh(g));
                st16(a.hidden + unit, BF16::store(act * u));
            };
            rsGU.run(xs, rowsGU, storeGU);
        }
        LdsStream<1, kDepthDown> rsF;
        rsF.init(ring1, rowsF, F, H, first, stride);
        issue_after_stores();
        if (worker) rsF.start(rowsF);
        grid_wait<kDepthDown>(gs, syncWave);

        // ---- F: down projection
        stage_vector(xs, a.hidden, F);
        if (worker) {
            auto storeF = [&](uint32_t unit, const float *sums) {
                if (lane == 0 && unit < H) st16(a.mlp + unit, BF16::store(sums[0]));
            };
            rsF.run(xs, rowsF, storeF);
        }
        if (l + 1u < L) {
            layer = l + 1u;
            rsA.init(ring0, rowsA, H, QKV, first, stride);
            issue_after_stores();
            if (worker) rsA.start(rowsA);
            grid_wait<kDepthQKV>(gs, syncWave);
        }
    }

    // The last block to finish zeroes the counters for the next launch: every
    // block that has arrived here has passed all of its waits.
    asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)" ::: "memory");
    asm volatile("s_barrier" ::: "memory");
    if (syncWave && lane == 0) {
        const uint32_t done = __hip_atomic_fetch_add(a.sync + kDoneWord, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (done + 1u == blocks) {
            for (int i = 0; i < kCounters; ++i) st32(a.sync + i * kLine, 0u);
            st32(a.sync + kDoneWord, 0u);
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
                                        uint16_t *mlp, uint16_t *x2, float *partials, uint32_t *sync,             \
                                        uint64_t *stamps, DecodeLayersConstants c) {                              \
        const Args a{x_in, wqkv, wo, wg, wu, wd, norms, kc, vc, position, q, attn, o, hidden, mlp, x2,           \
                     partials, sync, stamps};                                                                     \
        decode_layers<HD, G>(a, c);                                                                               \
    }

DECODE_LAYERS(256, 2)
DECODE_LAYERS(256, 1)
DECODE_LAYERS(128, 2)
DECODE_LAYERS(64, 2)
DECODE_LAYERS(64, 4)
