// Split-KV attention (FlashDecoding) and its log-sum-exp combine.
//
// Algorithm of Sources/Popcorn/Kernels/FlashDecoding.metal:28-231: the keys
// of each query row are split into P partitions of per = ceil(Sk/P) keys
// (:56-63); each partition runs the online softmax over its keys with Q
// pre-scaled (:65-68) and writes unnormalised O with its running max m and
// sum l (:165-173); the combine merges them with
//   m* = max m_k, l* = sum exp(m_k - m*) l_k, O = sum exp(m_k - m*) O_k / l*
// (:202-227). posQ = Sk - Sq + row (:73 for Sq = 1; FlashAttention.metal:72).
// Partition outputs: O [B, Nq, Sq, P, Hd], m and l [B, Nq, Sq, P] (f32).
//
// Layout for gfx950 (fast path, flash_decoding_partial_<t>_l<LPK>_c<CPL>_g<G>):
//  * one block (NW = 4 or 8 waves) per (partition, batch x KV head x head
//    group, query row): the G query heads that share a KV head (GQA) are processed
//    together, so each K/V byte is read once per block, not once per head;
//  * a key row is split across LPK lanes, each holding CPL 16-byte chunks, so
//    one wave-wide load instruction covers 64/LPK whole key rows (1 KB);
//  * a wave takes TILE = (64/LPK) * U keys per step: U rows of K and of V per
//    lane in flight, dot products reduced within the LPK-lane group by DPP,
//    tile max across the wave, then p = exp(s - m) and O += p V on the
//    lane's own dims; l and O stay group-local until the end of the range;
//  * waves take interleaved tiles of the partition's key range; the NW wave
//    states are merged in LDS and written as the partition's (O, m, l).
// Host names: flash_decoding_partial_<t>, flash_decoding_reduce_<t> and the
// plain flash_attention* keep the reference's names, parameter lists
// (FlashDecoding.metal:29-36, :181-187, FlashAttention.metal:31-36) and launch
// geometry (FlashDecoding.swift:155-160, :225-230, FlashAttention.swift:203),
// for raw launches built like the reference's; the descriptors use the fast
// kernels above, flash_decoding_partial_<t>_ext (any head dim, Sq rows,
// a KV row stride and a device position) and flash_decoding_reduce_<t>_ext.
// Keys outside the causal / sliding-window range are skipped by clamping
// the range; the per-key mask is still applied. A range with no allowed key
// writes m = -inf, l = 0, O = 0 (FlashDecoding.metal:78-87); a tile whose
// keys are all masked leaves the state unchanged instead of computing
// exp(-inf - -inf).
#include "common.hpp"

namespace {

constexpr int kWaves = 4;

struct FdGeom {
    uint32_t b, hkv, g0, gcount, qi, Sq, Sk, posQ, jLo, jHi;
    bool empty;
    bool owner;  // fresh-key variant: this block's partition holds key posQ
};

__device__ inline bool fd_allowed(const FlashDecodingPartialExtConstants &p, int posQ, int posK) {
    bool allowed = (p.maskKind == 2u) | (posK <= posQ);
    if (p.maskKind == 1u) allowed = allowed & ((posQ - posK) < p.slidingWindow);
    return allowed;
}

// Grid: x = partition, y = (b * Nkv + hkv) * ngroups + head group, z = row.
// With freshLast, key posQ is left out of the block's range (the fresh-key
// variant attends it from its prologue) and `owner` marks the block whose
// partition holds it.
__device__ inline FdGeom fd_geometry(const FlashDecodingPartialExtConstants &p, const int32_t *position, uint32_t gmax,
                                     bool freshLast = false) {
    FdGeom g;
    const uint32_t G = p.Nq / p.Nkv;
    const uint32_t ngroups = (G + gmax - 1) / gmax;
    const uint32_t hg = blockIdx.y % ngroups;
    const uint32_t bkv = blockIdx.y / ngroups;
    g.b = bkv / p.Nkv;
    g.hkv = bkv % p.Nkv;
    g.g0 = hg * gmax;
    g.gcount = min(gmax, G - g.g0);
    g.qi = blockIdx.z;
    g.Sq = p.Sq ? p.Sq : 1u;
    const uint32_t stride = p.kvStride ? p.kvStride : p.Sk;
    uint32_t Sk = p.Sk;
    bool inCache = true;  // the query rows' own keys lie inside the cache
    if (p.keyLenFromPosition) {
        int32_t pos = position[0];
        Sk = pos < 0 ? 0u : (uint32_t)pos + g.Sq;
        inCache = pos >= 0 && (uint64_t)pos + g.Sq <= stride;
    }
    if (Sk > stride) Sk = stride;  // never read past the cache
    g.Sk = Sk;
    const int posQ = (int)Sk - (int)g.Sq + (int)g.qi;
    g.posQ = (uint32_t)max(posQ, -1);
    const uint32_t P = p.P ? p.P : 1u;
    const uint32_t per = (Sk + P - 1) / P;
    int lo = (int)(blockIdx.x * per);
    int hi = min(lo + (int)per, (int)Sk);
    // a position past the cache writes no key row (and attends the clamped range)
    g.owner = freshLast && inCache && posQ >= 0 && (uint32_t)posQ < stride && lo <= posQ && posQ < hi;
    if (p.maskKind != 2u) hi = min(hi, posQ + 1);
    if (freshLast) hi = min(hi, posQ);
    if (p.maskKind == 1u) lo = max(lo, posQ - p.slidingWindow + 1);
    g.empty = hi <= lo;
    g.jLo = (uint32_t)max(lo, 0);
    g.jHi = g.empty ? g.jLo : (uint32_t)hi;
    return g;
}

// Writes one partition's state for `gcount` heads: wave states sm_* merged.
template <int GMAX, int HD, int NSLOTS = kWaves>
__device__ void fd_merge_store(const FlashDecodingPartialExtConstants &p, const FdGeom &geo, float (*sm_m)[GMAX],
                               float (*sm_l)[GMAX], float (*sm_o)[GMAX][HD], float *pO, float *pM, float *pL) {
    const uint32_t P = p.P ? p.P : 1u;
    const uint32_t G = p.Nq / p.Nkv;
    for (uint32_t idx = threadIdx.x; idx < geo.gcount * HD; idx += blockDim.x) {
        const uint32_t g = idx / HD, d = idx % HD;
        float mstar = -INFINITY;
#pragma unroll
        for (int w = 0; w < NSLOTS; ++w) mstar = fmaxf(mstar, sm_m[w][g]);
        float o = 0.0f, l = 0.0f;
        if (mstar != -INFINITY) {
#pragma unroll
            for (int w = 0; w < NSLOTS; ++w) {
                float a = pk::fast_exp(sm_m[w][g] - mstar);
                o += a * sm_o[w][g][d];
                l += a * sm_l[w][g];
            }
        }
        const uint32_t hq = geo.hkv * G + geo.g0 + g;
        const uint64_t slot = ((uint64_t)(geo.b * p.Nq + hq) * geo.Sq + geo.qi) * P + blockIdx.x;
        pO[slot * HD + d] = o;
        if (d == 0) {
            pM[slot] = mstar;
            pL[slot] = l;
        }
    }
}

// The fresh-key variant's extra inputs (DecodeAttentionConstants): the
// caches again as writable pointers for the new row, the per-head norm
// weights (f32 [Hd], read when their flag is set) and the RoPE frequencies.
template <typename T>
struct FreshArgs {
    typename T::storage *kw, *vw;
    const float *wq, *wk, *invFreq;
    DecodeAttentionConstants c;
};

struct NoFresh {};

// FRESH: the decode attention block of one token (DecodeAttentionConstants).
// Q is then the raw projection row; the prologue stages this block's query
// heads (and, in the block owning key posQ, the key and value heads) in LDS,
// applies the per-head RMSNorms and RoPE with the reference's rounding after
// each step, writes the new K/V row to the caches (head group 0 only), and
// turns the new key into one more softmax state (m = q.k, l = 1, O = v) that
// the merge folds in with the NW waves' states. The key loop covers keys
// below posQ only.
template <typename T, int LPK, int CPL, int GMAX, int U, bool FRESH = false, typename FA = NoFresh, int NW = kWaves>
__device__ void fd_partial_fast(const typename T::storage *__restrict__ Q, const typename T::storage *__restrict__ K,
                                const typename T::storage *__restrict__ V, float *__restrict__ pO,
                                float *__restrict__ pM, float *__restrict__ pL, const int32_t *__restrict__ position,
                                const FlashDecodingPartialExtConstants &p, const FA &fa = FA{}) {
    constexpr int kV = pk::Vec<T>::kVec;
    constexpr int DL = CPL * kV;   // dims per lane
    constexpr int HD = LPK * DL;   // head dim
    constexpr int KPW = 64 / LPK;  // key rows per wave-wide load
    constexpr int TILE = KPW * U;  // keys per wave step
    constexpr int NSLOTS = NW + (FRESH ? 1 : 0);
    constexpr int kUnits = FRESH ? GMAX + 2 : 1;  // query heads, key head, value head

    __shared__ float sm_m[NSLOTS][GMAX];
    __shared__ float sm_l[NSLOTS][GMAX];
    __shared__ float sm_o[NSLOTS][GMAX][HD];
    __shared__ float sm_x[kUnits][FRESH ? HD : 1];
    __shared__ float sm_ss[kUnits];

    const FdGeom geo = fd_geometry(p, position, GMAX, FRESH);
    const uint32_t lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const uint32_t kg = lane / LPK, dl = lane % LPK;
    const uint32_t G = p.Nq / p.Nkv;
    const uint32_t stride = p.kvStride ? p.kvStride : p.Sk;
    const uint64_t kvbase = (uint64_t)(geo.b * p.Nkv + geo.hkv) * stride * HD;

    if constexpr (FRESH) {
        const DecodeAttentionConstants &c = fa.c;
        const typename T::storage *row = Q + (uint64_t)geo.b * c.rowStride;
        const uint32_t hq0 = geo.hkv * G + geo.g0;
        auto live = [&](uint32_t u) { return u < (uint32_t)GMAX ? u < geo.gcount : geo.owner; };
        auto src = [&](uint32_t u) {
            return u < (uint32_t)GMAX ? row + (uint64_t)(hq0 + u) * HD
                 : u == (uint32_t)GMAX ? row + (uint64_t)(p.Nq + geo.hkv) * HD
                                       : row + (uint64_t)(p.Nq + p.Nkv + geo.hkv) * HD;
        };
        for (uint32_t idx = threadIdx.x; idx < (uint32_t)(kUnits * HD); idx += blockDim.x) {
            const uint32_t u = idx / HD, d = idx % HD;
            if (live(u)) sm_x[u][d] = T::load(src(u)[d]);
        }
        __syncthreads();
        for (uint32_t u = wave; u < (uint32_t)kUnits; u += NW) {
            if (!live(u)) continue;
            float acc = 0.0f;
            for (uint32_t d = lane; d < (uint32_t)HD; d += 64) acc += sm_x[u][d] * sm_x[u][d];
            acc = pk::wave_sum(acc);
            if (lane == 0) sm_ss[u] = acc;
        }
        __syncthreads();
        // one thread per (unit, rotation pair i, i + Hd/2): reads and writes
        // only its own two elements
        constexpr uint32_t H2 = HD / 2;
        const int32_t pos = (int32_t)geo.posQ;
        auto rnd = [](float x) { return T::load(T::store(x)); };
        for (uint32_t idx = threadIdx.x; idx < (uint32_t)kUnits * H2; idx += blockDim.x) {
            const uint32_t u = idx / H2, i = idx % H2;
            if (!live(u)) continue;
            const bool isQ = u < (uint32_t)GMAX, isK = u == (uint32_t)GMAX;
            float x1 = sm_x[u][i], x2 = sm_x[u][i + H2];
            if (c.flags & (isQ ? 1u : isK ? 2u : 4u)) {
                // RMSNorm.metal: (x * rsqrt(mean(x^2) + eps)) * w
                const float scale = 1.0f / sqrtf(sm_ss[u] / (float)HD + c.eps);
                x1 *= scale;
                x2 *= scale;
                if (isQ || isK) {  // the value norm has no weight
                    const float *w = isQ ? fa.wq : fa.wk;
                    x1 *= w[i];
                    x2 *= w[i + H2];
                }
                x1 = rnd(x1);
                x2 = rnd(x2);
            }
            if ((c.flags & 8u) && u <= (uint32_t)GMAX) {
                // RopeBuildCosSin.metal:17-20, RopeApply.metal:36-37
                const float angle = (float)pos * fa.invFreq[i];
                float sn, cs;
                sincosf(angle, &sn, &cs);
                cs *= c.ropeScaling;
                sn *= c.ropeScaling;
                const float o1 = x1 * cs - x2 * sn, o2 = x1 * sn + x2 * cs;
                x1 = rnd(o1);
                x2 = rnd(o2);
            }
            sm_x[u][i] = x1;
            sm_x[u][i + H2] = x2;
            if (!isQ && geo.g0 == 0) {
                typename T::storage *dst = (isK ? fa.kw : fa.vw) + kvbase + (uint64_t)pos * HD;
                dst[i] = T::store(x1);
                dst[i + H2] = T::store(x2);
            }
        }
        __syncthreads();
        // the new key's state per query head: m = q.k, l = 1, O = v
        for (uint32_t g = wave; g < (uint32_t)GMAX; g += NW) {
            const bool has = geo.owner && g < geo.gcount;
            float acc = 0.0f;
            if (has) {
                for (uint32_t d = lane; d < (uint32_t)HD; d += 64) acc += (sm_x[g][d] * p.scale) * sm_x[GMAX][d];
                acc = pk::wave_sum(acc);
            }
            if (lane == 0) {
                sm_m[NW][g] = has ? acc : -INFINITY;
                sm_l[NW][g] = has ? 1.0f : 0.0f;
            }
            for (uint32_t d = lane; d < (uint32_t)HD; d += 64) sm_o[NW][g][d] = has ? sm_x[GMAX + 1][d] : 0.0f;
        }
    }

    float q[GMAX][DL], o[GMAX][DL], m[GMAX], l[GMAX];
    pk::Vec<T> qv[GMAX][CPL];  // the query rows as loaded (converted in the key loop)
#pragma unroll
    for (int g = 0; g < GMAX; ++g) {
        m[g] = -INFINITY;
        l[g] = 0.0f;
        const uint32_t gg = min((uint32_t)g, geo.gcount - 1);
        if constexpr (FRESH) {
#pragma unroll
            for (int c = 0; c < CPL; ++c) {
#pragma unroll
                for (int e = 0; e < kV; ++e) {
                    q[g][c * kV + e] = sm_x[gg][(c * LPK + dl) * kV + e] * p.scale;
                    o[g][c * kV + e] = 0.0f;
                }
            }
        } else {
            const uint32_t hq = geo.hkv * G + geo.g0 + gg;
            const typename T::storage *qrow = Q + ((uint64_t)(geo.b * p.Nq + hq) * geo.Sq + geo.qi) * HD;
#pragma unroll
            for (int c = 0; c < CPL; ++c) {
                qv[g][c].load(qrow + (c * LPK + dl) * kV);
#pragma unroll
                for (int e = 0; e < kV; ++e) o[g][c * kV + e] = 0.0f;
            }
        }
    }

    const typename T::storage *Kh = K + kvbase;
    const typename T::storage *Vh = V + kvbase;
    const uint32_t nkeys = geo.jHi - geo.jLo;
    const uint32_t ntiles = (nkeys + TILE - 1) / TILE;

    for (uint32_t t = wave; t < ntiles; t += NW) {
        const uint32_t j0 = geo.jLo + t * TILE;
        pk::Vec<T> kv[U][CPL], vv[U][CPL];
        bool valid[U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const uint32_t j = j0 + u * KPW + kg;
            valid[u] = (j < geo.jHi) & fd_allowed(p, (int)geo.posQ, (int)j);
            const uint32_t jj = j < geo.jHi ? j : geo.jLo;
#pragma unroll
            for (int c = 0; c < CPL; ++c) {
                kv[u][c].load_nt(Kh + (uint64_t)jj * HD + (c * LPK + dl) * kV);
                vv[u][c].load_nt(Vh + (uint64_t)jj * HD + (c * LPK + dl) * kV);
            }
        }
        if constexpr (!FRESH) {
            __builtin_amdgcn_sched_barrier(0);  // every K/V load above issues first
            // The query rows are converted here, after this tile's K and V
            // loads are issued, so their round trip overlaps the keys'
            // (converted before the loop, they made every K/V load wait for
            // them). The empty volatile asm keeps the conversion from being
            // hoisted out of the loop and is a scheduling boundary.
#pragma unroll
            for (int g = 0; g < GMAX; ++g)
#pragma unroll
                for (int c = 0; c < CPL; ++c) {
                    pk::Vec<T> t = qv[g][c];
                    asm volatile("" : "+v"(t.raw));
#pragma unroll
                    for (int e = 0; e < kV; ++e) q[g][c * kV + e] = t.get(e) * p.scale;
                }
        }
        float s[GMAX][U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            float kf[DL];
#pragma unroll
            for (int c = 0; c < CPL; ++c) {
#pragma unroll
                for (int e = 0; e < kV; ++e) kf[c * kV + e] = kv[u][c].get(e);
            }
#pragma unroll
            for (int g = 0; g < GMAX; ++g) {
                float acc = 0.0f;
#pragma unroll
                for (int e = 0; e < DL; ++e) acc += q[g][e] * kf[e];
                s[g][u] = pk::group_sum<LPK>(acc);
            }
        }
#pragma unroll
        for (int g = 0; g < GMAX; ++g) {
            float mx = -INFINITY;
#pragma unroll
            for (int u = 0; u < U; ++u) {
                if (!valid[u]) s[g][u] = -INFINITY;
                mx = fmaxf(mx, s[g][u]);
            }
            if constexpr (KPW > 1) {
                // all lanes of a key group hold the same scores: reduce across groups
                mx = pk::wave_max(mx);
            }
            const float m_new = fmaxf(m[g], mx);
            if (m_new == -INFINITY) continue;  // nothing allowed yet
            const float alpha = pk::fast_exp(m[g] - m_new);
            float psum = 0.0f;
            float pu[U];
#pragma unroll
            for (int u = 0; u < U; ++u) {
                pu[u] = pk::fast_exp(s[g][u] - m_new);
                psum += pu[u];
            }
            l[g] = alpha * l[g] + psum;
            m[g] = m_new;
#pragma unroll
            for (int e = 0; e < DL; ++e) o[g][e] *= alpha;
#pragma unroll
            for (int u = 0; u < U; ++u) {
#pragma unroll
                for (int c = 0; c < CPL; ++c) {
#pragma unroll
                    for (int e = 0; e < kV; ++e) o[g][c * kV + e] += pu[u] * vv[u][c].get(e);
                }
            }
        }
    }

    // Merge the key groups of this wave (lanes dl, dl + LPK, ...): the xor-16
    // and xor-32 steps as register lane swaps
#pragma unroll
    for (int g = 0; g < GMAX; ++g) {
        if constexpr (LPK <= 8) {
            l[g] += __shfl_xor(l[g], 8, 64);
#pragma unroll
            for (int e = 0; e < DL; ++e) o[g][e] += __shfl_xor(o[g][e], 8, 64);
        }
        if constexpr (LPK <= 16) {
            l[g] = pk::pair16_sum(l[g]);
#pragma unroll
            for (int e = 0; e < DL; ++e) o[g][e] = pk::pair16_sum(o[g][e]);
        }
        if constexpr (LPK <= 32) {
            l[g] = pk::pair32_sum(l[g]);
#pragma unroll
            for (int e = 0; e < DL; ++e) o[g][e] = pk::pair32_sum(o[g][e]);
        }
    }
    if (kg == 0) {
#pragma unroll
        for (int g = 0; g < GMAX; ++g) {
#pragma unroll
            for (int c = 0; c < CPL; ++c) {
#pragma unroll
                for (int e = 0; e < kV; ++e) sm_o[wave][g][(c * LPK + dl) * kV + e] = o[g][c * kV + e];
            }
            if (dl == 0) {
                sm_m[wave][g] = m[g];
                sm_l[wave][g] = l[g];
            }
        }
    }
    __syncthreads();
    fd_merge_store<GMAX, HD, NSLOTS>(p, geo, sm_m, sm_l, sm_o, pO, pM, pL);
}

// Any head dim <= 512 and any dtype: one query head per block (GMAX = 1),
// lanes stride over the head dim, one key at a time per wave.
template <typename T>
__device__ void fd_partial_generic(const typename T::storage *__restrict__ Q, const typename T::storage *__restrict__ K,
                                   const typename T::storage *__restrict__ V, float *__restrict__ pO,
                                   float *__restrict__ pM, float *__restrict__ pL, const int32_t *__restrict__ position,
                                   const FlashDecodingPartialExtConstants &p) {
    constexpr int kMaxHd = 512, kDL = kMaxHd / 64;
    __shared__ float sm_m[kWaves][1];
    __shared__ float sm_l[kWaves][1];
    __shared__ float sm_o[kWaves][1][kMaxHd];
    const FdGeom geo = fd_geometry(p, position, 1);
    const uint32_t lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const uint32_t Hd = p.Hd;
    const uint32_t G = p.Nq / p.Nkv;
    const uint32_t hq = geo.hkv * G + geo.g0;
    const uint32_t stride = p.kvStride ? p.kvStride : p.Sk;
    const typename T::storage *qrow = Q + ((uint64_t)(geo.b * p.Nq + hq) * geo.Sq + geo.qi) * Hd;
    float q[kDL], o[kDL];
#pragma unroll
    for (int i = 0; i < kDL; ++i) {
        uint32_t d = lane + 64 * i;
        q[i] = d < Hd ? T::load(qrow[d]) * p.scale : 0.0f;
        o[i] = 0.0f;
    }
    float m = -INFINITY, l = 0.0f;
    const uint64_t kvbase = (uint64_t)(geo.b * p.Nkv + geo.hkv) * stride * Hd;
    for (uint32_t j = geo.jLo + wave; j < geo.jHi; j += kWaves) {
        if (!fd_allowed(p, (int)geo.posQ, (int)j)) continue;
        const typename T::storage *kr = K + kvbase + (uint64_t)j * Hd;
        const typename T::storage *vr = V + kvbase + (uint64_t)j * Hd;
        float acc = 0.0f;
#pragma unroll
        for (int i = 0; i < kDL; ++i) {
            uint32_t d = lane + 64 * i;
            if (d < Hd) acc += q[i] * T::load(kr[d]);
        }
        const float s = pk::wave_sum(acc);
        const float m_new = fmaxf(m, s);
        const float alpha = pk::fast_exp(m - m_new);
        const float pj = pk::fast_exp(s - m_new);
        l = alpha * l + pj;
        m = m_new;
#pragma unroll
        for (int i = 0; i < kDL; ++i) {
            uint32_t d = lane + 64 * i;
            o[i] = alpha * o[i] + (d < Hd ? pj * T::load(vr[d]) : 0.0f);
        }
    }
#pragma unroll
    for (int i = 0; i < kDL; ++i) sm_o[wave][0][lane + 64 * i] = o[i];
    if (lane == 0) {
        sm_m[wave][0] = m;
        sm_l[wave][0] = l;
    }
    __syncthreads();
    const uint32_t P = p.P ? p.P : 1u;
    for (uint32_t d = threadIdx.x; d < Hd; d += blockDim.x) {
        float mstar = -INFINITY;
#pragma unroll
        for (int w = 0; w < kWaves; ++w) mstar = fmaxf(mstar, sm_m[w][0]);
        float oo = 0.0f, ll = 0.0f;
        if (mstar != -INFINITY) {
#pragma unroll
            for (int w = 0; w < kWaves; ++w) {
                float a = pk::fast_exp(sm_m[w][0] - mstar);
                oo += a * sm_o[w][0][d];
                ll += a * sm_l[w][0];
            }
        }
        const uint64_t slot = ((uint64_t)(geo.b * p.Nq + hq) * geo.Sq + geo.qi) * P + blockIdx.x;
        pO[slot * Hd + d] = oo;
        if (d == 0) {
            pM[slot] = mstar;
            pL[slot] = ll;
        }
    }
}

// LSE combine, FlashDecoding.metal:179-228:
//   m* = max m_k, l* = sum exp(m_k - m*) l_k, O = sum exp(m_k - m*) O_k / l*.
// Grid: x = (b * Nq + hq) * Sq + row, y = 64-dim slice of the head. Lane =
// one dim; each wave takes a contiguous quarter of the partitions, a batch
// of kReduceBatch at a time: lane j loads batch entry j's m and l (one
// vector load each; read back with readlane) and every lane its dim of each
// entry's O, all in flight together, so a decode-sized combine (P <= 128)
// is one memory round trip. The batch's max is taken first, so each batch
// rescales the running state once; the 4 wave states are then merged in
// LDS. Empty partitions (m = -inf, l = 0) contribute nothing.
constexpr int kReduceBatch = 32;

template <typename O>
__device__ void fd_reduce(const float *__restrict__ pO, const float *__restrict__ pM, const float *__restrict__ pL,
                          typename O::storage *__restrict__ out, const FlashDecodingReduceExtConstants &p) {
    __shared__ float sm_m[kWaves], sm_l[kWaves];
    __shared__ float sm_o[kWaves][64];
    const uint32_t P = p.P, Hd = p.Hd;
    const uint64_t slot = blockIdx.x;
    const uint32_t lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const uint32_t d = blockIdx.y * 64 + lane;
    const uint32_t dc = min(d, Hd - 1);  // lanes past Hd read a valid dim and store nothing
    const float *m = pM + slot * P;
    const float *l = pL + slot * P;
    const float *o = pO + slot * P * Hd + dc;
    const uint32_t per = (P + kWaves - 1) / kWaves;
    const uint32_t kBeg = wave * per, kEnd = min(P, kBeg + per);

    float mr = -INFINITY, lr = 0.0f, acc = 0.0f;
    for (uint32_t k0 = kBeg; k0 < kEnd; k0 += kReduceBatch) {
        // entries past the range repeat the last one and are masked below
        const uint32_t kl = min(k0 + (lane % kReduceBatch), kEnd - 1);
        const float mv = m[kl], lv = l[kl];
        float ok[kReduceBatch];
#pragma unroll
        for (int i = 0; i < kReduceBatch; ++i) ok[i] = o[(uint64_t)min(k0 + i, kEnd - 1) * Hd];
        float mk[kReduceBatch];
        float mx = mr;
#pragma unroll
        for (int i = 0; i < kReduceBatch; ++i) {
            mk[i] = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, mv), i));
            if (k0 + i < kEnd) mx = fmaxf(mx, mk[i]);
        }
        // selects, not branches (a branch here lets the compiler sink the O
        // loads below it): while every partition so far is empty, mx = -inf
        // and every weight is 0
        const float a = mr == -INFINITY ? 0.0f : pk::fast_exp(mr - mx);
        acc *= a;
        lr *= a;
#pragma unroll
        for (int i = 0; i < kReduceBatch; ++i) {
            const float e = pk::fast_exp(mk[i] - mx);
            const float b = (k0 + i < kEnd && mk[i] != -INFINITY) ? e : 0.0f;
            acc += ok[i] * b;
            lr += __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, lv), i)) * b;
        }
        mr = mx;
    }
    if (lane == 0) {
        sm_m[wave] = mr;
        sm_l[wave] = lr;
    }
    sm_o[wave][lane] = acc;
    __syncthreads();
    if (wave != 0) return;
    float mstar = -INFINITY;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) mstar = fmaxf(mstar, sm_m[w]);
    float ls = 0.0f, os = 0.0f;
    if (mstar != -INFINITY) {
#pragma unroll
        for (int w = 0; w < kWaves; ++w) {
            const float e = pk::fast_exp(sm_m[w] - mstar);  // 0 for an empty wave (m = -inf)
            ls += e * sm_l[w];
            os += e * sm_o[w][lane];
        }
    }
    if (d < Hd) out[slot * Hd + d] = O::store(ls > 0.0f ? os / ls : 0.0f);
}

// ---- the reference's launch -----------------------------------------------
// One block per (b, hq, partition) for the partial (grid B x Nq x P) and per
// (b, hq) for the combine (grid B x Nq), any block size up to 1024 threads
// (the reference launches 128, FlashDecoding.swift:164, :234), with the
// reference's constants blocks. The partial walks its keys in tiles of
// kRefTile: each thread scores its keys of the tile over the whole head dim,
// the block reduces the tile's max and weight sum in LDS, then each thread
// updates its own dims of O (kept in LDS). Any head dim up to kRefMaxHd.

constexpr uint32_t kRefTile = 128, kRefMaxHd = 512;

__device__ inline uint32_t block_tid() { return threadIdx.x + blockDim.x * (threadIdx.y + blockDim.y * threadIdx.z); }
__device__ inline uint32_t block_size() { return blockDim.x * blockDim.y * blockDim.z; }

// Reduction over every thread of the block; every thread calls it and gets
// the result. buf holds one float per thread.
template <typename Op>
__device__ float block_reduce(float v, float *buf, Op op) {
    const uint32_t tid = block_tid();
    buf[tid] = v;
    __syncthreads();
    for (uint32_t n = block_size(); n > 1;) {
        const uint32_t half = (n + 1) / 2;
        if (tid < n - half) buf[tid] = op(buf[tid], buf[tid + half]);
        __syncthreads();
        n = half;
    }
    const float r = buf[0];
    __syncthreads();
    return r;
}

// The online softmax of one query row over keys [jLo, jHi) of one KV head,
// on the whole block: O (unnormalised) ends in o_sm[0, Hd), the running max
// and sum in m and l (every thread holds them). q_sm holds q * scale.
template <typename TKV>
__device__ void attend_ref(const float *q_sm, const typename TKV::storage *__restrict__ Kh,
                           const typename TKV::storage *__restrict__ Vh, uint32_t Hd, uint32_t jLo, uint32_t jHi, int posQ,
                           uint32_t maskKind, int32_t window, float *o_sm, float *w_sm, float *buf, float &m, float &l) {
    const uint32_t tid = block_tid(), bs = block_size();
    m = -INFINITY;
    l = 0.0f;
    for (uint32_t j0 = jLo; j0 < jHi; j0 += kRefTile) {
        const uint32_t n = min(kRefTile, jHi - j0);
        float tmax = -INFINITY;
        for (uint32_t i = tid; i < n; i += bs) {
            const uint32_t j = j0 + i;
            bool allowed = (maskKind == 2u) | ((int)j <= posQ);
            if (maskKind == 1u) allowed = allowed & ((posQ - (int)j) < window);
            float s = -INFINITY;
            if (allowed) {
                const typename TKV::storage *kr = Kh + (uint64_t)j * Hd;
                float acc = 0.0f;
                for (uint32_t d = 0; d < Hd; ++d) acc += q_sm[d] * TKV::load(kr[d]);
                s = acc;
            }
            w_sm[i] = s;
            tmax = fmaxf(tmax, s);
        }
        tmax = block_reduce(tmax, buf, [](float a, float c) { return fmaxf(a, c); });
        const float m_new = fmaxf(m, tmax);
        if (m_new == -INFINITY) continue;  // no allowed key yet
        const float alpha = pk::fast_exp(m - m_new);
        float ps = 0.0f;
        for (uint32_t i = tid; i < n; i += bs) {
            const float e = w_sm[i] == -INFINITY ? 0.0f : pk::fast_exp(w_sm[i] - m_new);
            w_sm[i] = e;
            ps += e;
        }
        ps = block_reduce(ps, buf, [](float a, float c) { return a + c; });
        l = alpha * l + ps;
        m = m_new;
        for (uint32_t d = tid; d < Hd; d += bs) {
            float o = o_sm[d] * alpha;
            for (uint32_t i = 0; i < n; ++i) o += w_sm[i] * TKV::load(Vh[(uint64_t)(j0 + i) * Hd + d]);
            o_sm[d] = o;
        }
        __syncthreads();
    }
}

template <typename T>
__device__ void fd_partial_ref(const typename T::storage *__restrict__ Q, const typename T::storage *__restrict__ K,
                               const typename T::storage *__restrict__ V, float *__restrict__ pO, float *__restrict__ pM,
                               float *__restrict__ pL, const FlashDecodingPartialConstants &p) {
    __shared__ float q_sm[kRefMaxHd], o_sm[kRefMaxHd], w_sm[kRefTile], buf[1024];
    const uint32_t b = blockIdx.x, hq = blockIdx.y, part = blockIdx.z;
    if (b >= p.B || hq >= p.Nq || part >= p.P || p.Hd > kRefMaxHd || p.Nkv == 0 || p.Nq % p.Nkv != 0) return;
    const uint32_t tid = block_tid(), bs = block_size();
    const uint32_t Hd = p.Hd, Sk = p.Sk, hkv = hq * p.Nkv / p.Nq;
    const uint32_t per = (Sk + p.P - 1) / p.P;
    const uint32_t jLo = min(part * per, Sk), jHi = min(jLo + per, Sk);
    const uint64_t slot = (uint64_t)(b * p.Nq + hq) * p.P + part;
    for (uint32_t d = tid; d < Hd; d += bs) {
        q_sm[d] = T::load(Q[(uint64_t)(b * p.Nq + hq) * Hd + d]) * p.scale;
        o_sm[d] = 0.0f;
    }
    __syncthreads();
    const uint64_t head = (uint64_t)(b * p.Nkv + hkv) * Sk * Hd;
    float m, l;
    // Sq = 1: the query sits at the last key, posQ = Sk - 1
    attend_ref<T>(q_sm, K + head, V + head, Hd, jLo, jHi, (int)Sk - 1, p.maskKind, p.slidingWindow, o_sm, w_sm, buf, m, l);
    for (uint32_t d = tid; d < Hd; d += bs) pO[slot * Hd + d] = o_sm[d];
    if (tid == 0) {
        pM[slot] = m;
        pL[slot] = l;
    }
}

// FlashAttention.metal:30-161 on the reference's launch (FlashAttention.swift:
// 203, :220-222): one block per (b, hq, query row), grid B x Nq x Sq, the row
// attending as position Sk - Sq + q over all Sk keys, O = O / l.
template <typename TQ, typename TKV, typename TO>
__device__ void fa_plain_ref(const typename TQ::storage *__restrict__ Q, const typename TKV::storage *__restrict__ K,
                             const typename TKV::storage *__restrict__ V, typename TO::storage *__restrict__ O,
                             const FlashAttentionConstants &p) {
    __shared__ float q_sm[kRefMaxHd], o_sm[kRefMaxHd], w_sm[kRefTile], buf[1024];
    const uint32_t b = blockIdx.x, hq = blockIdx.y, q = blockIdx.z;
    if (b >= p.B || hq >= p.Nq || q >= p.Sq || p.Hd > kRefMaxHd || p.Nkv == 0 || p.Nq % p.Nkv != 0) return;
    const uint32_t tid = block_tid(), bs = block_size();
    const uint32_t Hd = p.Hd, hkv = hq * p.Nkv / p.Nq;
    const uint64_t row = ((uint64_t)(b * p.Nq + hq) * p.Sq + q) * Hd;
    for (uint32_t d = tid; d < Hd; d += bs) {
        q_sm[d] = TQ::load(Q[row + d]) * p.scale;
        o_sm[d] = 0.0f;
    }
    __syncthreads();
    const uint64_t head = (uint64_t)(b * p.Nkv + hkv) * p.Sk * Hd;
    float m, l;
    attend_ref<TKV>(q_sm, K + head, V + head, Hd, 0, p.Sk, (int)p.Sk - (int)p.Sq + (int)q, p.maskKind, p.slidingWindow,
                    o_sm, w_sm, buf, m, l);
    const float inv = l > 0.0f ? 1.0f / l : 0.0f;
    for (uint32_t d = tid; d < Hd; d += bs) O[row + d] = TO::store(o_sm[d] * inv);
}

// FlashDecoding.metal:202-227 at one block per (b, hq): every thread takes
// the max and the weighted sum over the P partitions, then its dims.
template <typename O>
__device__ void fd_reduce_ref(const float *__restrict__ pO, const float *__restrict__ pM, const float *__restrict__ pL,
                              typename O::storage *__restrict__ out, const FlashDecodingReduceConstants &p) {
    const uint32_t b = blockIdx.x, hq = blockIdx.y;
    if (b >= p.B || hq >= p.Nq) return;
    const uint32_t tid = block_tid(), bs = block_size();
    const uint64_t s0 = (uint64_t)(b * p.Nq + hq) * p.P;
    float mstar = -INFINITY;
    for (uint32_t k = 0; k < p.P; ++k) mstar = fmaxf(mstar, pM[s0 + k]);
    float lstar = 0.0f;
    for (uint32_t k = 0; k < p.P; ++k)
        if (pM[s0 + k] != -INFINITY) lstar += pk::fast_exp(pM[s0 + k] - mstar) * pL[s0 + k];
    for (uint32_t d = tid; d < p.Hd; d += bs) {
        float acc = 0.0f;
        for (uint32_t k = 0; k < p.P; ++k)
            if (pM[s0 + k] != -INFINITY) acc += pk::fast_exp(pM[s0 + k] - mstar) * pO[(s0 + k) * p.Hd + d];
        out[(uint64_t)(b * p.Nq + hq) * p.Hd + d] = O::store(lstar > 0.0f ? acc / lstar : 0.0f);
    }
}

}  // namespace

#define FD_FAST(name, T, LPK, CPL, G, U, NW)                                                               \
    POPCORN_KERNEL void __launch_bounds__(64 * NW)                                                         \
        name(const T::storage *q, const T::storage *k, const T::storage *v, float *pO, float *pM, float *pL, \
             const int32_t *position, FlashDecodingPartialExtConstants p) {                                    \
        fd_partial_fast<T, LPK, CPL, G, U, false, NoFresh, NW>(q, k, v, pO, pM, pL, position, p);           \
    }

#define FD_FRESH(name, T, LPK, CPL, G, U, NW)                                                              \
    POPCORN_KERNEL void __launch_bounds__(64 * NW)                                                         \
        name(const T::storage *qkv, T::storage *k, T::storage *v, float *pO, float *pM, float *pL,          \
             const int32_t *position, const float *wq, const float *wk, const float *invFreq,                \
             FlashDecodingPartialExtConstants p, DecodeAttentionConstants c) {                                 \
        FreshArgs<T> fa{k, v, wq, wk, invFreq, c};                                                          \
        fd_partial_fast<T, LPK, CPL, G, U, true, FreshArgs<T>, NW>(qkv, k, v, pO, pM, pL, position, p, fa);  \
    }

#define FD_GENERIC(name, T)                                                                                 \
    POPCORN_KERNEL void __launch_bounds__(256)                                                             \
        name(const T::storage *q, const T::storage *k, const T::storage *v, float *pO, float *pM, float *pL, \
             const int32_t *position, FlashDecodingPartialExtConstants p) {                                    \
        fd_partial_generic<T>(q, k, v, pO, pM, pL, position, p);                                            \
    }

#define FD_REDUCE(name, O)                                                                                  \
    POPCORN_KERNEL void __launch_bounds__(256)                                                             \
        name(const float *pO, const float *pM, const float *pL, O::storage *out, FlashDecodingReduceExtConstants p) { \
        fd_reduce<O>(pO, pM, pL, out, p);                                                                   \
    }

#define FD_REF(pname, rname, T)                                                                             \
    POPCORN_KERNEL void __launch_bounds__(1024)                                                             \
        pname(const T::storage *q, const T::storage *k, const T::storage *v, float *pO, float *pM, float *pL, \
              FlashDecodingPartialConstants p) {                                                             \
        fd_partial_ref<T>(q, k, v, pO, pM, pL, p);                                                           \
    }                                                                                                        \
    POPCORN_KERNEL void __launch_bounds__(1024)                                                             \
        rname(const float *pO, const float *pM, const float *pL, T::storage *out, FlashDecodingReduceConstants p) { \
        fd_reduce_ref<T>(pO, pM, pL, out, p);                                                                \
    }

using pk::BF16;
using pk::F16;
using pk::F32;

FD_GENERIC(flash_decoding_partial_f32_ext, F32)
FD_GENERIC(flash_decoding_partial_bf16_ext, BF16)
FD_GENERIC(flash_decoding_partial_f16_ext, F16)

FD_REDUCE(flash_decoding_reduce_f32_ext, F32)
FD_REDUCE(flash_decoding_reduce_bf16_ext, BF16)
FD_REDUCE(flash_decoding_reduce_f16_ext, F16)

// FlashAttention.metal:164-167
#define FA_REF(name, TQ, TKV, TO)                                                                           \
    POPCORN_KERNEL void __launch_bounds__(1024)                                                             \
        name(const TQ::storage *q, const TKV::storage *k, const TKV::storage *v, TO::storage *o,           \
             FlashAttentionConstants p) {                                                                   \
        fa_plain_ref<TQ, TKV, TO>(q, k, v, o, p);                                                           \
    }
FA_REF(flash_attention, F32, F32, F32)
FA_REF(flash_attention_bf16, BF16, BF16, BF16)
FA_REF(flash_attention_bf16_to_f32, BF16, BF16, F32)
FA_REF(flash_attention_f32_bf16_to_bf16, F32, BF16, BF16)

FD_REF(flash_decoding_partial_f32, flash_decoding_reduce_f32, F32)
FD_REF(flash_decoding_partial_bf16, flash_decoding_reduce_bf16, BF16)
FD_REF(flash_decoding_partial_f16, flash_decoding_reduce_f16, F16)

// Fast path instantiations: 2-byte types (8 dims per 16B chunk):
// Hd 64 -> LPK 8, Hd 128 -> 16, Hd 256 -> 32, Hd 512 -> 64 (CPL 1).
// f32 (4 dims per chunk): Hd 64 -> LPK 16, 128 -> 32, 256 -> 64, 512 -> 64 with CPL 2.
// U (key rows per lane in flight, each for K and V) shrinks as G grows to keep
// the per-lane state (q, o for G heads) within the register file.
// Each partial kernel has a fresh-key twin (flash_decoding_fresh_*) for the
// decode attention block.
// The 2-byte types also get 8-wave twins (suffix _w8): the host gives them
// half the partitions of the 4-wave kernels, so the grid keeps its waves in
// half as many blocks, each covering twice the keys.
#define FD_W8_ON(T, t, LPK, CPL, G, U)                                                          \
    FD_FAST(flash_decoding_partial_##t##_l##LPK##_c##CPL##_g##G##_w8, T, LPK, CPL, G, U, 8)     \
    FD_FRESH(flash_decoding_fresh_##t##_l##LPK##_c##CPL##_g##G##_w8, T, LPK, CPL, G, U, 8)
#define FD_W8_OFF(T, t, LPK, CPL, G, U)
#define FD_W8_BF16 FD_W8_ON
#define FD_W8_F16 FD_W8_ON
#define FD_W8_F32 FD_W8_OFF
#define FD_W8(T, t, LPK, CPL, G, U) FD_W8_##T(T, t, LPK, CPL, G, U)
#define FD_BOTH(T, t, LPK, CPL, G, U)                                                \
    FD_FAST(flash_decoding_partial_##t##_l##LPK##_c##CPL##_g##G, T, LPK, CPL, G, U, 4)  \
    FD_FRESH(flash_decoding_fresh_##t##_l##LPK##_c##CPL##_g##G, T, LPK, CPL, G, U, 4)  \
    FD_W8(T, t, LPK, CPL, G, U)
#define FD_FAST_G4(T, t, LPK, CPL, U1, U2, U4) \
    FD_BOTH(T, t, LPK, CPL, 1, U1)              \
    FD_BOTH(T, t, LPK, CPL, 2, U2)              \
    FD_BOTH(T, t, LPK, CPL, 4, U4)
#define FD_FAST_G(T, t, LPK, CPL, U1, U2, U4, U8) \
    FD_FAST_G4(T, t, LPK, CPL, U1, U2, U4)         \
    FD_BOTH(T, t, LPK, CPL, 8, U8)

// Head dim 512 stops at G = 4 (the LDS merge buffer is 4 x G x Hd floats).
FD_FAST_G(BF16, bf16, 8, 1, 2, 2, 2, 1)
FD_FAST_G(BF16, bf16, 16, 1, 4, 4, 2, 1)
FD_FAST_G(BF16, bf16, 32, 1, 8, 8, 4, 2)
FD_FAST_G4(BF16, bf16, 64, 1, 8, 8, 4)
FD_FAST_G(F16, f16, 8, 1, 2, 2, 2, 1)
FD_FAST_G(F16, f16, 16, 1, 4, 4, 2, 1)
FD_FAST_G(F16, f16, 32, 1, 8, 8, 4, 2)
FD_FAST_G4(F16, f16, 64, 1, 8, 8, 4)
FD_FAST_G(F32, f32, 16, 1, 2, 2, 2, 1)
FD_FAST_G(F32, f32, 32, 1, 4, 4, 2, 1)
FD_FAST_G(F32, f32, 64, 1, 8, 8, 4, 2)
FD_FAST_G4(F32, f32, 64, 2, 4, 4, 2)
