// Prefill FlashAttention on the matrix cores (the reference's MPP path,
// FlashAttention.swift:236-425 and MPPFlashAttention.metal:38-256, whose
// role this takes; algorithm of FlashAttention.metal:30-167: online softmax
// over key tiles with posQ = Sk - Sq + q, FlashAttention.metal:72).
//
// A block of 4 waves takes 128 query rows of one (batch, query head); wave w
// owns rows q0 + 32 w .. +32. Per step of 32 keys:
//  * the block stages K [32 keys x Hd] row-major and V transposed,
//    Vt [Hd x 32 keys], in LDS;
//  * each wave computes S^T = K . Q^T (32 keys x 32 queries) with
//    v_mfma_f32_32x32x16: A = K rows from LDS, B = Q^T from registers (the
//    wave's Q rows, loaded once). In the C layout (mfma.hpp) lane l then
//    holds the 16 scores of query l % 32 for keys (i / 4) * 8 + (l / 32) * 4
//    + i % 4, so the row max and sum are a lane-local max over 16 values and
//    one exchange with lane l ^ 32;
//  * P^T (in the input dtype; for bf16 as a high part plus a bf16 remainder,
//    two products) is already the B operand of
//    O^T += Vt . P^T for k-step ks if the 16 key slots of the step are read
//    in the order the C layout holds them: slot (l / 32) * 8 + j is key
//    16 ks + (j / 4) * 8 + (l / 32) * 4 + j % 4; Vt rows keep the keys in
//    that order (vt_pos), so the A operand is one 16-byte read. O^T
//    accumulates per lane for one query, so the softmax rescale is
//    lane-local too.
// Causal / sliding-window keys outside the block's range are not visited;
// the rest are masked per query. Heavy (late) query tiles start first.
#include <type_traits>

#include "mfma.hpp"

namespace {

using pk::f32x16;
using pk::Mma;
using pk::u32x4;

constexpr int kWaves = 4;
constexpr int BQ = 32 * kWaves;  // query rows per block
constexpr int BKV = 32;          // keys per step
// How far (natural log) a score may pass a row's reference max before the
// reference moves: softmax weights stay below e^8 ~ 2981 (f16 holds 65504).
constexpr float kRescaleGap = 8.0f;
constexpr float kLog2e = 1.4426950408889634f;
// A buffer offset past every head's range (the host keeps Sk * Hd * 2 below
// 2^31, and a step's scalar offset below that too): the load returns zeros.
// Chunks of a row past the runtime head dim Hd read it, so a kernel compiled
// for HD > Hd multiplies zeros there.
constexpr int kOutOfRange = (int)0x80000000u;

// Partial state handed between the two blocks of a merged pair (pairTiles
// 2). The two blocks may run on different XCDs, whose L2 caches are not
// coherent with each other, so the exchange lives in uncached device memory
// (hipDeviceMallocUncached: every access goes to memory, whatever the
// instruction's cache policy), which the host allocates for it and never
// frees: 16-byte buffer stores and loads for O (with the agent-scope cache
// policy sc1 as well), single-copy atomic 64-bit words for (m, l).
//
// Ready flags: pairFlags[0] is the abort word, pairFlags[1 + tile] the flag
// of split tile `tile`: 0 while idle, the launch's ticket once the first
// block's part is published, kPoison once a merging block gave up on it.
// The first block publishes with a compare-and-swap from 0, so it never
// writes into a poisoned flag; the merging block takes the ticket and resets
// the flag to 0. A merging block whose wait ends without the ticket (0.2 s
// of the 100 MHz clock, or a flag holding anything but 0 or the ticket)
// poisons the flag with a compare-and-swap from 0, writes NaN rows and sets
// the abort word: a producer that publishes late then finds the flag
// poisoned and leaves it, so no later launch with the same ticket (a replayed
// graph) can take a stale part, and every later launch on that flag fails
// the same way until the host, reporting the abort, clears the flags. The
// wait cannot deadlock: the publishing block has the lower index, so it was
// dispatched first, and it waits for nothing.
constexpr int kSc1 = 16;
constexpr uint64_t kPoison = ~0ull;
constexpr uint64_t kWaitTicks = 20000000ull;  // 0.2 s of s_memrealtime (100 MHz)
constexpr uint32_t kFlagPolls = 1u << 22;     // a second bound on the polls
__device__ inline uint64_t ld64c(const void *p) {
    return __hip_atomic_load(reinterpret_cast<uint64_t *>(const_cast<void *>(p)), __ATOMIC_RELAXED,
                             __HIP_MEMORY_SCOPE_AGENT);
}
__device__ inline void st64c(void *p, uint64_t v) {
    __hip_atomic_store(reinterpret_cast<uint64_t *>(p), v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ inline bool cas64c(uint64_t *p, uint64_t &expected, uint64_t v) {
    return __hip_atomic_compare_exchange_strong(p, &expected, v, __ATOMIC_RELAXED, __ATOMIC_RELAXED,
                                                __HIP_MEMORY_SCOPE_AGENT);
}
// The first block of a pair, once every wave's stores of its part have
// completed: the flag goes from 0 to the ticket, or stays as it is.
__device__ inline void pair_publish(uint64_t *pairFlags, uint32_t tile, uint64_t ticket) {
    uint64_t expected = 0;
    (void)cas64c(pairFlags + 1 + tile, expected, ticket);
}
// The merging block (one thread): 1 when the partner's part of this launch
// is there (the flag is then reset to 0), 0 when the wait gave up (the flag
// is then poisoned and the abort word set).
__device__ inline uint32_t pair_take(uint64_t *pairFlags, uint32_t tile, uint64_t ticket) {
    uint64_t *flag = pairFlags + 1 + tile;
    const uint64_t t0 = __builtin_amdgcn_s_memrealtime();
    for (uint32_t i = 0; i < kFlagPolls; ++i) {
        const uint64_t v = ld64c(flag);
        if (v == ticket) {
            st64c(flag, 0u);
            return 1u;
        }
        if (v != 0u || __builtin_amdgcn_s_memrealtime() - t0 > kWaitTicks) break;
        __builtin_amdgcn_s_sleep(2);
    }
    uint64_t expected = 0;
    if (!cas64c(flag, expected, kPoison) && expected == ticket) {  // published meanwhile
        st64c(flag, 0u);
        return 1u;
    }
    st64c(pairFlags, 1u);
    return 0u;
}
// Vt rows hold a step's keys in the order of P^T's key slots (key index
// with bits 2 and 3 swapped): slots 8 h .. 8 h + 7 of k-step ks, which lane
// half h feeds to the product, are keys 16 ks + 4 h + 0..3 and
// 16 ks + 8 + 4 h + 0..3, so a lane's fragment is one 16-byte read. Rows of
// 40 elements (80 bytes) keep those reads 16-byte aligned and spread the
// 16 rows a quarter-wave reads over all 64 banks.
constexpr int LDV = BKV + 8;
__device__ inline uint32_t vt_pos(uint32_t key) { return (key & ~12u) | ((key & 4u) << 1) | ((key & 8u) >> 1); }

// Bitwise, not short-circuit, so a masked step's 16 keys become selects
// rather than 16 branches.
__device__ inline bool fa_allowed(const TiledFlashAttentionConstants &p, int posQ, int key) {
    return (key >= 0) & (key < (int)p.Sk) & ((p.maskKind == 2u) | (key <= posQ)) &
           ((p.maskKind != 1u) | (posQ - key < p.slidingWindow));
}

// Key steps of query tile qt: keys any query of the tile may see.
__device__ inline void fa_key_range(const TiledFlashAttentionConstants &p, uint32_t qt, int &kLo, int &kHi,
                                    uint32_t bq = BQ) {
    const int first = (int)p.Sk - (int)p.Sq + (int)(qt * bq);
    const int last = (int)p.Sk - (int)p.Sq + (int)min(qt * bq + bq - 1, p.Sq - 1);
    kLo = 0;
    kHi = (int)p.Sk;
    if (p.maskKind != 2u) kHi = min(kHi, last + 1);
    if (p.maskKind == 1u) kLo = max(0, first - p.slidingWindow + 1);
}

__device__ inline uint32_t fa_steps(const TiledFlashAttentionConstants &p, uint32_t qt, uint32_t bq = BQ) {
    int kLo, kHi;
    fa_key_range(p, qt, kLo, kHi, bq);
    return kHi > kLo ? (uint32_t)(kHi - kLo + BKV - 1) / BKV : 0u;
}

// Work of a block: one or two items, each a query tile qt over its key
// steps [lo, hi) (counted from the tile's first step), written whole or, for
// a split tile, as part `part` of two (partial O, m, l for the merge kernel).
//
// Without splits (splitFrom >= qTilesPerHead) a block takes one whole tile,
// the heaviest tiles first. With splits and pairTiles (at most one tile per
// CU), a causal head's tiles are paired, light tile a = i with heavy tile
// b = qTilesPerHead - 1 - i, and each pair runs as two blocks of equal work:
// the first takes tile a and the first x steps of tile b, the second the
// rest of tile b, where x makes the two halves of the pair's steps equal
// (pairTiles 2: the first block runs its steps of tile b first and
// publishes their partial state, which the second block merges itself)
// (the host uses this only where x >= 1 for every pair, so the b tiles,
// qt >= splitFrom, are exactly the split ones); an odd tile count leaves the
// middle tile whole, one block. Every block then holds about the mean work,
// so the CUs finish together. With splits and no pairTiles (up to two tiles
// per CU), the tiles from splitFrom on run as two blocks over the halves of
// their key steps and blocks take the items heaviest first (the larger of
// the next split half and the next whole tile), the (batch, head) index
// varying fastest, so the longest items start first on every CU.
struct FaWork {
    uint32_t bh, n;
    uint32_t qt[2], lo[2], hi[2], part[2];
    bool split[2];
};

__device__ inline FaWork fa_work(const TiledFlashAttentionConstants &p, uint32_t bq = BQ, bool whole = false) {
    const uint32_t BH = p.B * p.Nq, nQT = p.qTilesPerHead;
    const uint32_t rank = blockIdx.x / BH;
    FaWork w{};
    w.bh = blockIdx.x % BH;
    w.n = 1;
    if (whole || p.splitFrom >= nQT) {
        w.qt[0] = nQT - 1 - rank;
        w.hi[0] = fa_steps(p, w.qt[0], bq);
        return w;
    }
    if (!p.pairTiles) {
        const uint32_t sf = p.splitFrom, nItems = nQT + (nQT - sf);
        int a = (int)nQT - 1, b = (int)sf - 1;  // next split tile, next whole tile
        uint32_t halves = 2;
        for (uint32_t r = 0; r < nItems; ++r) {
            const bool takeSplit = a >= (int)sf && (b < 0 || (fa_steps(p, a, bq) + 1) / 2 >= fa_steps(p, b, bq));
            if (r == rank) {
                const uint32_t qt = (uint32_t)(takeSplit ? a : b), n = fa_steps(p, qt, bq), half = (n + 1) / 2;
                w.qt[0] = qt;
                w.split[0] = takeSplit;
                w.part[0] = takeSplit ? 2u - halves : 0u;
                w.lo[0] = takeSplit && w.part[0] == 1u ? half : 0u;
                w.hi[0] = takeSplit && w.part[0] == 0u ? half : n;
                break;
            }
            if (takeSplit) {
                if (--halves == 0) {
                    --a;
                    halves = 2;
                }
            } else {
                --b;
            }
        }
        return w;
    }
    const uint32_t pairs = nQT / 2;
    if (rank >= 2 * pairs) {  // the middle tile of an odd count
        w.qt[0] = pairs;
        w.hi[0] = fa_steps(p, pairs, bq);
        return w;
    }
    const uint32_t i = rank >> 1, a = i, bt = nQT - 1 - i;
    const uint32_t sa = fa_steps(p, a, bq), sb = fa_steps(p, bt, bq);
    const uint32_t x = (sa + sb + 1) / 2 - sa;
    if ((rank & 1u) == 0u && p.pairTiles == 2u) {
        // merged in the kernel: the partner's first steps come first, so
        // their partial state is published long before the second block
        // of the pair needs it
        w.n = 2;
        w.qt[0] = bt;
        w.hi[0] = x;
        w.split[0] = true;
        w.qt[1] = a;
        w.hi[1] = sa;
    } else if ((rank & 1u) == 0u) {
        w.n = 2;
        w.qt[0] = a;
        w.hi[0] = sa;
        w.qt[1] = bt;
        w.hi[1] = x;
        w.split[1] = true;
    } else {
        w.qt[0] = bt;
        w.lo[0] = x;
        w.hi[0] = sb;
        w.split[0] = true;
        w.part[0] = 1;
    }
    return w;
}

template <typename T, typename O, int HD>
__device__ void fa_tiled(const uint16_t *__restrict__ Q, const uint16_t *__restrict__ K,
                         const uint16_t *__restrict__ V, typename O::storage *__restrict__ out,
                         float *__restrict__ pO, float *__restrict__ pML, uint64_t *__restrict__ pairFlags,
                         const TiledFlashAttentionConstants &p) {
    constexpr int KS = HD / 16;  // k-steps of S^T = K . Q^T
    constexpr int DT = HD / 32;  // 32-row tiles of O^T
    constexpr int LDK = HD + 8;  // sK row (padded, elements)
    constexpr int kChunks = BKV * HD / 8;
    // softmax weights enter P.V in the input dtype; bf16 (8-bit significand)
    // carries them as a bf16 pair, f16 (11 bits) as one value
    constexpr bool kSplitP = std::is_same<T, pk::BF16>::value;
    // two LDS buffers: step s is multiplied from buffer s & 1 while the next
    // step is written into the other
    __shared__ __attribute__((aligned(16))) uint16_t sK[2][BKV * LDK];
    __shared__ __attribute__((aligned(16))) uint16_t sV[2][HD * LDV];
    __shared__ uint32_t sReady;  // a merged pair's partner state was seen

    const uint32_t lane = threadIdx.x & 63, h = lane >> 5, c32 = lane & 31;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const FaWork work = fa_work(p);
    const uint32_t bh = work.bh;  // b * Nq + hq
    const uint32_t b = bh / p.Nq, hq = bh % p.Nq;
    const uint32_t hkv = hq / (p.Nq / p.Nkv);
    const uint32_t stride = p.kvStride ? p.kvStride : p.Sk;
    const uint32_t D = p.Hd;  // runtime head dim (<= HD, a multiple of 8): rows are D apart
    const uint16_t *Qh = Q + (uint64_t)bh * p.Sq * D;
    const uint64_t kvoff = (uint64_t)(b * p.Nkv + hkv) * stride * D;
    const uint16_t *Kh = K + kvoff;
    const uint16_t *Vh = V + kvoff;
    // the current item's tile, this lane's query row and the wave's first
    uint32_t qt = 0, myq = 0;
    int posQ = 0, posQ0 = 0;
    // scores, m and the rescale gap are kept in log2 units: exp(x) = 2^(x log2 e)
    const float c2 = p.scale * kLog2e;
    u32x4 qf[KS];
    f32x16 acc[DT];
    float m = -INFINITY, l = 0.0f;

    // Staging of one step: K as 16-byte chunks (row-major), V as 4 keys x 8
    // dims per thread so its transpose is written as 8-byte runs of 4 keys.
    // A step's global loads go out before the previous step is computed.
    constexpr int kKC = (kChunks + 64 * kWaves - 1) / (64 * kWaves);
    constexpr int kVP = (BKV / 4) * (HD / 8);  // (key quad, dim block) pairs
    constexpr int kVC = (kVP + 64 * kWaves - 1) / (64 * kWaves);
    // Two register sets take alternate steps, so a step's loads go out two
    // steps before its LDS copy (one step of compute did not cover their
    // latency with every CU loading at once).
    using KRegs = u32x4[kKC];
    using VRegs = u32x4[kVC][4];
    u32x4 krA[kKC], vrA[kVC][4], krB[kKC], vrB[kVC][4];
    // K and V are read through buffer resources over the head's Sk rows
    // (the host keeps Sk * Hd * 2 below 2^31): a row past Sk reads as zeros
    // (its key is masked), the thread's offset within a step is fixed and
    // the step's offset k0 * Hd * 2 goes in the scalar offset, so a step's
    // loads need no address arithmetic.
    const __amdgpu_buffer_rsrc_t rsK = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t *>(Kh), 0,
                                                                          (int)(p.Sk * D * 2), 0x00020000);
    const __amdgpu_buffer_rsrc_t rsV = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t *>(Vh), 0,
                                                                          (int)(p.Sk * D * 2), 0x00020000);
    auto gload = [&](KRegs &kr, VRegs &vr, uint32_t k0) {
        const int so = (int)(k0 * D * 2);
#pragma unroll
        for (int i = 0; i < kKC; ++i) {
            const uint32_t c = threadIdx.x + i * 64 * kWaves;
            if (kChunks % (64 * kWaves) == 0 || c < (uint32_t)kChunks) {
                const uint32_t key = c / (HD / 8), dc = (c % (HD / 8)) * 8;
                const int off = dc < D ? (int)((key * D + dc) * 2) : kOutOfRange;
                kr[i] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rsK, off, so, 0));
            }
        }
#pragma unroll
        for (int i = 0; i < kVC; ++i) {
            const uint32_t pr = threadIdx.x + i * 64 * kWaves;
            if (kVP % (64 * kWaves) == 0 || pr < (uint32_t)kVP) {
                const uint32_t kq = pr % (BKV / 4), db = pr / (BKV / 4);
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const int off = db * 8 < D ? (int)(((4 * kq + j) * D + db * 8) * 2) : kOutOfRange;
                    vr[i][j] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rsV, off, so, 0));
                }
            }
        }
    };
    auto lstore = [&](const KRegs &kr, const VRegs &vr, int buf) {
#pragma unroll
        for (int i = 0; i < kKC; ++i) {
            const uint32_t c = threadIdx.x + i * 64 * kWaves;
            if (kChunks % (64 * kWaves) == 0 || c < (uint32_t)kChunks) {
                const uint32_t key = c / (HD / 8), dc = (c % (HD / 8)) * 8;
                *reinterpret_cast<u32x4 *>(&sK[buf][key * LDK + dc]) = kr[i];
            }
        }
#pragma unroll
        for (int i = 0; i < kVC; ++i) {
            const uint32_t pr = threadIdx.x + i * 64 * kWaves;
            if (kVP % (64 * kWaves) == 0 || pr < (uint32_t)kVP) {
                const uint32_t kq = pr % (BKV / 4), db = pr / (BKV / 4);
                // word j of each key row holds dims 2j (low half) and 2j + 1
                // (high half); v_perm_b32 pairs the halves of two keys
                // (selector bytes 0-3: second operand, 4-7: first)
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const uint32_t a = vr[i][0][j], b = vr[i][1][j], c = vr[i][2][j], e = vr[i][3][j];
                    *reinterpret_cast<uint2 *>(&sV[buf][(db * 8 + 2 * j) * LDV + vt_pos(4 * kq)]) =
                        uint2{__builtin_amdgcn_perm(b, a, 0x05040100u), __builtin_amdgcn_perm(e, c, 0x05040100u)};
                    *reinterpret_cast<uint2 *>(&sV[buf][(db * 8 + 2 * j + 1) * LDV + vt_pos(4 * kq)]) =
                        uint2{__builtin_amdgcn_perm(b, a, 0x07060302u), __builtin_amdgcn_perm(e, c, 0x07060302u)};
                }
            }
        }
    };

    auto compute = [&](uint32_t k0, int buf) {
        // All K fragments of the step are read before the first product (the
        // scheduler otherwise pairs each LDS read with its MFMA and waits on
        // every one); one accumulator chain.
        f32x16 st;
#pragma unroll
        for (int i = 0; i < 16; ++i) st[i] = 0.0f;
        u32x4 kf[KS];
#pragma unroll
        for (int s = 0; s < KS; ++s) kf[s] = *reinterpret_cast<const u32x4 *>(&sK[buf][c32 * LDK + s * 16 + h * 8]);
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int s = 0; s < KS; s += 2) {
            st = Mma<T>::run(kf[s], qf[s], st);
            st = Mma<T>::run(kf[s + 1], qf[s + 1], st);
        }
        // Vt fragments of the whole step, read now so they land while the
        // softmax below runs.
        u32x4 va[DT][2];
#pragma unroll
        for (int dt = 0; dt < DT; ++dt) {
            const uint16_t *vrow = &sV[buf][(dt * 32 + c32) * LDV];
#pragma unroll
            for (int ks = 0; ks < 2; ++ks) va[dt][ks] = *reinterpret_cast<const u32x4 *>(vrow + ks * 16 + h * 8);
        }
        __builtin_amdgcn_sched_barrier(0);
        // The whole step is visible to every row of the wave (keys in
        // range, at or before the wave's first query, inside the window of
        // its last): no per-key test.
        const bool full = (int)k0 + BKV <= (int)p.Sk && (p.maskKind == 2u || (int)k0 + BKV - 1 <= posQ0) &&
                          (p.maskKind != 1u || posQ0 + 31 - (int)k0 < (int)p.slidingWindow);
        // raw scores K.q: the scale (c2 > 0, in log2 units) is applied to the
        // row max and inside the exponent, exp2(s c2 - m)
        float sv[16];
        float mt = -INFINITY;
        if (full) {
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                sv[i] = st[i];
                mt = fmaxf(mt, sv[i]);
            }
        } else {
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                const int key = (int)k0 + (i >> 2) * 8 + (int)h * 4 + (i & 3);
                sv[i] = fa_allowed(p, posQ, key) ? st[i] : -INFINITY;
                mt = fmaxf(mt, sv[i]);
            }
        }
        mt = pk::pair32_max(mt) * c2;
        // Lazy rescaling: a row's reference max m moves only when a score
        // passes it by more than kRescaleGap, so the weights exp(s - m) stay
        // below e^kRescaleGap (inside f16's range) and the rescale of the
        // accumulators, a read-modify-write of all of them, is skipped by
        // every step in which no row of the wave moved.
        const bool move = mt > m + kRescaleGap * kLog2e;  // also when m is still -inf and a key is visible
        float alpha = 1.0f, ps = 0.0f;
        if (move) {
            const float mn = fmaxf(m, mt);
            alpha = __builtin_amdgcn_exp2f(m - mn);
            m = mn;
        }
        if (__ballot(move)) {
            // read-multiply-write in place: a plain `acc *= alpha` makes the
            // compiler carry every accumulator through VGPRs around the loop
            // (128 copies per step, taken or not); this way they stay in AGPRs
#pragma unroll
            for (int dt = 0; dt < DT; ++dt)
#pragma unroll
                for (int i = 0; i < 16; ++i) {
                    float x = acc[dt][i], t;
                    asm volatile("v_accvgpr_read_b32 %1, %0\n\tv_mul_f32 %1, %1, %2\n\tv_accvgpr_write_b32 %0, %1"
                                 : "+a"(x), "=&v"(t)
                                 : "v"(alpha));
                    acc[dt][i] = x;
                }
        }
        // P^T as the B operand: word j of pf[ks] holds the weights of slots
        // ks * 8 + 2j (low half) and + 1; the row sum takes the unrounded
        // weights (the rounding to 16 bits is below the output's precision)
        u32x4 pf[2], pfr[2];
        if (m == -INFINITY) {
#pragma unroll
            for (int ks = 0; ks < 2; ++ks) pf[ks] = pfr[ks] = u32x4{0u, 0u, 0u, 0u};
        } else {
#pragma unroll
            for (int ks = 0; ks < 2; ++ks)
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const int i = ks * 8 + 2 * j;
                    const float p0 = __builtin_amdgcn_exp2f(fmaf(sv[i], c2, -m));
                    const float p1 = __builtin_amdgcn_exp2f(fmaf(sv[i + 1], c2, -m));
                    ps += p0 + p1;
                    const uint32_t w = pk::pack2<T>(p0, p1);
                    pf[ks][j] = w;
                    if constexpr (kSplitP) {
                        // bf16 keeps 8 bits: the remainder goes in a second product
                        pfr[ks][j] = pk::pack2<T>(p0 - __uint_as_float(w << 16), p1 - __uint_as_float(w & 0xffff0000u));
                    } else {
                        pfr[ks][j] = 0u;
                    }
                }
        }
        ps = pk::pair32_sum(ps);
        l = l * alpha + ps;
#pragma unroll
        for (int dt = 0; dt < DT; ++dt) {
#pragma unroll
            for (int ks = 0; ks < 2; ++ks) {
                acc[dt] = Mma<T>::run(va[dt][ks], pf[ks], acc[dt]);
                if constexpr (kSplitP) acc[dt] = Mma<T>::run(va[dt][ks], pfr[ks], acc[dt]);
            }
        }
    };

    auto item = [&](uint32_t w) {
        qt = work.qt[w];
        myq = qt * BQ + wave * 32 + c32;
        posQ = (int)p.Sk - (int)p.Sq + (int)myq;
        posQ0 = (int)p.Sk - (int)p.Sq + (int)(qt * BQ + wave * 32);
        {
            const uint16_t *qrow = Qh + (uint64_t)min(myq, p.Sq - 1) * D + h * 8;
#pragma unroll
            for (int s = 0; s < KS; ++s)
                qf[s] = s * 16 + h * 8 < D ? *reinterpret_cast<const u32x4 *>(qrow + s * 16) : u32x4{0u, 0u, 0u, 0u};
        }
#pragma unroll
        for (int dt = 0; dt < DT; ++dt)
#pragma unroll
            for (int i = 0; i < 16; ++i) acc[dt][i] = 0.0f;
        m = -INFINITY;
        l = 0.0f;

        // keys any query of the tile may see, and the item's steps of them
        int kLo, kHi;
        fa_key_range(p, qt, kLo, kHi);
        const uint32_t nSteps = kHi > kLo ? (uint32_t)(kHi - kLo + BKV - 1) / BKV : 0u;
        const uint32_t itLo = work.lo[w], itHi = min(work.hi[w], nSteps);

        // Step s (counted from itLo) is multiplied from LDS buffer s & 1 and
        // staged through register set A (even s) or B (odd s). Each step: one
        // barrier (it publishes step s, written during step s - 1, and
        // retires the readers of the other buffer), then step s + 1 goes from
        // its registers into the other buffer, those registers take step
        // s + 3, and step s is multiplied: a step's loads go out two steps
        // before its LDS copy. Steps past the range re-read the last one, so
        // every pass issues the same loads.
        if (itLo < itHi) {
            auto kstep = [&](uint32_t it) { return (uint32_t)kLo + min(it, itHi - 1) * BKV; };
            __syncthreads();  // the previous item's readers of both buffers are done
            gload(krA, vrA, kstep(itLo));
            gload(krB, vrB, kstep(itLo + 1));
            lstore(krA, vrA, 0);
            gload(krA, vrA, kstep(itLo + 2));
            // two steps per pass and the odd last step outside the loop, so
            // the loop's back edge always follows the second register set's
            // loads and the wait before each LDS copy leaves the other set's
            // loads in flight
            uint32_t it = itLo;
            for (; it + 1 < itHi; it += 2) {
                __syncthreads();
                lstore(krB, vrB, 1);
                gload(krB, vrB, kstep(it + 3));
                compute(kstep(it), 0);
                __syncthreads();
                lstore(krA, vrA, 0);
                gload(krA, vrA, kstep(it + 4));
                compute(kstep(it + 1), 1);
            }
            if (it < itHi) {
                __syncthreads();
                compute(kstep(it), 0);
            }
        }

        // the lane's 4 consecutive dims d .. d + 3 of each (dt, i4) go out
        // as one store (16 bytes in f32, 8 in 16-bit types): a lane's row is
        // 64 lanes away from its neighbour's, so every element store would
        // be a separate memory transaction; value(dt, e) for accumulator
        // element e of acc[dt]
        auto store_dt = [&](int dt, auto &&value) {
            typename O::storage *orow = out + ((uint64_t)bh * p.Sq + myq) * D;
#pragma unroll
            for (int i4 = 0; i4 < 4; ++i4) {
                const uint32_t d = dt * 32 + i4 * 8 + h * 4;
                if (d >= D) continue;  // padding dims of a kernel compiled for HD > Hd
                const float v0 = value(dt, 4 * i4), v1 = value(dt, 4 * i4 + 1);
                const float v2 = value(dt, 4 * i4 + 2), v3 = value(dt, 4 * i4 + 3);
                if constexpr (std::is_same<O, pk::F32>::value) {
                    *reinterpret_cast<float4 *>(orow + d) = float4{v0, v1, v2, v3};
                } else {
                    auto b16 = [](float x) { return (uint32_t)__builtin_bit_cast(uint16_t, O::store(x)); };
                    *reinterpret_cast<uint2 *>(orow + d) = uint2{b16(v0) | (b16(v1) << 16), b16(v2) | (b16(v3) << 16)};
                }
            }
        };
        if (work.split[w] && p.pairTiles == 2u) {
            // a merged pair, as in fa_tiled16: the first block publishes its
            // part of the split tile and a ready flag, the second merges
            const uint32_t nSplit = p.qTilesPerHead - p.splitFrom;
            const uint32_t tile = bh * nSplit + (qt - p.splitFrom);
            const uint32_t rowsTotal = p.B * p.Nq * nSplit * BQ;
            const uint64_t row = (uint64_t)tile * BQ + wave * 32 + c32;
            const uint64_t ticket = ((uint64_t)p.ticketHi << 32) | p.ticketLo;
            const __amdgpu_buffer_rsrc_t rsO =
                __builtin_amdgcn_make_buffer_rsrc(pO, 0, (int)(rowsTotal * HD * 4u), 0x00020000);
            const int obase = (int)((row * HD + h * 4) * 4);
            if (work.part[w] == 0u) {
                if (myq < p.Sq) {
#pragma unroll
                    for (int dt = 0; dt < DT; ++dt)
#pragma unroll
                        for (int i4 = 0; i4 < 4; ++i4) {
                            const pk::f32x4 v = {acc[dt][4 * i4], acc[dt][4 * i4 + 1], acc[dt][4 * i4 + 2], acc[dt][4 * i4 + 3]};
                            __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, v), rsO,
                                                                   obase + (dt * 32 + i4 * 8) * 4, 0, kSc1);
                        }
                    if (h == 0) st64c(pML + 2 * row, (uint64_t)__float_as_uint(m) | ((uint64_t)__float_as_uint(l) << 32));
                }
                __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0): this wave's stores have completed
                __syncthreads();
                if (threadIdx.x == 0) pair_publish(pairFlags, tile, ticket);
            } else {
                if (threadIdx.x == 0) sReady = pair_take(pairFlags, tile, ticket);
                __syncthreads();
                asm volatile("" ::: "memory");  // the partner's state is read after the flag
                const bool ok = sReady != 0u;
                if (myq < p.Sq) {
                    const uint64_t ml = ld64c(pML + 2 * row);
                    const float m0 = __uint_as_float((uint32_t)ml), l0 = __uint_as_float((uint32_t)(ml >> 32));
                    const float M = fmaxf(m0, m);
                    const float w0 = m0 == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(m0 - M);
                    const float w1 = m == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(m - M);
                    const float L = w0 * l0 + w1 * l;
                    // a wait that gave up gives NaN rows, not stale data
                    const float inv = !ok ? __builtin_nanf("") : (L > 0.0f ? 1.0f / L : 0.0f);
                    // one 32-dim slice at a time (registers: the wave's
                    // accumulators already fill its AGPRs)
#pragma unroll
                    for (int dt = 0; dt < DT; ++dt) {
                        u32x4 oa[4];
#pragma unroll
                        for (int i4 = 0; i4 < 4; ++i4)
                            oa[i4] = __builtin_bit_cast(
                                u32x4, __builtin_amdgcn_raw_buffer_load_b128(rsO, obase + (dt * 32 + i4 * 8) * 4, 0, kSc1));
                        store_dt(dt, [&](int, int e) { return (w0 * __uint_as_float(oa[e / 4][e % 4]) + w1 * acc[dt][e]) * inv; });
                    }
                }
            }
        } else if (myq >= p.Sq) {
            // a row past Sq (ragged last tile) writes nothing
        } else if (work.split[w]) {
            // unnormalised O (f32), and m (log2 units) and l, of this half
            const uint32_t tile = (bh * (p.qTilesPerHead - p.splitFrom) + (qt - p.splitFrom)) * 2u + work.part[w];
            const uint64_t row = (uint64_t)tile * BQ + wave * 32 + c32;
            float *prow = pO + row * HD;
#pragma unroll
            for (int dt = 0; dt < DT; ++dt) {
#pragma unroll
                for (int i4 = 0; i4 < 4; ++i4) {
                    const uint32_t d = dt * 32 + i4 * 8 + h * 4;
                    *reinterpret_cast<float4 *>(prow + d) =
                        float4{acc[dt][4 * i4], acc[dt][4 * i4 + 1], acc[dt][4 * i4 + 2], acc[dt][4 * i4 + 3]};
                }
            }
            if (h == 0) *reinterpret_cast<float2 *>(pML + 2 * row) = float2{m, l};
        } else {
            const float inv = l > 0.0f ? 1.0f / l : 0.0f;
#pragma unroll
            for (int dt = 0; dt < DT; ++dt) store_dt(dt, [&](int, int e) { return acc[dt][e] * inv; });
        }
    };
    item(0);
    if (work.n > 1) item(1);
}

// ---- 16 query rows per wave -------------------------------------------------------
// The same tiles (128 rows), items, masks, lazy rescale and outputs as
// fa_tiled on 8 waves of 16 rows, with v_mfma_f32_16x16x32 (mfma.hpp). A
// wave's output is HD x 16 (HD / 4 accumulators per lane), which keeps a
// wave within 256 registers at Hd 256, so two waves share each SIMD; every
// wave runs the whole step for its own rows. Per step of 32 keys:
//  * S^T = K . Q^T as two 16-key tiles; lane l holds the scores of query
//    l % 16 for keys 4 g + i and 16 + 4 g + i (g = l / 16, i < 4), so the
//    row max and sum run over 8 values and the lanes l, l ^ 16, l ^ 32
//    (v_permlane16_swap, v_permlane32_swap);
//  * those 8 weights, in that order, are the lane's P^T slots 8 g .. 8 g + 7
//    for O^T += Vt . P^T; Vt rows hold the keys in the same slot order
//    (vt16_pos), so a lane's Vt fragment is one 16-byte read;
//  * K rows in LDS keep 16-byte chunk c of row r in slot c ^ (r % chunks),
//    so the 16 rows a quarter-wave reads fall in 16 distinct bank groups.

__device__ inline uint32_t vt16_pos(uint32_t key) {
    return key < 16u ? (key >> 2) * 8u + (key & 3u) : ((key - 16u) >> 2) * 8u + 4u + (key & 3u);
}
__device__ inline float quad16_max(float v) { return pk::pair32_max(pk::pair16_max(v)); }
__device__ inline float quad16_sum(float v) { return pk::pair32_sum(pk::pair16_sum(v)); }

template <typename T, typename O, int HD, int NW>
__device__ void fa_tiled16(const uint16_t *__restrict__ Q, const uint16_t *__restrict__ K,
                           const uint16_t *__restrict__ V, typename O::storage *__restrict__ out,
                           float *__restrict__ pO, float *__restrict__ pML, uint64_t *__restrict__ pairFlags,
                           const TiledFlashAttentionConstants &p) {
    constexpr int KS = HD / 32;   // k-steps of each S^T tile
    constexpr int DT = HD / 16;   // 16-row tiles of O^T
    constexpr int CH = HD / 8;    // 16-byte chunks per K row
    constexpr int kThreads = 64 * NW;
    constexpr uint32_t BQ16 = 16 * NW;  // query rows per block
    constexpr bool kSplitP = std::is_same<T, pk::BF16>::value;
    static_assert(CH >= 16, "the K swizzle needs 16 chunks per row");
    __shared__ __attribute__((aligned(16))) uint16_t sK[2][BKV * HD];
    __shared__ __attribute__((aligned(16))) uint16_t sV[2][HD * LDV];
    __shared__ uint32_t sReady;  // a merged pair's partner state was seen

    const uint32_t lane = threadIdx.x & 63, g = lane >> 4, c16 = lane & 15;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    // Hd 512 runs every tile whole, one block each (no split or paired tiles:
    // the merge paths' extra registers would spill)
    constexpr bool kSplits = HD < 512;
    const FaWork work = fa_work(p, BQ16, !kSplits);
    const uint32_t bh = work.bh;
    const uint32_t b = bh / p.Nq, hq = bh % p.Nq;
    const uint32_t hkv = hq / (p.Nq / p.Nkv);
    const uint32_t stride = p.kvStride ? p.kvStride : p.Sk;
    const uint32_t D = p.Hd;  // runtime head dim (<= HD, a multiple of 8): rows are D apart
    const uint16_t *Qh = Q + (uint64_t)bh * p.Sq * D;
    const uint64_t kvoff = (uint64_t)(b * p.Nkv + hkv) * stride * D;
    uint32_t qt = 0, myq = 0;
    int posQ = 0, posQ0 = 0;
    const float c2 = p.scale * kLog2e;
    u32x4 qf[KS];
    pk::f32x4 acc[DT];
    float m = -INFINITY, l = 0.0f;

    // Staging: K as 16-byte chunks (thread t takes chunks t + i kThreads),
    // V as two consecutive keys x 8 dims per (key pair, dim block), written
    // transposed as 32-bit words of two keys. Rows past Sk read as zeros.
    constexpr int kKC = (BKV * CH + kThreads - 1) / kThreads;
    constexpr int kVP = (BKV / 2) * (HD / 8);
    constexpr int kVC = (kVP + kThreads - 1) / kThreads;
    using KRegs = u32x4[kKC];
    using VRegs = u32x4[kVC][2];
    constexpr bool kOneSet = HD >= 512;
    u32x4 krA[kKC], vrA[kVC][2], krB[kOneSet ? 1 : kKC], vrB[kOneSet ? 1 : kVC][2];
    const __amdgpu_buffer_rsrc_t rsK = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t *>(K + kvoff), 0,
                                                                          (int)(p.Sk * D * 2), 0x00020000);
    const __amdgpu_buffer_rsrc_t rsV = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t *>(V + kvoff), 0,
                                                                          (int)(p.Sk * D * 2), 0x00020000);
    auto gload = [&](KRegs &kr, VRegs &vr, uint32_t k0) {
        const int so = (int)(k0 * D * 2);
#pragma unroll
        for (int i = 0; i < kKC; ++i) {
            const uint32_t c = threadIdx.x + i * kThreads;
            if ((BKV * CH) % kThreads == 0 || c < (uint32_t)(BKV * CH)) {
                const uint32_t key = c / CH, ch = c % CH;
                const int off = ch * 8 < D ? (int)((key * D + ch * 8) * 2) : kOutOfRange;
                kr[i] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rsK, off, so, 0));
            }
        }
#pragma unroll
        for (int i = 0; i < kVC; ++i) {
            const uint32_t pr = threadIdx.x + i * kThreads;
            if (kVP % kThreads == 0 || pr < (uint32_t)kVP) {
                const uint32_t kp = pr % (BKV / 2), db = pr / (BKV / 2);
#pragma unroll
                for (int j = 0; j < 2; ++j) {
                    const int off = db * 8 < D ? (int)(((2 * kp + j) * D + db * 8) * 2) : kOutOfRange;
                    vr[i][j] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rsV, off, so, 0));
                }
            }
        }
    };
    auto lstore = [&](const KRegs &kr, const VRegs &vr, int buf) {
#pragma unroll
        for (int i = 0; i < kKC; ++i) {
            const uint32_t c = threadIdx.x + i * kThreads;
            if ((BKV * CH) % kThreads == 0 || c < (uint32_t)(BKV * CH)) {
                const uint32_t key = c / CH, ch = c % CH;
                *reinterpret_cast<u32x4 *>(&sK[buf][key * HD + ((ch ^ (key % CH)) * 8)]) = kr[i];
            }
        }
#pragma unroll
        for (int i = 0; i < kVC; ++i) {
            const uint32_t pr = threadIdx.x + i * kThreads;
            if (kVP % kThreads == 0 || pr < (uint32_t)kVP) {
                const uint32_t kp = pr % (BKV / 2), db = pr / (BKV / 2);
                const uint32_t at = vt16_pos(2 * kp);
                // word j of a key row holds dims 2j (low half) and 2j + 1
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const uint32_t a = vr[i][0][j], e = vr[i][1][j];
                    *reinterpret_cast<uint32_t *>(&sV[buf][(db * 8 + 2 * j) * LDV + at]) = __builtin_amdgcn_perm(e, a, 0x05040100u);
                    *reinterpret_cast<uint32_t *>(&sV[buf][(db * 8 + 2 * j + 1) * LDV + at]) = __builtin_amdgcn_perm(e, a, 0x07060302u);
                }
            }
        }
    };

    auto compute = [&](uint32_t k0, int buf) {
        pk::f32x4 st[2];
#pragma unroll
        for (int mt = 0; mt < 2; ++mt) {
            st[mt] = pk::f32x4{0.0f, 0.0f, 0.0f, 0.0f};
            const uint32_t row = mt * 16 + c16;
            // K fragments four at a time (registers: two waves share a SIMD)
#pragma unroll
            for (int s0 = 0; s0 < KS; s0 += 4) {
                u32x4 kf[4];
#pragma unroll
                for (int s = 0; s < 4; ++s)
                    kf[s] = *reinterpret_cast<const u32x4 *>(&sK[buf][row * HD + ((((s0 + s) * 4 + g) ^ (row % CH)) * 8)]);
#pragma unroll
                for (int s = 0; s < 4; ++s) st[mt] = pk::Mma16<T>::run(kf[s], qf[s0 + s], st[mt]);
            }
        }
        const bool full = (int)k0 + BKV <= (int)p.Sk && (p.maskKind == 2u || (int)k0 + BKV - 1 <= posQ0) &&
                          (p.maskKind != 1u || posQ0 + 15 - (int)k0 < (int)p.slidingWindow);
        // one uniform branch per step: a step every row of the wave sees
        // takes the scores as they are, the others mask each key
        float sv[8];
        float mx = -INFINITY;
        if (full) {
#pragma unroll
            for (int mt = 0; mt < 2; ++mt)
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    sv[mt * 4 + i] = st[mt][i];
                    mx = fmaxf(mx, sv[mt * 4 + i]);
                }
        } else {
#pragma unroll
            for (int mt = 0; mt < 2; ++mt)
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const int key = (int)k0 + mt * 16 + (int)g * 4 + i;
                    sv[mt * 4 + i] = fa_allowed(p, posQ, key) ? st[mt][i] : -INFINITY;
                    mx = fmaxf(mx, sv[mt * 4 + i]);
                }
        }
        mx = quad16_max(mx) * c2;
        const bool move = mx > m + kRescaleGap * kLog2e;
        float alpha = 1.0f, ps = 0.0f;
        if (move) {
            const float mn = fmaxf(m, mx);
            alpha = __builtin_amdgcn_exp2f(m - mn);
            m = mn;
        }
        if (__ballot(move)) {
            // the accumulators stay in VGPRs here (a wave's 256 registers
            // hold all of its state), so a plain multiply
#pragma unroll
            for (int dt = 0; dt < DT; ++dt) acc[dt] *= alpha;
        }
        u32x4 pf, pfr;
        if (m == -INFINITY) {
            pf = pfr = u32x4{0u, 0u, 0u, 0u};
        } else {
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const float p0 = __builtin_amdgcn_exp2f(fmaf(sv[2 * j], c2, -m));
                const float p1 = __builtin_amdgcn_exp2f(fmaf(sv[2 * j + 1], c2, -m));
                ps += p0 + p1;
                const uint32_t w = pk::pack2<T>(p0, p1);
                pf[j] = w;
                if constexpr (kSplitP) {
                    pfr[j] = pk::pack2<T>(p0 - __uint_as_float(w << 16), p1 - __uint_as_float(w & 0xffff0000u));
                } else {
                    pfr[j] = 0u;
                }
            }
        }
        l = l * alpha + quad16_sum(ps);
#pragma unroll
        for (int dt = 0; dt < DT; ++dt) {
            const u32x4 va = *reinterpret_cast<const u32x4 *>(&sV[buf][(dt * 16 + c16) * LDV + g * 8]);
            acc[dt] = pk::Mma16<T>::run(va, pf, acc[dt]);
            if constexpr (kSplitP) acc[dt] = pk::Mma16<T>::run(va, pfr, acc[dt]);
        }
    };

    auto item = [&](uint32_t w) {
        qt = work.qt[w];
        myq = qt * BQ16 + wave * 16 + c16;
        posQ = (int)p.Sk - (int)p.Sq + (int)myq;
        posQ0 = (int)p.Sk - (int)p.Sq + (int)(qt * BQ16 + wave * 16);
        {
            const uint16_t *qrow = Qh + (uint64_t)min(myq, p.Sq - 1) * D + g * 8;
#pragma unroll
            for (int s = 0; s < KS; ++s)
                qf[s] = s * 32 + g * 8 < D ? *reinterpret_cast<const u32x4 *>(qrow + s * 32) : u32x4{0u, 0u, 0u, 0u};
        }
#pragma unroll
        for (int dt = 0; dt < DT; ++dt) acc[dt] = pk::f32x4{0.0f, 0.0f, 0.0f, 0.0f};
        m = -INFINITY;
        l = 0.0f;
        int kLo, kHi;
        fa_key_range(p, qt, kLo, kHi, BQ16);
        const uint32_t nSteps = kHi > kLo ? (uint32_t)(kHi - kLo + BKV - 1) / BKV : 0u;
        const uint32_t itLo = work.lo[w], itHi = min(work.hi[w], nSteps);
        // the double-buffered loop of fa_tiled: one barrier per step, a
        // step's loads two steps ahead of its LDS copy
        if constexpr (kOneSet) {
          if (itLo < itHi) {
            // one register set (Hd 512: a step's products take twice as
            // long, and the second set would not fit the registers): a
            // step's loads go out one step before its LDS copy
            auto kstep = [&](uint32_t it) { return (uint32_t)kLo + min(it, itHi - 1) * BKV; };
            __syncthreads();
            gload(krA, vrA, kstep(itLo));
            lstore(krA, vrA, 0);
            gload(krA, vrA, kstep(itLo + 1));
            uint32_t it = itLo;
            for (; it + 1 < itHi; it += 2) {
                __syncthreads();
                lstore(krA, vrA, 1);
                gload(krA, vrA, kstep(it + 2));
                compute(kstep(it), 0);
                __syncthreads();
                lstore(krA, vrA, 0);
                gload(krA, vrA, kstep(it + 3));
                compute(kstep(it + 1), 1);
            }
            if (it < itHi) {
                __syncthreads();
                compute(kstep(it), 0);
            }
          }
        } else if (itLo < itHi) {
            auto kstep = [&](uint32_t it) { return (uint32_t)kLo + min(it, itHi - 1) * BKV; };
            __syncthreads();
            gload(krA, vrA, kstep(itLo));
            gload(krB, vrB, kstep(itLo + 1));
            lstore(krA, vrA, 0);
            gload(krA, vrA, kstep(itLo + 2));
            // two steps per pass and the odd last step outside the loop, so
            // the loop's back edge always follows the second register set's
            // loads and the wait before each LDS copy leaves the other set's
            // loads in flight
            uint32_t it = itLo;
            for (; it + 1 < itHi; it += 2) {
                __syncthreads();
                lstore(krB, vrB, 1);
                gload(krB, vrB, kstep(it + 3));
                compute(kstep(it), 0);
                __syncthreads();
                lstore(krA, vrA, 0);
                gload(krA, vrA, kstep(it + 4));
                compute(kstep(it + 1), 1);
            }
            if (it < itHi) {
                __syncthreads();
                compute(kstep(it), 0);
            }
        }

        // this lane's 4 consecutive dims of each 16-dim slice of its row,
        // value(dt, i) for dim dt * 16 + 4 g + i
        auto store_out = [&](auto &&value) {
            typename O::storage *orow = out + ((uint64_t)bh * p.Sq + myq) * D;
#pragma unroll
            for (int dt = 0; dt < DT; ++dt) {
                const uint32_t d = dt * 16 + g * 4;
                if (d >= D) continue;  // padding dims of a kernel compiled for HD > Hd
                const float v0 = value(dt, 0), v1 = value(dt, 1), v2 = value(dt, 2), v3 = value(dt, 3);
                if constexpr (std::is_same<O, pk::F32>::value) {
                    *reinterpret_cast<float4 *>(orow + d) = float4{v0, v1, v2, v3};
                } else {
                    auto b16 = [](float x) { return (uint32_t)__builtin_bit_cast(uint16_t, O::store(x)); };
                    *reinterpret_cast<uint2 *>(orow + d) = uint2{b16(v0) | (b16(v1) << 16), b16(v2) | (b16(v3) << 16)};
                }
            }
        };
        if (kSplits && work.split[w] && p.pairTiles == 2u) {
            // A merged pair: the first block publishes its part of the split
            // tile (unnormalised O, then (m, l) per row, then the tile's
            // ready flag, set to this launch's ticket once every wave's
            // stores have completed); the second waits for the flag, resets
            // it for the next launch and combines the published part with
            // its own, as fa_split_merge does.
            const uint32_t nSplit = p.qTilesPerHead - p.splitFrom;
            const uint32_t tile = bh * nSplit + (qt - p.splitFrom);
            const uint32_t rowsTotal = p.B * p.Nq * nSplit * BQ16;
            const uint64_t row = (uint64_t)tile * BQ16 + wave * 16 + c16;
            const uint64_t ticket = ((uint64_t)p.ticketHi << 32) | p.ticketLo;
            const __amdgpu_buffer_rsrc_t rsO =
                __builtin_amdgcn_make_buffer_rsrc(pO, 0, (int)(rowsTotal * HD * 4u), 0x00020000);
            const int obase = (int)((row * HD + g * 4) * 4);
            if (work.part[w] == 0u) {
                if (myq < p.Sq) {
#pragma unroll
                    for (int dt = 0; dt < DT; ++dt)
                        __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, acc[dt]), rsO, obase + dt * 64, 0, kSc1);
                    if (g == 0) st64c(pML + 2 * row, (uint64_t)__float_as_uint(m) | ((uint64_t)__float_as_uint(l) << 32));
                }
                __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0): this wave's stores have completed
                __syncthreads();
                if (threadIdx.x == 0) pair_publish(pairFlags, tile, ticket);
            } else {
                if (threadIdx.x == 0) sReady = pair_take(pairFlags, tile, ticket);
                __syncthreads();
                asm volatile("" ::: "memory");  // the partner's state is read after the flag
                const bool ok = sReady != 0u;
                if (myq < p.Sq) {
                    u32x4 oa[DT];
#pragma unroll
                    for (int dt = 0; dt < DT; ++dt)
                        oa[dt] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rsO, obase + dt * 64, 0, kSc1));
                    const uint64_t ml = ld64c(pML + 2 * row);
                    const float m0 = __uint_as_float((uint32_t)ml), l0 = __uint_as_float((uint32_t)(ml >> 32));
                    const float M = fmaxf(m0, m);
                    const float w0 = m0 == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(m0 - M);
                    const float w1 = m == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(m - M);
                    const float L = w0 * l0 + w1 * l;
                    // a wait that gave up gives NaN rows, not stale data
                    const float inv = !ok ? __builtin_nanf("") : (L > 0.0f ? 1.0f / L : 0.0f);
                    store_out([&](int dt, int i) { return (w0 * __uint_as_float(oa[dt][i]) + w1 * acc[dt][i]) * inv; });
                }
            }
        } else if (myq >= p.Sq) {
            // a row past Sq (ragged last tile) writes nothing
        } else if (kSplits && work.split[w]) {
            const uint32_t tile = (bh * (p.qTilesPerHead - p.splitFrom) + (qt - p.splitFrom)) * 2u + work.part[w];
            const uint64_t row = (uint64_t)tile * BQ16 + wave * 16 + c16;
            float *prow = pO + row * HD;
#pragma unroll
            for (int dt = 0; dt < DT; ++dt)
                *reinterpret_cast<float4 *>(prow + dt * 16 + g * 4) = float4{acc[dt][0], acc[dt][1], acc[dt][2], acc[dt][3]};
            if (g == 0) *reinterpret_cast<float2 *>(pML + 2 * row) = float2{m, l};
        } else {
            const float inv = l > 0.0f ? 1.0f / l : 0.0f;
            store_out([&](int dt, int i) { return acc[dt][i] * inv; });
        }
    };
    item(0);
    if (work.n > 1) item(1);
}

// ---- f32 Q, K, V --------------------------------------------------------------------
// The reference's mpp_flash_attention_f32 (FlashAttention.swift:368-376,
// MPPFlashAttention.metal:251-256) on v_mfma_f32_16x16x4_f32, whose
// operands are single floats (lane l: A[l % 16][l / 16], B[l / 16][l % 16];
// C rows 4 (l / 16) + i, column l % 16). The masks and lazy rescale are the
// 16-bit kernels'; a block of 4 waves takes a whole tile of 64 query rows,
// a wave 16 of them, and a step 16 keys. Per step:
//  * S^T = K . Q^T (16 keys x 16 queries) in HD / 4 products; product
//    4 j + s takes dim 16 j + 4 (l / 16) + s from every lane, so a lane
//    feeds four consecutive products from one 16-byte K read (LDS) and one
//    16-byte chunk of its Q row (registers);
//  * lane l then holds the scores of query l % 16 for keys 4 (l / 16) + i;
//    ordering the keys of product s of P.V as 4 (l / 16) + s makes score s
//    the lane's own B operand, and the A operand V^T[dim][4 (l / 16) + s]
//    one 16-byte read of a Vt row for the four products.
// LDS rows are padded (K by 4 floats, Vt to 20) so the 16 rows a
// quarter-wave reads fall in distinct banks. Dims past the runtime Hd (a
// multiple of 4) and keys past Sk read as zeros (buffer loads out of range).
template <int HD, int NW, bool ZIGZAG>
__device__ void fa_tiled_f32(const float *__restrict__ Q, const float *__restrict__ K, const float *__restrict__ V,
                             float *__restrict__ out, const TiledFlashAttentionConstants &p) {
    constexpr int BK = 16;          // keys per step
    constexpr int DC = HD / 16;     // 16-byte chunks of a lane's Q row, and 16-dim tiles of O^T
    constexpr int LDK = HD + 4;     // sK row stride (floats)
    constexpr int LDT = BK + 4;     // sV (transposed: a row per dim) row stride
    constexpr int kThreads = 64 * NW;
    constexpr uint32_t BQ16 = 16 * NW;  // query rows per block
    constexpr int kChunks = BK * HD / 4;  // 16-byte chunks of K (and of V) per step
    constexpr int kC = (kChunks + kThreads - 1) / kThreads;
    constexpr bool kOneSet = HD >= 512;
    __shared__ __attribute__((aligned(16))) float sK[2][BK * LDK];
    __shared__ __attribute__((aligned(16))) float sV[2][HD * LDT];

    const uint32_t lane = threadIdx.x & 63, g = lane >> 4, c16 = lane & 15;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    // Tile of the block: the (batch, head) index varies fastest; by rank,
    // heaviest first, or (ZIGZAG) the heavy half heaviest first and then the
    // light half lightest first, so ranks r and r + half see a constant
    // number of keys together. With two blocks per CU (Hd <= 256) this
    // measured 30-38% faster at 16 heads x 2048 tokens (Hd 64-256) than one
    // 128-row tile per CU heaviest first, whose heaviest tiles, twice the
    // mean keys, set the time.
    const uint32_t BH = p.B * p.Nq, nQT = p.qTilesPerHead;
    const uint32_t bh = blockIdx.x % BH, rank = blockIdx.x / BH;
    const uint32_t half = (nQT + 1) / 2;
    const uint32_t qt = !ZIGZAG || rank < half ? nQT - 1 - rank : rank - half;
    const uint32_t b = bh / p.Nq, hq = bh % p.Nq;
    const uint32_t hkv = hq / (p.Nq / p.Nkv);
    const uint32_t stride = p.kvStride ? p.kvStride : p.Sk;
    const uint32_t D = p.Hd;
    const uint64_t kvoff = (uint64_t)(b * p.Nkv + hkv) * stride * D;
    const uint32_t myq = qt * BQ16 + wave * 16 + c16;
    const int posQ = (int)p.Sk - (int)p.Sq + (int)myq;
    const int posQ0 = (int)p.Sk - (int)p.Sq + (int)(qt * BQ16 + wave * 16);
    const float c2 = p.scale * kLog2e;

    using Regs = u32x4[kC];
    Regs krA, vrA, krB, vrB;
    const __amdgpu_buffer_rsrc_t rsK = __builtin_amdgcn_make_buffer_rsrc(const_cast<float *>(K + kvoff), 0,
                                                                          (int)(p.Sk * D * 4), 0x00020000);
    const __amdgpu_buffer_rsrc_t rsV = __builtin_amdgcn_make_buffer_rsrc(const_cast<float *>(V + kvoff), 0,
                                                                          (int)(p.Sk * D * 4), 0x00020000);
    // K chunk c: key c / (HD / 4), dims 4 (c % (HD / 4)) ..; V chunk c: key
    // c % 16, dims 4 (c / 16) .. (a wave's transposed stores then cover 64
    // distinct banks). The step's first key is part of the vector offset,
    // which the range check covers: keys past Sk read as zeros.
    auto gload = [&](Regs &kr, Regs &vr, uint32_t k0) {
#pragma unroll
        for (int i = 0; i < kC; ++i) {
            const uint32_t c = threadIdx.x + i * kThreads;
            if (kChunks % kThreads == 0 || c < (uint32_t)kChunks) {
                const uint32_t kk = c / (HD / 4), kd = (c % (HD / 4)) * 4;
                const uint32_t vk = c % BK, vd = (c / BK) * 4;
                const int ko = kd < D ? (int)(((k0 + kk) * D + kd) * 4) : kOutOfRange;
                const int vo = vd < D ? (int)(((k0 + vk) * D + vd) * 4) : kOutOfRange;
                kr[i] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rsK, ko, 0, 0));
                vr[i] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rsV, vo, 0, 0));
            }
        }
    };
    auto lstore = [&](const Regs &kr, const Regs &vr, int buf) {
#pragma unroll
        for (int i = 0; i < kC; ++i) {
            const uint32_t c = threadIdx.x + i * kThreads;
            if (kChunks % kThreads == 0 || c < (uint32_t)kChunks) {
                const uint32_t kk = c / (HD / 4), kd = (c % (HD / 4)) * 4;
                const uint32_t vk = c % BK, vd = (c / BK) * 4;
                *reinterpret_cast<u32x4 *>(&sK[buf][kk * LDK + kd]) = kr[i];
#pragma unroll
                for (int e = 0; e < 4; ++e) sV[buf][(vd + e) * LDT + vk] = __uint_as_float(vr[i][e]);
            }
        }
    };

    pk::f32x4 qf[DC], acc[DC];
    {
        const float *qrow = Q + ((uint64_t)bh * p.Sq + min(myq, p.Sq - 1)) * D + g * 4;
#pragma unroll
        for (int j = 0; j < DC; ++j)
            qf[j] = j * 16 + g * 4 < D ? *reinterpret_cast<const pk::f32x4 *>(qrow + j * 16) : pk::f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    }
#pragma unroll
    for (int dt = 0; dt < DC; ++dt) acc[dt] = pk::f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    float m = -INFINITY, l = 0.0f;
    auto compute = [&](uint32_t k0, int buf) {
        pk::f32x4 st = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int j = 0; j < DC; ++j) {
            const pk::f32x4 kf = *reinterpret_cast<const pk::f32x4 *>(&sK[buf][c16 * LDK + j * 16 + g * 4]);
#pragma unroll
            for (int s = 0; s < 4; ++s) st = __builtin_amdgcn_mfma_f32_16x16x4f32(kf[s], qf[j][s], st, 0, 0, 0);
        }
        const bool full = (int)k0 + BK <= (int)p.Sk && (p.maskKind == 2u || (int)k0 + BK - 1 <= posQ0) &&
                          (p.maskKind != 1u || posQ0 + 15 - (int)k0 < (int)p.slidingWindow);
        float sv[4];
        float mx = -INFINITY;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            sv[i] = full || fa_allowed(p, posQ, (int)k0 + (int)g * 4 + i) ? st[i] : -INFINITY;
            mx = fmaxf(mx, sv[i]);
        }
        mx = quad16_max(mx) * c2;
        const bool move = mx > m + kRescaleGap * kLog2e;
        float alpha = 1.0f;
        if (move) {
            const float mn = fmaxf(m, mx);
            alpha = __builtin_amdgcn_exp2f(m - mn);
            m = mn;
        }
        if (__ballot(move)) {
#pragma unroll
            for (int dt = 0; dt < DC; ++dt) acc[dt] *= alpha;
        }
        float pv[4], ps = 0.0f;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            pv[i] = m == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(fmaf(sv[i], c2, -m));
            ps += pv[i];
        }
        l = l * alpha + quad16_sum(ps);
#pragma unroll
        for (int dt = 0; dt < DC; ++dt) {
            const pk::f32x4 va = *reinterpret_cast<const pk::f32x4 *>(&sV[buf][(dt * 16 + c16) * LDT + g * 4]);
#pragma unroll
            for (int s = 0; s < 4; ++s) acc[dt] = __builtin_amdgcn_mfma_f32_16x16x4f32(va[s], pv[s], acc[dt], 0, 0, 0);
        }
    };

    int kLo, kHi;
    fa_key_range(p, qt, kLo, kHi, BQ16);
    const uint32_t nSteps = kHi > kLo ? (uint32_t)(kHi - kLo + BK - 1) / BK : 0u;
    // the double-buffered loop of the 16-bit kernels: one barrier per step;
    // a step's loads go out two steps (one at Hd 512, one register set)
    // before its LDS copy
    if (nSteps > 0) {
        auto kstep = [&](uint32_t it) { return (uint32_t)kLo + min(it, nSteps - 1) * BK; };
        uint32_t it = 0;
        if constexpr (kOneSet) {
            gload(krA, vrA, kstep(0));
            lstore(krA, vrA, 0);
            gload(krA, vrA, kstep(1));
            for (; it + 1 < nSteps; it += 2) {
                __syncthreads();
                lstore(krA, vrA, 1);
                gload(krA, vrA, kstep(it + 2));
                compute(kstep(it), 0);
                __syncthreads();
                lstore(krA, vrA, 0);
                gload(krA, vrA, kstep(it + 3));
                compute(kstep(it + 1), 1);
            }
        } else {
            gload(krA, vrA, kstep(0));
            gload(krB, vrB, kstep(1));
            lstore(krA, vrA, 0);
            gload(krA, vrA, kstep(2));
            for (; it + 1 < nSteps; it += 2) {
                __syncthreads();
                lstore(krB, vrB, 1);
                gload(krB, vrB, kstep(it + 3));
                compute(kstep(it), 0);
                __syncthreads();
                lstore(krA, vrA, 0);
                gload(krA, vrA, kstep(it + 4));
                compute(kstep(it + 1), 1);
            }
        }
        if (it < nSteps) {
            __syncthreads();
            compute(kstep(it), 0);
        }
    }
    if (myq >= p.Sq) return;  // a row past Sq (ragged last tile) writes nothing
    const float inv = l > 0.0f ? 1.0f / l : 0.0f;
    float *orow = out + ((uint64_t)bh * p.Sq + myq) * D;
#pragma unroll
    for (int dt = 0; dt < DC; ++dt) {
        const uint32_t d = dt * 16 + g * 4;
        if (d < D) *reinterpret_cast<float4 *>(orow + d) = float4{acc[dt][0] * inv, acc[dt][1] * inv, acc[dt][2] * inv, acc[dt][3] * inv};
    }
}

// Combine of a split tile's two halves (maxima in log2 units):
//   M = max(m0, m1), w_i = 2^(m_i - M) (0 for a half with no visible key),
//   O = (w0 O0 + w1 O1) / (w0 l0 + w1 l1),
// the log-sum-exp combine of FlashDecoding.metal:202-227 for two partitions.
// One block per 16 rows of a split tile; a thread takes 4 dims of a row.
constexpr int kMergeRows = 16;

template <typename O, int HD>
__device__ void fa_split_merge(const float *__restrict__ pO, const float *__restrict__ pML,
                               typename O::storage *__restrict__ out, const TiledFlashAttentionConstants &p) {
    const uint32_t nSplit = p.qTilesPerHead - p.splitFrom;
    const uint32_t tile = blockIdx.x / (BQ / kMergeRows);  // bh * nSplit + (qt - splitFrom)
    const uint32_t r0 = blockIdx.x % (BQ / kMergeRows) * kMergeRows;
    const uint32_t bh = tile / nSplit, qt = p.splitFrom + tile % nSplit;
    constexpr uint32_t kPerRow = HD / 4;
    for (uint32_t idx = threadIdx.x; idx < (uint32_t)kMergeRows * kPerRow; idx += blockDim.x) {
        const uint32_t r = r0 + idx / kPerRow, d = (idx % kPerRow) * 4;
        const uint32_t q = qt * BQ + r;
        if (q >= p.Sq) continue;
        const uint64_t row0 = (uint64_t)tile * 2 * BQ + r, row1 = row0 + BQ;
        const float2 ml0 = *reinterpret_cast<const float2 *>(pML + 2 * row0);
        const float2 ml1 = *reinterpret_cast<const float2 *>(pML + 2 * row1);
        const float M = fmaxf(ml0.x, ml1.x);
        const float w0 = ml0.x == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(ml0.x - M);
        const float w1 = ml1.x == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(ml1.x - M);
        const float L = w0 * ml0.y + w1 * ml1.y;
        const float inv = L > 0.0f ? 1.0f / L : 0.0f;
        const float4 a = *reinterpret_cast<const float4 *>(pO + row0 * HD + d);
        const float4 c = *reinterpret_cast<const float4 *>(pO + row1 * HD + d);
        if (d >= p.Hd) continue;  // padding dims of a kernel compiled for HD > Hd
        typename O::storage *orow = out + ((uint64_t)bh * p.Sq + q) * p.Hd + d;
        orow[0] = O::store((w0 * a.x + w1 * c.x) * inv);
        orow[1] = O::store((w0 * a.y + w1 * c.y) * inv);
        orow[2] = O::store((w0 * a.z + w1 * c.z) * inv);
        orow[3] = O::store((w0 * a.w + w1 * c.w) * inv);
    }
}

}  // namespace

#define FA_TILED(name, T, O, HD)                                                                       \
    POPCORN_KERNEL void __launch_bounds__(256)                                                         \
        name(const uint16_t *q, const uint16_t *k, const uint16_t *v, O::storage *out, float *pO,      \
             float *pML, uint64_t *pairFlags, TiledFlashAttentionConstants p) {                        \
        fa_tiled<T, O, HD>(q, k, v, out, pO, pML, pairFlags, p);                                       \
    }
#define FA_TILED_D(t, T, o, O)                                   \
    FA_TILED(flash_attention_tiled_##t##_##o##_d64, T, O, 64)    \
    FA_TILED(flash_attention_tiled_##t##_##o##_d128, T, O, 128)  \
    FA_TILED(flash_attention_tiled_##t##_##o##_d256, T, O, 256)
#define FA_TILED16(name, T, O, HD, NW)                                                                 \
    POPCORN_KERNEL void __launch_bounds__(64 * NW)                                                     \
        name(const uint16_t *q, const uint16_t *k, const uint16_t *v, O::storage *out, float *pO,      \
             float *pML, uint64_t *pairFlags, TiledFlashAttentionConstants p) {                        \
        fa_tiled16<T, O, HD, NW>(q, k, v, out, pO, pML, pairFlags, p);                                     \
    }
// Hd 512 on 4 waves (64 query rows per block): a wave's output and query
// fragments need up to 512 registers, one wave per SIMD
#define FA_TILED16_D(t, T, o, O)                                         \
    FA_TILED16(flash_attention_tiled16_##t##_##o##_d128, T, O, 128, 8)   \
    FA_TILED16(flash_attention_tiled16_##t##_##o##_d256, T, O, 256, 8)   \
    FA_TILED16(flash_attention_tiled16_##t##_##o##_d512, T, O, 512, 4)
// f32: 4 waves (64 query rows) per block, two blocks per CU below Hd 512
// (at Hd 512 a wave's Q chunks and accumulators alone take 256 registers);
// the partial-state arguments are never read (every tile whole)
#define FA_TILED_F32(name, HD, ZIGZAG)                                                                 \
    POPCORN_KERNEL void __launch_bounds__(256, HD < 512 ? 2 : 1)                                       \
        name(const float *q, const float *k, const float *v, float *out, float *, float *, uint64_t *, \
             TiledFlashAttentionConstants p) {                                                         \
        fa_tiled_f32<HD, 4, ZIGZAG>(q, k, v, out, p);                                                  \
    }
#define FA_MERGE(name, O, HD)                                                                       \
    POPCORN_KERNEL void __launch_bounds__(256)                                                         \
        name(const float *pO, const float *pML, O::storage *out, TiledFlashAttentionConstants p) {       \
        fa_split_merge<O, HD>(pO, pML, out, p);                                                        \
    }
#define FA_MERGE_D(o, O)                                         \
    FA_MERGE(flash_attention_split_merge_##o##_d64, O, 64)       \
    FA_MERGE(flash_attention_split_merge_##o##_d128, O, 128)     \
    FA_MERGE(flash_attention_split_merge_##o##_d256, O, 256)

using pk::BF16;
using pk::F16;
using pk::F32;

FA_TILED_D(f16, F16, f16, F16)
FA_TILED_D(f16, F16, f32, F32)
FA_TILED_D(bf16, BF16, bf16, BF16)
FA_TILED_D(bf16, BF16, f32, F32)
FA_TILED16_D(f16, F16, f16, F16)
FA_TILED16_D(f16, F16, f32, F32)
FA_TILED16_D(bf16, BF16, bf16, BF16)
FA_TILED16_D(bf16, BF16, f32, F32)
FA_MERGE_D(f16, F16)
FA_MERGE_D(bf16, BF16)
FA_MERGE_D(f32, F32)
FA_TILED_F32(flash_attention_tiled16_f32_f32_d64, 64, true)
FA_TILED_F32(flash_attention_tiled16_f32_f32_d128, 128, true)
FA_TILED_F32(flash_attention_tiled16_f32_f32_d256, 256, true)
FA_TILED_F32(flash_attention_tiled16_f32_f32_d512, 512, false)
