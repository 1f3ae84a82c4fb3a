// Prefill Matmul on the matrix cores: C[M, N] = A[M, K] . B[N, K]^T
// (the reference's transposeB layout, Matmul.swift:34-65 and
// MPPMatmul.metal:19-91, whose MPP tiles this replaces), f16 or bf16 inputs,
// f32 accumulation, output f32 or the input dtype (popcorn_store rounding).
//
// With the MFMA lane layout of mfma.hpp both operands are 16-byte runs
// along K of a row of A or of Bt.
//
// A block computes a BM x BN tile (128 or 256 each; 4 or 8 waves, each wave
// a 64 x 64 or 128 x 64 piece of 32 x 32 MFMA tiles; the host picks the tile
// shape per GEMM so the tile count fills the 256 CUs evenly). K advances 64
// at a time through two LDS stages
// (rows padded to 72 elements, so the 32 rows a fragment load touches fall
// in distinct banks); the next stage's global loads are in registers while
// the current stage is multiplied. Tiles are assigned XCD by XCD (blocks
// are dealt round-robin to the 8 XCDs, so block b runs on XCD b % 8) and,
// within an XCD's range, in groups of 8 tile rows, so the A and B panels a
// group shares stay in that XCD's L2.
#include <type_traits>

#include "mfma.hpp"

namespace {

using pk::f32x16;
using pk::Mma;
using pk::u32x4;

constexpr int BK = 64;
constexpr int LDK = BK + 8;  // padded LDS row, in elements
constexpr int kXcds = 8;
constexpr int kGroupM = 8;

__device__ inline void group_tile(uint32_t pid, uint32_t nM, uint32_t nN, uint32_t &pm, uint32_t &pn);
// Tile (pm, pn) of block b: XCD-contiguous ranges, grouped rows within.
__device__ inline void tile_of(uint32_t b, uint32_t nM, uint32_t nN, uint32_t &pm, uint32_t &pn) {
    const uint32_t total = nM * nN;
    uint32_t pid = b;
    if (total % kXcds == 0) pid = (b % kXcds) * (total / kXcds) + b / kXcds;
    group_tile(pid, nM, nN, pm, pn);
}
// Split-K grids (tiles x splits): the XCD-contiguous ranges run over the
// (split, tile) units, so an XCD's blocks share one split's K range and a
// band of tiles, whose A and B panels stay in that XCD's L2 (config-5
// down: 327 -> 314 us against ranges over the tiles alone, where every
// XCD read all of A).
__device__ inline void split_tile_of(uint32_t nM, uint32_t nN, uint32_t &pm, uint32_t &pn, uint32_t &split) {
    const uint32_t tiles = nM * nN, units = tiles * gridDim.y;
    const uint32_t b = blockIdx.x + blockIdx.y * gridDim.x;
    const uint32_t u = units % kXcds == 0 ? (b % kXcds) * (units / kXcds) + b / kXcds : b;
    split = u / tiles;
    group_tile(u % tiles, nM, nN, pm, pn);
}
// Tile pid of an XCD's range: groups of kGroupM tile rows, rows fastest.
__device__ inline void group_tile(uint32_t pid, uint32_t nM, uint32_t nN, uint32_t &pm, uint32_t &pn) {
    const uint32_t inGroup = kGroupM * nN;
    const uint32_t group = pid / inGroup;
    const uint32_t firstM = group * kGroupM;
    const uint32_t gm = min(nM - firstM, (uint32_t)kGroupM);
    pm = firstM + (pid % inGroup) % gm;
    pn = (pid % inGroup) / gm;
}

// BM x BN block tile on WM_N x WN_N waves; each wave a (BM / WM_N) x
// (BN / WN_N) tile of 32 x 32 MFMA tiles.
template <typename T, typename O, int BM, int BN, int WM_N, int WN_N>
__device__ void gemm_nt(const uint16_t *__restrict__ A, const uint16_t *__restrict__ B,
                        typename O::storage *__restrict__ C, const MatmulConstants &p) {
    constexpr int kThreads = 64 * WM_N * WN_N;
    constexpr int WM = BM / WM_N, WN = BN / WN_N;
    constexpr int TM = WM / 32, TN = WN / 32;
    constexpr int kChunksA = BM * BK / 8 / kThreads, kChunksB = BN * BK / 8 / kThreads;
    static_assert(kChunksA * kThreads * 8 == BM * BK && kChunksB * kThreads * 8 == BN * BK, "tile / thread count");
    // Two stages of [A rows | B rows], each row LDK elements. The array is
    // declared here (not passed in) so every access stays an LDS access.
    constexpr int kStage = (BM + BN) * LDK;
    __shared__ __attribute__((aligned(16))) uint16_t smem[2 * kStage];
    auto sA = [&](int buf) { return smem + buf * kStage; };
    auto sB = [&](int buf) { return smem + buf * kStage + BM * LDK; };

    const uint32_t M = p.M, N = p.N, K = p.K;
    const uint32_t nM = (M + BM - 1) / BM, nN = (N + BN - 1) / BN;
    uint32_t pm, pn;
    tile_of(blockIdx.x, nM, nN, pm, pn);
    const uint32_t bm = pm * BM, bn = pn * BN;
    const uint32_t t = threadIdx.x, lane = t & 63, wave = t >> 6;
    const uint32_t wm = (wave / WN_N) * WM, wn = (wave % WN_N) * WN;

    // Global chunk c of a stage: row c / 8 of the tile, elements (c % 8) * 8 .. +8
    // of the stage's K range. Rows past M (N) and K past the end read a valid
    // address and are zeroed when stored to LDS (the mask is applied there,
    // after the stage's multiply, so the loads stay in flight meanwhile).
    u32x4 ra[kChunksA], rb[kChunksB];
    uint32_t okA = 0, okB = 0;
    auto gload = [&](uint32_t k0) {
        okA = okB = 0;
#pragma unroll
        for (int i = 0; i < kChunksA; ++i) {
            const uint32_t c = t + i * kThreads, r = c >> 3, k = k0 + (c & 7) * 8;
            const uint32_t ar = bm + r;
            const bool kin = k < K;
            ra[i] = *reinterpret_cast<const u32x4 *>(A + (uint64_t)min(ar, M - 1) * K + (kin ? k : 0u));
            okA |= (ar < M && kin) ? 1u << i : 0u;
        }
#pragma unroll
        for (int i = 0; i < kChunksB; ++i) {
            const uint32_t c = t + i * kThreads, r = c >> 3, k = k0 + (c & 7) * 8;
            const uint32_t br = bn + r;
            const bool kin = k < K;
            rb[i] = *reinterpret_cast<const u32x4 *>(B + (uint64_t)min(br, N - 1) * K + (kin ? k : 0u));
            okB |= (br < N && kin) ? 1u << i : 0u;
        }
    };
    auto lstore = [&](int buf) {
        const u32x4 zero = {0u, 0u, 0u, 0u};
#pragma unroll
        for (int i = 0; i < kChunksA; ++i) {
            const uint32_t c = t + i * kThreads, r = c >> 3, kc = (c & 7) * 8;
            *reinterpret_cast<u32x4 *>(&sA(buf)[r * LDK + kc]) = (okA >> i) & 1u ? ra[i] : zero;
        }
#pragma unroll
        for (int i = 0; i < kChunksB; ++i) {
            const uint32_t c = t + i * kThreads, r = c >> 3, kc = (c & 7) * 8;
            *reinterpret_cast<u32x4 *>(&sB(buf)[r * LDK + kc]) = (okB >> i) & 1u ? rb[i] : zero;
        }
    };

    f32x16 acc[TM][TN];
#pragma unroll
    for (int mi = 0; mi < TM; ++mi)
#pragma unroll
        for (int ni = 0; ni < TN; ++ni)
#pragma unroll
            for (int i = 0; i < 16; ++i) acc[mi][ni][i] = 0.0f;

    auto compute = [&](int buf) {
#pragma unroll
        for (int kk = 0; kk < BK / 16; ++kk) {
            const uint32_t ko = kk * 16 + (lane >> 5) * 8;
            u32x4 fa[TM], fb[TN];
#pragma unroll
            for (int mi = 0; mi < TM; ++mi)
                fa[mi] = *reinterpret_cast<const u32x4 *>(&sA(buf)[(wm + mi * 32 + (lane & 31)) * LDK + ko]);
#pragma unroll
            for (int ni = 0; ni < TN; ++ni)
                fb[ni] = *reinterpret_cast<const u32x4 *>(&sB(buf)[(wn + ni * 32 + (lane & 31)) * LDK + ko]);
#pragma unroll
            for (int mi = 0; mi < TM; ++mi)
#pragma unroll
                for (int ni = 0; ni < TN; ++ni) acc[mi][ni] = Mma<T>::run(fa[mi], fb[ni], acc[mi][ni]);
        }
    };

    const uint32_t nk = (K + BK - 1) / BK;
    gload(0);
    lstore(0);
    __syncthreads();
    for (uint32_t kt = 0; kt < nk; ++kt) {
        const int cur = kt & 1;
        if (kt + 1 < nk) gload((kt + 1) * BK);
        compute(cur);
        if (kt + 1 < nk) lstore(cur ^ 1);
        __syncthreads();
    }

#pragma unroll
    for (int mi = 0; mi < TM; ++mi) {
#pragma unroll
        for (int ni = 0; ni < TN; ++ni) {
            const uint32_t col = bn + wn + ni * 32 + (lane & 31);
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                const uint32_t row = bm + wm + mi * 32 + (i >> 2) * 8 + (lane >> 5) * 4 + (i & 3);
                if (row < M && col < N) C[(uint64_t)row * N + col] = O::store(acc[mi][ni][i]);
            }
        }
    }
}

// ---- direct-to-LDS pipeline ----------------------------------------------------
// The same tile product with the operand tiles copied global -> LDS by
// global_load_lds_dwordx4 (lane l of a wave instruction writes 16 bytes at
// M0 + 16 l, checked on gfx950), kStagesD stages of BKD = 32 in flight and
// no staging registers. A stage holds BM + BN rows of 64 bytes (4 chunks);
// chunk kc of row r sits in slot kc ^ ((r >> 2) & 3), so the 16 rows a
// fragment read touches (lanes 16 at a time) fall in 16 distinct 4-bank
// groups. Needs K % 32 == 0 (a chunk past K cannot be zero-filled here).
constexpr int BKD = 32;
constexpr int kStagesD = 4;

typedef __attribute__((address_space(3))) void lds_void;

template <int N>
__device__ inline void wait_vmcnt() {
    // s_waitcnt vmcnt(N), expcnt and lgkmcnt left at their maximum (no wait)
    static_assert(N >= 0 && N < 64, "vmcnt range");
    __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}

// SPLITK: gridDim.y blocks share a tile, each over K / gridDim.y of the
// reduction (which split a block takes comes from split_tile_of), and
// write f32 partial products to P [gridDim.y][M][N] for
// gemm_splitk_reduce (C is then unused).
template <typename T, typename O, int BM, int BN, int WM_N, int WN_N, bool SPLITK = false>
__device__ void gemm_nt_direct(const uint16_t *__restrict__ A, const uint16_t *__restrict__ B,
                               typename O::storage *__restrict__ C, const MatmulConstants &p,
                               float *__restrict__ P = nullptr) {
    constexpr int NW = WM_N * WN_N;
    constexpr int WM = BM / WM_N, WN = BN / WN_N;
    constexpr int TM = WM / 32, TN = WN / 32;
    constexpr int kRowB = BKD * 2;                 // bytes per LDS row
    constexpr int kStageB = (BM + BN) * kRowB;     // bytes per stage
    constexpr int kInstA = BM / (16 * NW), kInstB = BN / (16 * NW);  // wave instructions per stage
    constexpr int kLPS = kInstA + kInstB;          // loads per stage per wave
    static_assert(kInstA * 16 * NW == BM && kInstB * 16 * NW == BN, "tile rows / waves");
    __shared__ __attribute__((aligned(16))) uint8_t smem[kStagesD * kStageB];

    const uint32_t M = p.M, N = p.N, K = p.K;
    const uint32_t nM = (M + BM - 1) / BM, nN = (N + BN - 1) / BN;
    uint32_t pm, pn, split = 0;
    if constexpr (SPLITK) split_tile_of(nM, nN, pm, pn, split);
    else tile_of(blockIdx.x, nM, nN, pm, pn);
    const uint32_t bm = pm * BM, bn = pn * BN;
    const uint32_t lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const uint32_t wm = (wave / WN_N) * WM, wn = (wave % WN_N) * WN;

    // this lane's source rows / chunk for each of its wave's instructions
    const uint32_t lr = lane >> 2, lpos = lane & 3;
    const uint32_t kBase = SPLITK ? split * (K / gridDim.y) : 0u;
    auto issue = [&](uint32_t kt) {
        const uint32_t k0 = kBase + kt * BKD;
        uint8_t *stage = smem + (kt % kStagesD) * kStageB;
#pragma unroll
        for (int i = 0; i < kInstA; ++i) {
            const uint32_t r0 = (i * NW + wave) * 16, r = r0 + lr;
            const uint32_t kc = lpos ^ ((r >> 2) & 3);
            const uint16_t *src = A + (uint64_t)min(bm + r, M - 1) * K + k0 + kc * 8;
            __builtin_amdgcn_global_load_lds(src, (lds_void *)(stage + r0 * kRowB), 16, 0, 0);
        }
#pragma unroll
        for (int i = 0; i < kInstB; ++i) {
            const uint32_t r0 = (i * NW + wave) * 16, r = r0 + lr;
            const uint32_t kc = lpos ^ ((r >> 2) & 3);
            const uint16_t *src = B + (uint64_t)min(bn + r, N - 1) * K + k0 + kc * 8;
            __builtin_amdgcn_global_load_lds(src, (lds_void *)(stage + (BM + r0) * kRowB), 16, 0, 0);
        }
    };

    f32x16 acc[TM][TN];
#pragma unroll
    for (int mi = 0; mi < TM; ++mi)
#pragma unroll
        for (int ni = 0; ni < TN; ++ni)
#pragma unroll
            for (int i = 0; i < 16; ++i) acc[mi][ni][i] = 0.0f;

    auto frag = [&](const uint8_t *base, uint32_t row, uint32_t kc) {
        return *reinterpret_cast<const u32x4 *>(base + row * kRowB + ((kc ^ ((row >> 2) & 3)) << 4));
    };
    // fragment mi of A / ni of B for K-16 half kk of stage kt
    auto fragA = [&](uint32_t kt, int kk, int mi) {
        return frag(smem + (kt % kStagesD) * kStageB, wm + mi * 32 + (lane & 31), kk * 2 + (lane >> 5));
    };
    auto fragB = [&](uint32_t kt, int kk, int ni) {
        return frag(smem + (kt % kStagesD) * kStageB + BM * kRowB, wn + ni * 32 + (lane & 31), kk * 2 + (lane >> 5));
    };
    // wait until at most `after` stages' copies issued after the awaited
    // one are outstanding (this wave's own copies of it have landed)
    auto wait_stage = [&](uint32_t after) {
        if (after >= 2) wait_vmcnt<2 * kLPS>();
        else if (after == 1) wait_vmcnt<kLPS>();
        else wait_vmcnt<0>();
    };

    // Each stage is two K-16 halves. The B fragments of the second half are
    // read at the start of the first (two B sets), and each A fragment is
    // re-read for the next half as soon as its MFMAs are issued, so a half's
    // fragments arrive while the previous half's products run. The stage
    // barrier sits between the halves: before it this wave has read all of
    // stage kt (lgkmcnt(0)) and its copies of stage kt + 1 have landed;
    // after it stage kt + 1 is visible, the buffer of stage kt is free for
    // the copies of stage kt + 4, and the first reads of stage kt + 1 overlap
    // the second half's products.
    const uint32_t nk = (SPLITK ? K / gridDim.y : K) / BKD;
    static_assert(kStagesD == 4, "the waits below count two stages in flight behind the awaited one");
#pragma unroll
    for (int s = 0; s < kStagesD - 1; ++s)
        if ((uint32_t)s < nk) issue(s);
    wait_stage(min((uint32_t)(kStagesD - 2), nk - 1));
    __builtin_amdgcn_s_barrier();
    if ((uint32_t)(kStagesD - 1) < nk) issue(kStagesD - 1);
    u32x4 fa[TM], fb[TN], fb2[TN];
    // Scalar loads (kernel arguments) also count in lgkmcnt and complete out
    // of order: with one still outstanding on entry, the wait before the
    // loop's first MFMA would have to be lgkmcnt(0) on every pass.
    __builtin_amdgcn_s_waitcnt(0xC07F);
    // in the order of the passes below (B, then A in order), held by
    // scheduling barriers: the wait before the first pass's first MFMA is
    // then the same on entry as around the loop, lgkmcnt(TM - 1)
#pragma unroll
    for (int ni = 0; ni < TN; ++ni) {
        fb[ni] = fragB(0, 0, ni);
        __builtin_amdgcn_sched_barrier(0);
    }
#pragma unroll
    for (int mi = 0; mi < TM; ++mi) {
        fa[mi] = fragA(0, 0, mi);
        __builtin_amdgcn_sched_barrier(0);
    }
    // The compiler would sink each fragment read to just before its first
    // use; the scheduling groups keep this order: per A fragment its MFMAs,
    // then its re-read (after the first group also the B reads).
    auto pin_order = [&] {
        __builtin_amdgcn_sched_group_barrier(0x008, TN, 0);      // MFMA
        __builtin_amdgcn_sched_group_barrier(0x100, TN + 1, 0);  // DS reads
#pragma unroll
        for (int mi = 1; mi < TM; ++mi) {
            __builtin_amdgcn_sched_group_barrier(0x008, TN, 0);  // MFMA
            __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);   // DS read
        }
    };
    for (uint32_t kt = 0; kt < nk; ++kt) {
#pragma unroll
        for (int ni = 0; ni < TN; ++ni) fb2[ni] = fragB(kt, 1, ni);
#pragma unroll
        for (int mi = 0; mi < TM; ++mi) {
#pragma unroll
            for (int ni = 0; ni < TN; ++ni) acc[mi][ni] = Mma<T>::run(fa[mi], fb[ni], acc[mi][ni]);
            fa[mi] = fragA(kt, 1, mi);
        }
        pin_order();
        // stages issued so far: up to min(kt + 3, nk - 1). In the last pass
        // nothing is outstanding, and the reads of "stage kt + 1" fetch a
        // buffer no copy is writing, unused (no branches inside the pass).
        wait_stage(kt + 2 < nk ? min((uint32_t)(kStagesD - 2), nk - 2 - kt) : 0u);
        __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): this wave's reads of stage kt are done
        __builtin_amdgcn_s_barrier();
        if (kt + kStagesD < nk) issue(kt + kStagesD);
#pragma unroll
        for (int ni = 0; ni < TN; ++ni) fb[ni] = fragB(kt + 1, 0, ni);
#pragma unroll
        for (int mi = 0; mi < TM; ++mi) {
#pragma unroll
            for (int ni = 0; ni < TN; ++ni) acc[mi][ni] = Mma<T>::run(fa[mi], fb2[ni], acc[mi][ni]);
            fa[mi] = fragA(kt + 1, 0, mi);
        }
        pin_order();
    }

#pragma unroll
    for (int mi = 0; mi < TM; ++mi) {
#pragma unroll
        for (int ni = 0; ni < TN; ++ni) {
            const uint32_t col = bn + wn + ni * 32 + (lane & 31);
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                const uint32_t row = bm + wm + mi * 32 + (i >> 2) * 8 + (lane >> 5) * 4 + (i & 3);
                if (row < M && col < N) {
                    if constexpr (SPLITK)
                        P[((uint64_t)split * M + row) * N + col] = acc[mi][ni][i];
                    else
                        C[(uint64_t)row * N + col] = O::store(acc[mi][ni][i]);
                }
            }
        }
    }
}

// ---- whole-line pipeline ("e" tiles, K % 64 == 0) ---------------------------
// The same tile product with K = 64 per stage: 128-byte LDS rows, so each
// copy instruction (8 lanes per row, buffer_load ... lds) requests whole
// 128-byte lines. The 64-byte rows of the pipeline above fetch each line
// twice, a stage apart, and the L2 -> LDS copy rate bounds those tiles
// (config-5 gate 283 -> 261 us, down 322 -> 290 us, bit for bit the same
// products). Two stage buffers; the copies of stage kt + 2 are issued at
// the barrier before the last K-16 quarter of stage kt. Chunk c of row r
// sits in slot c ^ ((r >> 1) & 7): the 16 rows a quarter-wave of a
// fragment read touches cover all 64 banks.
constexpr int BK64 = 64;
template <typename T, typename O, int BM, int BN, int WM_N, int WN_N, bool SPLITK = false>
__device__ void gemm_nt_lines(const uint16_t *__restrict__ A, const uint16_t *__restrict__ B,
                                 typename O::storage *__restrict__ C, const MatmulConstants &p,
                                 float *__restrict__ P = nullptr) {
    constexpr int NW = WM_N * WN_N;
    constexpr int WM = BM / WM_N, WN = BN / WN_N;
    constexpr int TM = WM / 32, TN = WN / 32;
    constexpr int kRowB = BK64 * 2;               // 128 bytes per LDS row
    constexpr int kStageB = (BM + BN) * kRowB;    // bytes per stage
    // A stage is kInst copy instructions of 8 rows each, A's rows then B's
    // (LDS row 8 j + r for instruction j); wave w issues j = w, w + NW, ...
    constexpr int kInst = (BM + BN) / 8, kInstA = BM / 8;
    constexpr int kPer = (kInst + NW - 1) / NW;  // per wave, rounded up
    static_assert(BM % 16 == 0 && BN % 8 == 0, "tile rows");
    __shared__ __attribute__((aligned(16))) uint8_t smem[2 * kStageB];

    const uint32_t M = p.M, N = p.N, K = p.K;
    const uint32_t nM = (M + BM - 1) / BM, nN = (N + BN - 1) / BN;
    uint32_t pm, pn, split = 0;
    if constexpr (SPLITK) split_tile_of(nM, nN, pm, pn, split);
    else tile_of(blockIdx.x, nM, nN, pm, pn);
    const uint32_t bm = pm * BM, bn = pn * BN;
    const uint32_t lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const uint32_t wm = (wave / WN_N) * WM, wn = (wave % WN_N) * WN;

    // Copies through buffer resources over the tile's rows: rows past M or
    // N fall outside the resource and read as zeros. A lane's byte offset
    // (its row within the 8, its chunk) is the same for every instruction
    // and both operands; the instruction's first row and the stage's K
    // offset go in the scalar offset.
    static_assert(NW % 2 == 0, "one chunk swizzle per lane for every instruction");
    const uint32_t lr = lane >> 3, lpos = lane & 7;
    const uint32_t kBase = SPLITK ? split * (K / gridDim.y) : 0u;
    const uint64_t rowB = (uint64_t)K * 2u;
    const uint32_t bytesA = (uint32_t)min((uint64_t)(M - bm) * rowB, (uint64_t)0xffffffffu);
    const uint32_t bytesB = (uint32_t)min((uint64_t)(N - bn) * rowB, (uint64_t)0xffffffffu);
    const __amdgpu_buffer_rsrc_t rsA = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t *>(A + (uint64_t)bm * K), 0, (int)bytesA, 0x00020000);
    const __amdgpu_buffer_rsrc_t rsB = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t *>(B + (uint64_t)bn * K), 0, (int)bytesB, 0x00020000);
    // row 8 j + lr of an operand: chunk swizzle (4 j + lr / 2) & 7, and j is
    // odd or even with the wave (NW and kInstA even)
    const uint32_t voff = lr * (uint32_t)rowB + ((lpos ^ (((wave & 1) * 4 + (lr >> 1)) & 7)) << 4);
    const uint32_t rows8 = 8 * (uint32_t)rowB;  // bytes per instruction's rows
    auto issue = [&](uint32_t kt) {
        const uint32_t kb = (kBase + kt * BK64) * 2u;
        uint8_t *stage = smem + (kt & 1) * kStageB;
#pragma unroll
        for (int i = 0; i < kPer; ++i) {
            const uint32_t j = i * NW + wave;
            if (kInst % NW != 0 && j >= (uint32_t)kInst) break;
            const bool isA = kInstA % NW == 0 ? i < kInstA / NW : j < (uint32_t)kInstA;
            __builtin_amdgcn_raw_ptr_buffer_load_lds(isA ? rsA : rsB, (lds_void *)(stage + j * 8 * kRowB), 16, voff,
                                                     kb + (isA ? j : j - kInstA) * rows8, 0, 0);
        }
    };
    // wait until only the copies of the stage after the awaited one are
    // outstanding (this wave issues kPer or kPer - 1 of them)
    auto wait_one_behind = [&] {
        if (kInst % NW == 0 || wave < (uint32_t)(kInst % NW)) wait_vmcnt<kPer>();
        else wait_vmcnt<kPer - 1>();
    };

    f32x16 acc[TM][TN];
#pragma unroll
    for (int mi = 0; mi < TM; ++mi)
#pragma unroll
        for (int ni = 0; ni < TN; ++ni)
#pragma unroll
            for (int i = 0; i < 16; ++i) acc[mi][ni][i] = 0.0f;

    auto frag = [&](const uint8_t *base, uint32_t row, uint32_t kc) {
        return *reinterpret_cast<const u32x4 *>(base + row * kRowB + ((kc ^ ((row >> 1) & 7)) << 4));
    };
    // fragment mi of A / ni of B for K-16 quarter kk of stage kt
    auto fragA = [&](uint32_t kt, int kk, int mi) {
        return frag(smem + (kt & 1) * kStageB, wm + mi * 32 + (lane & 31), kk * 2 + (lane >> 5));
    };
    auto fragB = [&](uint32_t kt, int kk, int ni) {
        return frag(smem + (kt & 1) * kStageB + BM * kRowB, wn + ni * 32 + (lane & 31), kk * 2 + (lane >> 5));
    };

    const uint32_t nk = (SPLITK ? K / gridDim.y : K) / BK64;
    issue(0);
    if (nk > 1) {
        issue(1);
        wait_one_behind();
    } else {
        wait_vmcnt<0>();
    }
    __builtin_amdgcn_s_barrier();
    u32x4 fa[TM], fb[TN], fb2[TN];
    __builtin_amdgcn_s_waitcnt(0xC07F);
#pragma unroll
    for (int ni = 0; ni < TN; ++ni) {
        fb[ni] = fragB(0, 0, ni);
        __builtin_amdgcn_sched_barrier(0);
    }
#pragma unroll
    for (int mi = 0; mi < TM; ++mi) {
        fa[mi] = fragA(0, 0, mi);
        __builtin_amdgcn_sched_barrier(0);
    }
    auto pin_order = [&] {
        __builtin_amdgcn_sched_group_barrier(0x008, TN, 0);      // MFMA
        __builtin_amdgcn_sched_group_barrier(0x100, TN + 1, 0);  // DS reads
#pragma unroll
        for (int mi = 1; mi < TM; ++mi) {
            __builtin_amdgcn_sched_group_barrier(0x008, TN, 0);  // MFMA
            __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);   // DS read
        }
    };
    // one K-16 quarter: products with (fa, fcur), while the next quarter's
    // B fragments go to fnext and each A fragment is re-read for it
    auto quarter = [&](u32x4 *fcur, u32x4 *fnext, uint32_t nkt, int nkk) {
#pragma unroll
        for (int ni = 0; ni < TN; ++ni) fnext[ni] = fragB(nkt, nkk, ni);
#pragma unroll
        for (int mi = 0; mi < TM; ++mi) {
#pragma unroll
            for (int ni = 0; ni < TN; ++ni) acc[mi][ni] = Mma<T>::run(fa[mi], fcur[ni], acc[mi][ni]);
            fa[mi] = fragA(nkt, nkk, mi);
        }
        pin_order();
    };
    for (uint32_t kt = 0; kt < nk; ++kt) {
        quarter(fb, fb2, kt, 1);
        quarter(fb2, fb, kt, 2);
        quarter(fb, fb2, kt, 3);
        // this wave's reads of stage kt are issued; wait for them and for
        // its copies of stage kt + 1 (the only ones outstanding), then the
        // buffer of stage kt takes the copies of stage kt + 2. In the last
        // pass the reads of "stage kt + 1" fetch a buffer no copy writes.
        wait_vmcnt<0>();
        __builtin_amdgcn_s_waitcnt(0xC07F);
        __builtin_amdgcn_s_barrier();
        if (kt + 2 < nk) issue(kt + 2);
        quarter(fb2, fb, kt + 1, 0);
    }

#pragma unroll
    for (int mi = 0; mi < TM; ++mi) {
#pragma unroll
        for (int ni = 0; ni < TN; ++ni) {
            const uint32_t col = bn + wn + ni * 32 + (lane & 31);
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                const uint32_t row = bm + wm + mi * 32 + (i >> 2) * 8 + (lane >> 5) * 4 + (i & 3);
                if (row < M && col < N) {
                    if constexpr (SPLITK)
                        P[((uint64_t)split * M + row) * N + col] = acc[mi][ni][i];
                    else
                        C[(uint64_t)row * N + col] = O::store(acc[mi][ni][i]);
                }
            }
        }
    }
}

// C = sum over the gridDim.y-way split of P [splits][M][N] (f32), rounded
// once to C's dtype; 4 elements per thread (M N % 4 == 0).
template <typename O>
__device__ void gemm_splitk_reduce(const float *__restrict__ P, typename O::storage *__restrict__ C,
                                   const MatmulConstants &p, uint32_t splits) {
    const uint64_t mn = (uint64_t)p.M * p.N;
    for (uint64_t i = ((uint64_t)blockIdx.x * blockDim.x + threadIdx.x) * 4; i < mn;
         i += (uint64_t)gridDim.x * blockDim.x * 4) {
        float4 a = *reinterpret_cast<const float4 *>(P + i);
        for (uint32_t s = 1; s < splits; ++s) {
            const float4 b = *reinterpret_cast<const float4 *>(P + s * mn + i);
            a.x += b.x;
            a.y += b.y;
            a.z += b.z;
            a.w += b.w;
        }
        if constexpr (std::is_same<O, pk::F32>::value) {
            *reinterpret_cast<float4 *>(C + i) = a;
        } else {
            // the four 16-bit results as one 8-byte store
            auto b16 = [](float x) { return (uint32_t)__builtin_bit_cast(uint16_t, O::store(x)); };
            *reinterpret_cast<uint2 *>(C + i) = uint2{b16(a.x) | (b16(a.y) << 16), b16(a.z) | (b16(a.w) << 16)};
        }
    }
}

}  // namespace

// A, B: 16-bit storage; the host requires K % 8 == 0 and 16-byte aligned A, B.
// Tile variants: _t<BM>x<BN> on 4 (128 x 128) or 8 waves; LDS is static.
#define GEMM_MFMA(name, T, O, BM, BN, WMN, WNN)                                                   \
    POPCORN_KERNEL void __launch_bounds__(64 * WMN * WNN)                                         \
        name(const uint16_t *a, const uint16_t *b, O::storage *c, MatmulConstants p) {            \
        gemm_nt<T, O, BM, BN, WMN, WNN>(a, b, c, p);                                              \
    }
#define GEMM_MFMA_D(name, T, O, BM, BN, WMN, WNN)                                                 \
    POPCORN_KERNEL void __launch_bounds__(64 * WMN * WNN)                                         \
        name(const uint16_t *a, const uint16_t *b, O::storage *c, MatmulConstants p) {            \
        gemm_nt_direct<T, O, BM, BN, WMN, WNN>(a, b, c, p);                                       \
    }
#define GEMM_MFMA_E(name, T, O, BM, BN, WMN, WNN)                                                 \
    POPCORN_KERNEL void __launch_bounds__(64 * WMN * WNN)                                         \
        name(const uint16_t *a, const uint16_t *b, O::storage *c, MatmulConstants p) {            \
        gemm_nt_lines<T, O, BM, BN, WMN, WNN>(a, b, c, p);                                        \
    }
#define GEMM_MFMA_TILES(base, T, O)                          \
    GEMM_MFMA_E(base##_e256x384, T, O, 256, 384, 2, 4)       \
    GEMM_MFMA_E(base##_e256x288, T, O, 256, 288, 4, 3)       \
    GEMM_MFMA_E(base##_e256x256, T, O, 256, 256, 2, 4)       \
    GEMM_MFMA_E(base##_e128x128, T, O, 128, 128, 2, 2)       \
    GEMM_MFMA_E(base##_e128x256, T, O, 128, 256, 2, 4)       \
    GEMM_MFMA_E(base##_e128x192, T, O, 128, 192, 2, 2)       \
    GEMM_MFMA_D(base##_d256x256, T, O, 256, 256, 2, 4)       \
    GEMM_MFMA_D(base##_d128x128, T, O, 128, 128, 2, 2)       \
    GEMM_MFMA_D(base##_d128x256, T, O, 128, 256, 2, 4)       \
    GEMM_MFMA_D(base##_d128x192, T, O, 128, 192, 2, 2)       \
    GEMM_MFMA_D(base##_d256x384, T, O, 256, 384, 2, 4)       \
    GEMM_MFMA(base##_t128x128, T, O, 128, 128, 2, 2)         \
    GEMM_MFMA(base##_t256x128, T, O, 256, 128, 4, 2)         \
    GEMM_MFMA(base##_t128x256, T, O, 128, 256, 2, 4)         \
    GEMM_MFMA(base##_t256x256, T, O, 256, 256, 2, 4)         \
    GEMM_MFMA(base##_t256x256w4, T, O, 256, 256, 2, 2)

using pk::BF16;
using pk::F16;
using pk::F32;

GEMM_MFMA_TILES(matmul_mfma_f16_f16_f16, F16, F16)
GEMM_MFMA_TILES(matmul_mfma_f16_f16_f32, F16, F32)
GEMM_MFMA_TILES(matmul_mfma_bf16_bf16_bf16, BF16, BF16)
GEMM_MFMA_TILES(matmul_mfma_bf16_bf16_f32, BF16, F32)

// Split-K forms of the 256 x 384 tile (f32 partials) and the reduction.
// B^T for a Matmul whose 16-bit B is [K, N] (not transposed): a block moves
// a 64 x 64 tile through LDS (66-element rows: a column read touches 32
// distinct banks). Whole tiles of 8-aligned shapes move as 16-byte runs (a
// thread takes two runs in and gathers two runs out); other tiles element
// by element.
__device__ void transpose2d_run(const uint16_t *__restrict__ in, uint16_t *__restrict__ out, const Transpose2DConstants &p) {
    __shared__ uint16_t tile[64][66];
    const uint32_t tr = blockIdx.y * 64, tc = blockIdx.x * 64;  // tile origin in `in`
    const bool vec = p.rows % 8 == 0 && p.cols % 8 == 0 && tr + 64 <= p.rows && tc + 64 <= p.cols &&
                     ((reinterpret_cast<uintptr_t>(in) | reinterpret_cast<uintptr_t>(out)) & 15) == 0;
    if (vec) {
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const uint32_t c = threadIdx.x + 256 * j, row = c >> 3, run = c & 7;
            const u32x4 v = *reinterpret_cast<const u32x4 *>(in + (uint64_t)(tr + row) * p.cols + tc + run * 8);
            uint32_t *dst = reinterpret_cast<uint32_t *>(&tile[row][run * 8]);
            dst[0] = v.x;
            dst[1] = v.y;
            dst[2] = v.z;
            dst[3] = v.w;
        }
        __syncthreads();
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const uint32_t c = threadIdx.x + 256 * j, orow = c >> 3, run = c & 7;  // out row tc + orow
            uint32_t w[4];
#pragma unroll
            for (int e = 0; e < 4; ++e)
                w[e] = (uint32_t)tile[run * 8 + 2 * e][orow] | ((uint32_t)tile[run * 8 + 2 * e + 1][orow] << 16);
            *reinterpret_cast<u32x4 *>(out + (uint64_t)(tc + orow) * p.rows + tr + run * 8) = u32x4{w[0], w[1], w[2], w[3]};
        }
        return;
    }
    const uint32_t tx = threadIdx.x & 31, ty = threadIdx.x >> 5;  // 2 elements per thread per row pass
    for (uint32_t r = ty; r < 64; r += 8) {
        const uint32_t row = tr + r, col = tc + 2 * tx;
        if (row < p.rows) {
            if (col < p.cols) tile[r][2 * tx] = in[(uint64_t)row * p.cols + col];
            if (col + 1 < p.cols) tile[r][2 * tx + 1] = in[(uint64_t)row * p.cols + col + 1];
        }
    }
    __syncthreads();
    for (uint32_t c = ty; c < 64; c += 8) {
        const uint32_t orow = tc + c, ocol = tr + 2 * tx;  // out[orow][ocol] = in[ocol][orow]
        if (orow < p.cols) {
            if (ocol < p.rows) out[(uint64_t)orow * p.rows + ocol] = tile[2 * tx][c];
            if (ocol + 1 < p.rows) out[(uint64_t)orow * p.rows + ocol + 1] = tile[2 * tx + 1][c];
        }
    }
}

POPCORN_KERNEL void __launch_bounds__(256) transpose2d_b16(const uint16_t *in, uint16_t *out, Transpose2DConstants p) {
    transpose2d_run(in, out, p);
}

#define GEMM_MFMA_SPLITK(name, T)                                                                 \
    POPCORN_KERNEL void __launch_bounds__(512)                                                    \
        name(const uint16_t *a, const uint16_t *b, float *partial, MatmulConstants p) {          \
        gemm_nt_direct<T, F32, 256, 384, 2, 4, true>(a, b, nullptr, p, partial);                  \
    }
#define GEMM_SPLITK_REDUCE(name, O)                                                                    \
    POPCORN_KERNEL void __launch_bounds__(256)                                                         \
        name(const float *partial, O::storage *c, MatmulConstants p, uint32_t splits) {                \
        gemm_splitk_reduce<O>(partial, c, p, splits);                                                  \
    }
#define GEMM_MFMA_SPLITK_E(name, T)                                                               \
    POPCORN_KERNEL void __launch_bounds__(512)                                                    \
        name(const uint16_t *a, const uint16_t *b, float *partial, MatmulConstants p) {          \
        gemm_nt_lines<T, F32, 256, 384, 2, 4, true>(a, b, nullptr, p, partial);                   \
    }
GEMM_MFMA_SPLITK(matmul_mfma_f16_splitk_d256x384, F16)
GEMM_MFMA_SPLITK(matmul_mfma_bf16_splitk_d256x384, BF16)
GEMM_MFMA_SPLITK_E(matmul_mfma_f16_splitk_e256x384, F16)
GEMM_MFMA_SPLITK_E(matmul_mfma_bf16_splitk_e256x384, BF16)
GEMM_SPLITK_REDUCE(matmul_splitk_reduce_f16, F16)
GEMM_SPLITK_REDUCE(matmul_splitk_reduce_bf16, BF16)
GEMM_SPLITK_REDUCE(matmul_splitk_reduce_f32, F32)
