// Skinny Matmul on the matrix cores, 2 <= M <= 64: C[M, N] = A[M, K] . B[N, K]^T
// with 16-bit A and B (the reference's transposeB layout), f32 accumulation,
// C in f32 or the input dtype (popcorn_store rounding). This is the role of
// the reference's small-M MPP tiles (TileM 8/16/32, Matmul.swift:175-196,
// MPPMatmul.metal:19-91): an 8-token prompt or an 8-wide decode batch, where
// B (the weights) is read once and the time is the stream of its bytes.
//
// The product is computed transposed, C^T = B . A^T, on
// v_mfma_f32_16x16x32_{f16,bf16} (lane layout in mfma.hpp): 16 rows of B
// are the A operand, 16 rows of A (M padded to 16, 32, 48 or 64 in MT
// tiles) the B operand, so both are 16-byte runs along K of one row and a
// lane's fragment is one 16-byte load: lane l reads row l % 16 at
// k0 + (l / 16) * 8. A block takes 32 rows of B (two 16-row tiles, so each
// A fragment serves two products), or 16 rows in the _r16 kernels, which
// the host picks when 32-row blocks would be fewer than the CUs (N < 8192:
// M 8, K 9216, N 2304 23.7 -> 15.8 us; M 32, K 2304, N 4096 12.5 -> 9.1
// us); its W waves split K, each wave a
// contiguous run of k-steps of 32 with U steps in flight, and sum their
// partial C^T tiles in LDS at the end. A (M x K, a few tens of KB) is read
// from L2 beside B. Rows past N or M read a valid row and are not stored;
// K % 8 == 0, so a chunk lies wholly inside or outside K and the chunks past
// it are zeros in both operands.
#include <type_traits>

#include "mfma.hpp"

namespace {

using pk::f32x4;
using pk::Mma16;
using pk::u32x4;

constexpr int U = 4;                  // k-steps in flight per wave
constexpr int kMaxWaves = 8;          // waves per block (K split)
constexpr int kRedFloats = 16384;     // LDS for the partial tiles: W x NT x MT x 256 floats

template <typename T, typename O, int MT, int NT>  // NT: 16-row tiles of B per block
__device__ void gemm_skinny(const uint16_t *__restrict__ A, const uint16_t *__restrict__ B,
                            typename O::storage *__restrict__ C, const MatmulConstants &p) {
    static_assert(kMaxWaves * NT * MT * 256 <= kRedFloats, "LDS for the partial tiles");
    __shared__ __attribute__((aligned(16))) float red[kRedFloats];

    const uint32_t lane = threadIdx.x & 63, wave = threadIdx.x >> 6, W = blockDim.x >> 6;
    const uint32_t M = p.M, K = p.K, N = p.N;
    const uint32_t r = lane & 15, g = lane >> 4;
    const uint32_t n0 = blockIdx.x * (16 * NT);
    // Buffer loads (the host keeps A and B under 4 GB): byte offsets of this
    // lane's rows. As intrinsic calls they also stay where they are issued
    // (plain loads of a loop-carried ring are folded into one load at the
    // point of use, which would drain the queue every step).
    const __amdgpu_buffer_rsrc_t rsB =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t *>(B), 0, (int)(N * K * 2u), 0x00020000);
    const __amdgpu_buffer_rsrc_t rsA =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t *>(A), 0, (int)(M * K * 2u), 0x00020000);
    uint32_t boff[NT], aoff[MT];
#pragma unroll
    for (int t = 0; t < NT; ++t) boff[t] = min(n0 + 16 * t + r, N - 1) * K * 2u;
#pragma unroll
    for (int u = 0; u < MT; ++u) aoff[u] = min(16u * u + r, M - 1) * K * 2u;

    f32x4 acc[NT][MT];
#pragma unroll
    for (int t = 0; t < NT; ++t)
#pragma unroll
        for (int u = 0; u < MT; ++u) acc[t][u] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};

    // this wave's k-steps: a contiguous run of KS / W (rounded up)
    const uint32_t KS = (K + 31) / 32;
    const uint32_t SPW = (KS + W - 1) / W;
    const uint32_t first = wave * SPW;
    const uint32_t nsteps = first < KS ? min(SPW, KS - first) : 0u;
    // Every load reads a valid address (a step past the wave's last reads
    // its last, a chunk past K the row's last chunk), so every path issues
    // the same loads and the wait counts stay exact; what lies outside is
    // replaced by zeros in both operands. The scheduling barriers hold the
    // loads in this order in the prologue and in the loop alike, so the
    // compiler's wait before each step counts the same loads in flight on
    // entry and around the loop (otherwise the loop header merges two orders
    // and waits for everything).
    u32x4 bf[U][NT], af[U][MT];
    auto issue = [&](int slot, uint32_t q) {
        const uint32_t s = first + min(q, nsteps ? nsteps - 1 : 0u);
        const uint32_t k2 = min(s * 32 + g * 8, K - 8) * 2u;
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int t = 0; t < NT; ++t)
            bf[slot][t] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rsB, boff[t] + k2, 0, 0));
#pragma unroll
        for (int u = 0; u < MT; ++u)
            af[slot][u] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rsA, aoff[u] + k2, 0, 0));
        __builtin_amdgcn_sched_barrier(0);
    };
    const u32x4 zero = {0u, 0u, 0u, 0u};
#pragma unroll
    for (int j = 0; j < U; ++j) issue(j, j);
    // Step q of slot j: data out of range replaced by zeros; the selects
    // also place real instructions on the slot's registers before the refill
    // reuses them, so each step waits only for its own loads.
    for (uint32_t q0 = 0; q0 < nsteps; q0 += U) {
#pragma unroll
        for (int j = 0; j < U; ++j) {
            const uint32_t q = q0 + j;
            const bool in = q < nsteps && (first + q) * 32 + g * 8 < K;
            u32x4 b[NT], a[MT];
#pragma unroll
            for (int t = 0; t < NT; ++t) b[t] = in ? bf[j][t] : zero;
#pragma unroll
            for (int u = 0; u < MT; ++u) a[u] = in ? af[j][u] : zero;
            issue(j, q + U);
#pragma unroll
            for (int t = 0; t < NT; ++t)
#pragma unroll
                for (int u = 0; u < MT; ++u) acc[t][u] = Mma16<T>::run(b[t], a[u], acc[t][u]);
        }
    }

    // partial tiles to LDS: [wave][t][u][element i][lane], then every
    // thread sums the waves' values of some (t, u, lane, i) and stores them:
    // C^T element i of lane l in tile (t, u) is row n0 + 16 t + (l / 16) * 4 + i
    // of B, row 16 u + l % 16 of A
    constexpr int kTile = NT * MT * 256;
#pragma unroll
    for (int t = 0; t < NT; ++t)
#pragma unroll
        for (int u = 0; u < MT; ++u)
#pragma unroll
            for (int i = 0; i < 4; ++i) red[wave * kTile + ((t * MT + u) * 4 + i) * 64 + lane] = acc[t][u][i];
    __syncthreads();
    for (uint32_t e = threadIdx.x; e < (uint32_t)kTile; e += blockDim.x) {
        float v = 0.0f;
        for (uint32_t w = 0; w < W; ++w) v += red[w * kTile + e];
        const uint32_t l = e & 63, i = (e >> 6) & 3, tu = e >> 8;
        const uint32_t t = tu / MT, u = tu % MT;
        const uint32_t n = n0 + 16 * t + (l >> 4) * 4 + i, m = 16 * u + (l & 15);
        if (n < N && m < M) C[(uint64_t)m * N + n] = O::store(v);
    }
}

// ---- A staged in LDS ("_lds", at least 512 tiles of 16 rows of B) ---------
// The kernel above loads each A fragment from L2 beside the B fragment it
// multiplies, and those loads slow the stream of B (4.45 -> 3.0 TB/s in a
// load-pattern test). Here each wave streams one 16-row tile of B over the
// whole of K with UL k-steps in flight, and the block's W waves stage A (M
// padded to 16 MT rows) in LDS one chunk of KC values of K at a time:
// double-buffered, direct buffer -> LDS copies of whole 512-byte row runs,
// chunk j of row a in slot j ^ (a & 15) so the 16 rows a fragment read
// touches cover all banks. Config shape M 8, K 2304, N 9216: 14.1 -> 11.4
// us; M 64: 30.9 -> 17.0 us.
constexpr int KC = 256;  // K values per A chunk: 8 k-steps
constexpr int UL = 16;   // k-steps of B in flight per wave
constexpr uint32_t kOOR = 0x80000000u;  // a buffer offset past every operand: zeros, no memory read
typedef __attribute__((address_space(3))) void lds_void;

template <int N>
__device__ inline void wait_vm() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}

template <typename T, typename O, int MT, int W>
__device__ void gemm_skinny_lds(const uint16_t *__restrict__ A, const uint16_t *__restrict__ B,
                                typename O::storage *__restrict__ C, const MatmulConstants &p) {
    constexpr int kChunkB = 16 * MT * KC * 2;  // bytes of A per chunk
    constexpr int kCopies = kChunkB / 1024;    // copy instructions per chunk, 2 rows each
    static_assert(kCopies % W == 0, "copies per wave");
    constexpr int kCPW = kCopies / W;
    // the two chunk buffers are separate arrays, so the compiler sees that
    // the copies into one do not feed the reads of the other
    __shared__ __attribute__((aligned(16))) uint8_t sA0[kChunkB];
    __shared__ __attribute__((aligned(16))) uint8_t sA1[kChunkB];

    const uint32_t lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const uint32_t M = p.M, K = p.K, N = p.N;
    const uint32_t r = lane & 15, g = lane >> 4;
    const uint32_t n0 = (blockIdx.x * W + wave) * 16;
    const __amdgpu_buffer_rsrc_t rsB =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t *>(B), 0, (int)(N * K * 2u), 0x00020000);
    const __amdgpu_buffer_rsrc_t rsA =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t *>(A), 0, (int)(M * K * 2u), 0x00020000);
    const uint32_t boff = n0 + r < N ? (n0 + r) * K * 2u : kOOR;

    u32x4 bq[UL];
    // loads held in issue order by scheduling barriers, so the compiler's
    // wait before each step counts the same loads in flight everywhere
    auto issueB = [&](int slot, uint32_t q) {
        const uint32_t k = q * 32 + g * 8;
        __builtin_amdgcn_sched_barrier(0);
        bq[slot] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rsB, k < K ? boff + 2 * k : kOOR, 0, 0));
        __builtin_amdgcn_sched_barrier(0);
    };
    auto copyA = [&](uint32_t c, int parity) {
        uint8_t *dst = parity ? sA1 : sA0;
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int t = 0; t < kCPW; ++t) {
            const uint32_t i = t * W + wave;
            const uint32_t a = 2 * i + (lane >> 5), j = (lane & 31) ^ (a & 15);
            const uint32_t kk = c * KC + 8 * j;
            const uint32_t off = (a < M && kk < K) ? (a * K + kk) * 2u : kOOR;
            __builtin_amdgcn_raw_ptr_buffer_load_lds(rsA, (lds_void *)(dst + i * 1024), 16, off, 0, 0, 0);
        }
        __builtin_amdgcn_sched_barrier(0);
    };

    f32x4 acc[MT];
#pragma unroll
    for (int u = 0; u < MT; ++u) acc[u] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};

    const uint32_t NC = (K + KC - 1) / KC;
    copyA(0, 0);
#pragma unroll
    for (int j = 0; j < UL; ++j) issueB(j, j);
    asm volatile("" ::: "memory");  // the prologue's loads stay ahead of the wait below
    wait_vm<UL>();  // this wave's copies of chunk 0 (issued before the UL steps of B)
    __builtin_amdgcn_s_barrier();
    // One chunk: its 8 k-steps use ring slots base .. base + 7 (chunks
    // alternate halves of the ring). The copies of the next chunk go out
    // first and land before the barrier that ends the chunk. Every path
    // issues the same loads (past K they read out of range: zeros, no
    // memory traffic), so the compiler's waits count the ring exactly
    // around the loop; the chunk count is rounded up to even.
    auto chunk = [&](uint32_t c, int base) {
        const int parity = (base / 8) & 1;  // chunk c's buffer: c and base / 8 have the same parity
        copyA(c + 1, parity ^ 1);
        const uint8_t *buf = parity ? sA1 : sA0;
#pragma unroll
        for (int s = 0; s < 8; ++s) {
            const uint32_t q = c * 8 + s;
            u32x4 af[MT];
#pragma unroll
            for (int u = 0; u < MT; ++u) {
                const uint32_t a = 16 * u + r, j = 4 * s + g;
                af[u] = *reinterpret_cast<const u32x4 *>(buf + a * (KC * 2) + ((j ^ (a & 15)) << 4));
            }
            // the slot's products first, then its refill: the refill can
            // reuse the slot's registers, so the ring stays in place around
            // the loop (no moves that would wait for every load)
#pragma unroll
            for (int u = 0; u < MT; ++u) acc[u] = Mma16<T>::run(bq[base + s], af[u], acc[u]);
            issueB(base + s, q + UL);
        }
        wait_vm<8>();  // the next chunk's copies: only this chunk's 8 refills may be outstanding
        __builtin_amdgcn_s_barrier();
    };
    static_assert(UL % 16 == 0, "an even number of chunks per ring (compile-time buffer parity)");
    // at least one pass (a wave with no K range reads zeros), so no branch
    // separates the prologue's loads from the loop
    uint32_t c = 0;
    do {
#pragma unroll
        for (int h = 0; h < UL / 8; ++h) chunk(c + h, 8 * h);
        c += UL / 8;
    } while (c < NC);
    wait_vm<0>();  // the ring's refills past K (zeros) before the wave ends

    // C^T element i of lane l in tile u: row n0 + 4 (l / 16) + i of B, row 16 u + l % 16 of A
#pragma unroll
    for (int u = 0; u < MT; ++u)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const uint32_t n = n0 + 4 * g + i, m = 16 * u + r;
            if (n < N && m < M) C[(uint64_t)m * N + n] = O::store(acc[u][i]);
        }
}

}  // namespace

#define GEMM_SKINNY(name, T, O, MT, NT)                                                                   \
    POPCORN_KERNEL void __launch_bounds__(64 * kMaxWaves)                                                 \
        name(const uint16_t *a, const uint16_t *b, O::storage *c, MatmulConstants p) {                    \
        gemm_skinny<T, O, MT, NT>(a, b, c, p);                                                            \
    }
#define GEMM_SKINNY_M(t, T, o, O)                                        \
    GEMM_SKINNY(matmul_skinny_##t##_##t##_##o##_m16, T, O, 1, 2)         \
    GEMM_SKINNY(matmul_skinny_##t##_##t##_##o##_m32, T, O, 2, 2)         \
    GEMM_SKINNY(matmul_skinny_##t##_##t##_##o##_m48, T, O, 3, 2)         \
    GEMM_SKINNY(matmul_skinny_##t##_##t##_##o##_m64, T, O, 4, 2)         \
    GEMM_SKINNY(matmul_skinny_##t##_##t##_##o##_m16_r16, T, O, 1, 1)     \
    GEMM_SKINNY(matmul_skinny_##t##_##t##_##o##_m32_r16, T, O, 2, 1)     \
    GEMM_SKINNY(matmul_skinny_##t##_##t##_##o##_m48_r16, T, O, 3, 1)     \
    GEMM_SKINNY(matmul_skinny_##t##_##t##_##o##_m64_r16, T, O, 4, 1)

using pk::BF16;
using pk::F16;
using pk::F32;

GEMM_SKINNY_M(f16, F16, f16, F16)
GEMM_SKINNY_M(f16, F16, f32, F32)
GEMM_SKINNY_M(bf16, BF16, bf16, BF16)
GEMM_SKINNY_M(bf16, BF16, f32, F32)

// A in LDS: one wave per block at M <= 16 (its A is 16 rows), four waves
// sharing the staged A above that
#define GEMM_SKINNY_LDS(name, T, O, MT, W)                                                                \
    POPCORN_KERNEL void __launch_bounds__(64 * W)                                                         \
        name(const uint16_t *a, const uint16_t *b, O::storage *c, MatmulConstants p) {                    \
        gemm_skinny_lds<T, O, MT, W>(a, b, c, p);                                                         \
    }
#define GEMM_SKINNY_LDS_M(t, T, o, O)                                         \
    GEMM_SKINNY_LDS(matmul_skinny_##t##_##t##_##o##_m16_lds, T, O, 1, 1)      \
    GEMM_SKINNY_LDS(matmul_skinny_##t##_##t##_##o##_m32_lds, T, O, 2, 4)      \
    GEMM_SKINNY_LDS(matmul_skinny_##t##_##t##_##o##_m48_lds, T, O, 3, 4)      \
    GEMM_SKINNY_LDS(matmul_skinny_##t##_##t##_##o##_m64_lds, T, O, 4, 4)

GEMM_SKINNY_LDS_M(f16, F16, f16, F16)
GEMM_SKINNY_LDS_M(f16, F16, f32, F32)
GEMM_SKINNY_LDS_M(bf16, BF16, bf16, BF16)
GEMM_SKINNY_LDS_M(bf16, BF16, f32, F32)
