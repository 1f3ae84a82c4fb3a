/*
 * popcorn_kernel_types.h — kernel parameter blocks shared by the host runtime
 * and the gfx950 kernels.
 *
 * A struct named as in the reference's
 * Sources/PopcornShaderTypes/PopcornKernelTypes.h (cited per struct) has
 * exactly the reference's fields in the reference's order, and the kernels
 * exported under the reference's host names take exactly it, so a caller
 * that packs the reference's constants for a raw launch packs these. Where a
 * kernel of this build needs more, it takes a struct of its own (suffix Ext,
 * or a name of its own): the reference's fields first, then the additions.
 * Fields are 4 bytes (FillNormalConstants' counters are 8); none of the
 * structs has padding.
 */
#ifndef POPCORN_KERNEL_TYPES_H
#define POPCORN_KERNEL_TYPES_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* PopcornKernelTypes.h:10-13 */
typedef struct {
    uint32_t N;
    uint32_t H;
} EmbeddingGatherConstants;

/* EmbeddingGatherConstants plus V (table rows; 0 = unchecked): an id outside
 * [0, V) yields a zero row instead of an out-of-bounds read
 * (embedding_gather*_ext). */
typedef struct {
    uint32_t N;
    uint32_t H;
    uint32_t V;
} EmbeddingGatherExtConstants;

/* PopcornKernelTypes.h:15-18 */
typedef struct {
    uint32_t count;
    float scalar;
} ScalarMulConstants;

/* PopcornKernelTypes.h:20-22 */
typedef struct {
    uint32_t count;
} MulConstants;

/* PopcornKernelTypes.h:24-26 */
typedef struct {
    uint32_t count;
} AddConstants;

/* PopcornKernelTypes.h:33-35 */
typedef struct {
    uint32_t count;
} GeluTanhConstants;

/* PopcornKernelTypes.h:46-51 */
typedef struct {
    uint32_t M;
    uint32_t K;
    uint32_t N;
    uint32_t transposeB;
} MatmulConstants;

/* PopcornKernelTypes.h:53-57 */
typedef struct {
    uint32_t K;
    uint32_t N;
    uint32_t transposeW;
} MatvecConstants;

/* PopcornKernelTypes.h:72-77 */
typedef struct {
    uint32_t H;
    uint32_t hasWeight;
    uint32_t addOneToWeight;
    float eps;
} RMSNormConstants;

/* PopcornKernelTypes.h:121-131 */
typedef struct {
    uint32_t B;
    uint32_t Nq;
    uint32_t Nkv;
    uint32_t Sq;
    uint32_t Sk;
    uint32_t Hd;
    uint32_t maskKind;
    int32_t slidingWindow;
    float scale;
} FlashAttentionConstants;

/* PopcornKernelTypes.h:133-144 (the reference's MPP kernels have no
 * counterpart here; kept for callers that pack it). */
typedef struct {
    uint32_t B;
    uint32_t Nq;
    uint32_t Nkv;
    uint32_t Sq;
    uint32_t Sk;
    uint32_t Hd;
    uint32_t qTilesPerHead;
    uint32_t maskKind;
    int32_t slidingWindow;
    float scale;
} MPPFlashAttentionConstants;

/* The MFMA prefill kernel's constants (flash_attention_tiled_*, the kernel
 * in the MPP route's place): MPPFlashAttentionConstants' fields, plus
 *   Hd         the head dim, at most the kernel's (_d64/_d128/_d256/_d512)
 *              and a multiple of 8: rows of Q, K, V and O are Hd apart, and
 *              the kernel's dims past Hd are zeros;
 *   kvStride   rows between consecutive KV heads in K/V (0 = Sk);
 *   splitFrom  splitFrom >= qTilesPerHead: one block per query tile.
 *              Otherwise tiles qt >= splitFrom are split in two parts, each
 *              written as partial (O, m, l) for the split-merge kernel:
 *   pairTiles  0: the split tiles run as two blocks over the halves of their
 *              key steps (qTilesPerHead + split tiles blocks per head);
 *              1 (causal, splitFrom = qTilesPerHead - qTilesPerHead / 2):
 *              tile i is paired with tile qTilesPerHead - 1 - i and each
 *              pair runs as two blocks of equal work, tile i and the first
 *              steps of its partner, then the partner's remaining steps
 *              (qTilesPerHead blocks per head);
 *              2: pairs as for 1, but the first
 *              block of a pair runs its steps of the partner first and
 *              publishes them (partial O and (m, l) of part 0 in the pO and
 *              pML buffers, then the split tile's 64-bit ready flag in
 *              pairFlags), and the second block merges them into the output
 *              itself: no split-merge kernel. pO, pML and pairFlags must be
 *              uncached device memory (popcorn_malloc_uncached): the two
 *              blocks may sit on XCDs whose L2 caches are not coherent.
 *              pairFlags (u64) holds the abort word at index 0 and the flag
 *              of split tile t at index 1 + t; all start at 0;
 *              The _d512 kernels (64 query rows per block, 256 threads)
 *              run every tile whole whatever splitFrom and pairTiles say;
 *   ticketLo, ticketHi  pairTiles 2: the 64-bit value (neither 0 nor
 *              ~0) the first block sets its flag to, by compare-and-swap
 *              from 0, distinct per launch; the merging block resets the
 *              flag to 0. A merging block that gives up (0.2 s, or a flag
 *              holding a value other than 0 and the ticket) sets the flag
 *              to ~0, the abort word to 1 and its rows to NaN. */
typedef struct {
    uint32_t B;
    uint32_t Nq;
    uint32_t Nkv;
    uint32_t Sq;
    uint32_t Sk;
    uint32_t Hd;
    uint32_t qTilesPerHead;
    uint32_t maskKind;
    int32_t slidingWindow;
    float scale;
    uint32_t kvStride;
    uint32_t splitFrom;
    uint32_t pairTiles;
    uint32_t ticketLo;
    uint32_t ticketHi;
} TiledFlashAttentionConstants;

/* PopcornKernelTypes.h:146-156 */
typedef struct {
    uint32_t B;
    uint32_t Nq;
    uint32_t Nkv;
    uint32_t Sk;
    uint32_t Hd;
    uint32_t P;
    uint32_t maskKind;
    int32_t slidingWindow;
    float scale;
} FlashDecodingPartialConstants;

/* FlashDecodingPartialConstants plus (flash_decoding_partial_*_ext, the fast
 * flash_decoding_partial_<t>_l*_c*_g* and flash_decoding_fresh_* kernels):
 *   kvStride       rows between consecutive KV heads in K/V (0 = Sk), so a
 *                  cache with spare capacity [B, Nkv, Smax, Hd] is read in
 *                  place;
 *   Sq             query rows (0 = 1); row r attends as position Sk - Sq + r;
 *   keyLenFromPosition  when 1, Sk = position[0] + Sq is read from the bound
 *                  position tensor (decode under graph replay). */
typedef struct {
    uint32_t B;
    uint32_t Nq;
    uint32_t Nkv;
    uint32_t Sk;
    uint32_t Hd;
    uint32_t P;
    uint32_t maskKind;
    int32_t slidingWindow;
    float scale;
    uint32_t kvStride;
    uint32_t Sq;
    uint32_t keyLenFromPosition;
} FlashDecodingPartialExtConstants;

/* No counterpart in the reference: the attention block of one decode token
 * with the per-head glue folded into the split-KV partial kernel
 * (flash_decoding_fresh_*). The projections arrive raw in one row per batch
 * entry of rowStride elements: Nq query heads, then Nkv key heads, then Nkv
 * value heads, Hd each. flags:
 *   bit 0  q = RMSNorm(q; w_q) per head   (Gemma4TextInference.swift:353)
 *   bit 1  k = RMSNorm(k; w_k) per head   (:367)
 *   bit 2  v = RMSNorm(v) per head, no weight (:368)
 *   bit 3  RoPE on q and k with angle = float(position) * inv_freq[i],
 *          tables scaled by ropeScaling (:354, :369; RopeBuildCosSin.metal)
 * Each step's result is rounded to the storage dtype, as the reference
 * stores each intermediate. The processed key and value rows are written to
 * the caches at row `position` and attended as the last key. */
typedef struct {
    uint32_t flags;
    float eps;
    float ropeScaling;
    uint32_t rowStride;
} DecodeAttentionConstants;

/* PopcornKernelTypes.h:158-163 */
typedef struct {
    uint32_t B;
    uint32_t Nq;
    uint32_t Hd;
    uint32_t P;
} FlashDecodingReduceConstants;

/* FlashDecodingReduceConstants plus Sq (query rows; 0 = 1)
 * (flash_decoding_reduce_*_ext). */
typedef struct {
    uint32_t B;
    uint32_t Nq;
    uint32_t Hd;
    uint32_t P;
    uint32_t Sq;
} FlashDecodingReduceExtConstants;

/* PopcornKernelTypes.h:165-172 */
typedef struct {
    uint32_t B;
    uint32_t Nkv;
    uint32_t Snew;
    uint32_t Smax;
    uint32_t Hd;
    uint32_t offset;
} KVCacheWriteConstants;

/* KVCacheWriteConstants plus offsetFromPosition (kv_cache_write*_ext): when 1
 * the write offset is read from the bound position tensor, and a range that
 * would leave the cache writes nothing. */
typedef struct {
    uint32_t B;
    uint32_t Nkv;
    uint32_t Snew;
    uint32_t Smax;
    uint32_t Hd;
    uint32_t offset;
    uint32_t offsetFromPosition;
} KVCacheWriteExtConstants;

/* PopcornKernelTypes.h:174-178: RoPE tables for T positions and Hd2 = Hd/2
 * frequencies, both scaled by `scaling`. */
typedef struct {
    uint32_t T;
    uint32_t Hd2;
    float scaling;
} RopeBuildCosSinConstants;

/* PopcornKernelTypes.h:180-185: half-rotation RoPE over x [B, T, Nh, 2*Hd2]. */
typedef struct {
    uint32_t B;
    uint32_t T;
    uint32_t Nh;
    uint32_t Hd2;
} RopeApplyConstants;

/* PopcornKernelTypes.h:216-221: [D0, D1, D2, D3] -> [D0, D2, D1, D3]. */
typedef struct {
    uint32_t D0;
    uint32_t D1;
    uint32_t D2;
    uint32_t D3;
} Transpose12Constants;

/* PopcornKernelTypes.h:240-247: y[M, N] = x[M, K] W^T with W block-affine
 * 4-bit (u32 words of 8 values, lowest index in the lowest bits; one
 * scale/bias pair per kGroups group of the row), wordsPerRow = K / 8. */
typedef struct {
    uint32_t M;
    uint32_t N;
    uint32_t K;
    uint32_t kGroups;
    uint32_t wordsPerRow;
    uint32_t hasBias;
} AffineQMatmulConstants;

/* PopcornKernelTypes.h:249-255: out[T, H] = dequantize(table[ids[t], :]). */
typedef struct {
    uint32_t T;
    uint32_t H;
    uint32_t kGroups;
    uint32_t wordsPerRow;
    uint32_t hasBias;
} AffineQEmbeddingGatherConstants;

/* AffineQEmbeddingGatherConstants plus V (table rows; 0 = unchecked): an id
 * outside [0, V) yields a zero row instead of an out-of-bounds read
 * (aq_embedding_gather_*_ext). */
typedef struct {
    uint32_t T;
    uint32_t H;
    uint32_t kGroups;
    uint32_t wordsPerRow;
    uint32_t hasBias;
    uint32_t V;
} AffineQEmbeddingGatherExtConstants;

/* PopcornKernelTypes.h:197-200 */
typedef struct {
    uint32_t rows;
    uint32_t N;
} ArgmaxConstants;

/* ArgmaxConstants plus slices: the number of row slices this build's
 * two-stage argmax (argmax_partial, argmax_finish) splits each row into. */
typedef struct {
    uint32_t rows;
    uint32_t N;
    uint32_t slices;
} ArgmaxSliceConstants;

/* No counterpart in the reference: the fused gated-MLP front half
 * (RMSNorm -> gate and up matvecs -> GELU-tanh(gate) * up), which replaces the
 * reference's five-dispatch composition. interDataType is the storage dtype of
 * the reference's intermediates (POPCORN_DTYPE_*): each intermediate is
 * rounded to it exactly where the reference stores a tensor. */
typedef struct {
    uint32_t H;
    uint32_t F;
    uint32_t hasWeight;
    uint32_t addOneToWeight;
    float eps;
    uint32_t interDataType;
    uint32_t residual;  /* 1: x = x_in + RMSNorm(delta; w_post) first (see below) */
} GatedMLPConstants;

/* No counterpart in the reference: the decode-step matvec y = W x (W [N, K])
 * with the neighbouring glue of a decoder layer folded in. flags:
 *   bit 0  residual: x = round(x_in + round(RMSNorm(delta; w_post))), the
 *          reference's post-norm + residual Add (Gemma4TextInference.swift:
 *          400-404, :430-434); block 0 stores x to x_out;
 *   bit 1  pre-norm: the vector multiplied is round(RMSNorm(x; w_pre)), the
 *          reference's input norm (:334, :416);
 *   bit 2  KV scatter: rows [qRows, qRows + kvRows) go to the K cache and the
 *          next kvRows rows to the V cache, at row position[0] of each KV
 *          head (head = (row - start) / headDim), the reference's KV-cache
 *          writes (:372-381); rows below qRows go to out.
 * Rounding points use interDataType (the storage dtype of the reference's
 * intermediates). */
typedef struct {
    uint32_t K;
    uint32_t N;
    float eps;
    uint32_t flags;
    uint32_t interDataType;
    uint32_t qRows;
    uint32_t kvRows;
    uint32_t headDim;
    uint32_t kvStride;
} DecodeMatvecConstants;

/* No counterpart in the reference: device-side fill of synthetic inputs
 * (counter-based normal generator) for benchmarks. */
typedef struct {
    uint64_t seed;
    uint64_t count;
    float mean;
    float stddev;
} FillNormalConstants;

/* No counterpart in the reference (GemmaCLI picks the token and writes the
 * position from the CPU, Gemma4TextInference.swift:95-99): the end of a
 * captured greedy decode step in one launch, so graph replays need no host
 * write. From stage-1 argmax candidates (slices of them, over N
 * logits) it picks the token (Argmax.metal's tie and NaN rules), records it
 * in the history ring (historyLen entries, index = position), advances the
 * position by delta, and writes the next step's input row: the token's
 * embedding row (H values; 4-bit rows dequantised as q * scale + bias,
 * rounded to bf16 as the gather stores it) times `scale`, rounded to bf16
 * (EmbeddingGather then ScalarMul, Gemma4TextInference.swift:184-185). */
typedef struct {
    uint32_t N;
    uint32_t slices;
    uint32_t H;
    uint32_t historyLen;
    int32_t delta;
    float scale;
    uint32_t hasBias;
} DecodeNextTokenConstants;

/* No counterpart in the reference: out[cols, rows] = in[rows, cols]^T for
 * 16-bit elements, so a Matmul with a non-transposed 16-bit B (the
 * reference's mpp_matmul without _tb, Matmul.swift:203-214) can run the
 * transposed-B matrix-core kernels. */
typedef struct {
    uint32_t rows;
    uint32_t cols;
} Transpose2DConstants;

#ifdef __cplusplus
}
#endif
#endif
