/*
 * popcorn_oracle.h — CPU restatement of the reference's decode hot path.
 *
 * TEST INFRASTRUCTURE ONLY. This library is the checker for the HIP kernels in
 * popcorn_amd/. Only tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg may load it; no product code path calls it.
 *
 * Every function restates, in scalar f32 C with sequential summation (built
 * with -ffp-contract=off, no fast-math), either the Swift CPU reference loop
 * the reference's tests use or the Metal kernel's documented semantics. The
 * cited file:line is relative to the reference tree (finnvoor/Popcorn).
 *
 * Pinning status of each function (what checks it besides its own formula):
 *   xorshift64 / fa_test_float  - first outputs vs a hand-computed golden
 *                                 fixture, and the reference's FA test inputs
 *   fill_normal                 - moments + tail fractions (closed form)
 *   bf16 / f16 conversions      - bit patterns vs numpy / IEEE special cases
 *   kv_cache_write              - reference KAT (KernelsTests.swift:551-564)
 *   rmsnorm                     - reference KATs (KernelsTests.swift:142-175)
 *                                 + constant-row closed form
 *   matmul / matvec             - reference KATs (58,64,139,154) + exact
 *                                 integer sums vs numpy int64
 *   gelu_tanh                   - reference KAT values (KernelsTests.swift:106-117)
 *   attention_naive             - one-hot GQA KAT (KernelsTests.swift:510-547),
 *                                 softmax of a constant row, numpy float64 brute force
 *   flash_decoding / flash_attention_rows - equal to attention_naive for every
 *                                 P / tile split (invariance), empty partitions
 *   gated_mlp                   - equal to its own composition of the pinned
 *                                 pieces (rmsnorm, matvec, gelu, mul) on the
 *                                 same inputs, and to numpy float64
 *   argmax / embedding_gather   - reference KAT (KernelsTests.swift:121-138),
 *                                 tie-break on equal values
 *   rope_build_cos_sin / rope_apply - reference KAT (KernelsTests.swift:438-489);
 *                                 cos^2 + sin^2 = scaling^2; rotation keeps each
 *                                 pair's norm; rotating by +p then -p, and by
 *                                 p1 then p2 vs p1 + p2 (numpy float64)
 *   transpose12                 - numpy transpose (0, 2, 1, 3); applied twice
 *                                 with swapped dims is the identity
 *   aq_unpack / aq_matmul / aq_embedding_gather - a hand-packed word's bit
 *                                 layout; numpy float64 of the dequantized
 *                                 product; exact integer products; the
 *                                 s*sum(xq) + b*sum(x) identity; numpy f32
 *                                 dequantization (the reference's tests hold
 *                                 no quantized case)
 *   decode_step                 - composition of the pinned pieces; numpy
 *                                 float64 forward of a tiny layer (with and
 *                                 without the q/k/v norms and RoPE)
 */
#ifndef POPCORN_ORACLE_H
#define POPCORN_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* dtype tags, same numbering as include/popcorn_hip.h (POPCORN_DTYPE_*) */
enum { ORACLE_F32 = 8, ORACLE_F16 = 9, ORACLE_BF16 = 10 };

/* ---- generators ---------------------------------------------------------- */
uint64_t oracle_xorshift64_next(uint64_t *state);
float oracle_fa_test_float(uint64_t *state);
void oracle_fill_fa_test(uint64_t seed, float *out, size_t n);
void oracle_fill_normal(uint64_t seed, float mean, float stddev, float *out, size_t n);

/* ---- element conversions ------------------------------------------------- */
uint16_t oracle_f32_to_bf16(float x);
float oracle_bf16_to_f32(uint16_t b);
uint16_t oracle_f32_to_f16(float x);
float oracle_f16_to_f32(uint16_t h);
void oracle_convert(const void *src, int src_dtype, void *dst, int dst_dtype, size_t n);

/* ---- kernels ------------------------------------------------------------- */
int oracle_kv_cache_write(const void *src, int src_dtype, void *cache, int cache_dtype,
                          uint32_t B, uint32_t Nkv, uint32_t Snew, uint32_t Smax,
                          uint32_t Hd, uint32_t offset);

void oracle_rmsnorm(const float *x, const float *weight, float *out, size_t rows,
                    size_t H, float eps, int add_one_to_weight);

void oracle_matmul(const float *a, const float *b, float *c, size_t M, size_t K,
                   size_t N, int transpose_b);

float oracle_gelu_tanh_scalar(float v);
void oracle_gelu_tanh(const float *x, float *out, size_t n);
void oracle_mul(const float *a, const float *b, float *out, size_t n);
void oracle_add(const float *a, const float *b, float *out, size_t n);
void oracle_scalar_mul(const float *a, float s, float *out, size_t n);

void oracle_gated_mlp(const float *x, const float *norm_w, float eps, int add_one,
                      const float *w_gate, const float *w_up, const float *w_down,
                      size_t H, size_t F, int inter_dtype, float *h_out, float *out);

void oracle_attention_naive(const float *q, const float *k, const float *v, float *out,
                            uint32_t B, uint32_t Nq, uint32_t Nkv, uint32_t Sq,
                            uint32_t Sk, uint32_t kv_stride, uint32_t Hd, float scale,
                            uint32_t mask_kind, int32_t window);

void oracle_flash_decoding(const float *q, const float *k, const float *v, float *out,
                           uint32_t B, uint32_t Nq, uint32_t Nkv, uint32_t Sk,
                           uint32_t kv_stride, uint32_t Hd, uint32_t P, float scale,
                           uint32_t mask_kind, int32_t window, float *partial_o,
                           float *partial_m, float *partial_l);

void oracle_flash_attention_rows(const float *q, const float *k, const float *v,
                                 float *out, uint32_t B, uint32_t Nq, uint32_t Nkv,
                                 uint32_t Sq, uint32_t Sk, uint32_t kv_stride,
                                 uint32_t Hd, uint32_t Bc, float scale,
                                 uint32_t mask_kind, int32_t window);

void oracle_rope_build_cos_sin(const int32_t *positions, const float *inv_freq, float *cos_out,
                               float *sin_out, uint32_t T, uint32_t Hd2, float scaling);
void oracle_rope_apply(const float *x, const float *cos_tab, const float *sin_tab, float *out,
                       uint32_t B, uint32_t T, uint32_t Nh, uint32_t Hd2);
void oracle_transpose12(const float *src, float *out, uint32_t D0, uint32_t D1, uint32_t D2,
                        uint32_t D3);

uint32_t oracle_aq_unpack(const uint32_t *words, size_t i, int bits);
void oracle_aq_matmul(const float *x, const uint32_t *packed, const float *scales, const float *biases,
                      float *y, size_t M, size_t N, size_t K, int bits, int group);
void oracle_aq_embedding_gather(const int32_t *ids, const uint32_t *packed, const float *scales,
                                const float *biases, float *out, size_t T, size_t H, int bits,
                                int group);

void oracle_argmax(const float *x, size_t rows, size_t N, int32_t *indices);
void oracle_embedding_gather(const int32_t *ids, const float *table, float *out,
                             size_t N, size_t H);

/* One decoder layer at batch 1 decode (Sq = 1), activations rounded to
 * `act_dtype` at every point where the reference stores a tensor. */
typedef struct {
    uint32_t H, Nq, Nkv, Hd, F;
    uint32_t kv_capacity;     /* row stride of the caches                       */
    float eps, scale;
    int act_dtype;            /* ORACLE_F32 or ORACLE_BF16                      */
    const float *w_in_norm;   /* [H]                                            */
    const float *w_qkv;       /* [(Nq+2Nkv)*Hd, H]                              */
    const float *w_o;         /* [H, Nq*Hd]                                     */
    const float *w_post_attn_norm; /* [H]                                       */
    const float *w_pre_ffn_norm;   /* [H]                                       */
    const float *w_gate, *w_up;    /* [F, H]                                    */
    const float *w_down;      /* [H, F]                                         */
    const float *w_post_ffn_norm;  /* [H]                                       */
    /* a real attention block (all optional: NULL / 0 = left out) */
    const float *w_q_norm;    /* [Hd] per-head RMSNorm of q                     */
    const float *w_k_norm;    /* [Hd] per-head RMSNorm of k                     */
    int v_norm;               /* 1: per-head RMSNorm of v without weight        */
    const float *inv_freq;    /* [Hd/2]: RoPE on q and k at position pos        */
    float rope_scaling;
} oracle_layer_t;

void oracle_decoder_layer(const oracle_layer_t *L, float *x, float *k_cache,
                          float *v_cache, uint32_t pos);

#ifdef __cplusplus
}
#endif
#endif
