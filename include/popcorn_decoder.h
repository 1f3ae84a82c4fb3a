/*
 * popcorn_decoder.h — the batch-1 greedy decode loop over the hot-path
 * kernels (a Gemma-shaped decoder with random weights), as one native
 * component with a C ABI.
 *
 * It restates the per-token op sequence of the reference's example app
 * (Examples/GemmaCLI/Sources/GemmaCLI/Gemma4TextInference.swift:172-207 for
 * the forward, :312-436 for a layer) without the per-layer inputs and layer
 * scalars:
 *
 *   x = EmbeddingGather(token) * sqrt(H)                       (:184-185)
 *   per layer:  n = RMSNorm(x); qkv = n W_qkv^T;
 *               [attention_block: q = RoPE(RMSNorm_h(q)), k = RoPE(RMSNorm_h(k)),
 *                v = RMSNorm_h(v) per head                     (:352-371)]
 *               KVCacheWrite(k, v) at pos;
 *               a = FlashAttention(q, K[:pos+1], V[:pos+1]); o = a W_o^T;
 *               x = x + RMSNorm(o)                             (:334-404)
 *               x = x + RMSNorm(GatedMLP(x))                   (:408-436)
 *   logits = RMSNorm(x) E^T (tied embedding); token = Argmax(logits)
 *                                                              (:201-206)
 *
 * With attention_block = 0 the layer is the benchmark layer of the headline
 * decode configuration (no per-head norms or RoPE).
 *
 * The position and the token live in device memory and the step ends with a
 * kernel that picks the token, advances the position and writes the next
 * step's input row, so a step (or several) is captured once as a HIP graph
 * and replayed with no host work per token.
 */
#ifndef POPCORN_DECODER_H
#define POPCORN_DECODER_H

#include "popcorn_hip.h"

#ifdef __cplusplus
extern "C" {
#endif

typedef struct {
    int32_t layers;
    int32_t hidden;
    int32_t query_heads;
    int32_t kv_heads;
    int32_t head_dim;
    int32_t ffn;
    int32_t vocab;
    int32_t max_seq;      /* KV-cache capacity (rows per KV head)                */
    float eps;            /* RMSNorm epsilon                                     */
    float attn_scale;     /* attention scale                                     */
    int32_t history_len;  /* ring of generated tokens kept on the device         */
    int32_t graph_steps;  /* decode steps captured per HIP graph (0 = 1)         */
    int32_t attention_block; /* 1: per-head q/k RMSNorm (f32 weights), v RMSNorm
                                without weight and RoPE on q and k              */
    float rope_theta;     /* RoPE base: inv_freq[i] = theta^(-2i/head_dim)       */
    int32_t weight_bits;  /* 16 (or 0): bf16 weights; 4: block-affine 4-bit, group
                             64, bf16 scales and biases (the MLX format of
                             AffineQuantizedTensor.swift), embedding included  */
} popcorn_decoder_config_t;

typedef struct popcorn_decoder_s *popcorn_decoder_t;

popcorn_status_t popcorn_decoder_create(popcorn_library_t library, popcorn_stream_t stream,
                                        const popcorn_decoder_config_t *config, popcorn_decoder_t *decoder);
popcorn_status_t popcorn_decoder_destroy(popcorn_decoder_t decoder);

/* Synthetic state on the device: weights N(0, 0.02), norm weights
 * 1 + N(0, 0.1) (f32), embedding N(0, 0.02), KV caches N(0, 1). */
popcorn_status_t popcorn_decoder_randomize(popcorn_decoder_t decoder, uint64_t seed);

/* A view of an internal tensor: "embedding", "final_norm", "w_qkv", "w_o",
 * "w_gate", "w_up", "w_down", "norm_in", "norm_post_attn", "norm_pre_ffn",
 * "norm_post_ffn", "k_cache", "v_cache" and, with attention_block, "q_norm"
 * and "k_norm" (per `layer`); "inv_freq" (attention_block), "x", "logits",
 * "token", "position", "history", plus the last layer's step buffers
 * "q", "qkv", "attn", "o", "mlp", "hidden" and "x2" (the residual stream
 * the last layer's MLP and the head read: after a step it holds the stream
 * after the last attention block, while "x" holds the next step's input
 * row). With weight_bits 4 a weight name
 * ("embedding", "w_qkv", ...) is its packed u32 values [N, K/8], and
 * "<name>.scales" / "<name>.biases" its bf16 [N, K/64] groups. */
popcorn_status_t popcorn_decoder_tensor(popcorn_decoder_t decoder, const char *name, int32_t layer,
                                        popcorn_tensor_t *tensor);

/* Sets the input token and the position of the next step (host write). */
popcorn_status_t popcorn_decoder_reset(popcorn_decoder_t decoder, int32_t token, int32_t position);

/* Enqueues `steps` decode steps on the decoder's stream (no host sync):
 * through captured graphs when use_graph != 0, else dispatch by dispatch.
 * The first step starts from the token and position in device memory (its
 * input row is gathered first); "logits" then holds the last step's. Steps
 * that would decode at a position >= max_seq (write past the KV cache) are
 * refused with -1007 (tensorShapeMismatch) before anything is enqueued; the
 * position is tracked on the host from reset and read. */
popcorn_status_t popcorn_decoder_step(popcorn_decoder_t decoder, int32_t steps, int32_t use_graph);

/* Waits for the stream, then reads the current token and position. */
popcorn_status_t popcorn_decoder_read(popcorn_decoder_t decoder, int32_t *token, int32_t *position);

/* Dispatches of one step, in order, joined by ','; and their count. */
popcorn_status_t popcorn_decoder_describe(popcorn_decoder_t decoder, char *buffer, size_t capacity,
                                          int32_t *dispatches_per_step);

/* Bytes one step reads at a given position: weights + KV rows + activations
 * (the algorithmic traffic a decode step is priced by). */
int64_t popcorn_decoder_step_bytes(popcorn_decoder_t decoder, int32_t position);

/* Times one kernel of the step in isolation: every dispatch of the step
 * whose function is `function_name` (one per layer, say) is launched back to
 * back `reps` times between two events on the decoder's stream, all other
 * dispatches skipped (captured once as a graph and replayed, so no host work
 * sits between the launches). Reports the mean duration per launch and the number of
 * launches timed. State other than those kernels' outputs is unchanged; the
 * token and position are restored afterwards. */
popcorn_status_t popcorn_decoder_time_kernel(popcorn_decoder_t decoder, const char *function_name, int32_t reps,
                                             float *mean_ms, int32_t *launches);

/* Times one kernel inside the step: runs `steps` eager decode steps from the
 * current position (advancing it, like popcorn_decoder_step without a graph)
 * with a stop event attached to every launch of `function_name` and to the
 * launch just before each (hipExtModuleLaunchKernel; events without the
 * system-scope fence), and reports the mean of end(kernel) - end(previous
 * launch): the kernel's dispatch and run as the step pays for them, after its
 * neighbours and with their cache state. These times add up to the step.
 * A bounded wait kernel (hold_stream) runs first, so that every step is
 * enqueued before the GPU reaches it and no host gap falls between launches.
 * steps: 1..16. */
popcorn_status_t popcorn_decoder_time_kernel_in_step(popcorn_decoder_t decoder, const char *function_name,
                                                     int32_t steps, float *mean_ms, int32_t *launches);

#ifdef __cplusplus
}
#endif
#endif
