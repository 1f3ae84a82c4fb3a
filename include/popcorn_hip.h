/*
 * popcorn_hip.h — the C ABI of the MI355X (gfx950) build of Popcorn's decode
 * hot path.
 *
 * Two layers, both plain C (pointers, sizes, int32 status codes):
 *
 *  1. The thin shim the reference's Swift runtime core binds through a module
 *     map: device memory, streams/events, the kernel library (gfx950 code
 *     objects loaded by name) and the raw launch. Each entry cites the Swift
 *     member it replaces.
 *  2. The `Kernels.*` operation descriptors with the reference's validation,
 *     routing and dispatch geometry, plus `KernelCommandEncoder`. A descriptor
 *     is created (validated) once and encoded any number of times, as the
 *     reference's value-typed kernels are.
 *
 * Status codes are the raw values of the reference's PopcornError.Code
 * (Sources/Popcorn/PopcornError.swift:23-42). No C++ exception crosses this
 * boundary; the message of the last failure on the calling thread is
 * returned by popcorn_last_error_message().
 */
#ifndef POPCORN_HIP_H
#define POPCORN_HIP_H

#include <stddef.h>
#include <stdint.h>

#include "popcorn_kernel_types.h"

#ifdef __cplusplus
extern "C" {
#endif

/* ---- status ------------------------------------------------------------ */

typedef int32_t popcorn_status_t;

/* PopcornError.swift:23-42, same raw values. */
enum {
    POPCORN_OK = 0,
    POPCORN_ERR_CONSTANT_ALLOCATION_FAILED = -1001,
    POPCORN_ERR_TENSOR_ALLOCATION_FAILED = -1003,
    POPCORN_ERR_TENSOR_SHAPE_UNSUPPORTED_FOR_VIEW = -1004,
    POPCORN_ERR_TENSOR_DATA_TYPE_UNSUPPORTED_FOR_VIEW = -1005,
    POPCORN_ERR_KERNEL_FUNCTION_NOT_FOUND = -1006,
    POPCORN_ERR_TENSOR_SHAPE_MISMATCH = -1007,
    POPCORN_ERR_TENSOR_INVALID_RANK = -1008,
    POPCORN_ERR_TENSOR_INVALID_AXIS = -1009,
    POPCORN_ERR_UNSUPPORTED_DATA_TYPE_COMBINATION = -1010,
    POPCORN_ERR_HEAP_ALLOCATION_FAILED = -1011,
    POPCORN_ERR_WORKSPACE_EXHAUSTED = -1012,
    POPCORN_ERR_GPU_OUT_OF_MEMORY = -1013,
    POPCORN_ERR_GPU_TIMEOUT = -1014,
    POPCORN_ERR_GPU_PAGE_FAULT = -1015,
    POPCORN_ERR_GPU_INVALID_RESOURCE = -1016,
    POPCORN_ERR_GPU_DEVICE_REMOVED = -1017,
    POPCORN_ERR_GPU_ACCESS_REVOKED = -1018,
    POPCORN_ERR_GPU_INTERNAL = -1019,
    /* not in the reference (Swift reports these as preconditions) */
    POPCORN_ERR_INVALID_ARGUMENT = -1100
};

/* Message of the last failed call on this thread ("" if none). */
const char *popcorn_last_error_message(void);

/* Maps a hipError_t value to a status (the hipError -> PopcornError table
 * that replaces PopcornError.fromMetalError, PopcornError.swift:240-266). */
popcorn_status_t popcorn_status_from_hip_error(int hip_error);

/* ---- tensors (Tensor.swift:5-22, :134-178) ------------------------------ */

/* Tensor.DataType, declaration order of Tensor.swift:136-148. */
enum {
    POPCORN_DTYPE_U8 = 0,
    POPCORN_DTYPE_U16 = 1,
    POPCORN_DTYPE_U32 = 2,
    POPCORN_DTYPE_U64 = 3,
    POPCORN_DTYPE_I8 = 4,
    POPCORN_DTYPE_I16 = 5,
    POPCORN_DTYPE_I32 = 6,
    POPCORN_DTYPE_I64 = 7,
    POPCORN_DTYPE_F32 = 8,
    POPCORN_DTYPE_F16 = 9,
    POPCORN_DTYPE_BF16 = 10
};

#define POPCORN_MAX_RANK 8

/* Tensor{buffer, shape, dataType}: a non-owning view of device memory. */
typedef struct {
    void *data;
    int32_t dtype;
    int32_t rank;
    int64_t shape[POPCORN_MAX_RANK];
} popcorn_tensor_t;

/* ---- block-affine 4-bit weights (AffineQuantizedTensor.swift:19-84) ------
 * w = q * scale + bias, q unsigned `bits` wide, packed least-significant
 * first into little-endian u32 words (AffineQuantizationFormat.swift:24-30),
 * one scale/bias pair per `group_size` values along the inner axis.
 * packed_values u32 [..., out, in * bits / 32]; scales and biases
 * [..., out, in / group_size]; biases.data == NULL for none; shape is the
 * logical (dequantized) shape, rank >= 2. The kernels take bits 4, group 64,
 * bf16 scales. */
typedef struct {
    popcorn_tensor_t packed_values;
    popcorn_tensor_t scales;
    popcorn_tensor_t biases;
    int32_t rank;
    int64_t shape[POPCORN_MAX_RANK];
    int32_t bits;
    int32_t group_size;
} popcorn_affine_quantized_tensor_t;

/* Tensor.DataType.stride (Tensor.swift:152-159); 0 for an unknown tag. */
int32_t popcorn_dtype_stride(int32_t dtype);

/* ---- device and memory (MTLDevice+Extensions.swift:14-46) --------------- */

typedef struct {
    char name[64];
    char arch[32];          /* e.g. "gfx950"                                 */
    int32_t compute_units;
    int32_t wave_size;
    int32_t max_threads_per_block;
    int32_t lds_bytes_per_block;
    int64_t global_memory_bytes;
    int32_t l2_bytes;
    int32_t clock_khz;
} popcorn_device_info_t;

popcorn_status_t popcorn_device_count(int32_t *count);
popcorn_status_t popcorn_set_device(int32_t device);
popcorn_status_t popcorn_device_info(int32_t device, popcorn_device_info_t *info);
/* Waits for the device; then, like popcorn_stream_synchronize, reports a
 * merged-pair wait of the tiled prefill attention that gave up on any stream
 * of the device (-1019). */
popcorn_status_t popcorn_device_synchronize(void);

/* makeTensor's allocation; -1003 (tensorAllocationFailed) on failure. */
popcorn_status_t popcorn_malloc(size_t bytes, void **ptr);
popcorn_status_t popcorn_free(void *ptr);

/* No counterpart in the reference (Metal buffers have no per-XCD caches):
 * uncached device memory (hipDeviceMallocUncached), for buffers that blocks
 * on different XCDs of one launch exchange data through, such as the
 * pO/pML/pairFlags buffers of a raw launch of flash_attention_tiled*_ with
 * pairTiles 2. popcorn_free_uncached returns the block to a process-wide
 * pool for reuse by a later request of the same size on the same device;
 * such memory is never given back to the driver (memory of this kind, once
 * read by a kernel, is not freed before the process ends). */
popcorn_status_t popcorn_malloc_uncached(size_t bytes, void **ptr);
popcorn_status_t popcorn_free_uncached(void *ptr);

typedef struct popcorn_stream_s *popcorn_stream_t; /* NULL = default stream */

popcorn_status_t popcorn_memcpy_h2d(void *dst, const void *src, size_t bytes, popcorn_stream_t stream);
popcorn_status_t popcorn_memcpy_d2h(void *dst, const void *src, size_t bytes, popcorn_stream_t stream);
popcorn_status_t popcorn_memcpy_d2d(void *dst, const void *src, size_t bytes, popcorn_stream_t stream);
popcorn_status_t popcorn_memset(void *dst, int32_t value, size_t bytes, popcorn_stream_t stream);

/* ---- streams and events ------------------------------------------------
 * An in-order stream replaces the command buffer + hazard barriers
 * (KernelCommandEncoder.swift:71-85, :155-168); events replace the
 * command-buffer completion handler (GemmaCLI CommitFeedbackBox.swift:9-22). */

typedef struct popcorn_event_s *popcorn_event_t;

popcorn_status_t popcorn_stream_create(popcorn_stream_t *stream);
popcorn_status_t popcorn_stream_destroy(popcorn_stream_t stream);
/* Waits for the stream; then reports -1019 (gpuInternal) when a merged pair
 * of the tiled prefill attention (pairTiles 2) gave up waiting for its
 * partner block on this stream since the last check (its rows were written
 * as NaN; the stream's ready flags are cleared before returning), the way
 * the reference reports a command buffer's GPU error on completion
 * (PopcornError.swift:240-266). */
popcorn_status_t popcorn_stream_synchronize(popcorn_stream_t stream);

/* No counterpart in the reference: the ready flags of the tiled prefill
 * attention's merged pairs on `stream` (created on first use): u64
 * [count], index 0 the abort word, 1 + t the flag of split tile t, in
 * uncached device memory. For inspection and tests. */
popcorn_status_t popcorn_attention_pair_flags(popcorn_stream_t stream, void **flags, int32_t *count);

popcorn_status_t popcorn_event_create(popcorn_event_t *event);
popcorn_status_t popcorn_event_destroy(popcorn_event_t event);
popcorn_status_t popcorn_event_record(popcorn_event_t event, popcorn_stream_t stream);
popcorn_status_t popcorn_event_wait(popcorn_stream_t stream, popcorn_event_t event);
popcorn_status_t popcorn_event_synchronize(popcorn_event_t event);
popcorn_status_t popcorn_event_elapsed_ms(popcorn_event_t start, popcorn_event_t stop, float *ms);

/* ---- kernel library (KernelLibrary.swift:4-41) --------------------------
 * A library is a set of gfx950 code objects. `path` names one code object
 * file or a directory of them; NULL loads the kernels that ship next to this
 * shared library (the reference's default metallib, KernelLibrary.swift:7-14).
 * Function lookup is cached behind a mutex and fails with -1006
 * (kernelFunctionNotFound) for an unknown name, as pipelineState(for:) does. */

typedef struct popcorn_library_s *popcorn_library_t;
typedef struct popcorn_function_s *popcorn_function_t;

typedef struct {
    int32_t max_threads_per_block;  /* maxTotalThreadsPerThreadgroup         */
    int32_t wave_size;              /* threadExecutionWidth: 64 on gfx950    */
    int32_t static_lds_bytes;
    int32_t num_vgprs;
    int32_t num_sgprs;
    int32_t private_bytes;
} popcorn_function_attrs_t;

popcorn_status_t popcorn_library_load(const char *path, popcorn_library_t *library);
popcorn_status_t popcorn_library_destroy(popcorn_library_t library);
popcorn_status_t popcorn_library_function(popcorn_library_t library, const char *name,
                                          popcorn_function_t *function);
popcorn_status_t popcorn_function_attributes(popcorn_function_t function,
                                             popcorn_function_attrs_t *attrs);
/* Number of functions found so far (the pipeline-state cache size). */
int32_t popcorn_library_cached_function_count(popcorn_library_t library);

/* A kernel's parameter list as its code object's metadata states it: the
 * leading device pointers, then the by-value constants blocks (no
 * counterpart in the reference, where Metal reflects it; the checks below
 * use it). */
#define POPCORN_MAX_CONSTANT_BLOCKS 8
typedef struct {
    int32_t nbuffers;       /* leading device-pointer parameters */
    int32_t nconstants;     /* parameters after them */
    uint32_t constant_sizes[POPCORN_MAX_CONSTANT_BLOCKS]; /* bytes; 8 for a pointer
                                                      among them (trailing_pointers) */
    int32_t trailing_pointers; /* pointers after the first constants block (0 here) */
    uint32_t max_threads_per_block;
} popcorn_kernel_layout_t;

popcorn_status_t popcorn_function_layout(popcorn_function_t function, popcorn_kernel_layout_t *layout);
/* The same read from a code-object file without a GPU (-1006 if the file
 * holds no kernel of that name, -1100 for an unreadable file). */
popcorn_status_t popcorn_code_object_layout(const char *path, const char *kernel, popcorn_kernel_layout_t *layout);

/* Raw launch (replaces setBuffer/setBytes/dispatchThreads,
 * KernelCommandEncoder.swift:193-208): the kernel's parameters are the
 * `nbuffers` device pointers in order, then each constants block by value.
 * grid and block are in blocks and threads (not threads and threads).
 * The launch must bind exactly the kernel's parameter list (pointer count
 * and each block's size, popcorn_function_layout) and at most its block
 * size, else -1100 (invalidArgument) and nothing runs. Kernels under the
 * reference's host names take the reference's parameter list and compute
 * the reference's result under its launch geometry (threads converted to
 * blocks). */
popcorn_status_t popcorn_launch(popcorn_stream_t stream, popcorn_function_t function,
                                const uint32_t grid[3], const uint32_t block[3],
                                void *const *buffers, int32_t nbuffers,
                                const void *const *constants, const size_t *constant_sizes,
                                int32_t nconstants, size_t dynamic_lds_bytes);

/* ---- scratch (KernelResources.swift:5-36, ScratchSpec.swift:10-26) ------- */

/* KernelScratchAllocator: borrow returns device memory of >= length bytes and
 * whether it may hold earlier writes (KernelTemporaryBuffer.wasReused). */
typedef struct {
    void *context;
    popcorn_status_t (*borrow)(void *context, size_t length, void **buffer, int32_t *was_reused);
    void (*release)(void *context, void *buffer);
} popcorn_scratch_allocator_t;

/* A best-fit pool (the GemmaCLI ScratchPool, ScratchPool.swift:42-71) bound to
 * one stream: buffers return to the pool on release and are reused by later
 * borrows; work on that stream is ordered, so reuse needs no barrier. */
typedef struct popcorn_scratch_pool_s *popcorn_scratch_pool_t;
popcorn_status_t popcorn_scratch_pool_create(popcorn_scratch_pool_t *pool);
popcorn_status_t popcorn_scratch_pool_destroy(popcorn_scratch_pool_t pool);
popcorn_status_t popcorn_scratch_pool_allocator(popcorn_scratch_pool_t pool,
                                                popcorn_scratch_allocator_t *allocator);
size_t popcorn_scratch_pool_bytes(popcorn_scratch_pool_t pool);

/* ScratchSpec.byteCount: max(1, prod(shape) * stride). */
size_t popcorn_scratch_spec_byte_count(const int64_t *shape, int32_t rank, int32_t dtype);

/* ---- command encoder (KernelCommandEncoder.swift:4-208) ------------------ */

typedef struct popcorn_encoder_s *popcorn_encoder_t;
typedef struct popcorn_kernel_s *popcorn_kernel_t;

/* `scratch` may be NULL: the encoder then owns a pool on `stream`. */
popcorn_status_t popcorn_encoder_create(popcorn_library_t library, popcorn_stream_t stream,
                                        const popcorn_scratch_allocator_t *scratch,
                                        popcorn_encoder_t *encoder);
popcorn_status_t popcorn_encoder_destroy(popcorn_encoder_t encoder);
/* encode(_:) and the result-builder form encode { k1; k2; ... }. */
popcorn_status_t popcorn_encoder_encode(popcorn_encoder_t encoder, popcorn_kernel_t kernel);
popcorn_status_t popcorn_encoder_encode_all(popcorn_encoder_t encoder,
                                            const popcorn_kernel_t *kernels, int32_t count);
/* barrier(): on one in-order stream every dispatch already sees the writes of
 * the ones before it, so this only resets the hazard map. */
popcorn_status_t popcorn_encoder_barrier(popcorn_encoder_t encoder);

typedef struct {
    int64_t dispatches;
    int64_t hazards;      /* RAW/WAR/WAW pairs the reference would barrier on */
    int64_t scratch_borrows;
} popcorn_encoder_stats_t;
popcorn_status_t popcorn_encoder_stats(popcorn_encoder_t encoder, popcorn_encoder_stats_t *stats);

/* ---- operation descriptors (Kernels.*) ---------------------------------- */

/* AttentionMask (AttentionMask.swift:17-41): kind 0 causal, 1 causal +
 * sliding window (window used), 2 bidirectional. */
typedef struct {
    uint32_t kind;
    int32_t window;
} popcorn_attention_mask_t;

/* FlashAttention.Path (FlashAttention.swift:94-98); `tiled` is the MFMA
 * prefill kernel that takes the place of the reference's MPP path. */
enum { POPCORN_ATTENTION_PLAIN = 0, POPCORN_ATTENTION_TILED = 1, POPCORN_ATTENTION_DECODING = 2 };

/* Kernels.FlashAttention.route(sq:hd:supportsMPP:) (FlashAttention.swift:109-113). */
int32_t popcorn_flash_attention_route(int64_t query_len, int64_t head_dim, int32_t q_dtype);

/* Kernels.FlashAttention(q:k:v:into:scale:mask:) (FlashAttention.swift:51-90). */
popcorn_status_t popcorn_kernel_flash_attention(const popcorn_tensor_t *q, const popcorn_tensor_t *k,
                                                const popcorn_tensor_t *v, const popcorn_tensor_t *out,
                                                float scale, popcorn_attention_mask_t mask,
                                                popcorn_kernel_t *kernel);

/* Kernels.FlashAttention(q:k:v:out:batch:...:scale:mask:) (FlashAttention.swift:13-49)
 * with two additions: `key_capacity` (>= key_len; 0 = key_len) is the row
 * stride of K/V, so a cache [B, Nkv, Smax, Hd] is read in place; `position`
 * (may be NULL) is an i32 tensor whose element 0 + query_len replaces
 * key_len at run time (a decode step replayed from a captured graph). */
popcorn_status_t popcorn_kernel_flash_attention_dims(
    const popcorn_tensor_t *q, const popcorn_tensor_t *k, const popcorn_tensor_t *v,
    const popcorn_tensor_t *out, int64_t batch, int64_t query_heads, int64_t kv_heads,
    int64_t query_len, int64_t key_len, int64_t head_dim, float scale,
    popcorn_attention_mask_t mask, int64_t key_capacity, const popcorn_tensor_t *position,
    popcorn_kernel_t *kernel);

/* No counterpart in the reference: popcorn_kernel_flash_attention_dims'
 * split-KV attention (the partial kernel and the log-sum-exp combine) in one
 * call that allocates nothing, for callers that cannot call hipMalloc (code
 * under HIP graph capture, tight serving loops, harnesses that forbid
 * allocation). The partials live in a static device array of
 * POPCORN_NO_ALLOC_SCRATCH_BYTES per GPU, part of this library and held
 * until the process ends, instead of a borrowed scratch buffer; a call needing
 * more (B * Nq * Sq * P * (Hd + 2) * 4 bytes, P the partitions chosen for the
 * shape) fails with -1012 (workspaceExhausted) and launches nothing. Same
 * arguments, validation, kernels and results as the split-KV route of the
 * descriptor (whatever route the descriptor would take for the shape);
 * enqueued on `stream`. Calls that overlap on one GPU share the array and
 * race: order them on one stream. */
#define POPCORN_NO_ALLOC_SCRATCH_BYTES ((size_t)4 << 20)
popcorn_status_t popcorn_flash_decoding_no_alloc(popcorn_library_t library, popcorn_stream_t stream,
                                                 const popcorn_tensor_t *q, const popcorn_tensor_t *k,
                                                 const popcorn_tensor_t *v, const popcorn_tensor_t *out, int64_t batch,
                                                 int64_t query_heads, int64_t kv_heads, int64_t query_len,
                                                 int64_t key_len, int64_t head_dim, float scale,
                                                 popcorn_attention_mask_t mask, int64_t key_capacity,
                                                 const popcorn_tensor_t *position);

/* Kernels.Matmul(_:_:into:transposeB:) (Matmul.swift:68-93); m == 1 routes to
 * the matvec (Matmul.swift:22-32). */
popcorn_status_t popcorn_kernel_matmul(const popcorn_tensor_t *a, const popcorn_tensor_t *b,
                                       const popcorn_tensor_t *c, int32_t transpose_b,
                                       popcorn_kernel_t *kernel);
/* Kernels.Matmul(a:b:c:m:k:n:transposeB:) (Matmul.swift:9-66). */
popcorn_status_t popcorn_kernel_matmul_dims(const popcorn_tensor_t *a, const popcorn_tensor_t *b,
                                            const popcorn_tensor_t *c, int64_t m, int64_t k,
                                            int64_t n, int32_t transpose_b, popcorn_kernel_t *kernel);

/* Kernels.RMSNorm(_:weight:into:axis:eps:addOneToWeight:) (RMSNorm.swift:39-70);
 * weight may be NULL. */
popcorn_status_t popcorn_kernel_rmsnorm(const popcorn_tensor_t *x, const popcorn_tensor_t *weight,
                                        const popcorn_tensor_t *out, int32_t axis, float eps,
                                        int32_t add_one_to_weight, popcorn_kernel_t *kernel);
/* Kernels.RMSNorm(x:weight:out:rowCount:hiddenSize:eps:addOneToWeight:) (RMSNorm.swift:10-37). */
popcorn_status_t popcorn_kernel_rmsnorm_dims(const popcorn_tensor_t *x, const popcorn_tensor_t *weight,
                                             const popcorn_tensor_t *out, int64_t row_count,
                                             int64_t hidden_size, float eps,
                                             int32_t add_one_to_weight, popcorn_kernel_t *kernel);

/* Kernels.KVCacheWrite(source:cache:offset:) (KVCacheWrite.swift:37-48). */
popcorn_status_t popcorn_kernel_kv_cache_write(const popcorn_tensor_t *source,
                                               const popcorn_tensor_t *cache, int64_t offset,
                                               popcorn_kernel_t *kernel);
/* Kernels.KVCacheWrite(source:cache:batch:kvHeads:newLen:maxLen:headDim:offset:)
 * (KVCacheWrite.swift:7-35); `position` (may be NULL) is an i32 tensor whose
 * element 0 replaces `offset` at run time. */
popcorn_status_t popcorn_kernel_kv_cache_write_dims(const popcorn_tensor_t *source,
                                                    const popcorn_tensor_t *cache, int64_t batch,
                                                    int64_t kv_heads, int64_t new_len,
                                                    int64_t max_len, int64_t head_dim,
                                                    int64_t offset, const popcorn_tensor_t *position,
                                                    popcorn_kernel_t *kernel);

/* Kernels.GeluTanh(_:into:) (GeluTanh.swift:28-33), Kernels.Mul(_:_:into:)
 * (Mul.swift:28-37), Kernels.Add (Add.swift), Kernels.ScalarMul (ScalarMul.swift). */
popcorn_status_t popcorn_kernel_gelu_tanh(const popcorn_tensor_t *x, const popcorn_tensor_t *out,
                                          popcorn_kernel_t *kernel);
popcorn_status_t popcorn_kernel_mul(const popcorn_tensor_t *a, const popcorn_tensor_t *b,
                                    const popcorn_tensor_t *out, popcorn_kernel_t *kernel);
popcorn_status_t popcorn_kernel_add(const popcorn_tensor_t *a, const popcorn_tensor_t *b,
                                    const popcorn_tensor_t *out, popcorn_kernel_t *kernel);
popcorn_status_t popcorn_kernel_scalar_mul(const popcorn_tensor_t *x, float scalar,
                                           const popcorn_tensor_t *out, popcorn_kernel_t *kernel);

/* Kernels.RopeBuildCosSin(positions:invFreq:cosOut:sinOut:attentionScaling:)
 * (RopeBuildCosSin.swift:30-50) and the explicit init (:8-28): positions i32
 * [T], inv_freq f32 [Hd/2] -> cos, sin f32 [T, Hd/2] =
 * cos/sin(float(position) * inv_freq) * attention_scaling. */
popcorn_status_t popcorn_kernel_rope_build_cos_sin(const popcorn_tensor_t *positions, const popcorn_tensor_t *inv_freq,
                                                 const popcorn_tensor_t *cos_out, const popcorn_tensor_t *sin_out,
                                                 float attention_scaling, popcorn_kernel_t *kernel);
popcorn_status_t popcorn_kernel_rope_build_cos_sin_dims(const popcorn_tensor_t *positions, const popcorn_tensor_t *inv_freq,
                                                      const popcorn_tensor_t *cos_out, const popcorn_tensor_t *sin_out,
                                                      int64_t seq_len, int64_t half_head_dim, float attention_scaling,
                                                      popcorn_kernel_t *kernel);

/* Kernels.RopeApply(_:cos:sin:into:) (RopeApply.swift:46-60) and the explicit
 * init (:8-44): half-rotation RoPE of x [B, T, Nh, Hd] with tables [T, Hd/2];
 * (x, table) dtypes (f32, f32), (bf16, bf16) or (bf16, f32), out of x's dtype. */
popcorn_status_t popcorn_kernel_rope_apply(const popcorn_tensor_t *x, const popcorn_tensor_t *cos_table,
                                         const popcorn_tensor_t *sin_table, const popcorn_tensor_t *out,
                                         popcorn_kernel_t *kernel);
popcorn_status_t popcorn_kernel_rope_apply_dims(const popcorn_tensor_t *x, const popcorn_tensor_t *cos_table,
                                              const popcorn_tensor_t *sin_table, const popcorn_tensor_t *out, int64_t batch,
                                              int64_t seq_len, int64_t head_count, int64_t head_dim,
                                              popcorn_kernel_t *kernel);

/* Kernels.Transpose12(_:into:) (Transpose12.swift:27-35) and the explicit init
 * (:8-25): [D0, D1, D2, D3] -> [D0, D2, D1, D3] for f32, f16, bf16. */
popcorn_status_t popcorn_kernel_transpose12(const popcorn_tensor_t *src, const popcorn_tensor_t *out,
                                          popcorn_kernel_t *kernel);
popcorn_status_t popcorn_kernel_transpose12_dims(const popcorn_tensor_t *src, const popcorn_tensor_t *out, int64_t d0,
                                               int64_t d1, int64_t d2, int64_t d3, popcorn_kernel_t *kernel);

/* The gated MLP of Gemma4TextInference.swift:416-429 (RMSNorm -> gate, up ->
 * GeluTanh(gate) * up -> down) as two dispatches: a fused kernel for
 * everything up to the gated product, then the down matvec. No single
 * counterpart in the reference, which runs it as five dispatches; `hidden`
 * (may be NULL; [F], x's dtype) receives the gated product. */
popcorn_status_t popcorn_kernel_gated_mlp(const popcorn_tensor_t *x, const popcorn_tensor_t *norm_weight,
                                          const popcorn_tensor_t *w_gate, const popcorn_tensor_t *w_up,
                                          const popcorn_tensor_t *w_down, const popcorn_tensor_t *out,
                                          float eps, int32_t add_one_to_weight,
                                          const popcorn_tensor_t *hidden, popcorn_kernel_t *kernel);

/* The gated MLP with the attention block's post-norm and residual Add in
 * front (Gemma4TextInference.swift:400-404 then :416-429):
 * x = x_in + RMSNorm(delta) * w_post is stored to x_out (which must not alias
 * x_in), then out = GatedMLP(x). No single counterpart in the reference. */
popcorn_status_t popcorn_kernel_gated_mlp_residual(const popcorn_tensor_t *x_in, const popcorn_tensor_t *delta,
                                                   const popcorn_tensor_t *w_post, const popcorn_tensor_t *x_out,
                                                   const popcorn_tensor_t *norm_weight, const popcorn_tensor_t *w_gate,
                                                   const popcorn_tensor_t *w_up, const popcorn_tensor_t *w_down,
                                                   const popcorn_tensor_t *out, float eps, int32_t add_one_to_weight,
                                                   const popcorn_tensor_t *hidden, popcorn_kernel_t *kernel);

/* popcorn_kernel_gated_mlp_residual with block-affine 4-bit gate, up and down
 * weights (bf16 x/out, bf16 scales, group 64) and an f32 pre-FFN norm weight;
 * delta, w_post and x_out all NULL for the plain form. No single counterpart
 * in the reference (its quantized Matmul dispatches, Matmul.swift:99-130, in
 * the composition of Gemma4TextInference.swift:416-429). */
popcorn_status_t popcorn_kernel_gated_mlp_residual_quantized(
    const popcorn_tensor_t *x_in, const popcorn_tensor_t *delta, const popcorn_tensor_t *w_post,
    const popcorn_tensor_t *x_out, const popcorn_tensor_t *norm_weight, const popcorn_affine_quantized_tensor_t *w_gate,
    const popcorn_affine_quantized_tensor_t *w_up, const popcorn_affine_quantized_tensor_t *w_down,
    const popcorn_tensor_t *out, float eps, const popcorn_tensor_t *hidden, popcorn_kernel_t *kernel);

/* The decode-step matvec out = W v (W [N, K], one token) with the layer glue
 * around it (DecodeMatvecConstants in popcorn_kernel_types.h): with delta,
 * x = x + RMSNorm(delta) * w_post is formed and stored to x_out; with w_pre,
 * v = RMSNorm(x) * w_pre, else v = x; with the caches, rows past q_rows are
 * written to the K then V cache at row position[0] of each KV head. Every
 * stored intermediate is rounded to the weight dtype. NULL = absent. No
 * single counterpart in the reference (its RMSNorm, Add, Matmul and
 * KVCacheWrite dispatches, Gemma4TextInference.swift:334-404). */
typedef struct {
    const popcorn_tensor_t *x;
    const popcorn_tensor_t *delta;
    const popcorn_tensor_t *w_post;
    const popcorn_tensor_t *x_out;
    const popcorn_tensor_t *w_pre;
    const popcorn_tensor_t *weight;
    const popcorn_tensor_t *out;
    const popcorn_tensor_t *k_cache;
    const popcorn_tensor_t *v_cache;
    const popcorn_tensor_t *position;
    int64_t q_rows;
    float eps;
    /* in place of `weight`: a block-affine 4-bit weight [N, K] (bf16 x, bf16
     * scales, group 64, K a multiple of 64 and at most 8192) */
    const popcorn_affine_quantized_tensor_t *qweight;
} popcorn_decode_matvec_args_t;

popcorn_status_t popcorn_kernel_decode_matvec(const popcorn_decode_matvec_args_t *args, popcorn_kernel_t *kernel);

/* The attention block of one decode token with its per-head glue folded into
 * the split-KV kernel (DecodeAttentionConstants in popcorn_kernel_types.h):
 * qkv [B, (Nq + 2 Nkv) * Hd] holds the raw projections; q_norm / k_norm (f32
 * [Hd]) apply the per-head RMSNorms, v_norm the weightless one, inv_freq (f32
 * [Hd/2]) RoPE at position[0] with tables scaled by rope_scaling; the
 * processed key and value rows are written to the caches [B, Nkv, S, Hd] at
 * row position[0], and out [B, Nq, 1, Hd] = attention over keys
 * 0..position[0] (mask as for FlashAttention). Every intermediate is rounded
 * to the cache dtype where the reference stores a tensor. NULL = absent.
 * Replaces the reference's RMSNorm, RopeApply, Transpose12, KVCacheWrite and
 * FlashAttention dispatches of one token (Gemma4TextInference.swift:352-399);
 * no single counterpart. Needs the fast split-KV path: 16-byte aligned data,
 * head dim 64/128/256/512 for f16/bf16 (128/256/512 for f32). */
typedef struct {
    const popcorn_tensor_t *qkv;
    const popcorn_tensor_t *k_cache;
    const popcorn_tensor_t *v_cache;
    const popcorn_tensor_t *out;
    const popcorn_tensor_t *position;
    const popcorn_tensor_t *q_norm;
    const popcorn_tensor_t *k_norm;
    const popcorn_tensor_t *inv_freq;
    int32_t v_norm;
    int32_t query_heads;
    int32_t kv_heads;
    float eps;
    float scale;
    float rope_scaling;
    popcorn_attention_mask_t mask;
} popcorn_decode_attention_args_t;

popcorn_status_t popcorn_kernel_decode_attention(const popcorn_decode_attention_args_t *args,
                                                 popcorn_kernel_t *kernel);

/* Kernels.EmbeddingGather(ids:table:out:tokenCount:hiddenSize:)
 * (EmbeddingGather.swift) and Kernels.Argmax(_:indices:axis:) (Argmax.swift:24-37):
 * the decode loop's token in / token out. */
popcorn_status_t popcorn_kernel_embedding_gather(const popcorn_tensor_t *ids, const popcorn_tensor_t *table,
                                                 const popcorn_tensor_t *out, popcorn_kernel_t *kernel);
popcorn_status_t popcorn_kernel_argmax(const popcorn_tensor_t *x, const popcorn_tensor_t *indices,
                                       popcorn_kernel_t *kernel);


/* AffineQuantizedTensor.init's checks (AffineQuantizedTensor.swift:29-48). */
popcorn_status_t popcorn_affine_quantized_validate(const popcorn_affine_quantized_tensor_t *tensor);

/* Kernels.Matmul(_:_:into:) with a quantized RHS (Matmul.swift:99-130,
 * :279-332): c[m, n] = a[m, k] b^T; (a, scales, c) dtypes (bf16, bf16, bf16),
 * (bf16, bf16, f32) or (f32, bf16, f32); m == 1 runs aq_qmv_fast_*. */
popcorn_status_t popcorn_kernel_matmul_quantized(const popcorn_tensor_t *a, const popcorn_affine_quantized_tensor_t *b,
                                                 const popcorn_tensor_t *c, popcorn_kernel_t *kernel);

/* Kernels.EmbeddingGather(ids:table:into:) with a quantized table
 * (EmbeddingGather.swift:45-88): out[t, :] = dequantize(table[ids[t], :]);
 * an id outside the table gives a zero row. */
popcorn_status_t popcorn_kernel_embedding_gather_quantized(const popcorn_tensor_t *ids,
                                                           const popcorn_affine_quantized_tensor_t *table,
                                                           const popcorn_tensor_t *out, popcorn_kernel_t *kernel);

/* A DispatchKernel built by the caller (Kernel.swift:54-70): function name,
 * bound tensors with their access (1 read, 2 write, 3 both), constants blocks,
 * and the launch geometry in blocks/threads. */
popcorn_status_t popcorn_kernel_custom(const char *function_name, const popcorn_tensor_t *tensors,
                                       const uint8_t *access, int32_t ntensors,
                                       const void *const *constants, const size_t *constant_sizes,
                                       int32_t nconstants, const uint32_t grid[3],
                                       const uint32_t block[3], popcorn_kernel_t *kernel);

popcorn_status_t popcorn_kernel_destroy(popcorn_kernel_t kernel);

/* Introspection: the function names the descriptor dispatches, joined by
 * ',', in order (e.g. "flash_decoding_partial_bf16,flash_decoding_reduce_bf16"). */
popcorn_status_t popcorn_kernel_describe(popcorn_kernel_t kernel, char *buffer, size_t capacity);

/* ---- synthetic inputs ---------------------------------------------------- */

/* Fills `count` elements of `data` (dtype f32/f16/bf16) with N(mean, std)
 * from a counter-based generator keyed by seed (device side; for benchmarks,
 * not bit-identical to the CPU oracle's generator). */
popcorn_status_t popcorn_fill_normal(popcorn_library_t library, popcorn_stream_t stream, void *data,
                                     int32_t dtype, uint64_t count, uint64_t seed, float mean,
                                     float stddev);

#ifdef __cplusplus
}
#endif
#endif
