// extern "C" entry points of include/popcorn_hip.h. Every function converts
// exceptions to status codes and records the message for
// popcorn_last_error_message(); nothing throws across the boundary.
#include <cstring>
#include <new>

#include "handles.hpp"
#include "uncached.hpp"

using namespace popcorn;

struct popcorn_function_s {
    const Function *fn;
};
struct popcorn_scratch_pool_s {
    ScratchPool pool;
};
struct popcorn_encoder_s {
    std::unique_ptr<KernelScratchAllocator> ownedScratch;
    std::unique_ptr<KernelCommandEncoder> enc;
};
struct popcorn_kernel_s {
    std::unique_ptr<Kernel> k;
};

namespace {

template <typename F>
popcorn_status_t guarded(F &&f) {
    try {
        f();
        setLastError("");
        return POPCORN_OK;
    } catch (const Error &e) {
        setLastError(e.what());
        return e.code();
    } catch (const std::bad_alloc &) {
        setLastError("host allocation failed");
        return POPCORN_ERR_TENSOR_ALLOCATION_FAILED;
    } catch (const std::exception &e) {
        setLastError(e.what());
        return POPCORN_ERR_GPU_INTERNAL;
    } catch (...) {
        setLastError("unknown error");
        return POPCORN_ERR_GPU_INTERNAL;
    }
}

void need(const void *p, const char *what) {
    if (!p) throw Error::invalidArgument(std::string(what) + " must not be NULL");
}

Tensor T(const popcorn_tensor_t *t, const char *what) {
    need(t, what);
    return Tensor::fromC(*t);
}

popcorn_status_t emit(popcorn_kernel_t *out, std::unique_ptr<Kernel> k) {
    need(out, "kernel");
    *out = new popcorn_kernel_s{std::move(k)};
    return POPCORN_OK;
}

hipStream_t S(popcorn_stream_t s) { return reinterpret_cast<hipStream_t>(s); }

}  // namespace

extern "C" {

const char *popcorn_last_error_message(void) { return lastError(); }

popcorn_status_t popcorn_status_from_hip_error(int e) {
    switch (e) {
    case hipSuccess: return POPCORN_OK;
    case hipErrorOutOfMemory: return POPCORN_ERR_GPU_OUT_OF_MEMORY;
    case hipErrorLaunchTimeOut: return POPCORN_ERR_GPU_TIMEOUT;
    case hipErrorIllegalAddress: return POPCORN_ERR_GPU_PAGE_FAULT;
    case hipErrorInvalidHandle: return POPCORN_ERR_GPU_INVALID_RESOURCE;
    case hipErrorNoDevice:
    case hipErrorInvalidDevice: return POPCORN_ERR_GPU_DEVICE_REMOVED;
    case hipErrorNotFound:
    case hipErrorInvalidDeviceFunction: return POPCORN_ERR_KERNEL_FUNCTION_NOT_FOUND;
    case hipErrorInvalidValue: return POPCORN_ERR_INVALID_ARGUMENT;
    default: return POPCORN_ERR_GPU_INTERNAL;
    }
}

int32_t popcorn_dtype_stride(int32_t dtype) {
    switch (dtype) {
    case POPCORN_DTYPE_U8:
    case POPCORN_DTYPE_I8: return 1;
    case POPCORN_DTYPE_U16:
    case POPCORN_DTYPE_I16:
    case POPCORN_DTYPE_F16:
    case POPCORN_DTYPE_BF16: return 2;
    case POPCORN_DTYPE_U32:
    case POPCORN_DTYPE_I32:
    case POPCORN_DTYPE_F32: return 4;
    case POPCORN_DTYPE_U64:
    case POPCORN_DTYPE_I64: return 8;
    default: return 0;
    }
}

// ---- device and memory ---------------------------------------------------------

popcorn_status_t popcorn_device_count(int32_t *count) {
    return guarded([&] {
        need(count, "count");
        int n = 0;
        hipError_t e = hipGetDeviceCount(&n);
        if (e == hipErrorNoDevice) {
            (void)hipGetLastError();
            n = 0;
        } else {
            checkHip(e, "hipGetDeviceCount");
        }
        *count = n;
    });
}

popcorn_status_t popcorn_set_device(int32_t device) {
    return guarded([&] { checkHip(hipSetDevice(device), "hipSetDevice"); });
}

popcorn_status_t popcorn_device_info(int32_t device, popcorn_device_info_t *info) {
    return guarded([&] {
        need(info, "info");
        hipDeviceProp_t p;
        checkHip(hipGetDeviceProperties(&p, device), "hipGetDeviceProperties");
        std::memset(info, 0, sizeof(*info));
        std::strncpy(info->name, p.name, sizeof(info->name) - 1);
        std::strncpy(info->arch, p.gcnArchName, sizeof(info->arch) - 1);
        info->compute_units = p.multiProcessorCount;
        info->wave_size = p.warpSize;
        info->max_threads_per_block = p.maxThreadsPerBlock;
        info->lds_bytes_per_block = (int32_t)p.sharedMemPerBlock;
        info->global_memory_bytes = (int64_t)p.totalGlobalMem;
        info->l2_bytes = p.l2CacheSize;
        info->clock_khz = p.clockRate;
    });
}

popcorn_status_t popcorn_device_synchronize(void) {
    return guarded([&] {
        checkHip(hipDeviceSynchronize(), "hipDeviceSynchronize");
        checkPairExchange(nullptr, true);
    });
}

popcorn_status_t popcorn_malloc(size_t bytes, void **ptr) {
    return guarded([&] {
        need(ptr, "ptr");
        size_t n = bytes ? bytes : 1;
        if (hipMalloc(ptr, n) != hipSuccess) {
            (void)hipGetLastError();
            *ptr = nullptr;
            throw Error::tensorAllocationFailed(n);
        }
    });
}

popcorn_status_t popcorn_free(void *ptr) {
    return guarded([&] {
        if (ptr) checkHip(hipFree(ptr), "hipFree");
    });
}

popcorn_status_t popcorn_malloc_uncached(size_t bytes, void **ptr) {
    return guarded([&] {
        need(ptr, "ptr");
        *ptr = nullptr;
        *ptr = UncachedPool::take(bytes ? bytes : 1);
    });
}

popcorn_status_t popcorn_free_uncached(void *ptr) {
    return guarded([&] {
        if (ptr && !UncachedPool::give(ptr))
            throw Error::invalidArgument("popcorn_free_uncached: the pointer was not returned by popcorn_malloc_uncached");
    });
}

static popcorn_status_t copy(void *dst, const void *src, size_t bytes, hipMemcpyKind kind, popcorn_stream_t stream) {
    return guarded([&] {
        if (!bytes) return;
        need(dst, "dst");
        need(src, "src");
        checkHip(hipMemcpyAsync(dst, src, bytes, kind, S(stream)), "hipMemcpyAsync");
        if (kind == hipMemcpyDeviceToHost || kind == hipMemcpyHostToDevice)
            checkHip(hipStreamSynchronize(S(stream)), "hipStreamSynchronize");
    });
}

popcorn_status_t popcorn_memcpy_h2d(void *dst, const void *src, size_t bytes, popcorn_stream_t stream) {
    return copy(dst, src, bytes, hipMemcpyHostToDevice, stream);
}
popcorn_status_t popcorn_memcpy_d2h(void *dst, const void *src, size_t bytes, popcorn_stream_t stream) {
    return copy(dst, src, bytes, hipMemcpyDeviceToHost, stream);
}
popcorn_status_t popcorn_memcpy_d2d(void *dst, const void *src, size_t bytes, popcorn_stream_t stream) {
    return copy(dst, src, bytes, hipMemcpyDeviceToDevice, stream);
}

popcorn_status_t popcorn_memset(void *dst, int32_t value, size_t bytes, popcorn_stream_t stream) {
    return guarded([&] {
        if (!bytes) return;
        need(dst, "dst");
        checkHip(hipMemsetAsync(dst, value, bytes, S(stream)), "hipMemsetAsync");
    });
}

// ---- streams and events ------------------------------------------------------------

popcorn_status_t popcorn_stream_create(popcorn_stream_t *stream) {
    return guarded([&] {
        need(stream, "stream");
        hipStream_t s = nullptr;
        checkHip(hipStreamCreateWithFlags(&s, hipStreamNonBlocking), "hipStreamCreate");
        *stream = reinterpret_cast<popcorn_stream_t>(s);
    });
}
popcorn_status_t popcorn_stream_destroy(popcorn_stream_t stream) {
    return guarded([&] {
        if (stream) checkHip(hipStreamDestroy(S(stream)), "hipStreamDestroy");
    });
}
popcorn_status_t popcorn_stream_synchronize(popcorn_stream_t stream) {
    return guarded([&] {
        checkHip(hipStreamSynchronize(S(stream)), "hipStreamSynchronize");
        checkPairExchange(S(stream));
    });
}

popcorn_status_t popcorn_attention_pair_flags(popcorn_stream_t stream, void **flags, int32_t *count) {
    return guarded([&] {
        need(flags, "flags");
        need(count, "count");
        const PairExchange &x = pairExchange(S(stream), 0);
        *flags = x.flags;
        *count = (int32_t)PairExchange::kFlags;
    });
}

popcorn_status_t popcorn_event_create(popcorn_event_t *event) {
    return guarded([&] {
        need(event, "event");
        hipEvent_t e = nullptr;
        checkHip(hipEventCreate(&e), "hipEventCreate");
        *event = reinterpret_cast<popcorn_event_t>(e);
    });
}
popcorn_status_t popcorn_event_destroy(popcorn_event_t event) {
    return guarded([&] {
        if (event) checkHip(hipEventDestroy(reinterpret_cast<hipEvent_t>(event)), "hipEventDestroy");
    });
}
popcorn_status_t popcorn_event_record(popcorn_event_t event, popcorn_stream_t stream) {
    return guarded([&] {
        need(event, "event");
        checkHip(hipEventRecord(reinterpret_cast<hipEvent_t>(event), S(stream)), "hipEventRecord");
    });
}
popcorn_status_t popcorn_event_wait(popcorn_stream_t stream, popcorn_event_t event) {
    return guarded([&] {
        need(event, "event");
        checkHip(hipStreamWaitEvent(S(stream), reinterpret_cast<hipEvent_t>(event), 0), "hipStreamWaitEvent");
    });
}
popcorn_status_t popcorn_event_synchronize(popcorn_event_t event) {
    return guarded([&] {
        need(event, "event");
        checkHip(hipEventSynchronize(reinterpret_cast<hipEvent_t>(event)), "hipEventSynchronize");
    });
}
popcorn_status_t popcorn_event_elapsed_ms(popcorn_event_t start, popcorn_event_t stop, float *ms) {
    return guarded([&] {
        need(start, "start");
        need(stop, "stop");
        need(ms, "ms");
        checkHip(hipEventElapsedTime(ms, reinterpret_cast<hipEvent_t>(start), reinterpret_cast<hipEvent_t>(stop)),
                 "hipEventElapsedTime");
    });
}

// ---- library -------------------------------------------------------------------------

popcorn_status_t popcorn_library_load(const char *path, popcorn_library_t *library) {
    return guarded([&] {
        need(library, "library");
        *library = nullptr;
        auto l = std::make_unique<KernelLibrary>(path ? path : "");
        *library = new popcorn_library_s{std::move(l)};
    });
}

popcorn_status_t popcorn_library_destroy(popcorn_library_t library) {
    return guarded([&] { delete library; });
}

popcorn_status_t popcorn_library_function(popcorn_library_t library, const char *name, popcorn_function_t *function) {
    return guarded([&] {
        need(library, "library");
        need(name, "name");
        need(function, "function");
        const Function &f = library->lib->function(name);
        // handles are owned by the library; the cache keeps them stable
        *function = reinterpret_cast<popcorn_function_t>(const_cast<Function *>(&f));
    });
}

popcorn_status_t popcorn_function_attributes(popcorn_function_t function, popcorn_function_attrs_t *attrs) {
    return guarded([&] {
        need(function, "function");
        need(attrs, "attrs");
        const Function *f = reinterpret_cast<const Function *>(function);
        attrs->max_threads_per_block = f->attrs.maxThreadsPerBlock;
        attrs->wave_size = f->attrs.waveSize;
        attrs->static_lds_bytes = f->attrs.staticLds;
        attrs->num_vgprs = f->attrs.numVgprs;
        attrs->num_sgprs = f->attrs.numSgprs;
        attrs->private_bytes = f->attrs.privateBytes;
    });
}

int32_t popcorn_library_cached_function_count(popcorn_library_t library) {
    return library ? (int32_t)library->lib->cachedCount() : 0;
}

static void fillLayout(const KernelLayout &L, popcorn_kernel_layout_t *out) {
    std::memset(out, 0, sizeof(*out));
    size_t i = 0;
    while (i < L.args.size() && L.args[i].pointer) ++i;
    out->nbuffers = (int32_t)i;
    out->nconstants = (int32_t)(L.args.size() - i);
    for (size_t j = i; j < L.args.size(); ++j) {
        if (j - i < POPCORN_MAX_CONSTANT_BLOCKS) out->constant_sizes[j - i] = L.args[j].size;
        if (L.args[j].pointer) ++out->trailing_pointers;
    }
    out->max_threads_per_block = L.maxThreads;
}

popcorn_status_t popcorn_function_layout(popcorn_function_t function, popcorn_kernel_layout_t *layout) {
    return guarded([&] {
        need(function, "function");
        need(layout, "layout");
        const Function *f = reinterpret_cast<const Function *>(function);
        if (!f->layout) throw Error::invalidArgument("no parameter metadata for " + f->name);
        fillLayout(*f->layout, layout);
    });
}

popcorn_status_t popcorn_code_object_layout(const char *path, const char *kernel, popcorn_kernel_layout_t *layout) {
    return guarded([&] {
        need(path, "path");
        need(kernel, "kernel");
        need(layout, "layout");
        const auto all = readKernelLayouts(std::string(path));
        auto it = all.find(kernel);
        if (it == all.end()) throw Error::kernelFunctionNotFound(kernel);
        fillLayout(it->second, layout);
    });
}

popcorn_status_t popcorn_launch(popcorn_stream_t stream, popcorn_function_t function, const uint32_t grid[3],
                                const uint32_t block[3], void *const *buffers, int32_t nbuffers,
                                const void *const *constants, const size_t *constant_sizes, int32_t nconstants,
                                size_t dynamic_lds_bytes) {
    return guarded([&] {
        need(function, "function");
        need(grid, "grid");
        need(block, "block");
        if (nbuffers < 0 || nconstants < 0) throw Error::invalidArgument("negative argument count");
        if (nbuffers) need(buffers, "buffers");
        if (nconstants) {
            need(constants, "constants");
            need(constant_sizes, "constant_sizes");
        }
        const Function *f = reinterpret_cast<const Function *>(function);
        if (f->layout) f->layout->check(f->name, (size_t)nbuffers, std::vector<size_t>(constant_sizes, constant_sizes + nconstants));
        if ((uint64_t)block[0] * block[1] * block[2] > (uint64_t)f->attrs.maxThreadsPerBlock)
            throw Error::invalidArgument("block of " + std::to_string((uint64_t)block[0] * block[1] * block[2]) +
                                         " threads exceeds the limit of " + f->name + " (" +
                                         std::to_string(f->attrs.maxThreadsPerBlock) + ")");
        std::vector<void *> ptrs(buffers, buffers + nbuffers);
        std::vector<void *> params;
        for (int32_t i = 0; i < nbuffers; ++i) params.push_back(&ptrs[(size_t)i]);
        for (int32_t i = 0; i < nconstants; ++i) params.push_back(const_cast<void *>(constants[i]));
        checkHip(hipModuleLaunchKernel(f->fn, grid[0], grid[1], grid[2], block[0], block[1], block[2],
                                       (unsigned)dynamic_lds_bytes, S(stream), params.data(), nullptr),
                 "hipModuleLaunchKernel");
    });
}

// ---- scratch ----------------------------------------------------------------------------

static popcorn_status_t pool_borrow(void *ctx, size_t length, void **buffer, int32_t *was_reused) {
    return guarded([&] {
        KernelTemporaryBuffer t = static_cast<ScratchPool *>(ctx)->borrowTemporaryBuffer(length);
        *buffer = t.buffer;
        if (was_reused) *was_reused = t.wasReused ? 1 : 0;
    });
}

static void pool_release(void *ctx, void *buffer) {
    try {
        static_cast<ScratchPool *>(ctx)->releaseTemporaryBuffer(KernelTemporaryBuffer{buffer, 0, false});
    } catch (...) {
    }
}

popcorn_status_t popcorn_scratch_pool_create(popcorn_scratch_pool_t *pool) {
    return guarded([&] {
        need(pool, "pool");
        *pool = new popcorn_scratch_pool_s();
    });
}

popcorn_status_t popcorn_scratch_pool_destroy(popcorn_scratch_pool_t pool) {
    return guarded([&] { delete pool; });
}

popcorn_status_t popcorn_scratch_pool_allocator(popcorn_scratch_pool_t pool, popcorn_scratch_allocator_t *allocator) {
    return guarded([&] {
        need(pool, "pool");
        need(allocator, "allocator");
        allocator->context = &pool->pool;
        allocator->borrow = pool_borrow;
        allocator->release = pool_release;
    });
}

size_t popcorn_scratch_pool_bytes(popcorn_scratch_pool_t pool) { return pool ? pool->pool.bytes() : 0; }

size_t popcorn_scratch_spec_byte_count(const int64_t *shape, int32_t rank, int32_t dtype) {
    ScratchSpec s{std::vector<int64_t>(shape, shape + (rank > 0 ? rank : 0)), (DataType)dtype};
    return s.byteCount();
}

// ---- encoder ------------------------------------------------------------------------------

popcorn_status_t popcorn_encoder_create(popcorn_library_t library, popcorn_stream_t stream,
                                        const popcorn_scratch_allocator_t *scratch, popcorn_encoder_t *encoder) {
    return guarded([&] {
        need(library, "library");
        need(encoder, "encoder");
        auto e = std::make_unique<popcorn_encoder_s>();
        if (scratch) {
            if (!scratch->borrow) throw Error::invalidArgument("scratch->borrow must not be NULL");
            e->ownedScratch = std::make_unique<CScratchAllocator>(*scratch);
        } else {
            e->ownedScratch = std::make_unique<ScratchPool>();
        }
        e->enc = std::make_unique<KernelCommandEncoder>(*library->lib, S(stream), *e->ownedScratch);
        *encoder = e.release();
    });
}

popcorn_status_t popcorn_encoder_destroy(popcorn_encoder_t encoder) {
    return guarded([&] {
        if (!encoder) return;
        // pooled scratch may still be in use by queued work
        (void)hipStreamSynchronize(encoder->enc->stream());
        delete encoder;
    });
}

popcorn_status_t popcorn_encoder_encode(popcorn_encoder_t encoder, popcorn_kernel_t kernel) {
    return guarded([&] {
        need(encoder, "encoder");
        need(kernel, "kernel");
        encoder->enc->encode(*kernel->k);
    });
}

popcorn_status_t popcorn_encoder_encode_all(popcorn_encoder_t encoder, const popcorn_kernel_t *kernels, int32_t count) {
    return guarded([&] {
        need(encoder, "encoder");
        if (count) need(kernels, "kernels");
        for (int32_t i = 0; i < count; ++i) {
            need(kernels[i], "kernel");
            encoder->enc->encode(*kernels[i]->k);
        }
    });
}

popcorn_status_t popcorn_encoder_barrier(popcorn_encoder_t encoder) {
    return guarded([&] {
        need(encoder, "encoder");
        encoder->enc->barrier();
    });
}

popcorn_status_t popcorn_encoder_stats(popcorn_encoder_t encoder, popcorn_encoder_stats_t *stats) {
    return guarded([&] {
        need(encoder, "encoder");
        need(stats, "stats");
        *stats = encoder->enc->stats();
    });
}

// ---- descriptors ----------------------------------------------------------------------------

int32_t popcorn_flash_attention_route(int64_t query_len, int64_t head_dim, int32_t q_dtype) {
    return (int32_t)Kernels::route(query_len, head_dim, (DataType)q_dtype);
}

static AttentionMask M(popcorn_attention_mask_t m) { return AttentionMask{m.kind, m.window}; }

popcorn_status_t popcorn_kernel_flash_attention(const popcorn_tensor_t *q, const popcorn_tensor_t *k,
                                                const popcorn_tensor_t *v, const popcorn_tensor_t *out, float scale,
                                                popcorn_attention_mask_t mask, popcorn_kernel_t *kernel) {
    return guarded([&] {
        emit(kernel, Kernels::FlashAttention(T(q, "q"), T(k, "k"), T(v, "v"), T(out, "out"), scale, M(mask)));
    });
}

popcorn_status_t popcorn_kernel_flash_attention_dims(const popcorn_tensor_t *q, const popcorn_tensor_t *k,
                                                     const popcorn_tensor_t *v, const popcorn_tensor_t *out, int64_t batch,
                                                     int64_t query_heads, int64_t kv_heads, int64_t query_len,
                                                     int64_t key_len, int64_t head_dim, float scale,
                                                     popcorn_attention_mask_t mask, int64_t key_capacity,
                                                     const popcorn_tensor_t *position, popcorn_kernel_t *kernel) {
    return guarded([&] {
        Tensor pos;
        if (position) pos = Tensor::fromC(*position);
        emit(kernel, Kernels::FlashAttention(T(q, "q"), T(k, "k"), T(v, "v"), T(out, "out"), batch, query_heads, kv_heads,
                                             query_len, key_len, head_dim, scale, M(mask), key_capacity,
                                             position ? &pos : nullptr));
    });
}

popcorn_status_t popcorn_flash_decoding_no_alloc(popcorn_library_t library, popcorn_stream_t stream,
                                                 const popcorn_tensor_t *q, const popcorn_tensor_t *k,
                                                 const popcorn_tensor_t *v, const popcorn_tensor_t *out, int64_t batch,
                                                 int64_t query_heads, int64_t kv_heads, int64_t query_len,
                                                 int64_t key_len, int64_t head_dim, float scale,
                                                 popcorn_attention_mask_t mask, int64_t key_capacity,
                                                 const popcorn_tensor_t *position) {
    return guarded([&] {
        need(library, "library");
        Tensor pos;
        if (position) pos = Tensor::fromC(*position);
        Kernels::FlashDecodingNoAlloc(*library->lib, S(stream), T(q, "q"), T(k, "k"), T(v, "v"), T(out, "out"), batch,
                                      query_heads, kv_heads, query_len, key_len, head_dim, scale, M(mask), key_capacity,
                                      position ? &pos : nullptr);
    });
}

popcorn_status_t popcorn_kernel_matmul(const popcorn_tensor_t *a, const popcorn_tensor_t *b, const popcorn_tensor_t *c,
                                       int32_t transpose_b, popcorn_kernel_t *kernel) {
    return guarded([&] { emit(kernel, Kernels::Matmul(T(a, "a"), T(b, "b"), T(c, "c"), transpose_b != 0)); });
}

popcorn_status_t popcorn_kernel_matmul_dims(const popcorn_tensor_t *a, const popcorn_tensor_t *b, const popcorn_tensor_t *c,
                                            int64_t m, int64_t k, int64_t n, int32_t transpose_b, popcorn_kernel_t *kernel) {
    return guarded([&] { emit(kernel, Kernels::Matmul(T(a, "a"), T(b, "b"), T(c, "c"), m, k, n, transpose_b != 0)); });
}

popcorn_status_t popcorn_kernel_rmsnorm(const popcorn_tensor_t *x, const popcorn_tensor_t *weight,
                                        const popcorn_tensor_t *out, int32_t axis, float eps, int32_t add_one_to_weight,
                                        popcorn_kernel_t *kernel) {
    return guarded([&] {
        Tensor w;
        if (weight) w = Tensor::fromC(*weight);
        emit(kernel, Kernels::RMSNorm(T(x, "x"), weight ? &w : nullptr, T(out, "out"), axis, eps, add_one_to_weight != 0));
    });
}

popcorn_status_t popcorn_kernel_rmsnorm_dims(const popcorn_tensor_t *x, const popcorn_tensor_t *weight,
                                             const popcorn_tensor_t *out, int64_t row_count, int64_t hidden_size,
                                             float eps, int32_t add_one_to_weight, popcorn_kernel_t *kernel) {
    return guarded([&] {
        Tensor w;
        if (weight) w = Tensor::fromC(*weight);
        emit(kernel, Kernels::RMSNorm(T(x, "x"), weight ? &w : nullptr, T(out, "out"), row_count, hidden_size, eps,
                                      add_one_to_weight != 0));
    });
}

popcorn_status_t popcorn_kernel_kv_cache_write(const popcorn_tensor_t *source, const popcorn_tensor_t *cache, int64_t offset,
                                               popcorn_kernel_t *kernel) {
    return guarded([&] { emit(kernel, Kernels::KVCacheWrite(T(source, "source"), T(cache, "cache"), offset)); });
}

popcorn_status_t popcorn_kernel_kv_cache_write_dims(const popcorn_tensor_t *source, const popcorn_tensor_t *cache,
                                                    int64_t batch, int64_t kv_heads, int64_t new_len, int64_t max_len,
                                                    int64_t head_dim, int64_t offset, const popcorn_tensor_t *position,
                                                    popcorn_kernel_t *kernel) {
    return guarded([&] {
        Tensor pos;
        if (position) pos = Tensor::fromC(*position);
        emit(kernel, Kernels::KVCacheWrite(T(source, "source"), T(cache, "cache"), batch, kv_heads, new_len, max_len,
                                           head_dim, offset, position ? &pos : nullptr));
    });
}

popcorn_status_t popcorn_kernel_gelu_tanh(const popcorn_tensor_t *x, const popcorn_tensor_t *out, popcorn_kernel_t *kernel) {
    return guarded([&] { emit(kernel, Kernels::GeluTanh(T(x, "x"), T(out, "out"))); });
}
popcorn_status_t popcorn_kernel_mul(const popcorn_tensor_t *a, const popcorn_tensor_t *b, const popcorn_tensor_t *out,
                                    popcorn_kernel_t *kernel) {
    return guarded([&] { emit(kernel, Kernels::Mul(T(a, "a"), T(b, "b"), T(out, "out"))); });
}
popcorn_status_t popcorn_kernel_add(const popcorn_tensor_t *a, const popcorn_tensor_t *b, const popcorn_tensor_t *out,
                                    popcorn_kernel_t *kernel) {
    return guarded([&] { emit(kernel, Kernels::Add(T(a, "a"), T(b, "b"), T(out, "out"))); });
}
popcorn_status_t popcorn_kernel_scalar_mul(const popcorn_tensor_t *x, float scalar, const popcorn_tensor_t *out,
                                           popcorn_kernel_t *kernel) {
    return guarded([&] { emit(kernel, Kernels::ScalarMul(T(x, "x"), scalar, T(out, "out"))); });
}

popcorn_status_t popcorn_kernel_rope_build_cos_sin(const popcorn_tensor_t *positions, const popcorn_tensor_t *inv_freq,
                                                 const popcorn_tensor_t *cos_out, const popcorn_tensor_t *sin_out,
                                                 float attention_scaling, popcorn_kernel_t *kernel) {
    return guarded([&] {
        emit(kernel, Kernels::RopeBuildCosSin(T(positions, "positions"), T(inv_freq, "invFreq"), T(cos_out, "cosOut"),
                                              T(sin_out, "sinOut"), attention_scaling));
    });
}
popcorn_status_t popcorn_kernel_rope_build_cos_sin_dims(const popcorn_tensor_t *positions, const popcorn_tensor_t *inv_freq,
                                                      const popcorn_tensor_t *cos_out, const popcorn_tensor_t *sin_out,
                                                      int64_t seq_len, int64_t half_head_dim, float attention_scaling,
                                                      popcorn_kernel_t *kernel) {
    return guarded([&] {
        emit(kernel, Kernels::RopeBuildCosSin(T(positions, "positions"), T(inv_freq, "invFreq"), T(cos_out, "cosOut"),
                                              T(sin_out, "sinOut"), seq_len, half_head_dim, attention_scaling));
    });
}
popcorn_status_t popcorn_kernel_rope_apply(const popcorn_tensor_t *x, const popcorn_tensor_t *cos_table,
                                         const popcorn_tensor_t *sin_table, const popcorn_tensor_t *out,
                                         popcorn_kernel_t *kernel) {
    return guarded([&] {
        emit(kernel, Kernels::RopeApply(T(x, "x"), T(cos_table, "cos"), T(sin_table, "sin"), T(out, "out")));
    });
}
popcorn_status_t popcorn_kernel_rope_apply_dims(const popcorn_tensor_t *x, const popcorn_tensor_t *cos_table,
                                              const popcorn_tensor_t *sin_table, const popcorn_tensor_t *out, int64_t batch,
                                              int64_t seq_len, int64_t head_count, int64_t head_dim,
                                              popcorn_kernel_t *kernel) {
    return guarded([&] {
        emit(kernel, Kernels::RopeApply(T(x, "x"), T(cos_table, "cos"), T(sin_table, "sin"), T(out, "out"), batch, seq_len,
                                        head_count, head_dim));
    });
}
popcorn_status_t popcorn_kernel_transpose12(const popcorn_tensor_t *src, const popcorn_tensor_t *out, popcorn_kernel_t *kernel) {
    return guarded([&] { emit(kernel, Kernels::Transpose12(T(src, "src"), T(out, "out"))); });
}
popcorn_status_t popcorn_kernel_transpose12_dims(const popcorn_tensor_t *src, const popcorn_tensor_t *out, int64_t d0,
                                               int64_t d1, int64_t d2, int64_t d3, popcorn_kernel_t *kernel) {
    return guarded([&] { emit(kernel, Kernels::Transpose12(T(src, "src"), T(out, "out"), d0, d1, d2, d3)); });
}

popcorn_status_t popcorn_kernel_gated_mlp(const popcorn_tensor_t *x, const popcorn_tensor_t *norm_weight,
                                          const popcorn_tensor_t *w_gate, const popcorn_tensor_t *w_up,
                                          const popcorn_tensor_t *w_down, const popcorn_tensor_t *out, float eps,
                                          int32_t add_one_to_weight, const popcorn_tensor_t *hidden,
                                          popcorn_kernel_t *kernel) {
    return guarded([&] {
        Tensor nw, h;
        if (norm_weight) nw = Tensor::fromC(*norm_weight);
        if (hidden) h = Tensor::fromC(*hidden);
        emit(kernel, Kernels::GatedMLP(T(x, "x"), norm_weight ? &nw : nullptr, T(w_gate, "w_gate"), T(w_up, "w_up"),
                                       T(w_down, "w_down"), T(out, "out"), eps, add_one_to_weight != 0,
                                       hidden ? &h : nullptr));
    });
}

popcorn_status_t popcorn_kernel_gated_mlp_residual(const popcorn_tensor_t *x_in, const popcorn_tensor_t *delta,
                                                   const popcorn_tensor_t *w_post, const popcorn_tensor_t *x_out,
                                                   const popcorn_tensor_t *norm_weight, const popcorn_tensor_t *w_gate,
                                                   const popcorn_tensor_t *w_up, const popcorn_tensor_t *w_down,
                                                   const popcorn_tensor_t *out, float eps, int32_t add_one_to_weight,
                                                   const popcorn_tensor_t *hidden, popcorn_kernel_t *kernel) {
    return guarded([&] {
        Tensor nw, h;
        if (norm_weight) nw = Tensor::fromC(*norm_weight);
        if (hidden) h = Tensor::fromC(*hidden);
        emit(kernel, Kernels::GatedMLPResidual(T(x_in, "x_in"), T(delta, "delta"), T(w_post, "w_post"), T(x_out, "x_out"),
                                               norm_weight ? &nw : nullptr, T(w_gate, "w_gate"), T(w_up, "w_up"),
                                               T(w_down, "w_down"), T(out, "out"), eps, add_one_to_weight != 0,
                                               hidden ? &h : nullptr));
    });
}

namespace {
AffineQuantizedTensor quantized(const popcorn_affine_quantized_tensor_t *q, const char *what) {
    need(q, what);
    AffineQuantizedTensor t;
    t.packedValues = Tensor::fromC(q->packed_values);
    t.scales = Tensor::fromC(q->scales);
    t.hasBiases = q->biases.data != nullptr;
    if (t.hasBiases) t.biases = Tensor::fromC(q->biases);
    if (q->rank < 0 || q->rank > POPCORN_MAX_RANK) throw Error::invalidArgument(std::string(what) + ": rank out of range");
    std::vector<int64_t> dims(q->shape, q->shape + q->rank);
    t.shape = Shape(std::move(dims));
    t.bits = q->bits;
    t.groupSize = q->group_size;
    return t;
}
}  // namespace

popcorn_status_t popcorn_kernel_decode_attention(const popcorn_decode_attention_args_t *args, popcorn_kernel_t *kernel) {
    return guarded([&] {
        need(args, "args");
        Tensor t[8];
        const popcorn_tensor_t *src[8] = {args->qkv,    args->k_cache, args->v_cache, args->out,
                                          args->position, args->q_norm, args->k_norm, args->inv_freq};
        const Tensor *p[8];
        for (int i = 0; i < 8; ++i) {
            p[i] = nullptr;
            if (src[i]) {
                t[i] = Tensor::fromC(*src[i]);
                p[i] = &t[i];
            }
        }
        Kernels::DecodeAttentionArgs a;
        a.qkv = p[0];
        a.kCache = p[1];
        a.vCache = p[2];
        a.out = p[3];
        a.position = p[4];
        a.qNorm = p[5];
        a.kNorm = p[6];
        a.invFreq = p[7];
        a.vNorm = args->v_norm != 0;
        a.queryHeads = args->query_heads;
        a.kvHeads = args->kv_heads;
        a.eps = args->eps;
        a.scale = args->scale;
        a.ropeScaling = args->rope_scaling;
        a.mask = AttentionMask{args->mask.kind, args->mask.window};
        emit(kernel, Kernels::DecodeAttention(a));
    });
}

popcorn_status_t popcorn_kernel_decode_matvec(const popcorn_decode_matvec_args_t *args, popcorn_kernel_t *kernel) {
    return guarded([&] {
        need(args, "args");
        Tensor t[10];
        const popcorn_tensor_t *src[10] = {args->x, args->delta, args->w_post, args->x_out, args->w_pre,
                                           args->weight, args->out, args->k_cache, args->v_cache, args->position};
        const Tensor *p[10];
        for (int i = 0; i < 10; ++i) {
            p[i] = nullptr;
            if (src[i]) {
                t[i] = Tensor::fromC(*src[i]);
                p[i] = &t[i];
            }
        }
        Kernels::DecodeMatvecArgs a;
        a.x = p[0];
        a.delta = p[1];
        a.wPost = p[2];
        a.xOut = p[3];
        a.wPre = p[4];
        a.weight = p[5];
        a.out = p[6];
        a.kCache = p[7];
        a.vCache = p[8];
        a.position = p[9];
        a.qRows = args->q_rows;
        a.eps = args->eps;
        AffineQuantizedTensor qw;
        if (args->qweight) {
            qw = quantized(args->qweight, "qweight");
            a.qweight = &qw;
        }
        emit(kernel, Kernels::DecodeMatvec(a));
    });
}


popcorn_status_t popcorn_kernel_gated_mlp_residual_quantized(
    const popcorn_tensor_t *x_in, const popcorn_tensor_t *delta, const popcorn_tensor_t *w_post,
    const popcorn_tensor_t *x_out, const popcorn_tensor_t *norm_weight, const popcorn_affine_quantized_tensor_t *w_gate,
    const popcorn_affine_quantized_tensor_t *w_up, const popcorn_affine_quantized_tensor_t *w_down,
    const popcorn_tensor_t *out, float eps, const popcorn_tensor_t *hidden, popcorn_kernel_t *kernel) {
    return guarded([&] {
        Tensor d, w, xo, h;
        if (delta) d = Tensor::fromC(*delta);
        if (w_post) w = Tensor::fromC(*w_post);
        if (x_out) xo = Tensor::fromC(*x_out);
        if (hidden) h = Tensor::fromC(*hidden);
        emit(kernel, Kernels::GatedMLPResidual(T(x_in, "x_in"), delta ? &d : nullptr, w_post ? &w : nullptr,
                                               x_out ? &xo : nullptr, T(norm_weight, "norm_weight"), quantized(w_gate, "w_gate"),
                                               quantized(w_up, "w_up"), quantized(w_down, "w_down"), T(out, "out"), eps,
                                               hidden ? &h : nullptr));
    });
}

popcorn_status_t popcorn_affine_quantized_validate(const popcorn_affine_quantized_tensor_t *tensor) {
    return guarded([&] { quantized(tensor, "tensor").validate(); });
}

popcorn_status_t popcorn_kernel_matmul_quantized(const popcorn_tensor_t *a, const popcorn_affine_quantized_tensor_t *b,
                                                 const popcorn_tensor_t *c, popcorn_kernel_t *kernel) {
    return guarded([&] { emit(kernel, Kernels::Matmul(T(a, "a"), quantized(b, "b"), T(c, "c"))); });
}

popcorn_status_t popcorn_kernel_embedding_gather_quantized(const popcorn_tensor_t *ids,
                                                           const popcorn_affine_quantized_tensor_t *table,
                                                           const popcorn_tensor_t *out, popcorn_kernel_t *kernel) {
    return guarded([&] { emit(kernel, Kernels::EmbeddingGather(T(ids, "ids"), quantized(table, "table"), T(out, "out"))); });
}

popcorn_status_t popcorn_kernel_embedding_gather(const popcorn_tensor_t *ids, const popcorn_tensor_t *table,
                                                 const popcorn_tensor_t *out, popcorn_kernel_t *kernel) {
    return guarded([&] { emit(kernel, Kernels::EmbeddingGather(T(ids, "ids"), T(table, "table"), T(out, "out"))); });
}

popcorn_status_t popcorn_kernel_argmax(const popcorn_tensor_t *x, const popcorn_tensor_t *indices, popcorn_kernel_t *kernel) {
    return guarded([&] { emit(kernel, Kernels::Argmax(T(x, "x"), T(indices, "indices"))); });
}

popcorn_status_t popcorn_kernel_custom(const char *function_name, const popcorn_tensor_t *tensors, const uint8_t *access,
                                       int32_t ntensors, const void *const *constants, const size_t *constant_sizes,
                                       int32_t nconstants, const uint32_t grid[3], const uint32_t block[3],
                                       popcorn_kernel_t *kernel) {
    return guarded([&] {
        need(function_name, "function_name");
        need(grid, "grid");
        need(block, "block");
        if (ntensors < 0 || nconstants < 0) throw Error::invalidArgument("negative count");
        std::vector<Binding> b;
        for (int32_t i = 0; i < ntensors; ++i) {
            uint8_t acc = access ? access[i] : (uint8_t)kReadWrite;
            if (acc == 0 || acc > 3) throw Error::invalidArgument("tensor binding access must not be empty");  // Tensor.swift:208
            b.push_back({Tensor::fromC(tensors[i]), acc});
        }
        std::vector<std::vector<uint8_t>> c;
        for (int32_t i = 0; i < nconstants; ++i) {
            const uint8_t *p = static_cast<const uint8_t *>(constants[i]);
            c.emplace_back(p, p + constant_sizes[i]);
        }
        emit(kernel, Kernels::Custom(function_name, std::move(b), std::move(c), dim3(grid[0], grid[1], grid[2]),
                                     dim3(block[0], block[1], block[2])));
    });
}

popcorn_status_t popcorn_kernel_destroy(popcorn_kernel_t kernel) {
    return guarded([&] { delete kernel; });
}

popcorn_status_t popcorn_kernel_describe(popcorn_kernel_t kernel, char *buffer, size_t capacity) {
    return guarded([&] {
        need(kernel, "kernel");
        need(buffer, "buffer");
        std::string s = kernel->k->describe();
        if (capacity == 0) throw Error::invalidArgument("capacity must be positive");
        std::strncpy(buffer, s.c_str(), capacity - 1);
        buffer[capacity - 1] = '\0';
    });
}

popcorn_status_t popcorn_fill_normal(popcorn_library_t library, popcorn_stream_t stream, void *data, int32_t dtype,
                                     uint64_t count, uint64_t seed, float mean, float stddev) {
    return guarded([&] {
        need(library, "library");
        ScratchPool none;
        KernelCommandEncoder enc(*library->lib, S(stream), none);
        enc.encode(*Kernels::FillNormal(data, (DataType)dtype, count, seed, mean, stddev));
    });
}

}  // extern "C"
