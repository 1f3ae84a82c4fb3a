// KV-cache write: cache[b, h, offset + s, d] = store(load(src[b, h, s, d])).
// Semantics of Sources/Popcorn/Kernels/KVCacheWrite.metal:6-58 (pairs
// f32->f32, bf16->bf16, f32->bf16 of KVCacheWrite.swift:20-25, plus f16->f16).
// Bit-exact: bf16->bf16 and f16->f16 copy bits; f32->bf16 applies the
// reference's RNE formula.
//
// Each thread moves one run of up to kRun consecutive elements of one cache
// row (kRun = 8 for 2-byte sources, 4 for f32: one 16B load). A run never
// crosses a row, so the destination of a run is contiguous. The grid strides
// over the runs, so any launch shape covers the whole source (the
// reference's one thread per 4 elements, KVCacheWrite.swift:33-34, included).
//
// kv_cache_write* keep the reference's host names and parameter list
// (src, cache, KVCacheWriteConstants; KVCacheWrite.metal:6-11);
// kv_cache_write*_ext take a position tensor and KVCacheWriteExtConstants:
// when the write offset comes from the position (decode replayed from a
// graph) and the range would leave the cache, they write nothing.
#include "common.hpp"

namespace {

template <typename S, typename C>
__device__ void kv_write(const typename S::storage *__restrict__ src, typename C::storage *__restrict__ cache,
                         const int32_t *__restrict__ position, const KVCacheWriteExtConstants &p) {
    constexpr uint32_t kRun = 16 / sizeof(typename S::storage);
    uint32_t offset = p.offset;
    if (p.offsetFromPosition) {
        int32_t pos = position[0];
        if (pos < 0 || (uint64_t)pos + p.Snew > p.Smax) return;
        offset = (uint32_t)pos;
    }
    const uint32_t runs_per_row = (p.Hd + kRun - 1) / kRun;
    const uint64_t rows = (uint64_t)p.B * p.Nkv * p.Snew;
    const uint64_t total_runs = rows * runs_per_row;
    const bool vec_ok = (p.Hd % kRun) == 0 && (reinterpret_cast<uintptr_t>(src) % 16) == 0 &&
                        (reinterpret_cast<uintptr_t>(cache) % (kRun * sizeof(typename C::storage))) == 0;
    for (uint64_t r = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; r < total_runs;
         r += (uint64_t)gridDim.x * blockDim.x) {
        const uint64_t row = r / runs_per_row;
        const uint32_t d0 = (uint32_t)(r % runs_per_row) * kRun;
        const uint32_t s = (uint32_t)(row % p.Snew);
        const uint64_t bh = row / p.Snew;  // b * Nkv + h
        const typename S::storage *srow = src + row * p.Hd;
        typename C::storage *drow = cache + (bh * p.Smax + offset + s) * (uint64_t)p.Hd;
        if constexpr (sizeof(typename S::storage) == sizeof(typename C::storage) && S::kTag != 8) {
            // same 2-byte dtype: bit copy
            if (vec_ok) {
                *reinterpret_cast<pk::u32x4 *>(drow + d0) = *reinterpret_cast<const pk::u32x4 *>(srow + d0);
            } else {
                for (uint32_t d = d0; d < d0 + kRun && d < p.Hd; ++d) drow[d] = srow[d];
            }
        } else {
            if (vec_ok) {
                pk::Vec<S> v;
                v.load(srow + d0);
                typename C::storage out[kRun];
#pragma unroll
                for (uint32_t i = 0; i < kRun; ++i) out[i] = C::store(v.get(i));
                if constexpr (sizeof(out) == 16) {
                    *reinterpret_cast<pk::u32x4 *>(drow + d0) = *reinterpret_cast<const pk::u32x4 *>(out);
                } else {
                    *reinterpret_cast<pk::u32x2 *>(drow + d0) = *reinterpret_cast<const pk::u32x2 *>(out);
                }
            } else {
                for (uint32_t d = d0; d < d0 + kRun && d < p.Hd; ++d) drow[d] = C::store(S::load(srow[d]));
            }
        }
    }
}

}  // namespace

#define KV_WRITE(name, S, C)                                                                                  \
    POPCORN_KERNEL void __launch_bounds__(1024) name(const S::storage *src, C::storage *cache, KVCacheWriteConstants p) { \
        const KVCacheWriteExtConstants e{p.B, p.Nkv, p.Snew, p.Smax, p.Hd, p.offset, 0u};                   \
        kv_write<S, C>(src, cache, nullptr, e);                                                               \
    }                                                                                                         \
    POPCORN_KERNEL void __launch_bounds__(1024)                                                               \
        name##_ext(const S::storage *src, C::storage *cache, const int32_t *position, KVCacheWriteExtConstants p) { \
        kv_write<S, C>(src, cache, position, p);                                                              \
    }

using pk::BF16;
using pk::F16;
using pk::F32;

KV_WRITE(kv_cache_write, F32, F32)
KV_WRITE(kv_cache_write_bf16, BF16, BF16)
KV_WRITE(kv_cache_write_f32_to_bf16, F32, BF16)
KV_WRITE(kv_cache_write_f16, F16, F16)
