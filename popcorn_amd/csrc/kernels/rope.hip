// The pieces of a real attention block around the projections: the RoPE
// tables (RopeBuildCosSin.metal:5-21), the half-rotation RoPE
// (RopeApply.metal:7-49) and the [D0, D1, D2, D3] -> [D0, D2, D1, D3] head
// transpose (Transpose12.metal:7-25). All three are one pass over HBM: each
// lane moves 16-byte runs along the contiguous last axis when the shape and
// the pointers allow it, single elements otherwise.
#include "common.hpp"

namespace {

constexpr int kThreads = 256;

__device__ inline uint64_t first_index() { return (uint64_t)blockIdx.x * kThreads + threadIdx.x; }
__device__ inline uint64_t grid_stride() { return (uint64_t)gridDim.x * kThreads; }

bool __device__ inline aligned16(const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

// V consecutive elements widened to f32 / rounded from f32, in 16-byte pieces.
template <typename T, int V>
__device__ inline void load_run(const typename T::storage *p, float *f) {
    constexpr int kPer = pk::Vec<T>::kVec;
    static_assert(V % kPer == 0, "a run is whole 16-byte pieces");
#pragma unroll
    for (int c = 0; c < V / kPer; ++c) {
        pk::Vec<T> v;
        v.load(p + c * kPer);
        v.to_float(f + c * kPer);
    }
}

template <typename T, int V>
__device__ inline void store_run(typename T::storage *p, const float *f) {
    constexpr int kPer = pk::Vec<T>::kVec;
#pragma unroll
    for (int c = 0; c < V / kPer; ++c) {
        typename T::storage r[kPer];
#pragma unroll
        for (int e = 0; e < kPer; ++e) r[e] = T::store(f[c * kPer + e]);
        *reinterpret_cast<pk::u32x4 *>(p + c * kPer) = *reinterpret_cast<const pk::u32x4 *>(r);
    }
}

// out[..., i] = x1 c - x2 s, out[..., Hd2 + i] = x1 s + x2 c, with x1 =
// x[..., i], x2 = x[..., Hd2 + i] and (c, s) the table row of the token
// (RopeApply.metal:36-37). Work item = one run of kRun pair indices of one
// head; the last, partial run of a head and unaligned data go element by
// element with the same arithmetic.
template <typename X, typename Tab, typename O>
__device__ void rope_apply_run(const typename X::storage *__restrict__ x, const typename Tab::storage *__restrict__ cos_tab,
                           const typename Tab::storage *__restrict__ sin_tab, typename O::storage *__restrict__ out,
                           const RopeApplyConstants &p) {
    constexpr int kRun = 8;
    const uint32_t runs = (p.Hd2 + kRun - 1) / kRun;
    const uint64_t total = (uint64_t)p.B * p.T * p.Nh * runs;
    const bool vec = (p.Hd2 % kRun) == 0 && aligned16(x) && aligned16(out) && aligned16(cos_tab) && aligned16(sin_tab);
    for (uint64_t id = first_index(); id < total; id += grid_stride()) {
        const uint32_t run = (uint32_t)(id % runs);
        const uint64_t head = id / runs;  // (b * T + t) * Nh + h
        const uint32_t t = (uint32_t)((head / p.Nh) % p.T);
        const uint64_t base = head * 2ull * p.Hd2;
        const uint64_t tab = (uint64_t)t * p.Hd2;
        const uint32_t i0 = run * kRun;
        if (vec) {
            float x1[kRun], x2[kRun], c[kRun], s[kRun], o1[kRun], o2[kRun];
            load_run<X, kRun>(x + base + i0, x1);
            load_run<X, kRun>(x + base + p.Hd2 + i0, x2);
            load_run<Tab, kRun>(cos_tab + tab + i0, c);
            load_run<Tab, kRun>(sin_tab + tab + i0, s);
#pragma unroll
            for (int e = 0; e < kRun; ++e) {
                o1[e] = x1[e] * c[e] - x2[e] * s[e];
                o2[e] = x1[e] * s[e] + x2[e] * c[e];
            }
            store_run<O, kRun>(out + base + i0, o1);
            store_run<O, kRun>(out + base + p.Hd2 + i0, o2);
        } else {
            const uint32_t end = min(i0 + kRun, p.Hd2);
            for (uint32_t i = i0; i < end; ++i) {
                const float x1 = X::load(x[base + i]), x2 = X::load(x[base + p.Hd2 + i]);
                const float c = Tab::load(cos_tab[tab + i]), s = Tab::load(sin_tab[tab + i]);
                out[base + i] = O::store(x1 * c - x2 * s);
                out[base + p.Hd2 + i] = O::store(x1 * s + x2 * c);
            }
        }
    }
}

// out[d0][d2][d1][d3] = src[d0][d1][d2][d3] (Transpose12.metal:16-24); a work
// item is one 16-byte run of d3 when D3 fills whole runs, else one element.
template <typename E>
__device__ void transpose12_run(const E *__restrict__ src, E *__restrict__ out, const Transpose12Constants &p) {
    constexpr uint32_t kRun = 16 / sizeof(E);
    const bool vec = (p.D3 % kRun) == 0 && aligned16(src) && aligned16(out);
    const uint32_t run = vec ? kRun : 1;
    const uint32_t perRow = p.D3 / run;
    const uint64_t total = (uint64_t)p.D0 * p.D1 * p.D2 * perRow;
    for (uint64_t id = first_index(); id < total; id += grid_stride()) {
        const uint32_t c = (uint32_t)(id % perRow);
        uint64_t r = id / perRow;
        const uint32_t d2 = (uint32_t)(r % p.D2);
        r /= p.D2;
        const uint32_t d1 = (uint32_t)(r % p.D1);
        const uint64_t d0 = r / p.D1;
        const uint64_t from = id * run;
        const uint64_t to = (((d0 * p.D2 + d2) * p.D1 + d1) * p.D3) + (uint64_t)c * run;
        if (vec)
            *reinterpret_cast<pk::u32x4 *>(out + to) = __builtin_nontemporal_load(reinterpret_cast<const pk::u32x4 *>(src + from));
        else
            out[to] = src[from];
    }
}

}  // namespace

using pk::BF16;
using pk::F16;
using pk::F32;

// cos/sin of angle = float(position) * inv_freq, times `scaling`
// (RopeBuildCosSin.metal:17-20). sincosf is the full-precision library
// routine (argument reduction valid for every float angle).
POPCORN_KERNEL void __launch_bounds__(256)
    rope_build_cos_sin(const int32_t *__restrict__ positions, const float *__restrict__ inv_freq, float *__restrict__ cos_out,
                       float *__restrict__ sin_out, RopeBuildCosSinConstants p) {
    const uint64_t total = (uint64_t)p.T * p.Hd2;
    for (uint64_t id = first_index(); id < total; id += grid_stride()) {
        const uint32_t t = (uint32_t)(id / p.Hd2), i = (uint32_t)(id % p.Hd2);
        const float angle = (float)positions[t] * inv_freq[i];
        float s, c;
        sincosf(angle, &s, &c);
        cos_out[id] = c * p.scaling;
        sin_out[id] = s * p.scaling;
    }
}

#define ROPE(name, X, TAB, O)                                                                                   \
    POPCORN_KERNEL void __launch_bounds__(256) name(const X::storage *x, const TAB::storage *c, const TAB::storage *s, \
                                                    O::storage *out, RopeApplyConstants p) {                    \
        rope_apply_run<X, TAB, O>(x, c, s, out, p);                                                                 \
    }

// RopeApply.swift:25-30 (RopeApply.metal:51-53)
ROPE(rope_apply, F32, F32, F32)
ROPE(rope_apply_bf16, BF16, BF16, BF16)
ROPE(rope_apply_f32_tables_bf16, BF16, F32, BF16)

// Transpose12.swift:15-20 (Transpose12.metal:27-29)
POPCORN_KERNEL void __launch_bounds__(256) transpose12(const float *src, float *out, Transpose12Constants p) {
    transpose12_run<float>(src, out, p);
}
POPCORN_KERNEL void __launch_bounds__(256) transpose12_f16(const uint16_t *src, uint16_t *out, Transpose12Constants p) {
    transpose12_run<uint16_t>(src, out, p);
}
POPCORN_KERNEL void __launch_bounds__(256) transpose12_bf16(const uint16_t *src, uint16_t *out, Transpose12Constants p) {
    transpose12_run<uint16_t>(src, out, p);
}
