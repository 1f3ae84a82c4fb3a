// Building blocks of the block-affine 4-bit matvecs (affine_quant.hip):
// weights w = q * scale + bias with q an unsigned 4-bit value, 8 values per
// little-endian u32 word (value i in bits 4(i % 8) .. 4(i % 8) + 3,
// AffineQuantizationFormat.swift:25-29) and one bf16 scale/bias pair per group
// of 64 values along the row (AffineQuantizedTensor.swift:5-17).
//
// Per group g of a row: sum_k x_k (q_k s + b) = s * sum_k x_k q_k + b * X_g with
// X_g = sum_k x_k (the identity the reference's aq_qmv_fast uses,
// AffineQuantizedMatmul.metal:75-82), so the inner loop is a plain dot product
// of x with the raw nibbles and the group sums X_g are computed once per block.
//
// For bf16 activations the dot product runs on v_dot2_f32_bf16 (two bf16
// products accumulated in f32 per instruction; bf16 x bf16 products are exact
// in f32). A nibble pair becomes a bf16 pair with one mask and one OR: bf16
// 0x4300 is 128.0 and its 7-bit mantissa step is 1, so 0x4300 | q = 128 + q
// exactly. One AND with 0x000F000F takes nibbles p and p + 4 of a word into
// the two halves, hence x is staged in LDS as the bf16 pairs (x[8j + p],
// x[8j + p + 4]). The dot then holds sum x (128 + q) and the group's result is
// s * dot + (b - 128 s) * X_g.
#pragma once

#include "stream.hpp"

namespace pk {

constexpr uint32_t kQ4Group = 64;          // values per scale/bias group
constexpr uint32_t kQ4GroupWords = 8;      // packed u32 words per group
constexpr uint32_t kQ4PairBase = 0x43004300u;  // bf16 pair (128, 128)
// LDS words per group of staged x: 32 pair words + 4 of padding, so that the
// 16-byte reads of 8 consecutive groups (8 lanes of one row, or one lane of
// 8 rows... any 8 lanes served together) start in 8 different 4-bank slots
// instead of all in the same one (a stride of 32 words is 32 banks).
constexpr uint32_t kQ4GroupStride = 36;

typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));

__device__ inline float dot2_bf16(uint32_t a, uint32_t b, float c) {
    return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, a), __builtin_bit_cast(bf16x2_t, b), c, false);
}

__device__ inline float bf16_lo(uint32_t v) { return __uint_as_float(v << 16); }
// The bf16 of group g in the word that holds groups g & ~1 and g | 1.
__device__ inline float bf16_half(uint32_t v, uint32_t g) { return __uint_as_float((g & 1u) ? (v & 0xffff0000u) : (v << 16)); }

// Staged activations of one row of x for the 4-bit stream, in LDS.
//   bf16 x (XF32 = false): xw[K / 64 * kQ4GroupStride] pair words (see
//                          above), gsum[K / 64];
//   f32 x  (XF32 = true):  xf[K] floats, gsum[K / 64].
// One thread per octet of 8 values: the octet sums meet in groups of 8 lanes.
template <bool XF32>
struct Q4Staging {
    // From 8 f32 values of octet o (already rounded as the caller stores x).
    __device__ static void put_octet(uint32_t *xw, float *xf, uint32_t o, const float *v) {
        if constexpr (XF32) {
            *reinterpret_cast<float4 *>(xf + 8 * o) = float4{v[0], v[1], v[2], v[3]};
            *reinterpret_cast<float4 *>(xf + 8 * o + 4) = float4{v[4], v[5], v[6], v[7]};
        } else {
            u32x4 w;
            w.x = (__float_as_uint(v[0]) >> 16) | (__float_as_uint(v[4]) & 0xffff0000u);
            w.y = (__float_as_uint(v[1]) >> 16) | (__float_as_uint(v[5]) & 0xffff0000u);
            w.z = (__float_as_uint(v[2]) >> 16) | (__float_as_uint(v[6]) & 0xffff0000u);
            w.w = (__float_as_uint(v[3]) >> 16) | (__float_as_uint(v[7]) & 0xffff0000u);
            *reinterpret_cast<u32x4 *>(xw + (o / 8) * kQ4GroupStride + 4 * (o % 8)) = w;
        }
    }

    // Octets o = tid + 256 j (pass j); `get(j, o, v)` fills the 8 values of
    // octet o. Ends with a barrier. K is a multiple of 64, so every group's 8
    // octets are 8 consecutive threads of one pass.
    template <class Get>
    __device__ static void build(uint32_t K, uint32_t *xw, float *xf, float *gsum, const Get &get) {
        const uint32_t octets = K / 8;
        for (uint32_t base = 0, j = 0; base < octets; base += kStreamThreads, ++j) {
            const uint32_t o = base + threadIdx.x;
            float v[8] = {0, 0, 0, 0, 0, 0, 0, 0};
            float s = 0.0f;
            if (o < octets) {
                get(j, o, v);
                put_octet(xw, xf, o, v);
#pragma unroll
                for (int e = 0; e < 8; ++e) s += v[e];
            }
            s = group_sum<8>(s);
            if (o < octets && (o & 7u) == 0) gsum[o / 8] = s;
        }
        __syncthreads();
    }
};

// One 4-bit matrix of N rows: its packed words, scales and biases (biases ==
// scales when the tensor has none; hasBias says so). Read through buffer
// resources with 32-bit byte offsets, so each array stays under 2 GB (the
// host checks); the scale and bias rows start 4-byte aligned (an even number
// of groups per row).
struct Q4Mat {
    const uint32_t *w;
    const uint16_t *s;
    const uint16_t *b;
};

// A buffer load at this byte offset is out of range: it returns zeros and
// reads no memory.
constexpr uint32_t kQ4OutOfRange = 0x80000000u;

// Streams units of kRows = 64 / LPR rows through a wave: lane l serves row
// l / LPR of the unit and groups g = l % LPR + LPR i of that row, one group
// (two 16-byte loads of words, one scale, one bias) per step; NS rows (of NS
// weight matrices of one shape, same row index) per lane. U steps stay in
// flight and each slot is refilled as soon as it is consumed (in issue
// order, as in RowStream). A unit's per-row results are summed over its LPR
// lanes.
// The sum over the LPR lanes of a row, in the row's first lane (LPR a power
// of two: in every lane of the row). LPR that is not a power of two is a
// multiple of 4, so rows start on quad boundaries: quads sum over DPP, and
// the row's first lane adds its row's other quads through ds_bpermute.
template <int LPR>
__device__ inline float row_sum(float v) {
    if constexpr ((LPR & (LPR - 1)) == 0) {
        return group_sum<LPR>(v);
    } else {
        static_assert(LPR % 4 == 0, "a row of lanes starts on a quad");
        const float q = group_sum<4>(v);
        const int lane = (int)(threadIdx.x & 63);
        float t = q;
#pragma unroll
        for (int k = 1; k < LPR / 4; ++k)
            t += __int_as_float(__builtin_amdgcn_ds_bpermute(((lane + 4 * k) & 63) * 4, __float_as_int(q)));
        return t;
    }
}

// Streams units of kRows = 64 / LPR rows through a wave (lanes past kRows x
// LPR idle: they read a valid row, and their sums are not stored).
template <int LPR, int NS, int U, bool XF32>
struct Q4Stream {
    static_assert(LPR >= 4 && LPR <= 64 && ((LPR & (LPR - 1)) == 0 || LPR % 4 == 0),
                  "LPR is a power of two or a multiple of 4 in [4, 64]");
    static constexpr int kRows = 64 / LPR;
    u32x4 wv[U][NS][2];
    // Scale and bias of the step's group, as the aligned 32-bit word that
    // holds the bf16 (groups 2i and 2i + 1 share a word; rows hold an even
    // number of groups, so words never straddle rows). A full-word load
    // needs no arithmetic at issue time: any (a 16-bit load's zero
    // extension included) makes the compiler wait for the load right there,
    // and as loads retire in order the whole queue would drain.
    uint32_t sv[U][NS], bv[U][NS];
    __amdgpu_buffer_rsrc_t rw[NS], rs[NS], rb[NS];
    uint32_t G, cpl, steps, first, stride, is, ii, iu, gl;
    uint32_t orow, srow;  // byte offsets of this lane's row of the unit being issued (words, scales)
    bool hasBias;
    // The nibble-pair mask and the bf16 (128, 128) base, held in registers so
    // that each pair is one v_and_or_b32 (which cannot take two literals).
    uint32_t pairMask, pairBase;

    // rowOf(unit): this lane's row of the unit (clamped to N - 1 by the caller).
    template <class RowOf>
    __device__ void init(const RowOf &rowOf, const Q4Mat (&m)[NS], uint32_t N, uint32_t K, uint32_t units,
                         uint32_t first_, uint32_t stride_, bool hasBias_) {
        asm volatile("v_mov_b32 %0, 0x000f000f" : "=v"(pairMask));
        asm volatile("v_mov_b32 %0, 0x43004300" : "=v"(pairBase));
        G = K / kQ4Group;
        gl = (threadIdx.x & 63) % LPR;
        cpl = (G + LPR - 1) / LPR;
        first = first_;
        stride = stride_;
        hasBias = hasBias_;
        const uint32_t nu = first < units ? (units - first + stride - 1) / stride : 0u;
        steps = nu * cpl;
        is = 0;
        ii = 0;
        iu = first;
        const int wordBytes = (int)(N * (K / 8) * 4u), scaleBytes = (int)(N * G * 2u);
#pragma unroll
        for (int s = 0; s < NS; ++s) {
            rw[s] = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint32_t *>(m[s].w), 0, wordBytes, 0x00020000);
            rs[s] = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t *>(m[s].s), 0, scaleBytes, 0x00020000);
            rb[s] = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t *>(m[s].b), 0, scaleBytes, 0x00020000);
        }
        set_row(rowOf(iu));
    }

    __device__ inline void set_row(uint32_t row) {
        orow = row * (G * kQ4GroupWords * 4u);
        srow = row * (G * 2u);
    }

    // Loads step `is` into `slot`. Once every step is issued, a slot is
    // filled from out-of-range offsets instead (zeros, no memory read), so
    // every path through the kernel issues the same loads and the compiler's
    // wait counts stay exact.
    template <class RowOf>
    __device__ inline void issue(int slot, const RowOf &rowOf) {
        const bool real = is < steps;
        const uint32_t g = min(gl + LPR * ii, G - 1);
        const uint32_t ow = real ? orow + g * (kQ4GroupWords * 4u) : kQ4OutOfRange;
        const uint32_t os = real ? srow + (g >> 1) * 4u : kQ4OutOfRange;
#pragma unroll
        for (int s = 0; s < NS; ++s) {
            wv[slot][s][0] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rw[s], ow, 0, 2));
            wv[slot][s][1] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rw[s], ow + 16u, 0, 2));
            sv[slot][s] = __builtin_amdgcn_raw_buffer_load_b32(rs[s], os, 0, 0);
            bv[slot][s] = __builtin_amdgcn_raw_buffer_load_b32(rb[s], os, 0, 0);
        }
        if (real) {
            ++is;
            if (++ii == cpl) {
                ii = 0;
                iu += stride;
                if (is < steps) set_row(rowOf(iu));
            }
        }
    }

    // Issues slots FROM .. TO - 1 (all of them by default). A kernel that
    // builds its vector with block barriers in between issues a first slot
    // before and the rest after: a wave whose loads back up in the memory
    // pipeline stalls at the issue, and the barrier would wait for the
    // slowest wave's last load, i.e. for nearly all of the block's stream.
    template <int FROM = 0, int TO = U, class RowOf>
    __device__ void start(const RowOf &rowOf) {
#pragma unroll
        for (int u = FROM; u < TO; ++u) issue(u, rowOf);
    }

    __device__ static inline uint32_t word(const u32x4 (&w)[2], int j) {
        const u32x4 &h = w[j >> 2];
        return (j & 3) == 0 ? h.x : (j & 3) == 1 ? h.y : (j & 3) == 2 ? h.z : h.w;
    }

    template <class Store>
    __device__ inline void consume(int slot, const uint32_t *xw, const float *xf, const float *gsum, float (&acc)[NS],
                                   uint32_t &ci, uint32_t &cu, Store &store) {
        const uint32_t g = gl + LPR * ci;
        if (g < G) {
            const float xg = gsum[g];
            if constexpr (!XF32) {
                u32x4 xv[8];
#pragma unroll
                for (int j = 0; j < 8; ++j) xv[j] = *reinterpret_cast<const u32x4 *>(xw + g * kQ4GroupStride + 4 * j);
#pragma unroll
                for (int s = 0; s < NS; ++s) {
                    float d0 = 0.0f, d1 = 0.0f, d2 = 0.0f, d3 = 0.0f;
#pragma unroll
                    for (int j = 0; j < 8; ++j) {
                        const uint32_t w = word(wv[slot][s], j);
                        d0 = dot2_bf16((w & pairMask) | pairBase, xv[j].x, d0);
                        d1 = dot2_bf16(((w >> 4) & pairMask) | pairBase, xv[j].y, d1);
                        d2 = dot2_bf16(((w >> 8) & pairMask) | pairBase, xv[j].z, d2);
                        d3 = dot2_bf16(((w >> 12) & pairMask) | pairBase, xv[j].w, d3);
                    }
                    const float dot = (d0 + d1) + (d2 + d3);
                    const float sc = bf16_half(sv[slot][s], g);
                    const float bi = hasBias ? bf16_half(bv[slot][s], g) : 0.0f;
                    acc[s] += sc * dot + (bi - 128.0f * sc) * xg;
                }
            } else {
#pragma unroll
                for (int s = 0; s < NS; ++s) {
                    float qd = 0.0f;
#pragma unroll
                    for (int j = 0; j < 8; ++j) {
                        const uint32_t w = word(wv[slot][s], j);
                        const float4 a = *reinterpret_cast<const float4 *>(xf + (uint64_t)g * 64 + 8 * j);
                        const float4 b = *reinterpret_cast<const float4 *>(xf + (uint64_t)g * 64 + 8 * j + 4);
                        qd += a.x * (float)(w & 15u) + a.y * (float)((w >> 4) & 15u) + a.z * (float)((w >> 8) & 15u) +
                              a.w * (float)((w >> 12) & 15u) + b.x * (float)((w >> 16) & 15u) +
                              b.y * (float)((w >> 20) & 15u) + b.z * (float)((w >> 24) & 15u) + b.w * (float)(w >> 28);
                    }
                    const float sc = bf16_half(sv[slot][s], g);
                    const float bi = hasBias ? bf16_half(bv[slot][s], g) : 0.0f;
                    acc[s] += sc * qd + bi * xg;
                }
            }
        }
        if (++ci == cpl) {
            float sums[NS];
#pragma unroll
            for (int s = 0; s < NS; ++s) {
                sums[s] = row_sum<LPR>(acc[s]);
                acc[s] = 0.0f;
            }
            store(cu, sums);
            ci = 0;
            cu += stride;
        }
    }

    template <class RowOf, class Store>
    __device__ void run(const uint32_t *xw, const float *xf, const float *gsum, const RowOf &rowOf, Store &store) {
        float acc[NS];
#pragma unroll
        for (int s = 0; s < NS; ++s) acc[s] = 0.0f;
        uint32_t cs = 0, ci = 0, cu = first;
        while (cs + 2 * U <= steps) {
#pragma unroll
            for (int u = 0; u < U; ++u) {
                consume(u, xw, xf, gsum, acc, ci, cu, store);
                issue(u, rowOf);
            }
            cs += U;
        }
        while (cs < steps) {
#pragma unroll
            for (int u = 0; u < U; ++u) {
                if (cs + u < steps) consume(u, xw, xf, gsum, acc, ci, cu, store);
                issue(u, rowOf);
            }
            cs += U;
        }
    }
};

}  // namespace pk
