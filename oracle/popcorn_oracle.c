/*
 * popcorn_oracle.c — CPU restatement of the reference's decode hot path.
 *
 * TEST INFRASTRUCTURE ONLY: the checker for the HIP kernels, never the thing
 * measured or shipped. Only tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg load it.
 *
 * Build: gcc -O2 -ffp-contract=off -fPIC -shared (no fast-math), so every sum
 * below is a sequential f32 sum, as in the reference's Swift CPU loops.
 * Citations are file:line in the reference tree (finnvoor/Popcorn).
 */
#include "popcorn_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

/* ------------------------------------------------------------------------ */
/* Generators                                                                */
/* ------------------------------------------------------------------------ */

/* Tests/PopcornTests/Kernels/BidirectionalFATests.swift:100
 *   rng ^= rng << 13; rng ^= rng >> 7; rng ^= rng << 17 */
uint64_t oracle_xorshift64_next(uint64_t *state) {
    uint64_t x = *state;
    x ^= x << 13;
    x ^= x >> 7;
    x ^= x << 17;
    *state = x;
    return x;
}

/* BidirectionalFATests.swift:101
 *   Float(Int64(bitPattern: rng) >> 32) / Float(Int32.max) * 0.2 */
float oracle_fa_test_float(uint64_t *state) {
    uint64_t x = oracle_xorshift64_next(state);
    int64_t s = (int64_t)x >> 32; /* arithmetic shift, as Swift's >> on Int64 */
    float num = (float)s;
    float den = (float)2147483647; /* Float(Int32.max) rounds to 2^31 */
    return num / den * 0.2f;
}

/* Fills n values exactly as the reference FA test fills q, then k, then v
 * (BidirectionalFATests.swift:98-114) when called three times on one state. */
void oracle_fill_fa_test(uint64_t seed, float *out, size_t n) {
    uint64_t st = seed;
    for (size_t i = 0; i < n; ++i) out[i] = oracle_fa_test_float(&st);
}

/* Seeded N(mean, std): the reference has no normal generator, so this build
 * defines one — the xorshift64 above for uniforms, then Box–Muller (G. E. P.
 * Box and M. E. Muller, 1958) evaluated in double, both outputs used. */
void oracle_fill_normal(uint64_t seed, float mean, float stddev, float *out, size_t n) {
    uint64_t st = seed * 0x9E3779B97F4A7C15ull + 0xdeadbeefcafebabeull;
    if (st == 0) st = 0xdeadbeefcafebabeull;
    const double two_pi = 6.283185307179586476925286766559;
    size_t i = 0;
    while (i < n) {
        uint64_t a = oracle_xorshift64_next(&st);
        uint64_t b = oracle_xorshift64_next(&st);
        double u1 = ((double)(a >> 11) + 1.0) * (1.0 / 9007199254740992.0); /* (0,1] */
        double u2 = (double)(b >> 11) * (1.0 / 9007199254740992.0);         /* [0,1) */
        double r = sqrt(-2.0 * log(u1));
        double z0 = r * cos(two_pi * u2);
        double z1 = r * sin(two_pi * u2);
        out[i++] = (float)(mean + stddev * z0);
        if (i < n) out[i++] = (float)(mean + stddev * z1);
    }
}

/* ------------------------------------------------------------------------ */
/* Element conversions                                                       */
/* ------------------------------------------------------------------------ */

static uint32_t f32_bits(float x) { uint32_t u; memcpy(&u, &x, 4); return u; }
static float bits_f32(uint32_t u) { float x; memcpy(&x, &u, 4); return x; }

/* Sources/Popcorn/PopcornDTypes.h:29-34 — round-to-nearest-even by adding
 * 0x7fff + lsb, with no NaN special case (some NaNs become ±Inf). */
uint16_t oracle_f32_to_bf16(float x) {
    uint32_t bits = f32_bits(x);
    uint32_t lsb = (bits >> 16) & 1u;
    return (uint16_t)((bits + 0x7fffu + lsb) >> 16);
}

/* PopcornDTypes.h:11 — as_type<float>(uint(p[i]) << 16) */
float oracle_bf16_to_f32(uint16_t b) { return bits_f32((uint32_t)b << 16); }

/* IEEE 754 binary32 -> binary16, round to nearest even (Metal's half(x),
 * PopcornDTypes.h:37). NaN becomes the quiet NaN 0x7e00 with the sign kept. */
static uint32_t rne_shift(uint32_t m, uint32_t s) {
    if (s == 0) return m;
    if (s >= 32) return 0;
    uint32_t r = m >> s;
    uint32_t rem = m & ((1u << s) - 1u);
    uint32_t half = 1u << (s - 1u);
    if (rem > half || (rem == half && (r & 1u))) r++;
    return r;
}

uint16_t oracle_f32_to_f16(float x) {
    uint32_t u = f32_bits(x);
    uint16_t sign = (uint16_t)((u >> 16) & 0x8000u);
    uint32_t exp = (u >> 23) & 0xffu;
    uint32_t mant = u & 0x7fffffu;
    if (exp == 0xffu) return (uint16_t)(sign | (mant ? 0x7e00u : 0x7c00u));
    int e = (int)exp - 127 + 15;
    if (e >= 31) return (uint16_t)(sign | 0x7c00u);
    if (e <= 0) {
        if (exp == 0) return sign; /* f32 zero/subnormal: far below f16 range */
        uint32_t m = mant | 0x800000u;
        uint32_t s = (uint32_t)(14 - e);
        return (uint16_t)(sign | rne_shift(m, s));
    }
    uint32_t r = ((uint32_t)e << 10) | (mant >> 13);
    uint32_t rem = mant & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (r & 1u))) r++; /* carry may reach inf */
    return (uint16_t)(sign | r);
}

float oracle_f16_to_f32(uint16_t h) {
    uint32_t sign = ((uint32_t)h & 0x8000u) << 16;
    uint32_t exp = ((uint32_t)h >> 10) & 0x1fu;
    uint32_t mant = (uint32_t)h & 0x3ffu;
    if (exp == 0) {
        if (mant == 0) return bits_f32(sign);
        float v = (float)mant * (1.0f / 16777216.0f); /* 2^-24 exact */
        return sign ? -v : v;
    }
    if (exp == 31) return bits_f32(sign | 0x7f800000u | (mant << 13));
    return bits_f32(sign | ((exp - 15 + 127) << 23) | (mant << 13));
}

static float load_elem(const void *p, int dtype, size_t i) {
    switch (dtype) {
    case ORACLE_F32: return ((const float *)p)[i];
    case ORACLE_BF16: return oracle_bf16_to_f32(((const uint16_t *)p)[i]);
    case ORACLE_F16: return oracle_f16_to_f32(((const uint16_t *)p)[i]);
    default: return NAN;
    }
}

static void store_elem(void *p, int dtype, size_t i, float v) {
    switch (dtype) {
    case ORACLE_F32: ((float *)p)[i] = v; break;
    case ORACLE_BF16: ((uint16_t *)p)[i] = oracle_f32_to_bf16(v); break;
    case ORACLE_F16: ((uint16_t *)p)[i] = oracle_f32_to_f16(v); break;
    default: break;
    }
}

void oracle_convert(const void *src, int src_dtype, void *dst, int dst_dtype, size_t n) {
    for (size_t i = 0; i < n; ++i) store_elem(dst, dst_dtype, i, load_elem(src, src_dtype, i));
}

/* Round-trips v through `dtype` storage (the value a kernel reads back after
 * the reference stores an intermediate tensor of that dtype). */
static float round_to(int dtype, float v) {
    switch (dtype) {
    case ORACLE_BF16: return oracle_bf16_to_f32(oracle_f32_to_bf16(v));
    case ORACLE_F16: return oracle_f16_to_f32(oracle_f32_to_f16(v));
    default: return v;
    }
}

static void round_array(int dtype, float *v, size_t n) {
    if (dtype == ORACLE_F32) return;
    for (size_t i = 0; i < n; ++i) v[i] = round_to(dtype, v[i]);
}

/* ------------------------------------------------------------------------ */
/* KV-cache write                                                            */
/* ------------------------------------------------------------------------ */

/* Sources/Popcorn/Kernels/KVCacheWrite.metal:6-58 — cache[b,h,offset+s,d] =
 * store(load(src[b,h,s,d])). Pairs (f32,f32), (bf16,bf16), (f32,bf16) as in
 * KVCacheWrite.swift:20-25; (f16,f16) is this build's extension. bf16->bf16
 * goes through load (bits<<16) and the RNE store, which is the identity on
 * bits. Returns -1007 (tensorShapeMismatch) when offset+Snew > Smax
 * (KVCacheWrite.swift:45-47). */
int oracle_kv_cache_write(const void *src, int src_dtype, void *cache, int cache_dtype,
                          uint32_t B, uint32_t Nkv, uint32_t Snew, uint32_t Smax,
                          uint32_t Hd, uint32_t offset) {
    if ((uint64_t)offset + Snew > Smax) return -1007;
    uint64_t total = (uint64_t)B * Nkv * Snew * Hd;
    for (uint64_t i = 0; i < total; ++i) {
        uint64_t d = i % Hd;
        uint64_t rest = i / Hd;
        uint64_t s = rest % Snew;
        rest /= Snew;
        uint64_t h = rest % Nkv;
        uint64_t b = rest / Nkv;
        uint64_t dst = ((b * Nkv + h) * Smax + offset + s) * Hd + d;
        if (src_dtype == cache_dtype && src_dtype != ORACLE_F32) {
            ((uint16_t *)cache)[dst] = ((const uint16_t *)src)[i]; /* bitwise identity */
        } else {
            store_elem(cache, cache_dtype, dst, load_elem(src, src_dtype, i));
        }
    }
    return 0;
}

/* ------------------------------------------------------------------------ */
/* RMSNorm                                                                   */
/* ------------------------------------------------------------------------ */

/* Sources/Popcorn/Kernels/RMSNorm.metal:16-41, sum taken sequentially as in
 * the test's closed form (KernelsTests.swift:156-157):
 *   scale = 1/sqrt(sum(x^2)/H + eps);  y = (x*scale) * (addOne ? 1+w : w) */
void oracle_rmsnorm(const float *x, const float *weight, float *out, size_t rows,
                    size_t H, float eps, int add_one_to_weight) {
    for (size_t r = 0; r < rows; ++r) {
        const float *xr = x + r * H;
        float acc = 0.0f;
        for (size_t i = 0; i < H; ++i) acc += xr[i] * xr[i];
        float scale = 1.0f / sqrtf(acc / (float)H + eps);
        for (size_t i = 0; i < H; ++i) {
            float v = xr[i] * scale;
            if (weight) {
                float w = weight[i];
                if (add_one_to_weight) w = 1.0f + w;
                v *= w;
            }
            out[r * H + i] = v;
        }
    }
}

/* ------------------------------------------------------------------------ */
/* Matmul / matvec                                                           */
/* ------------------------------------------------------------------------ */

/* Tests/PopcornTests/Kernels/KernelsTests.swift:254-265 (runMatmul's CPU
 * loop): acc += a[i*K+kk] * (transposeB ? b[j*K+kk] : b[kk*N+j]).
 * M == 1 is the matvec (Matvec.metal:6-30, W [N,K] when transposed). */
void oracle_matmul(const float *a, const float *b, float *c, size_t M, size_t K,
                   size_t N, int transpose_b) {
    for (size_t i = 0; i < M; ++i) {
        for (size_t j = 0; j < N; ++j) {
            float acc = 0.0f;
            for (size_t kk = 0; kk < K; ++kk) {
                float av = a[i * K + kk];
                float bv = transpose_b ? b[j * K + kk] : b[kk * N + j];
                acc += av * bv;
            }
            c[i * N + j] = acc;
        }
    }
}

/* ------------------------------------------------------------------------ */
/* Elementwise                                                               */
/* ------------------------------------------------------------------------ */

/* Sources/Popcorn/Kernels/GeluTanh.metal:6-11 */
float oracle_gelu_tanh_scalar(float v) {
    const float k0 = 0.7978845608028654f;
    const float k1 = 0.044715f;
    float inner = k0 * (v + k1 * v * v * v);
    if (inner < -20.0f) inner = -20.0f;
    if (inner > 20.0f) inner = 20.0f;
    return 0.5f * v * (1.0f + tanhf(inner));
}

void oracle_gelu_tanh(const float *x, float *out, size_t n) {
    for (size_t i = 0; i < n; ++i) out[i] = oracle_gelu_tanh_scalar(x[i]);
}

/* Mul.metal:6-29, Add.metal:6-29, ScalarMul.metal */
void oracle_mul(const float *a, const float *b, float *out, size_t n) {
    for (size_t i = 0; i < n; ++i) out[i] = a[i] * b[i];
}
void oracle_add(const float *a, const float *b, float *out, size_t n) {
    for (size_t i = 0; i < n; ++i) out[i] = a[i] + b[i];
}
void oracle_scalar_mul(const float *a, float s, float *out, size_t n) {
    for (size_t i = 0; i < n; ++i) out[i] = a[i] * s;
}

/* ------------------------------------------------------------------------ */
/* Gated MLP                                                                 */
/* ------------------------------------------------------------------------ */

/* The reference's gated MLP is a composition of dispatches
 * (Examples/GemmaCLI/Sources/GemmaCLI/Gemma4TextInference.swift:416-429):
 *   n = RMSNorm(x); g = n·Wg^T; u = n·Wu^T; a = GeluTanh(g); h = a*u;
 *   out = h·Wd^T
 * with every intermediate stored as a tensor of the activation dtype
 * (Gemma4Workspace.swift:37-42). `inter_dtype` selects that storage dtype
 * (ORACLE_F32 keeps every intermediate in f32). `out` is the f32 value of the
 * down projection before its own store; h_out (optional) receives h. */
void oracle_gated_mlp(const float *x, const float *norm_w, float eps, int add_one,
                      const float *w_gate, const float *w_up, const float *w_down,
                      size_t H, size_t F, int inter_dtype, float *h_out, float *out) {
    float *n = (float *)malloc(H * sizeof(float));
    float *g = (float *)malloc(F * sizeof(float));
    float *u = (float *)malloc(F * sizeof(float));
    float *h = h_out ? h_out : (float *)malloc(F * sizeof(float));
    oracle_rmsnorm(x, norm_w, n, 1, H, eps, add_one);
    round_array(inter_dtype, n, H);
    oracle_matmul(n, w_gate, g, 1, H, F, 1);
    oracle_matmul(n, w_up, u, 1, H, F, 1);
    round_array(inter_dtype, g, F);
    round_array(inter_dtype, u, F);
    for (size_t i = 0; i < F; ++i) {
        float a = round_to(inter_dtype, oracle_gelu_tanh_scalar(g[i]));
        h[i] = round_to(inter_dtype, a * u[i]);
    }
    oracle_matmul(h, w_down, out, 1, F, H, 1);
    free(n);
    free(g);
    free(u);
    if (!h_out) free(h);
}

/* ------------------------------------------------------------------------ */
/* Attention                                                                 */
/* ------------------------------------------------------------------------ */

/* Mask predicate of FlashAttention.metal:72 and :85-87 (and
 * FlashDecoding.metal:73, :97-99): kind 0 causal, 1 causal + sliding window,
 * 2 bidirectional. */
static int mask_allows(uint32_t kind, int32_t window, int pos_q, int pos_k) {
    int allowed = (kind == 2u) || (pos_k <= pos_q);
    if (kind == 1u) allowed = allowed && ((pos_q - pos_k) < window);
    return allowed;
}

/* Naive attention: Tests/PopcornTests/Kernels/BidirectionalFATests.swift:9-53
 * (scores = (q·k)*scale, row max, expf, sum, divide, then P·V), generalised
 * with the kernels' GQA head map hkv = hq*Nkv/Nq (FlashAttention.metal:57),
 * the causal position posQ = Sk-Sq+i (FlashAttention.metal:72) and a KV row
 * stride `kv_stride` (>= Sk) for caches with spare capacity. A row whose keys
 * are all masked yields zeros here (the reference divides 0/0). */
void oracle_attention_naive(const float *q, const float *k, const float *v, float *out,
                            uint32_t B, uint32_t Nq, uint32_t Nkv, uint32_t Sq,
                            uint32_t Sk, uint32_t kv_stride, uint32_t Hd, float scale,
                            uint32_t mask_kind, int32_t window) {
    float *scores = (float *)malloc((Sk ? Sk : 1) * sizeof(float));
    for (uint32_t b = 0; b < B; ++b) {
        for (uint32_t hq = 0; hq < Nq; ++hq) {
            uint32_t hkv = hq * Nkv / Nq;
            const float *kh = k + (size_t)(b * Nkv + hkv) * kv_stride * Hd;
            const float *vh = v + (size_t)(b * Nkv + hkv) * kv_stride * Hd;
            for (uint32_t i = 0; i < Sq; ++i) {
                const float *qi = q + (((size_t)b * Nq + hq) * Sq + i) * Hd;
                float *oi = out + (((size_t)b * Nq + hq) * Sq + i) * Hd;
                int pos_q = (int)Sk - (int)Sq + (int)i;
                float row_max = -INFINITY;
                for (uint32_t j = 0; j < Sk; ++j) {
                    if (!mask_allows(mask_kind, window, pos_q, (int)j)) {
                        scores[j] = -INFINITY;
                        continue;
                    }
                    float s = 0.0f;
                    for (uint32_t d = 0; d < Hd; ++d) s += qi[d] * kh[(size_t)j * Hd + d];
                    scores[j] = s * scale;
                    if (scores[j] > row_max) row_max = scores[j];
                }
                if (row_max == -INFINITY) {
                    for (uint32_t d = 0; d < Hd; ++d) oi[d] = 0.0f;
                    continue;
                }
                float sum_exp = 0.0f;
                for (uint32_t j = 0; j < Sk; ++j) {
                    scores[j] = expf(scores[j] - row_max);
                    sum_exp += scores[j];
                }
                for (uint32_t j = 0; j < Sk; ++j) scores[j] /= sum_exp;
                for (uint32_t d = 0; d < Hd; ++d) {
                    float acc = 0.0f;
                    for (uint32_t j = 0; j < Sk; ++j) acc += scores[j] * vh[(size_t)j * Hd + d];
                    oi[d] = acc;
                }
            }
        }
    }
    free(scores);
}

/* Online-softmax state over one key range [j_lo, j_hi) in tiles of Bc keys,
 * the loop of FlashDecoding.metal:89-163 / FlashAttention.metal:74-154: per
 * tile, m_new = max(m, max s), scale_old = exp(m - m_new), p = exp(s - m_new),
 * l = scale_old*l + sum p, O = scale_old*O + sum p*V. Q is pre-scaled
 * (FlashDecoding.metal:65-68). A tile whose keys are all masked while m is
 * still -inf is skipped (the reference would compute exp(-inf - -inf)). */
static void online_softmax_range(const float *qs, const float *kh, const float *vh,
                                 uint32_t Hd, uint32_t j_lo, uint32_t j_hi, uint32_t Bc,
                                 int pos_q, uint32_t mask_kind, int32_t window,
                                 float *s_tile, float *m_io, float *l_io, float *o_io) {
    float m = *m_io, l = *l_io;
    for (uint32_t j0 = j_lo; j0 < j_hi; j0 += Bc) {
        uint32_t n = (j_hi - j0 < Bc) ? (j_hi - j0) : Bc;
        float tile_max = -INFINITY;
        for (uint32_t i = 0; i < n; ++i) {
            uint32_t j = j0 + i;
            float acc = -INFINITY;
            if (mask_allows(mask_kind, window, pos_q, (int)j)) {
                acc = 0.0f;
                for (uint32_t d = 0; d < Hd; ++d) acc += qs[d] * kh[(size_t)j * Hd + d];
            }
            s_tile[i] = acc;
            if (acc > tile_max) tile_max = acc;
        }
        float m_new = m > tile_max ? m : tile_max;
        if (m_new == -INFINITY) continue;
        float scale_old = expf(m - m_new);
        float psum = 0.0f;
        for (uint32_t i = 0; i < n; ++i) {
            s_tile[i] = expf(s_tile[i] - m_new);
            psum += s_tile[i];
        }
        l = scale_old * l + psum;
        m = m_new;
        for (uint32_t d = 0; d < Hd; ++d) {
            float acc = 0.0f;
            for (uint32_t i = 0; i < n; ++i) acc += s_tile[i] * vh[(size_t)(j0 + i) * Hd + d];
            o_io[d] = scale_old * o_io[d] + acc;
        }
    }
    *m_io = m;
    *l_io = l;
}

/* Split-KV decoding, Sources/Popcorn/Kernels/FlashDecoding.metal:28-231:
 * partition `part` of (b, hq) covers [part*per, min(+per, Sk)) with
 * per = ceil(Sk/P) (:56-63); posQ = Sk-1 (:73); a partition starting past
 * posQ writes m=-inf, l=0, O=0 (:78-87); otherwise the online softmax over
 * Bc=128 tiles (:89-163) leaves unnormalised O, m, l (:165-173). The combine
 * (:202-227): m* = max m_k, l* = sum exp(m_k-m*) l_k,
 * O = sum exp(m_k-m*) O_k / l*. partial_* may be NULL. */
void oracle_flash_decoding(const float *q, const float *k, const float *v, float *out,
                           uint32_t B, uint32_t Nq, uint32_t Nkv, uint32_t Sk,
                           uint32_t kv_stride, uint32_t Hd, uint32_t P, float scale,
                           uint32_t mask_kind, int32_t window, float *partial_o,
                           float *partial_m, float *partial_l) {
    const uint32_t Bc = 128;
    size_t npart = (size_t)B * Nq * P;
    float *po = partial_o ? partial_o : (float *)malloc(npart * Hd * sizeof(float));
    float *pm = partial_m ? partial_m : (float *)malloc(npart * sizeof(float));
    float *pl = partial_l ? partial_l : (float *)malloc(npart * sizeof(float));
    float *qs = (float *)malloc((Hd ? Hd : 1) * sizeof(float));
    float *s_tile = (float *)malloc(Bc * sizeof(float));
    uint32_t per = (Sk + P - 1u) / P;
    int pos_q = (int)Sk - 1;
    for (uint32_t b = 0; b < B; ++b) {
        for (uint32_t hq = 0; hq < Nq; ++hq) {
            uint32_t hkv = hq * Nkv / Nq;
            const float *kh = k + (size_t)(b * Nkv + hkv) * kv_stride * Hd;
            const float *vh = v + (size_t)(b * Nkv + hkv) * kv_stride * Hd;
            const float *qi = q + ((size_t)b * Nq + hq) * Hd;
            for (uint32_t d = 0; d < Hd; ++d) qs[d] = qi[d] * scale;
            for (uint32_t part = 0; part < P; ++part) {
                size_t idx = ((size_t)b * Nq + hq) * P + part;
                float *o = po + idx * Hd;
                for (uint32_t d = 0; d < Hd; ++d) o[d] = 0.0f;
                float m = -INFINITY, l = 0.0f;
                uint32_t j_lo = part * per;
                uint32_t j_hi = j_lo + per < Sk ? j_lo + per : Sk;
                if ((int64_t)j_lo <= (int64_t)pos_q)
                    online_softmax_range(qs, kh, vh, Hd, j_lo, j_hi, Bc, pos_q, mask_kind,
                                         window, s_tile, &m, &l, o);
                pm[idx] = m;
                pl[idx] = l;
            }
            /* combine */
            size_t base = ((size_t)b * Nq + hq) * P;
            float m_g = -INFINITY;
            for (uint32_t p = 0; p < P; ++p)
                if (pm[base + p] > m_g) m_g = pm[base + p];
            float *oo = out + ((size_t)b * Nq + hq) * Hd;
            if (m_g == -INFINITY) {
                for (uint32_t d = 0; d < Hd; ++d) oo[d] = 0.0f;
                continue;
            }
            float l_g = 0.0f;
            for (uint32_t p = 0; p < P; ++p) l_g += expf(pm[base + p] - m_g) * pl[base + p];
            float inv_l = 1.0f / l_g;
            for (uint32_t d = 0; d < Hd; ++d) {
                float acc = 0.0f;
                for (uint32_t p = 0; p < P; ++p)
                    acc += expf(pm[base + p] - m_g) * po[(base + p) * Hd + d];
                oo[d] = acc * inv_l;
            }
        }
    }
    free(qs);
    free(s_tile);
    if (!partial_o) free(po);
    if (!partial_m) free(pm);
    if (!partial_l) free(pl);
}

/* Fused attention, one query row at a time over the whole key range
 * (Sources/Popcorn/Kernels/FlashAttention.metal:30-162), tiles of Bc keys,
 * final O * (1/l) (:157-161). */
void oracle_flash_attention_rows(const float *q, const float *k, const float *v,
                                 float *out, uint32_t B, uint32_t Nq, uint32_t Nkv,
                                 uint32_t Sq, uint32_t Sk, uint32_t kv_stride,
                                 uint32_t Hd, uint32_t Bc, float scale,
                                 uint32_t mask_kind, int32_t window) {
    float *qs = (float *)malloc((Hd ? Hd : 1) * sizeof(float));
    float *s_tile = (float *)malloc((Bc ? Bc : 1) * sizeof(float));
    for (uint32_t b = 0; b < B; ++b) {
        for (uint32_t hq = 0; hq < Nq; ++hq) {
            uint32_t hkv = hq * Nkv / Nq;
            const float *kh = k + (size_t)(b * Nkv + hkv) * kv_stride * Hd;
            const float *vh = v + (size_t)(b * Nkv + hkv) * kv_stride * Hd;
            for (uint32_t i = 0; i < Sq; ++i) {
                const float *qi = q + (((size_t)b * Nq + hq) * Sq + i) * Hd;
                float *oi = out + (((size_t)b * Nq + hq) * Sq + i) * Hd;
                for (uint32_t d = 0; d < Hd; ++d) {
                    qs[d] = qi[d] * scale;
                    oi[d] = 0.0f;
                }
                float m = -INFINITY, l = 0.0f;
                int pos_q = (int)Sk - (int)Sq + (int)i;
                online_softmax_range(qs, kh, vh, Hd, 0, Sk, Bc, pos_q, mask_kind, window,
                                     s_tile, &m, &l, oi);
                float inv_l = l > 0.0f ? 1.0f / l : 0.0f;
                for (uint32_t d = 0; d < Hd; ++d) oi[d] *= inv_l;
            }
        }
    }
    free(qs);
    free(s_tile);
}

/* ------------------------------------------------------------------------ */
/* RoPE and head transposes                                                  */
/* ------------------------------------------------------------------------ */

/* Sources/Popcorn/Kernels/RopeBuildCosSin.metal:17-20:
 *   angle = float(positions[t]) * inv_freq[i]
 *   cos_out[t*Hd2+i] = cos(angle) * scaling, sin_out likewise.
 * The angle is the f32 product; cos/sin of it are taken in double and rounded
 * once to f32 (the correctly rounded value the GPU's library routine is
 * within an ulp or two of). */
void oracle_rope_build_cos_sin(const int32_t *positions, const float *inv_freq, float *cos_out,
                               float *sin_out, uint32_t T, uint32_t Hd2, float scaling) {
    for (uint32_t t = 0; t < T; ++t) {
        for (uint32_t i = 0; i < Hd2; ++i) {
            float angle = (float)positions[t] * inv_freq[i];
            float c = (float)cos((double)angle);
            float s = (float)sin((double)angle);
            cos_out[(size_t)t * Hd2 + i] = c * scaling;
            sin_out[(size_t)t * Hd2 + i] = s * scaling;
        }
    }
}

/* Sources/Popcorn/Kernels/RopeApply.metal:15-48: for each (b, t, h) head of
 * x [B, T, Nh, 2*Hd2] and each i < Hd2, with x1 = x[..., i], x2 =
 * x[..., Hd2 + i], c = cos[t, i], s = sin[t, i]:
 *   out[..., i] = x1*c - x2*s,  out[..., Hd2 + i] = x1*s + x2*c.
 * Values are f32 (widened from the storage dtype); the caller rounds. */
void oracle_rope_apply(const float *x, const float *cos_tab, const float *sin_tab, float *out,
                       uint32_t B, uint32_t T, uint32_t Nh, uint32_t Hd2) {
    for (uint32_t b = 0; b < B; ++b)
        for (uint32_t t = 0; t < T; ++t)
            for (uint32_t h = 0; h < Nh; ++h) {
                size_t base = (((size_t)b * T + t) * Nh + h) * 2 * Hd2;
                for (uint32_t i = 0; i < Hd2; ++i) {
                    float x1 = x[base + i], x2 = x[base + Hd2 + i];
                    float c = cos_tab[(size_t)t * Hd2 + i], s = sin_tab[(size_t)t * Hd2 + i];
                    float p1 = x1 * c, p2 = x2 * s, p3 = x1 * s, p4 = x2 * c;
                    out[base + i] = p1 - p2;
                    out[base + Hd2 + i] = p3 + p4;
                }
            }
}

/* Sources/Popcorn/Kernels/Transpose12.metal:13-24:
 *   out[((d0*D2 + d2)*D1 + d1)*D3 + d3] = src[((d0*D1 + d1)*D2 + d2)*D3 + d3]. */
void oracle_transpose12(const float *src, float *out, uint32_t D0, uint32_t D1, uint32_t D2,
                        uint32_t D3) {
    for (uint32_t a = 0; a < D0; ++a)
        for (uint32_t b = 0; b < D1; ++b)
            for (uint32_t c = 0; c < D2; ++c)
                for (uint32_t d = 0; d < D3; ++d)
                    out[(((size_t)a * D2 + c) * D1 + b) * D3 + d] =
                        src[(((size_t)a * D1 + b) * D2 + c) * D3 + d];
}

/* ------------------------------------------------------------------------ */
/* Block-affine quantized weights                                           */
/* ------------------------------------------------------------------------ */

/* Sources/Popcorn/Quantization/AffineQuantizationFormat.swift:25-29 and
 * PopcornDTypes.h:55-63: value i of a packed stream sits in bits
 * (i % vpw) * bits .. + bits of word i / vpw, vpw = 32 / bits. */
uint32_t oracle_aq_unpack(const uint32_t *words, size_t i, int bits) {
    const size_t vpw = (size_t)(32 / bits);
    const uint32_t mask = bits == 32 ? 0xffffffffu : ((1u << bits) - 1u);
    return (words[i / vpw] >> ((i % vpw) * (size_t)bits)) & mask;
}

/* Sources/Popcorn/Kernels/Quantized/AffineQuantizedMatmul.metal:34-58
 * (aq_matvec_simd4): y[m, n] = sum_k x[m, k] * (float(q[n, k]) * s[n, g] +
 * b[n, g]), g = k / group, summed in k order; biases NULL = no bias
 * (hasBias 0). Rows of packed values hold K * bits / 32 words. */
void oracle_aq_matmul(const float *x, const uint32_t *packed, const float *scales, const float *biases,
                      float *y, size_t M, size_t N, size_t K, int bits, int group) {
    const size_t words = K * (size_t)bits / 32, groups = K / (size_t)group;
    for (size_t m = 0; m < M; ++m)
        for (size_t n = 0; n < N; ++n) {
            float acc = 0.0f;
            for (size_t k = 0; k < K; ++k) {
                const size_t g = k / (size_t)group;
                const float s = scales[n * groups + g];
                const float b = biases ? biases[n * groups + g] : 0.0f;
                const float q = (float)oracle_aq_unpack(packed + n * words, k, bits);
                const float w = q * s + b;
                acc += x[m * K + k] * w;
            }
            y[m * N + n] = acc;
        }
}

/* Sources/Popcorn/Kernels/Quantized/AffineQuantizedEmbeddingGather.metal:16-26:
 * out[t, h] = float(q[ids[t], h]) * s + b. */
void oracle_aq_embedding_gather(const int32_t *ids, const uint32_t *packed, const float *scales,
                                const float *biases, float *out, size_t T, size_t H, int bits,
                                int group) {
    const size_t words = H * (size_t)bits / 32, groups = H / (size_t)group;
    for (size_t t = 0; t < T; ++t) {
        const size_t row = (size_t)(uint32_t)ids[t];
        for (size_t h = 0; h < H; ++h) {
            const size_t g = h / (size_t)group;
            const float s = scales[row * groups + g];
            const float b = biases ? biases[row * groups + g] : 0.0f;
            out[t * H + h] = (float)oracle_aq_unpack(packed + row * words, h, bits) * s + b;
        }
    }
}

/* ------------------------------------------------------------------------ */
/* Decode-loop glue                                                          */
/* ------------------------------------------------------------------------ */

/* Sources/Popcorn/Kernels/Argmax.metal:7-27: first maximum wins (a later
 * equal value never replaces an earlier index). */
void oracle_argmax(const float *x, size_t rows, size_t N, int32_t *indices) {
    for (size_t r = 0; r < rows; ++r) {
        const float *xr = x + r * N;
        float best = xr[0];
        int32_t bi = 0;
        for (size_t i = 1; i < N; ++i) {
            float v = xr[i];
            if (v > best || (v == best && (int32_t)i < bi)) {
                best = v;
                bi = (int32_t)i;
            }
        }
        indices[r] = bi;
    }
}

/* Sources/Popcorn/Kernels/EmbeddingGather.metal:6-23 */
void oracle_embedding_gather(const int32_t *ids, const float *table, float *out,
                             size_t N, size_t H) {
    for (size_t n = 0; n < N; ++n) {
        size_t row = (size_t)(uint32_t)ids[n];
        for (size_t h = 0; h < H; ++h) out[n * H + h] = table[row * H + h];
    }
}

/* One decoder layer at Sq = 1, following the op order of
 * Examples/GemmaCLI/Sources/GemmaCLI/Gemma4TextInference.swift:334-436 with
 * the per-layer inputs left out: RMSNorm -> QKV matvec (one [Nq+2Nkv]*Hd x H
 * weight, row-identical to the three separate projections at :335-343) ->
 * when given, per-head RMSNorm of q (:353), k (:367) and v without weight
 * (:368) and RoPE of q (:354) and k (:369) at position pos (tables as
 * RopeBuildCosSin.metal:17-20; the head transposes :355, :370-371 move no
 * value at one token) -> KV-cache write at `pos` (:372-381) -> attention
 * over pos+1 keys (:394-398) -> O projection -> post-attention RMSNorm ->
 * residual Add (:400-404) -> gated MLP (:416-429) -> post-FFN RMSNorm ->
 * residual Add (:430-434). Every stored tensor is rounded to L->act_dtype;
 * the caches hold act_dtype values in f32 storage here. x is updated in
 * place. */
void oracle_decoder_layer(const oracle_layer_t *L, float *x, float *k_cache,
                          float *v_cache, uint32_t pos) {
    const uint32_t H = L->H, Hd = L->Hd, Nq = L->Nq, Nkv = L->Nkv, F = L->F;
    const uint32_t QW = Nq * Hd, KW = Nkv * Hd, QKV = QW + 2 * KW;
    const int dt = L->act_dtype;
    float *n = (float *)malloc(H * sizeof(float));
    float *qkv = (float *)malloc(QKV * sizeof(float));
    float *attn = (float *)malloc(QW * sizeof(float));
    float *o = (float *)malloc(H * sizeof(float));
    float *tmp = (float *)malloc(H * sizeof(float));

    oracle_rmsnorm(x, L->w_in_norm, n, 1, H, L->eps, 0);
    round_array(dt, n, H);
    oracle_matmul(n, L->w_qkv, qkv, 1, H, QKV, 1);
    round_array(dt, qkv, QKV);
    if (L->w_q_norm) {
        oracle_rmsnorm(qkv, L->w_q_norm, qkv, Nq, Hd, L->eps, 0);
        round_array(dt, qkv, QW);
    }
    if (L->w_k_norm) {
        oracle_rmsnorm(qkv + QW, L->w_k_norm, qkv + QW, Nkv, Hd, L->eps, 0);
        round_array(dt, qkv + QW, KW);
    }
    if (L->v_norm) {
        oracle_rmsnorm(qkv + QW + KW, NULL, qkv + QW + KW, Nkv, Hd, L->eps, 0);
        round_array(dt, qkv + QW + KW, KW);
    }
    if (L->inv_freq) {
        float *cs = (float *)malloc(Hd * sizeof(float));
        const int32_t p32 = (int32_t)pos;
        oracle_rope_build_cos_sin(&p32, L->inv_freq, cs, cs + Hd / 2, 1, Hd / 2, L->rope_scaling);
        oracle_rope_apply(qkv, cs, cs + Hd / 2, qkv, 1, 1, Nq, Hd / 2);
        round_array(dt, qkv, QW);
        oracle_rope_apply(qkv + QW, cs, cs + Hd / 2, qkv + QW, 1, 1, Nkv, Hd / 2);
        round_array(dt, qkv + QW, KW);
        free(cs);
    }
    for (uint32_t h = 0; h < Nkv; ++h) {
        for (uint32_t d = 0; d < Hd; ++d) {
            size_t dst = ((size_t)h * L->kv_capacity + pos) * Hd + d;
            k_cache[dst] = qkv[QW + h * Hd + d];
            v_cache[dst] = qkv[QW + KW + h * Hd + d];
        }
    }
    oracle_attention_naive(qkv, k_cache, v_cache, attn, 1, Nq, Nkv, 1, pos + 1,
                           L->kv_capacity, Hd, L->scale, 0, -1);
    round_array(dt, attn, QW);
    oracle_matmul(attn, L->w_o, o, 1, QW, H, 1);
    round_array(dt, o, H);
    oracle_rmsnorm(o, L->w_post_attn_norm, tmp, 1, H, L->eps, 0);
    round_array(dt, tmp, H);
    for (uint32_t i = 0; i < H; ++i) x[i] = round_to(dt, x[i] + tmp[i]);

    oracle_gated_mlp(x, L->w_pre_ffn_norm, L->eps, 0, L->w_gate, L->w_up, L->w_down, H, F,
                     dt, NULL, o);
    round_array(dt, o, H);
    oracle_rmsnorm(o, L->w_post_ffn_norm, tmp, 1, H, L->eps, 0);
    round_array(dt, tmp, H);
    for (uint32_t i = 0; i < H; ++i) x[i] = round_to(dt, x[i] + tmp[i]);

    free(n);
    free(qkv);
    free(attn);
    free(o);
    free(tmp);
}
