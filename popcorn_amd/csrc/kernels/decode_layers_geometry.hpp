// Launch geometry and memory layout of the persistent decode-layers kernel
// (decode_layers.hip), shared by the kernel and the host code that launches
// it.
#pragma once

#include <stdint.h>

namespace pk {
namespace layers {

#ifndef POPCORN_LAYER_WORK_WAVES
#define POPCORN_LAYER_WORK_WAVES 9
#endif
// Streaming waves per block, plus one staging wave (the last).
constexpr int kWork = POPCORN_LAYER_WORK_WAVES;
constexpr int kWaves = kWork + 1;
constexpr int kThreads = kWaves * 64;

// Sync words (uint32), each on a 256-byte line of its own: 8 arrival
// counters (block b arrives on counter b % 8, the blocks of one XCD), the
// done counter, the abort word and the launch epoch.
constexpr uint32_t kLine = 64;
constexpr int kCounters = 8;
constexpr uint32_t kDoneWord = kLine * kCounters;
constexpr uint32_t kAbortWord = kLine * (kCounters + 1);
constexpr uint32_t kEpochWord = kLine * (kCounters + 2);
constexpr uint32_t kSyncBytes = kLine * (kCounters + 3) * 4;

// Per worker wave: a 12 KB LDS region; ring 0 is its first 8 KB, ring 1 the
// last 4 KB. The QKV and down streams use the whole region, gate/up ring 0,
// the O projection ring 1.
constexpr uint32_t kRing0 = 8192, kRing1 = 4096, kRegion = kRing0 + kRing1;
// Longest vector the staging wave holds (H and Nq Hd): 9 16-byte groups of
// four per lane.
constexpr int kStagedGroups = 9;
constexpr int64_t kMaxStaged = 4 * 64 * kStagedGroups;
// Split-KV partitions per KV head: at most one per lane of the combine.
constexpr uint32_t kMaxPartitions = 64;
// Block-wide barriers per layer (phases A, B, D, E, F1, F2) and the stamps
// kept per block when timing is on (one per barrier release).
constexpr uint32_t kBarriersPerLayer = 6;
constexpr uint32_t kStampsPerBlock = 2048;

constexpr uint32_t align16(uint32_t b) { return (b + 15u) & ~15u; }
constexpr uint32_t align256(uint64_t b) { return (uint32_t)((b + 255u) & ~(uint64_t)255u); }
constexpr uint32_t umax(uint32_t a, uint32_t b) { return a > b ? a : b; }

// Dynamic LDS (byte offsets): the residual stream xres (bf16 [H]: every value
// of it is bf16-rounded); two staged vectors of the small phases (bf16
// [max(H, Nq Hd)]); the big staged vector (bf16 [F]; during the attention
// phase the workers' softmax states, f32 [kWork][G][Hd]); the query heads of
// the block's KV head and the new key and value rows (bf16 [(G + 2) Hd]);
// the two norm weight vectors of the next glue (f32 [2][H]); the workers'
// ring regions.
struct Lds {
    uint32_t xres, small0, small1, big, qbuf, normw, rings, bytes;
};
constexpr Lds ldsLayout(uint32_t H, uint32_t QW, uint32_t F, uint32_t G, uint32_t Hd) {
    Lds l{};
    const uint32_t small = align16(umax(H, QW) * 2u);
    l.xres = 0;
    l.small0 = align16(H * 2u);
    l.small1 = l.small0 + small;
    l.big = l.small1 + small;
    l.qbuf = l.big + align16(umax(F * 2u, (uint32_t)kWork * G * Hd * 4u));
    l.normw = l.qbuf + align16((G + 2u) * Hd * 2u);
    l.rings = l.normw + 2u * H * 4u;
    l.bytes = l.rings + (uint32_t)kWork * kRegion;
    return l;
}

// Device workspace of the activations exchanged inside a launch, every
// element tagged: bf16 vectors as 32-bit words (tag << 16 | bits) and the
// attention partials as 64-bit words (tag << 32 | f32 bits). Byte offsets.
struct Tagged {
    uint64_t qkv, attn, o, hidden, mlp, pO, pML, bytes;
};
constexpr Tagged taggedLayout(uint32_t H, uint32_t Nq, uint32_t Nkv, uint32_t Hd, uint32_t F, uint32_t P) {
    Tagged t{};
    const uint64_t QW = (uint64_t)Nq * Hd, QKV = QW + 2ull * Nkv * Hd;
    t.qkv = 0;
    t.attn = t.qkv + align256(QKV * 4);
    t.o = t.attn + align256(QW * 4);
    t.hidden = t.o + align256((uint64_t)H * 4);
    t.mlp = t.hidden + align256((uint64_t)F * 4);
    t.pO = t.mlp + align256((uint64_t)H * 4);
    t.pML = t.pO + align256((uint64_t)Nq * P * Hd * 8);
    t.bytes = t.pML + align256((uint64_t)Nq * P * 2 * 8);
    return t;
}

// Head dims and GQA group sizes with a compiled kernel
// (decode_layers_bf16_h<Hd>_g<G>).
constexpr bool compiled(int hd, int g) {
    return (hd == 256 && (g == 1 || g == 2)) || (hd == 128 && g == 2) || (hd == 64 && (g == 2 || g == 4));
}

}  // namespace layers
}  // namespace pk
