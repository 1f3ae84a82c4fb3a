// Launch geometry of the persistent decode-layers kernel (decode_layers.hip),
// shared by the kernel and the host code that launches it.
#pragma once

#include <stdint.h>

namespace pk {
namespace layers {

#ifndef POPCORN_LAYER_WORK_WAVES
#define POPCORN_LAYER_WORK_WAVES 11
#endif
// Streaming waves per block, plus one wave that only synchronises.
constexpr int kWork = POPCORN_LAYER_WORK_WAVES;
constexpr int kWaves = kWork + 1;
constexpr int kThreads = kWaves * 64;

// Sync words (uint32): 16 arrival counters, one per 256-byte line; then the
// done counter and the abort word, each on a line of its own.
constexpr int kCounters = 16;
constexpr uint32_t kLine = 64;
constexpr uint32_t kDoneWord = kLine * kCounters;
constexpr uint32_t kAbortWord = kLine * (kCounters + 1);
constexpr uint32_t kSyncBytes = kLine * (kCounters + 2) * 4;

// Per worker wave: ring 0 (QKV and gate/up streams) and ring 1 (O and down).
constexpr uint32_t kRing0 = 8192, kRing1 = 4096;
// Split-KV partitions per KV head: at most one per lane of the combine.
constexpr uint32_t kMaxPartitions = 64;
// Arrival/release stamps kept per block when timing is on (two per wait).
constexpr uint32_t kStampsPerBlock = 2048;

constexpr uint32_t align16(uint32_t b) { return (b + 15u) & ~15u; }

// Dynamic LDS of a launch (bytes): the residual stream (f32 [H]), the
// staged vector (bf16 [max(H, Nq Hd, F)]) and the rings of every worker wave.
constexpr uint32_t ldsBytes(uint32_t H, uint32_t maxK) {
    return align16(H * 4u) + align16(maxK * 2u) + (uint32_t)kWork * (kRing0 + kRing1);
}

// Head dims and GQA group sizes with a compiled kernel
// (decode_layers_bf16_h<Hd>_g<G>).
constexpr bool compiled(int hd, int g) {
    return (hd == 256 && (g == 1 || g == 2)) || (hd == 128 && g == 2) || (hd == 64 && (g == 2 || g == 4));
}

}  // namespace layers
}  // namespace pk
