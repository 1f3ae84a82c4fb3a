// Kernels.* operation descriptors: validation and routing of the reference's
// Swift descriptors (Sources/Popcorn/Kernels/*.swift, cited per descriptor),
// with dispatch geometry chosen for wave64 and the device's CU count.
#include <algorithm>
#include <atomic>
#include <chrono>
#include <cstdlib>
#include <cstring>
#include <map>
#include <mutex>

#include "popcorn.hpp"
#include "uncached.hpp"

namespace popcorn {
namespace {

constexpr int kBlock = 256;

int deviceCUs() {
    static thread_local int cached_dev = -1, cached_cus = 256;
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) {
        (void)hipGetLastError();
        return cached_cus;
    }
    if (dev != cached_dev) {
        int cus = 0;
        if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess && cus > 0) cached_cus = cus;
        (void)hipGetLastError();
        cached_dev = dev;
    }
    return cached_cus;
}

int64_t cdiv(int64_t a, int64_t b) { return (a + b - 1) / b; }

bool isFloat(DataType t) { return t == DataType::f32 || t == DataType::f16 || t == DataType::bf16; }

void requireElements(const Tensor &t, int64_t n, const char *what) {
    if (n < 0) throw Error::invalidArgument(std::string(what) + ": negative size");
    if (n > 0 && !t.data) throw Error::invalidArgument(std::string(what) + ": null data pointer");
    if (t.shape.elementCount() < n)
        throw Error::tensorShapeMismatch(std::string(what) + " holds " + std::to_string(t.shape.elementCount()) +
                                         " elements; the operation reads or writes " + std::to_string(n) + ".");
}

bool aligned16(const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

// A single dispatch whose function, bindings, constants and geometry are all
// fixed at init (the common case of the reference's DispatchKernel structs).
class FixedDispatch : public DispatchKernel {
public:
    FixedDispatch(std::string fn, std::vector<Binding> b, std::vector<std::vector<uint8_t>> c, DispatchSize ds)
        : fn_(std::move(fn)), b_(std::move(b)), c_(std::move(c)), ds_(ds) {}
    std::string functionName() const override { return fn_; }
    std::vector<Binding> tensors() const override { return b_; }
    std::vector<std::vector<uint8_t>> constants() const override { return c_; }
    DispatchSize dispatchSize(const FunctionAttributes &) const override { return ds_; }

private:
    std::string fn_;
    std::vector<Binding> b_;
    std::vector<std::vector<uint8_t>> c_;
    DispatchSize ds_;
};

DispatchSize grid1(int64_t blocks, int threads, size_t lds = 0) {
    DispatchSize d;
    d.grid = dim3((unsigned)std::max<int64_t>(blocks, 0), 1, 1);
    d.block = dim3((unsigned)threads, 1, 1);
    d.dynamicLds = lds;
    return d;
}

const char *tag(DataType t) { return name(t); }

// ---------------------------------------------------------------------------
// FlashAttention / FlashDecoding (FlashAttention.swift, FlashDecoding.swift)
// ---------------------------------------------------------------------------

// FlashDecoding partition sizing: blocks per CU to aim for (default 2) and
// the fewest keys a partition takes (default 64); POPCORN_FD_BLOCKS_PER_CU
// and POPCORN_FD_MIN_KEYS override them for tuning.
int envInt(const char *name, int lo, int hi, int dflt) {
    const char *e = std::getenv(name);
    const int v = e ? std::atoi(e) : 0;
    return v >= lo && v <= hi ? v : dflt;
}
int fdBlocksPerCU() {
    static const int v = envInt("POPCORN_FD_BLOCKS_PER_CU", 1, 64, 2);
    return v;
}
int fdMinKeys() {
    static const int v = envInt("POPCORN_FD_MIN_KEYS", 1, 4096, 64);
    return v;
}
// Waves per block of the 16-bit split-KV kernels: 0 (chosen per shape, the
// default), or forced to 4 or 8 for tuning.
int fdWaves16() {
    static const int v = envInt("POPCORN_FD_WAVES", 4, 8, 0);
    return v == 4 || v == 8 ? v : 0;
}

struct AttnDims {
    int64_t B, Nq, Nkv, Sq, Sk, Hd, cap;
};

// The split-KV launch plan: the fast kernel's lanes per key row (0 = the
// generic kernel), chunks per lane, query heads per block, head groups per
// KV head and partitions per query row.
struct FdPlan {
    int lpk = 0, cpl = 1, gmax = 1, waves = 4;
    int64_t ngroups = 1, P = 1;
    std::string suffix() const {  // "<t>_l<LPK>_c<CPL>_g<G>[_w8]" without the dtype
        return "_l" + std::to_string(lpk) + "_c" + std::to_string(cpl) + "_g" + std::to_string(gmax) +
               (waves == 8 ? "_w8" : "");
    }
    int64_t block() const { return 64 * waves; }
};

FdPlan fdPlan(DataType t, const AttnDims &d, bool alignedOk, int64_t keys) {
    FdPlan f;
    const int64_t G = d.Nq / d.Nkv;
    const int kV = 16 / stride(t);
    if (alignedOk && d.Hd % kV == 0) {
        const int64_t chunks = d.Hd / kV;
        if (chunks == 8 || chunks == 16 || chunks == 32 || chunks == 64) f.lpk = (int)chunks;
        if (chunks == 128 && t == DataType::f32) {
            f.lpk = 64;
            f.cpl = 2;
        }
        if (t == DataType::f32 && chunks == 8) f.lpk = 0;  // f32 Hd 32: generic
    }
    if (f.lpk) {
        f.gmax = G <= 1 ? 1 : G <= 2 ? 2 : G <= 4 ? 4 : 8;
        if (d.Hd == 512 && f.gmax > 4) f.gmax = 4;  // 4 waves x G x Hd f32 of LDS stays <= 32 KB
    }
    f.ngroups = cdiv(G, f.gmax);
    // Partitions: enough blocks to cover every CU fdBlocksPerCU() times,
    // but at least fdMinKeys() keys per block (the reference fixes P = 8,
    // FlashDecoding.swift:77).
    const int64_t base = d.B * d.Nkv * f.ngroups * d.Sq;
    const int64_t want = cdiv(fdBlocksPerCU() * deviceCUs(), base);
    const int64_t maxByKeys = cdiv(std::max<int64_t>(keys, 1), fdMinKeys());
    f.P = std::clamp<int64_t>(std::min(want, maxByKeys), 1, 1024);
    // 16-bit kernels: 8 waves per block over half the partitions (the same
    // waves, each block twice the keys) when the keys set P and the 4-wave
    // grid would put more than one block on some CU. Measured at config 4
    // (68 -> 34 partitions): 6.85-7.07 us against 7.57-7.75 in the decode
    // step; where the 4-wave grid fits the CUs (B 1, 2048 keys) or P is set
    // by the CU count, 8 waves measured no faster or slower.
    if (f.lpk && t != DataType::f32) {
        const int forced = fdWaves16();
        const bool pick = forced ? forced == 8 : maxByKeys < want && base * f.P > deviceCUs();
        if (pick) {
            f.waves = 8;
            f.P = cdiv(f.P, 2);
        }
    }
    return f;
}

class FlashAttentionKernel : public Kernel {
public:
    FlashAttentionKernel(const Tensor &q, const Tensor &k, const Tensor &v, const Tensor &out, AttnDims d, float scale,
                         AttentionMask mask, const Tensor *position)
        : q_(q), k_(k), v_(v), out_(out), d_(d), scale_(scale), mask_(mask), hasPos_(position != nullptr) {
        if (position) pos_ = *position;
        // FlashAttention.swift:27-36
        if (d.Nkv <= 0 || d.Nq % d.Nkv != 0)
            throw Error::tensorShapeMismatch("FlashAttention query heads must be divisible by KV heads; got " +
                                             std::to_string(d.Nq) + " and " + std::to_string(d.Nkv) + ".");
        if (d.Hd > 512)
            throw Error::tensorShapeMismatch("FlashAttention head dim must be <= 512 (kernel limit); got " +
                                             std::to_string(d.Hd) + ".");
        if (d.B <= 0 || d.Nq <= 0 || d.Sq <= 0 || d.Hd <= 0 || d.Sk < 0)
            throw Error::tensorShapeMismatch("FlashAttention dimensions must be positive.");
        if (d.cap < d.Sk) throw Error::tensorShapeMismatch("FlashAttention key capacity is smaller than the key length.");
        if (mask.kind > 2) throw Error::invalidArgument("unknown attention mask kind");
        // FlashDecoding.swift:119-125 and :199-205, FlashAttention.swift:181-190,
        // extended with f16; Q, K and V share one dtype.
        if (!(q.dataType == k.dataType && k.dataType == v.dataType && isFloat(q.dataType) && isFloat(out.dataType)))
            throw Error::unsupportedDataTypeCombination(std::string("Unsupported FlashAttention data type combination: ") +
                                                        tag(q.dataType) + ", " + tag(k.dataType) + ", " + tag(out.dataType) + ".");
        requireElements(q, d.B * d.Nq * d.Sq * d.Hd, "FlashAttention q");
        requireElements(k, d.B * d.Nkv * d.cap * d.Hd, "FlashAttention k");
        requireElements(v, d.B * d.Nkv * d.cap * d.Hd, "FlashAttention v");
        requireElements(out, d.B * d.Nq * d.Sq * d.Hd, "FlashAttention out");
        if (hasPos_) {
            if (pos_.dataType != DataType::i32) throw Error::unsupportedDataTypeCombination("position tensor must be i32");
            requireElements(pos_, 1, "position");
        }
        path_ = Kernels::route(d.Sq, d.Hd, q.dataType);
        // the tiled kernel reads Q/K/V and writes O as 8- and 16-byte runs,
        // takes a fixed key length (no device-side position), addresses a
        // head's keys with 32-bit buffer offsets and tracks row maxima on
        // unscaled scores (scale > 0)
        if (path_ == Kernels::AttentionPath::tiled &&
            (hasPos_ || !aligned16(q.data) || !aligned16(k.data) || !aligned16(v.data) || !aligned16(out.data) ||
             !(out.dataType == q.dataType || out.dataType == DataType::f32) || !(scale > 0.0f) ||
             d.Sk * d.Hd * (int64_t)stride(q.dataType) >= (int64_t{1} << 31)))
            path_ = Kernels::AttentionPath::plain;
        if (path_ == Kernels::AttentionPath::tiled) {
            // Hd 128 and 256 run 16 query rows per wave (two waves per SIMD);
            // POPCORN_FA_ROWS=32 selects the 32-row kernel there (a tuning
            // override)
            const char *e = std::getenv("POPCORN_FA_ROWS");
            hdp_ = d.Hd <= 64 ? 64 : d.Hd <= 128 ? 128 : d.Hd <= 256 ? 256 : 512;
            // f32 has only the 16-row kernel (v_mfma_f32_16x16x4_f32)
            rows16_ = q.dataType == DataType::f32 || hdp_ == 512 ||
                      ((hdp_ == 128 || hdp_ == 256) && !(e && std::string(e) == "32"));
            // POPCORN_FA_PAIR_MERGE=0: paired tiles merged by the merge
            // kernel instead of the pair's second block (a tuning override)
            const char *pm = std::getenv("POPCORN_FA_PAIR_MERGE");
            pairMergeInKernel_ = !(pm && std::string(pm) == "0");
            tiledName_ = std::string(rows16_ ? "flash_attention_tiled16_" : "flash_attention_tiled_") + tag(q.dataType) +
                         "_" + tag(out.dataType) + "_d" + std::to_string(hdp_);
            planTileSplit();
        }
        planSplit();
    }

    std::vector<Binding> tensors() const override {
        std::vector<Binding> b = {{q_, kRead}, {k_, kRead}, {v_, kRead}, {out_, kWrite}};
        if (hasPos_) b.push_back({pos_, kRead});
        return b;
    }

    std::string describe() const override {
        if (path_ == Kernels::AttentionPath::tiled) return nSplit_ && !mergedPairs() ? tiledName_ + "," + mergeName_ : tiledName_;
        return partialName_ + "," + reduceName_;
    }

    void encode(KernelCommandEncoder &enc) const override {
        if (path_ == Kernels::AttentionPath::tiled) {
            // TiledFlashAttentionConstants (the fields of
            // PopcornKernelTypes.h:133-144 and two more): one block per 128
            // query rows of each (batch, query head)
            TiledFlashAttentionConstants c{};
            c.B = (uint32_t)d_.B;
            c.Nq = (uint32_t)d_.Nq;
            c.Nkv = (uint32_t)d_.Nkv;
            c.Sq = (uint32_t)d_.Sq;
            c.Sk = (uint32_t)d_.Sk;
            c.Hd = (uint32_t)d_.Hd;
            c.qTilesPerHead = (uint32_t)cdiv(d_.Sq, tileRows());
            c.maskKind = mask_.kind;
            c.slidingWindow = mask_.kind == 1 ? mask_.window : -1;
            c.scale = scale_;
            c.kvStride = (uint32_t)d_.cap;
            c.splitFrom = (uint32_t)(c.qTilesPerHead - nSplit_);
            c.pairTiles = pairTiles_ ? (mergedPairs() ? 2u : 1u) : 0u;
            // one block per tile; a split tile's two halves take two, a pair
            // of tiles two in all
            const int64_t items = d_.B * d_.Nq * ((int64_t)c.qTilesPerHead + (pairTiles_ ? 0 : nSplit_));
            if (!nSplit_) {
                // no split tile: the partial-state arguments are never touched
                FixedDispatch fa(tiledName_,
                                 {{q_, kRead}, {k_, kRead}, {v_, kRead}, {out_, kWrite}, {q_, kRead}, {q_, kRead},
                                  {q_, kRead}},
                                 {bytesOf(c)}, grid1(items, tiledBlock()));
                enc.dispatch(fa);
                return;
            }
            if (mergedPairs()) {
                // the published part of each split tile (unnormalised O, then
                // (m, l) per row) and its ready flag, in the stream's
                // uncached pair exchange; the second block of each pair
                // merges, so no merge kernel
                const int64_t tiles = d_.B * d_.Nq * nSplit_;
                const size_t oBytes = (size_t)(tiles * 128 * hdp_) * 4;
                const PairExchange &x = pairExchange(enc.stream(), oBytes + (size_t)(tiles * 128 * 2) * 4);
                const uint64_t ticket = nextTicket();
                c.ticketLo = (uint32_t)ticket;
                c.ticketHi = (uint32_t)(ticket >> 32);
                Tensor pO(x.data, Shape({tiles * 128, hdp_}), DataType::f32);
                Tensor pML(static_cast<uint8_t *>(x.data) + oBytes, Shape({tiles * 128 * 2}), DataType::f32);
                Tensor flags(x.flags, Shape({(int64_t)PairExchange::kFlags}), DataType::u64);
                FixedDispatch fa(tiledName_,
                                 {{q_, kRead}, {k_, kRead}, {v_, kRead}, {out_, kWrite}, {pO, kReadWrite},
                                  {pML, kReadWrite}, {flags, kReadWrite}},
                                 {bytesOf(c)}, grid1(items, tiledBlock()));
                enc.dispatch(fa);
                return;
            }
            // the two parts of each split tile: unnormalised O, then (m, l) per row
            const int64_t rows = d_.B * d_.Nq * nSplit_ * 2 * 128;
            enc.withTemporaryTensor(ScratchSpec{{rows, hdp_}, DataType::f32}, [&](Tensor pO) {
                enc.withTemporaryTensor(ScratchSpec{{rows, 2}, DataType::f32}, [&](Tensor pML) {
                    FixedDispatch fa(tiledName_,
                                     {{q_, kRead}, {k_, kRead}, {v_, kRead}, {out_, kWrite}, {pO, kWrite}, {pML, kWrite},
                                      {q_, kRead}},
                                     {bytesOf(c)}, grid1(items, tiledBlock()));
                    enc.dispatch(fa);
                    // one block per 16 rows of a split tile
                    FixedDispatch merge(mergeName_, {{pO, kRead}, {pML, kRead}, {out_, kWrite}}, {bytesOf(c)},
                                        grid1(d_.B * d_.Nq * nSplit_ * 8, kBlock));
                    enc.dispatch(merge);
                });
            });
            return;
        }
        // FlashDecoding.swift:54-73: borrow partial O, m, l; partial; combine.
        const int64_t slots = d_.B * d_.Nq * d_.Sq * P_;
        enc.withTemporaryTensor(ScratchSpec{{slots, d_.Hd}, DataType::f32}, [&](Tensor pO) {
            enc.withTemporaryTensor(ScratchSpec{{slots}, DataType::f32}, [&](Tensor pM) {
                enc.withTemporaryTensor(ScratchSpec{{slots}, DataType::f32}, [&](Tensor pL) {
                    encodeSplit(enc, pO, pM, pL);
                });
            });
        });
    }

    // The split-KV path's partial (O, m, l) in f32: slots x (Hd + 2) floats.
    size_t splitScratchBytes() const { return (size_t)(d_.B * d_.Nq * d_.Sq * P_) * (size_t)(d_.Hd + 2) * 4; }

    // The split-KV path on caller-given partial buffers (no scratch borrowed):
    // O [slots, Hd], then m and l [slots] each, inside `bytes` at `scratch`.
    void encodeSplitInto(KernelCommandEncoder &enc, void *scratch, size_t bytes) const {
        const int64_t slots = d_.B * d_.Nq * d_.Sq * P_;
        if (splitScratchBytes() > bytes)
            throw Error(POPCORN_ERR_WORKSPACE_EXHAUSTED,
                        "split-KV attention needs " + std::to_string(splitScratchBytes()) +
                            " bytes of partials; the static scratch holds " + std::to_string(bytes) + ".");
        float *base = static_cast<float *>(scratch);
        Tensor pO(base, Shape({slots, d_.Hd}), DataType::f32);
        Tensor pM(base + slots * d_.Hd, Shape({slots}), DataType::f32);
        Tensor pL(base + slots * (d_.Hd + 1), Shape({slots}), DataType::f32);
        encodeSplit(enc, pO, pM, pL);
    }

    bool tiled() const { return path_ == Kernels::AttentionPath::tiled; }

    // Forces the split-KV kernels (the plain/decoding routes) whatever route
    // the shape would take.
    void useSplitPath() { path_ = Kernels::AttentionPath::decoding; }

    void encodeSplit(KernelCommandEncoder &enc, const Tensor &pO, const Tensor &pM, const Tensor &pL) const {
        FlashDecodingPartialExtConstants pc{};
        pc.B = (uint32_t)d_.B;
        pc.Nq = (uint32_t)d_.Nq;
        pc.Nkv = (uint32_t)d_.Nkv;
        pc.Sk = (uint32_t)d_.Sk;
        pc.Hd = (uint32_t)d_.Hd;
        pc.P = (uint32_t)P_;
        pc.maskKind = mask_.kind;
        pc.slidingWindow = mask_.kind == 1 ? mask_.window : -1;
        pc.scale = scale_;
        pc.kvStride = (uint32_t)d_.cap;
        pc.Sq = (uint32_t)d_.Sq;
        pc.keyLenFromPosition = hasPos_ ? 1u : 0u;
        DispatchSize ds;
        ds.grid = dim3((unsigned)P_, (unsigned)(d_.B * d_.Nkv * ngroups_), (unsigned)d_.Sq);
        ds.block = dim3((unsigned)partialBlock_, 1, 1);
        // the position binding is read only when keyLenFromPosition
        Tensor posOrDummy = hasPos_ ? pos_ : q_;
        FixedDispatch partial(partialName_,
                              {{q_, kRead}, {k_, kRead}, {v_, kRead}, {pO, kWrite}, {pM, kWrite}, {pL, kWrite},
                               {posOrDummy, kRead}},
                              {bytesOf(pc)}, ds);
        enc.dispatch(partial);
        FlashDecodingReduceExtConstants rc{};
        rc.B = (uint32_t)d_.B;
        rc.Nq = (uint32_t)d_.Nq;
        rc.Hd = (uint32_t)d_.Hd;
        rc.P = (uint32_t)P_;
        rc.Sq = (uint32_t)d_.Sq;
        // one block per (query row, 64-dim slice of the head)
        DispatchSize rs;
        rs.grid = dim3((unsigned)(d_.B * d_.Nq * d_.Sq), (unsigned)cdiv(d_.Hd, 64), 1);
        rs.block = dim3(kBlock, 1, 1);
        FixedDispatch reduce(reduceName_, {{pO, kRead}, {pM, kRead}, {pL, kRead}, {out_, kWrite}}, {bytesOf(rc)}, rs);
        enc.dispatch(reduce);
    }

private:
    // Causal prefill with few tiles per CU: the last query tiles see up to
    // twice the mean number of keys and, one tile per CU, set the kernel's
    // time. Tiles with more than half the largest tile's key steps run as
    // two blocks over the halves of their keys, merged by a second kernel.
    // Causal prefill with at most two tiles per CU splits tiles in two
    // (flash_attention_tiled.hip, fa_work). With at most one tile per CU a
    // head's query tiles are paired light with heavy (tile i with nQT - 1 - i)
    // and each pair runs as two blocks of equal work, when every pair splits
    // its heavy tile (x >= 1 steps in the first block); otherwise the tiles
    // with more than half the heaviest tile's steps run as two halves.
    void planTileSplit() {
        nSplit_ = 0;
        pairTiles_ = false;
        const int64_t nQT = cdiv(d_.Sq, 128);
        const int64_t tiles = d_.B * d_.Nq * nQT;
        // the Hd 512 and f32 kernels run every tile whole
        if (hdp_ == 512 || q_.dataType == DataType::f32 || mask_.kind != 0 || nQT < 4 || tiles > 2 * (int64_t)deviceCUs()) return;
        auto steps = [&](int64_t qt) {
            const int64_t last = d_.Sk - d_.Sq + std::min(qt * 128 + 127, d_.Sq - 1);
            const int64_t hi = std::min(d_.Sk, last + 1);
            return hi > 0 ? cdiv(hi, 32) : int64_t(0);
        };
        mergeName_ = std::string("flash_attention_split_merge_") + tag(out_.dataType) + "_d" + std::to_string(hdp_);
        bool pairs = tiles <= (int64_t)deviceCUs();
        for (int64_t i = 0; pairs && i < nQT / 2; ++i) {
            const int64_t sa = steps(i), sb = steps(nQT - 1 - i);
            const int64_t x = (sa + sb + 1) / 2 - sa;
            pairs = x >= 1 && x < sb;
        }
        // one ready flag per split tile in the stream's pair exchange
        pairs = pairs && d_.B * d_.Nq * (nQT / 2) < (int64_t)PairExchange::kFlags;
        if (pairs) {
            pairTiles_ = true;
            nSplit_ = nQT / 2;
            return;
        }
        const int64_t most = steps(nQT - 1);
        int64_t from = nQT;
        while (from > 0 && steps(from - 1) * 2 > most) --from;
        if (most < 4 || from == nQT) return;
        nSplit_ = nQT - from;
    }

    void planSplit() {
        const DataType t = q_.dataType;
        const bool alignedOk = aligned16(q_.data) && aligned16(k_.data) && aligned16(v_.data);
        const FdPlan f = fdPlan(t, d_, alignedOk, hasPos_ ? d_.cap : d_.Sk);
        partialName_ = std::string("flash_decoding_partial_") + tag(t) + (f.lpk ? f.suffix() : std::string("_ext"));
        partialBlock_ = f.lpk ? f.block() : kBlock;
        reduceName_ = std::string("flash_decoding_reduce_") + tag(out_.dataType) + "_ext";
        ngroups_ = f.ngroups;
        P_ = f.P;
    }

    Tensor q_, k_, v_, out_, pos_;
    AttnDims d_;
    float scale_;
    AttentionMask mask_;
    bool hasPos_;
    Kernels::AttentionPath path_ = Kernels::AttentionPath::plain;
    std::string partialName_, reduceName_, tiledName_, mergeName_;
    int64_t partialBlock_ = kBlock;
    int64_t nSplit_ = 0;
    bool pairTiles_ = false;
    bool rows16_ = false;  // the 16-rows-per-wave kernel: 8 waves per 128-row tile (4 per 64 at Hd 512 and in f32)
    int64_t hdp_ = 0;      // the tiled kernel's head dim: Hd padded to 64, 128, 256 or 512
    bool tiles64() const { return hdp_ == 512 || q_.dataType == DataType::f32; }
    int64_t tiledBlock() const { return tiles64() ? 256 : rows16_ ? 512 : kBlock; }
    int64_t tileRows() const { return tiles64() ? 64 : 128; }
    // Paired tiles are merged inside the tiled kernels (pairTiles 2).
    bool pairMergeInKernel_ = true;
    bool mergedPairs() const { return pairTiles_ && pairMergeInKernel_; }
    // A 64-bit value, never 0 or ~0 and distinct per launch, for the ready flags
    // of merged pairs: a counter, started from the clock so that processes
    // differ, through the splitmix64 finaliser.
    static uint64_t nextTicket() {
        static std::atomic<uint64_t> counter{(uint64_t)std::chrono::steady_clock::now().time_since_epoch().count()};
        for (;;) {
            uint64_t z = (counter.fetch_add(1, std::memory_order_relaxed) + 1) * 0x9E3779B97F4A7C15ull;
            z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
            z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
            z ^= z >> 31;
            if (z != 0 && z != ~0ull) return z;
        }
    }
    int64_t ngroups_ = 1, P_ = 1;
};

// The attention block of one decode token (DecodeAttentionConstants): the
// fresh-key split-KV partial kernel, then the same LSE combine.
class DecodeAttentionKernel : public Kernel {
public:
    explicit DecodeAttentionKernel(const Kernels::DecodeAttentionArgs &a) {
        if (!a.qkv || !a.kCache || !a.vCache || !a.out || !a.position)
            throw Error::invalidArgument("DecodeAttention needs qkv, both caches, out and position");
        qkv_ = *a.qkv;
        k_ = *a.kCache;
        v_ = *a.vCache;
        out_ = *a.out;
        pos_ = *a.position;
        if (k_.shape.rank() != 4) throw Error::tensorInvalidRank(4, k_.shape.rank());
        if (v_.shape != k_.shape) throw Error::tensorShapeMismatch("DecodeAttention K and V caches must have one shape.");
        d_.B = k_.shape[0];
        d_.Nkv = k_.shape[1];
        d_.cap = k_.shape[2];
        d_.Hd = k_.shape[3];
        d_.Nq = a.queryHeads;
        d_.Sq = 1;
        d_.Sk = d_.cap;
        if (d_.Nkv != a.kvHeads) throw Error::tensorShapeMismatch("DecodeAttention kv_heads must match the caches' dim 1.");
        if (d_.Nkv <= 0 || d_.Nq <= 0 || d_.Nq % d_.Nkv != 0)
            throw Error::tensorShapeMismatch("DecodeAttention query heads must be a positive multiple of the KV heads.");
        if (d_.B <= 0 || d_.cap <= 0 || d_.Hd <= 0 || d_.Hd % 2 != 0)
            throw Error::tensorShapeMismatch("DecodeAttention needs B, capacity > 0 and an even head dim.");
        if (a.mask.kind > 2) throw Error::invalidArgument("unknown attention mask kind");
        const DataType t = k_.dataType;
        if (!isFloat(t) || qkv_.dataType != t || v_.dataType != t || !(out_.dataType == t || out_.dataType == DataType::f32))
            throw Error::unsupportedDataTypeCombination("DecodeAttention: qkv and the caches of one float dtype, out of it or f32.");
        if (pos_.dataType != DataType::i32) throw Error::unsupportedDataTypeCombination("position tensor must be i32");
        requireElements(pos_, 1, "position");
        const int64_t rowStride = (d_.Nq + 2 * d_.Nkv) * d_.Hd;
        requireElements(qkv_, d_.B * rowStride, "DecodeAttention qkv");
        requireElements(k_, d_.B * d_.Nkv * d_.cap * d_.Hd, "DecodeAttention k_cache");
        requireElements(out_, d_.B * d_.Nq * d_.Hd, "DecodeAttention out");
        auto f32vec = [&](const Tensor *w, int64_t n, const char *what) {
            if (!w) return;
            if (w->dataType != DataType::f32) throw Error::unsupportedDataTypeCombination(std::string(what) + " must be f32.");
            requireElements(*w, n, what);
        };
        f32vec(a.qNorm, d_.Hd, "DecodeAttention q_norm");
        f32vec(a.kNorm, d_.Hd, "DecodeAttention k_norm");
        f32vec(a.invFreq, d_.Hd / 2, "DecodeAttention inv_freq");
        dc_.flags = (a.qNorm ? 1u : 0u) | (a.kNorm ? 2u : 0u) | (a.vNorm ? 4u : 0u) | (a.invFreq ? 8u : 0u);
        dc_.eps = a.eps;
        dc_.ropeScaling = a.ropeScaling;
        dc_.rowStride = (uint32_t)rowStride;
        const Tensor &dummy = qkv_;  // bound in place of an absent optional input; never read
        wq_ = a.qNorm ? *a.qNorm : dummy;
        wk_ = a.kNorm ? *a.kNorm : dummy;
        invf_ = a.invFreq ? *a.invFreq : dummy;
        mask_ = a.mask;
        scale_ = a.scale;
        const bool alignedOk = aligned16(qkv_.data) && aligned16(k_.data) && aligned16(v_.data) && (rowStride * stride(t)) % 16 == 0;
        plan_ = fdPlan(t, d_, alignedOk, d_.cap);
        if (!plan_.lpk)
            throw Error::unsupportedDataTypeCombination(
                "DecodeAttention needs 16-byte aligned f16/bf16 data with head dim 64, 128, 256 or 512 (f32: 128, 256, 512).");
        partialName_ = std::string("flash_decoding_fresh_") + tag(t) + plan_.suffix();
        reduceName_ = std::string("flash_decoding_reduce_") + tag(out_.dataType) + "_ext";
    }

    std::vector<Binding> tensors() const override {
        return {{qkv_, kRead}, {k_, kReadWrite}, {v_, kReadWrite}, {out_, kWrite}, {pos_, kRead},
                {wq_, kRead}, {wk_, kRead}, {invf_, kRead}};
    }
    std::string describe() const override { return partialName_ + "," + reduceName_; }

    void encode(KernelCommandEncoder &enc) const override {
        const int64_t P = plan_.P;
        const int64_t slots = d_.B * d_.Nq * P;
        enc.withTemporaryTensor(ScratchSpec{{slots, d_.Hd}, DataType::f32}, [&](Tensor pO) {
            enc.withTemporaryTensor(ScratchSpec{{slots}, DataType::f32}, [&](Tensor pM) {
                enc.withTemporaryTensor(ScratchSpec{{slots}, DataType::f32}, [&](Tensor pL) {
                    FlashDecodingPartialExtConstants pc{};
                    pc.B = (uint32_t)d_.B;
                    pc.Nq = (uint32_t)d_.Nq;
                    pc.Nkv = (uint32_t)d_.Nkv;
                    pc.Sk = (uint32_t)d_.cap;
                    pc.Hd = (uint32_t)d_.Hd;
                    pc.P = (uint32_t)P;
                    pc.maskKind = mask_.kind;
                    pc.slidingWindow = mask_.kind == 1 ? mask_.window : -1;
                    pc.scale = scale_;
                    pc.kvStride = (uint32_t)d_.cap;
                    pc.Sq = 1;
                    pc.keyLenFromPosition = 1;
                    DispatchSize ds;
                    ds.grid = dim3((unsigned)P, (unsigned)(d_.B * d_.Nkv * plan_.ngroups), 1);
                    ds.block = dim3((unsigned)plan_.block(), 1, 1);
                    FixedDispatch partial(partialName_,
                                          {{qkv_, kRead}, {k_, kReadWrite}, {v_, kReadWrite}, {pO, kWrite}, {pM, kWrite},
                                           {pL, kWrite}, {pos_, kRead}, {wq_, kRead}, {wk_, kRead}, {invf_, kRead}},
                                          {bytesOf(pc), bytesOf(dc_)}, ds);
                    enc.dispatch(partial);
                    FlashDecodingReduceExtConstants rc{};
                    rc.B = (uint32_t)d_.B;
                    rc.Nq = (uint32_t)d_.Nq;
                    rc.Hd = (uint32_t)d_.Hd;
                    rc.P = (uint32_t)P;
                    rc.Sq = 1;
                    DispatchSize rs;
                    rs.grid = dim3((unsigned)(d_.B * d_.Nq), (unsigned)cdiv(d_.Hd, 64), 1);
                    rs.block = dim3(kBlock, 1, 1);
                    FixedDispatch reduce(reduceName_, {{pO, kRead}, {pM, kRead}, {pL, kRead}, {out_, kWrite}},
                                         {bytesOf(rc)}, rs);
                    enc.dispatch(reduce);
                });
            });
        });
    }

private:
    Tensor qkv_, k_, v_, out_, pos_, wq_, wk_, invf_;
    AttnDims d_{};
    DecodeAttentionConstants dc_{};
    AttentionMask mask_{0, -1};
    float scale_ = 1.0f;
    FdPlan plan_;
    std::string partialName_, reduceName_;
};

// ---------------------------------------------------------------------------
// Matmul (Matmul.swift)
// ---------------------------------------------------------------------------

// The streaming matvec for a transposeB product with m == 1 (the triples of
// Matmul.swift:362-374, plus f16 triples): matvec_nk_stream_<x>_<w>_<o>,
// suffixed _r<R> by the caller.
std::string matvecNKName(DataType x, DataType w, DataType o) {
    using D = DataType;
    const bool ok = (x == D::f32 && w == D::f32 && o == D::f32) || (x == D::f32 && w == D::bf16 && o == D::f32) ||
                    (x == D::bf16 && w == D::bf16 && o == D::f32) || (x == D::bf16 && w == D::bf16 && o == D::bf16) ||
                    (x == D::f32 && w == D::f16 && o == D::f32) || (x == D::f16 && w == D::f16 && o == D::f32) ||
                    (x == D::f16 && w == D::f16 && o == D::f16);
    if (!ok) return "";
    return std::string("matvec_nk_stream_") + tag(x) + "_" + tag(w) + "_" + tag(o);
}

std::string plainName(const char *base, DataType x, DataType w, DataType o) {
    using D = DataType;
    std::string b = base;
    // Matmul.swift:222-229 and :381-388, plus f16 triples
    if (x == D::f32 && w == D::f32 && o == D::f32) return b;
    if (x == D::f32 && w == D::f16 && o == D::f32) return b + "_f16";
    if (x == D::f32 && w == D::bf16 && o == D::f32) return b + "_bf16";
    if (x == D::bf16 && w == D::bf16 && o == D::f32) return b + "_bf16_bf16_f32";
    if (x == D::bf16 && w == D::bf16 && o == D::bf16) return b + "_bf16_bf16_bf16";
    if (x == D::f16 && w == D::f16 && o == D::f32) return b + "_f16_f16_f32";
    if (x == D::f16 && w == D::f16 && o == D::f16) return b + "_f16_f16_f16";
    return "";
}

// Rows per unit of the streaming matvecs (stream.hpp): 4 for long outputs
// (one LDS read of x feeds 4 rows), 1 otherwise (finer units balance better).
int matvecRows(int64_t N) { return N >= 32768 ? 4 : 1; }

// Waves per CU the streaming kernels are sized for: 12 (3 blocks of 4 waves,
// 3 waves per SIMD), measured best on MI355X for the decode matvecs with 4
// steps in flight per wave (stream.hpp); POPCORN_STREAM_WAVES_PER_CU
// overrides it (1..32) for tuning.
int streamWavesPerCU() {
    static const int w = [] {
        const char *e = std::getenv("POPCORN_STREAM_WAVES_PER_CU");
        const int v = e ? std::atoi(e) : 0;
        return v >= 1 && v <= 32 ? v : 12;
    }();
    return w;
}

// Blocks (of 4 waves) for `units` units: each wave's share is
// ceil(units / maxWaves), and just enough waves are launched to cover the
// units at that share, so every wave streams the same number of units give
// or take one.
int64_t streamBlocks(int64_t units) {
    if (units <= 0) return 0;
    const int64_t maxWaves = (int64_t)deviceCUs() * streamWavesPerCU();
    const int64_t per = cdiv(units, maxWaves);
    return cdiv(cdiv(units, per), kBlock / 64);
}

// The 4-bit fast kernels' launch shape: lanes per row LPR (8, 12, 16 or 32;
// a unit is floor(64 / LPR) rows and a row's K / 64 groups are dealt to its
// LPR lanes, one group per lane and step) and x octets per thread J (2 or
// 8). LPR minimises the steps of the busiest SIMD, waves per SIMD x units
// per wave x steps per unit, at the grid's waves per CU (the 4-bit inner
// loop is bound by its vector ALU work): short matrices want many small
// units, long ones full lanes (12 lanes fit rows of 36 groups, K 2304, in 3
// whole steps, where 16 lanes take 3 steps with a quarter of them idle).
// Ties go to the higher lane occupancy.
struct Q4Shape {
    int lpr = 0, j = 0;
};

Q4Shape q4Shape(int64_t N, int64_t K, bool xF32) {
    Q4Shape q;
    const int64_t G = K / 64;
    const int64_t kMax = xF32 ? 4096 : 16384;
    // the fast kernels read a row's scales and biases as 32-bit words, and
    // the packed words through 32-bit byte offsets
    if (N <= 0 || G <= 0 || G % 2 != 0 || K > kMax || N * (K / 2) >= (int64_t{1} << 31)) return q;
    q.j = K <= 4096 ? 2 : 8;
    const int64_t waves = (int64_t)deviceCUs() * streamWavesPerCU();
    int64_t bestSteps = INT64_MAX;
    double bestEff = 0.0;
    const int64_t simds = (int64_t)deviceCUs() * 4;
    for (int lpr : {32, 16, 12, 8}) {
        const int64_t cpl = cdiv(G, lpr), rows = 64 / lpr, units = cdiv(N, rows);
        const int64_t used = std::min(units, waves);
        const int64_t steps = cdiv(used, simds) * cdiv(units, used) * cpl;
        const double eff = (double)G / (double)(lpr * cpl) * (double)(rows * lpr) / 64.0;
        if (steps < bestSteps || (steps == bestSteps && eff > bestEff)) {
            bestSteps = steps;
            bestEff = eff;
            q.lpr = lpr;
        }
    }
    return q;
}

// MFMA GEMM tile shapes (gemm_mfma.hip): BM x BN and the block size.
struct GemmTile {
    int bm, bn, threads;
    const char *suffix;
};

// "d" tiles copy operands global -> LDS directly (4 stages of K 32); they
// need K % 32 == 0. Their "e" forms copy whole 128-byte lines (2 stages of
// K 64, buffer loads whose byte offsets stay below 2^31 over a tile's rows);
// they need K % 64 == 0 and take every such shape.
bool gemmLinesFit(int64_t k, int bn) { return k % 64 == 0 && (int64_t)(bn + 16) * k * 2 < (int64_t{1} << 31); }

// The whole-line tiles are chosen by a score: the share of the CU slots
// their grid keeps busy over its rounds (two blocks per CU for the tiles
// of at most 80 KB of LDS; such a tile alone on a CU counts 0.6 of a
// slot), times the share of the grid's tiles that lies inside C, times the
// tile's measured throughput per CU relative to 256 x 384 when the CUs are
// full (bf16, 33 Gemma-family prefill shapes, M 512-4096: the score's pick
// was within 3% of the fastest tile on 31 and within 5% on the others,
// 5% faster than the rules of the 64-byte-row tiles over all of them).
struct ScoredTile {
    GemmTile tile;
    int blocksPerCU;
    double weight;
};
const ScoredTile kLineTiles[] = {
    {{256, 384, 512, "e256x384"}, 1, 1.0},  {{256, 256, 512, "e256x256"}, 1, 0.97}, {{256, 288, 768, "e256x288"}, 1, 0.94},
    {{128, 192, 256, "e128x192"}, 2, 0.92}, {{128, 128, 256, "e128x128"}, 2, 0.87}, {{128, 256, 512, "e128x256"}, 1, 0.75}};

double lineTileScore(const ScoredTile &t, int64_t m, int64_t n) {
    const int64_t cus = deviceCUs();
    const int64_t tm = cdiv(m, t.tile.bm), tn = cdiv(n, t.tile.bn), tiles = tm * tn;
    const int64_t slots = cus * t.blocksPerCU;
    double fill = (double)tiles / (double)(cdiv(tiles, slots) * slots);
    if (t.blocksPerCU > 1 && tiles <= cus) fill = 0.6 * (double)tiles / (double)cus;
    const double inside = (double)(m * n) / (double)(tm * t.tile.bm * tn * t.tile.bn);
    return fill * inside * t.weight;
}

const ScoredTile &bestLineTile(int64_t m, int64_t n) {
    const ScoredTile *best = &kLineTiles[0];
    double bestScore = -1.0;
    for (const ScoredTile &t : kLineTiles) {
        const double sc = lineTileScore(t, m, n);
        if (sc > bestScore) {
            bestScore = sc;
            best = &t;
        }
    }
    return *best;
}

GemmTile gemmTileForm(int64_t m, int64_t n, int64_t k);
GemmTile gemmTile(int64_t m, int64_t n, int64_t k) {
    if (!std::getenv("POPCORN_GEMM_TILE") && gemmLinesFit(k, 384)) return bestLineTile(m, n).tile;
    return gemmTileForm(m, n, k);
}

GemmTile gemmTileForm(int64_t m, int64_t n, int64_t k) {
    static const GemmTile tiles[] = {{256, 256, 512, "t256x256"}, {256, 256, 256, "t256x256w4"},
                                     {256, 128, 512, "t256x128"}, {128, 256, 512, "t128x256"},
                                     {128, 128, 256, "t128x128"}, {256, 256, 512, "d256x256"},
                                     {128, 128, 256, "d128x128"}, {128, 256, 512, "d128x256"},
                                     {128, 192, 256, "d128x192"}, {256, 384, 512, "d256x384"},
                                     {256, 256, 512, "e256x256"}, {128, 128, 256, "e128x128"},
                                     {128, 256, 512, "e128x256"}, {128, 192, 256, "e128x192"},
                                     {256, 384, 512, "e256x384"}, {256, 288, 768, "e256x288"}};
    if (const char *e = std::getenv("POPCORN_GEMM_TILE")) {  // tuning override, e.g. "t256x128"
        for (const GemmTile &t : tiles)
            if (std::string(t.suffix) == e && (t.suffix[0] != 'd' || k % 32 == 0) && (t.suffix[0] != 'e' || gemmLinesFit(k, t.bn)))
                return t;
    }
    // 256 x 256 on 8 waves reuses each LDS stage for twice the MFMA work of
    // 128 x 128 but runs one block per CU, so it only pays when the tiles
    // fill the CUs several times over; below that the 128 x 128 grid (two
    // blocks per CU) balances better. The direct-to-LDS forms beat the
    // register-staged ones on every config-5 shape (f16, M 2048; us):
    //                      d256  d128  t256  t128
    //   QKV  N 9216  K 3072   177   162   203   186
    //   gate N 24576 K 3072   319   422   375   431
    //   down N 3072  K 24576  589   430   712   485
    const bool big = cdiv(m, 256) * cdiv(n, 256) >= 3 * deviceCUs();
    if (k % 32 == 0) {
        // 256 x 384 (8 waves of 128 x 96: 7 fragment reads per 12 MFMAs) when
        // its grid keeps at least 70% of the CUs busy in every round
        // (config-5 QKV, 192 tiles: 136 -> 127 us; gate and up, 512 tiles:
        // 294-303 -> 284-288 us)
        const int64_t cus = deviceCUs();
        const int64_t t384 = cdiv(m, 256) * cdiv(n, 384);
        if (t384 * 10 >= cus * 7 && t384 * 10 >= cdiv(t384, cus) * cus * 7) return tiles[9];
        if (big) return tiles[5];
        // 128 x 192 tiles when their grid is whole rounds of one tile per CU
        // (config-5 QKV, N 9216: 768 tiles, 155 -> 135 us; down, N 3072:
        // 256 tiles, 397 -> 352 us)
        const int64_t t192 = cdiv(m, 128) * cdiv(n, 192);
        if (n % 192 == 0 && t192 % deviceCUs() == 0) return tiles[8];
        // a 128 x 128 grid between one and two tiles per CU leaves half the
        // CUs with a second tile; one 128 x 256 tile per CU (8 waves) ends
        // sooner (config-5 down: 379 against 423 us before 128 x 192 took it)
        const int64_t t128 = cdiv(m, 128) * cdiv(n, 128);
        if (t128 > deviceCUs() && t128 < 2 * (int64_t)deviceCUs() && n >= 256) return tiles[7];
        return tiles[6];
    }
    return big ? tiles[0] : tiles[4];
}

// Split-K for a GEMM whose 256 x 384 tiles are too few to fill the CUs:
// the number of K splits that makes the grid whole rounds of one tile per
// CU, each split at least 2048 deep, or 0. Config-5 down (M 2048, N 3072,
// K 24576): 64 tiles x 4 splits of K 6144.
int64_t gemmSplitK(int64_t m, int64_t n, int64_t k) {
    if (std::getenv("POPCORN_GEMM_TILE") || k % 32 != 0 || (m * n) % 4 != 0) return 0;
    const int64_t cus = deviceCUs();
    const int64_t t384 = cdiv(m, 256) * cdiv(n, 384);
    if (t384 * 10 >= cus * 7) return 0;
    for (int64_t s = 2; s <= 8; ++s)
        if ((t384 * s) % cus == 0 && k % (32 * s) == 0 && k / s >= 2048) {
            // with whole-line tiles, split only when it beats the best tile's
            // score: the split grid fills the CUs, less the share of time its
            // partials' round trip through HBM adds (8 s bytes per element
            // at ~7 TB/s against 2 K flop at ~1.2 PFLOP/s: ~700 s / K)
            if (gemmLinesFit(k, 384)) {
                const ScoredTile &t = bestLineTile(m, n);
                if (1.0 - 700.0 * (double)s / (double)k <= lineTileScore(t, m, n)) return 0;
            }
            return s;
        }
    return 0;
}

// The split-K GEMM: f32 partial products per split in scratch, then one
// pass that sums them and rounds to C's dtype.
class SplitKMatmulKernel : public Kernel {
public:
    SplitKMatmulKernel(const Tensor &a, const Tensor &b, const Tensor &c, int64_t m, int64_t k, int64_t n, int64_t splits)
        : a_(a), b_(b), c_(c), m_(m), k_(k), n_(n), splits_(splits) {}
    std::vector<Binding> tensors() const override { return {{a_, kRead}, {b_, kRead}, {c_, kWrite}}; }
    std::string describe() const override { return mainName() + "," + reduceName(); }
    void encode(KernelCommandEncoder &enc) const override {
        MatmulConstants mc{(uint32_t)m_, (uint32_t)k_, (uint32_t)n_, 1u};
        enc.withTemporaryTensor(ScratchSpec{{splits_ * m_, n_}, DataType::f32}, [&](Tensor part) {
            DispatchSize ds;
            ds.grid = dim3((unsigned)(cdiv(m_, 256) * cdiv(n_, 384)), (unsigned)splits_, 1);
            ds.block = dim3(512, 1, 1);
            FixedDispatch s1(mainName(), {{a_, kRead}, {b_, kRead}, {part, kWrite}}, {bytesOf(mc)}, ds);
            enc.dispatch(s1);
            const uint32_t splits = (uint32_t)splits_;
            const int64_t blocks = std::clamp<int64_t>(cdiv(m_ * n_ / 4, kBlock), 1, 8 * deviceCUs());
            FixedDispatch s2(reduceName(), {{part, kRead}, {c_, kWrite}}, {bytesOf(mc), bytesOf(splits)}, grid1(blocks, kBlock));
            enc.dispatch(s2);
        });
    }

private:
    std::string mainName() const {
        // each split's K a whole number of 64-deep stages; offsets span the full rows
        const bool lines = gemmLinesFit(k_, 384) && k_ % (64 * splits_) == 0;
        return std::string("matmul_mfma_") + tag(a_.dataType) + (lines ? "_splitk_e256x384" : "_splitk_d256x384");
    }
    std::string reduceName() const { return std::string("matmul_splitk_reduce_") + tag(c_.dataType); }
    Tensor a_, b_, c_;
    int64_t m_, k_, n_, splits_;
};

constexpr int64_t kMaxStagedK = 16384;  // x staged as f32 in 64 KB of LDS
// A Matmul with a non-transposed 16-bit B [K, N] and m > 1: B^T into
// scratch (transpose2d_b16), then the transposed-B route (the MFMA or
// skinny kernels) on it.
std::unique_ptr<Kernel> makeMatmul(const Tensor &a, const Tensor &b, const Tensor &c, int64_t m, int64_t k, int64_t n,
                                   bool transposeB);
class TransposeBMatmulKernel : public Kernel {
public:
    TransposeBMatmulKernel(const Tensor &a, const Tensor &b, const Tensor &c, int64_t m, int64_t k, int64_t n)
        : a_(a), b_(b), c_(c), m_(m), k_(k), n_(n) {}
    std::vector<Binding> tensors() const override { return {{a_, kRead}, {b_, kRead}, {c_, kWrite}}; }
    std::string describe() const override {
        // the inner route's kernels, for B^T in (256-byte aligned) scratch
        Tensor bt(reinterpret_cast<void *>(uintptr_t{1} << 20), Shape({n_, k_}), b_.dataType);
        return "transpose2d_b16," + makeMatmul(a_, bt, c_, m_, k_, n_, true)->describe();
    }
    void encode(KernelCommandEncoder &enc) const override {
        enc.withTemporaryTensor(ScratchSpec{{n_, k_}, b_.dataType}, [&](Tensor bt) {
            Transpose2DConstants tc{(uint32_t)k_, (uint32_t)n_};
            DispatchSize ds;
            ds.grid = dim3((unsigned)cdiv(n_, 64), (unsigned)cdiv(k_, 64), 1);
            ds.block = dim3(kBlock, 1, 1);
            FixedDispatch t("transpose2d_b16", {{b_, kRead}, {bt, kWrite}}, {bytesOf(tc)}, ds);
            enc.dispatch(t);
            makeMatmul(a_, bt, c_, m_, k_, n_, true)->encode(enc);
        });
    }

private:
    Tensor a_, b_, c_;
    int64_t m_, k_, n_;
};


std::unique_ptr<Kernel> makeMatmul(const Tensor &a, const Tensor &b, const Tensor &c, int64_t m, int64_t k, int64_t n,
                                   bool transposeB) {
    if (m < 0 || k < 0 || n < 0) throw Error::tensorShapeMismatch("Matmul dimensions must be non-negative.");
    requireElements(a, m * k, "Matmul a");
    requireElements(b, k * n, "Matmul b");
    requireElements(c, m * n, "Matmul c");
    std::vector<Binding> binds = {{a, kRead}, {b, kRead}, {c, kWrite}};
    if (m == 1) {
        // Matmul.swift:233-277
        MatvecConstants mc{(uint32_t)k, (uint32_t)n, transposeB ? 1u : 0u};
        if (transposeB) {
            std::string fn = matvecNKName(a.dataType, b.dataType, c.dataType);
            if (fn.empty())
                throw Error::unsupportedDataTypeCombination(std::string("Unsupported matvec data type combination: ") +
                                                            tag(a.dataType) + ", " + tag(b.dataType) + ", " + tag(c.dataType) + ".");
            if (k > kMaxStagedK) throw Error::tensorShapeMismatch("matvec K above " + std::to_string(kMaxStagedK) + " is not supported.");
            const int R = matvecRows(n);
            fn += "_r" + std::to_string(R);
            return std::make_unique<FixedDispatch>(fn, binds, std::vector<std::vector<uint8_t>>{bytesOf(mc)},
                                                   grid1(streamBlocks(cdiv(n, R)), kBlock, (size_t)std::max<int64_t>(k, 1) * 4));
        }
        std::string fn = plainName("matvec", a.dataType, b.dataType, c.dataType);
        if (fn.empty())
            throw Error::unsupportedDataTypeCombination(std::string("Unsupported matvec data type combination: ") +
                                                        tag(a.dataType) + ", " + tag(b.dataType) + ", " + tag(c.dataType) + ".");
        return std::make_unique<FixedDispatch>(fn, binds, std::vector<std::vector<uint8_t>>{bytesOf(mc)}, grid1(cdiv(n, kBlock), kBlock));
    }
    // m > 1, transposeB, 16-bit operands: the MFMA tiles (the reference's MPP
    // GEMM path, Matmul.swift:175-196); 16-byte rows needed (K % 8 == 0).
    {
        const DataType t = a.dataType;
        // a [K, N] B (the reference's mpp_matmul without _tb): transposed
        // into scratch first, then this route (the scratch is 256-byte aligned)
        if (!transposeB && (t == DataType::f16 || t == DataType::bf16) && b.dataType == t &&
            (c.dataType == t || c.dataType == DataType::f32) && k % 8 == 0 && k > 0 && aligned16(a.data) &&
            k < 65536 * 64 && n < 65536 * 64)
            return std::make_unique<TransposeBMatmulKernel>(a, b, c, m, k, n);
        if (transposeB && (t == DataType::f16 || t == DataType::bf16) && b.dataType == t &&
            (c.dataType == t || c.dataType == DataType::f32) && k % 8 == 0 && k > 0 && aligned16(a.data) &&
            aligned16(b.data)) {
            // 2 <= M <= 64: the skinny kernel (gemm_skinny.hip), which
            // streams B once with its K split over a block's waves: about
            // 3 waves per CU in all, at most 4 per block (measured best on
            // MI355X for N 2304..24576 x K 2304..9216)
            if (m <= 64 && !std::getenv("POPCORN_GEMM_TILE") && n * k * 2 <= INT32_MAX && m * k * 2 <= INT32_MAX) {
                const int mt = (int)cdiv(m, 16);
                MatmulConstants mc{(uint32_t)m, (uint32_t)k, (uint32_t)n, 1u};
                // at least 512 tiles of 16 rows of B: A staged in LDS, one
                // tile per wave (one wave per block at M <= 16, else four)
                if (cdiv(n, 16) >= 2 * (int64_t)deviceCUs()) {
                    const int w = mt == 1 ? 1 : 4;
                    const std::string fn = std::string("matmul_skinny_") + tag(t) + "_" + tag(t) + "_" + tag(c.dataType) +
                                           "_m" + std::to_string(16 * mt) + "_lds";
                    return std::make_unique<FixedDispatch>(fn, binds, std::vector<std::vector<uint8_t>>{bytesOf(mc)},
                                                           grid1(cdiv(cdiv(n, 16), w), 64 * w));
                }
                // 16-row blocks (_r16) when 32-row ones would be fewer than the CUs
                const int rows = cdiv(n, 32) < deviceCUs() ? 16 : 32;
                const int64_t blocks = cdiv(n, rows);
                const int64_t want = 3 * (int64_t)deviceCUs() / blocks;
                int64_t w = 1;
                while (2 * w <= want && w < 4 && 2 * w <= cdiv(k, 32)) w *= 2;
                const std::string fn = std::string("matmul_skinny_") + tag(t) + "_" + tag(t) + "_" + tag(c.dataType) +
                                       "_m" + std::to_string(16 * mt) + (rows == 16 ? "_r16" : "");
                return std::make_unique<FixedDispatch>(fn, binds, std::vector<std::vector<uint8_t>>{bytesOf(mc)},
                                                       grid1(blocks, (int)(64 * w)));
            }
            // the split-K reduction stores 4 results of C at a time
            if (const int64_t splits = aligned16(c.data) ? gemmSplitK(m, n, k) : 0)
                return std::make_unique<SplitKMatmulKernel>(a, b, c, m, k, n, splits);
            MatmulConstants mc{(uint32_t)m, (uint32_t)k, (uint32_t)n, 1u};
            const GemmTile tile = gemmTile(m, n, k);
            const std::string fn =
                std::string("matmul_mfma_") + tag(t) + "_" + tag(t) + "_" + tag(c.dataType) + "_" + tile.suffix;
            return std::make_unique<FixedDispatch>(fn, binds, std::vector<std::vector<uint8_t>>{bytesOf(mc)},
                                                   grid1(cdiv(m, tile.bm) * cdiv(n, tile.bn), tile.threads));
        }
    }
    // m > 1 with f32 output and an f32 operand (the reference's MPP f32
    // combinations f32 x f32, f32 x bf16, bf16 x f32, Matmul.swift:203-214):
    // the f32 matrix-core tiles (gemm_f32.hip), B either way round; rows of
    // 4 values in 16-byte-aligned buffers
    {
        const DataType ta = a.dataType, tb = b.dataType, f32 = DataType::f32, bf16 = DataType::bf16;
        const bool combo = c.dataType == f32 && ((ta == f32 && (tb == f32 || tb == bf16)) || (ta == bf16 && tb == f32));
        if (combo && m > 1 && k % 4 == 0 && (transposeB || n % 4 == 0) && aligned16(a.data) && aligned16(b.data)) {
            MatmulConstants mc{(uint32_t)m, (uint32_t)k, (uint32_t)n, transposeB ? 1u : 0u};
            const std::string fn = std::string("matmul_mfma_") + tag(ta) + "_" + tag(tb) + "_f32" + (transposeB ? "_tb" : "");
            return std::make_unique<FixedDispatch>(fn, binds, std::vector<std::vector<uint8_t>>{bytesOf(mc)},
                                                   grid1(cdiv(m, 128) * cdiv(n, 128), kBlock));
        }
    }
    // the SIMT tiles (matmul.hip) in the place of the reference's matmul_typed
    std::string fn = plainName("matmul_tiled", a.dataType, b.dataType, c.dataType);
    if (fn.empty())
        throw Error::unsupportedDataTypeCombination(std::string("Unsupported matmul data type combination: ") +
                                                    tag(a.dataType) + ", " + tag(b.dataType) + ", " + tag(c.dataType) + ".");
    MatmulConstants mc{(uint32_t)m, (uint32_t)k, (uint32_t)n, transposeB ? 1u : 0u};
    DispatchSize ds;
    ds.grid = dim3((unsigned)cdiv(n, 64), (unsigned)cdiv(m, 64), 1);
    ds.block = dim3(kBlock, 1, 1);
    return std::make_unique<FixedDispatch>(fn, binds, std::vector<std::vector<uint8_t>>{bytesOf(mc)}, ds);
}

// ---------------------------------------------------------------------------
// Gated MLP (Gemma4TextInference.swift:416-429 as two dispatches)
// ---------------------------------------------------------------------------

class GatedMLPKernel : public Kernel {
public:
    GatedMLPKernel(const Tensor &x, const Tensor *nw, const Tensor &wg, const Tensor &wu, const Tensor &wd, const Tensor &out,
                   float eps, bool addOne, const Tensor *hidden)
        : x_(x), wg_(wg), wu_(wu), wd_(wd), out_(out), eps_(eps), addOne_(addOne) {
        if (nw) {
            nw_ = *nw;
            hasNorm_ = true;
        }
        if (hidden) {
            h_ = *hidden;
            hasHidden_ = true;
        }
        if (wg.shape.rank() != 2) throw Error::tensorInvalidRank(2, wg.shape.rank());
        F_ = wg.shape[0];
        H_ = wg.shape[1];
        if (wu.shape != wg.shape) throw Error::tensorShapeMismatch("GatedMLP up weight shape must match gate weight " + wg.shape.str() + ".");
        if (wd.shape != Shape({H_, F_})) throw Error::tensorShapeMismatch("GatedMLP down weight must be [" + std::to_string(H_) + ", " + std::to_string(F_) + "].");
        if (x.shape.rank() < 1 || x.shape.dims.back() != H_ || x.shape.elementCount() != H_)
            throw Error::tensorShapeMismatch("GatedMLP decodes one row: x must hold [" + std::to_string(H_) + "].");
        if (out.shape != x.shape) throw Error::tensorShapeMismatch("GatedMLP output shape must match x.");
        const DataType t = x.dataType;
        if (!isFloat(t) || wg.dataType != t || wu.dataType != t || wd.dataType != t || out.dataType != t)
            throw Error::unsupportedDataTypeCombination("GatedMLP needs x, weights and out of one float dtype.");
        if (hasNorm_) {
            if (nw_.dataType != DataType::f32) throw Error::unsupportedDataTypeCombination("GatedMLP norm weight must be f32.");
            requireElements(nw_, H_, "GatedMLP norm weight");
        }
        if (hasHidden_) {
            if (h_.dataType != t) throw Error::unsupportedDataTypeCombination("GatedMLP hidden must have x's dtype.");
            requireElements(h_, F_, "GatedMLP hidden");
        }
        if (H_ > kMaxStagedK || F_ > kMaxStagedK) throw Error::tensorShapeMismatch("GatedMLP H and F must be <= 16384.");
        requireElements(x, H_, "x");
        requireElements(wg, F_ * H_, "w_gate");
        requireElements(wu, F_ * H_, "w_up");
        requireElements(wd, H_ * F_, "w_down");
        R_ = F_ >= 32768 ? 2 : 1;
        down_ = makeMatmul(wd_, wd_, out_, 1, F_, H_, true);  // name/geometry probe only
    }

    // Residual form: x_ is the incoming residual stream; x = x_ +
    // RMSNorm(delta) * wPost is stored to xOut and feeds the MLP.
    void setResidual(const Tensor &delta, const Tensor &wPost, const Tensor &xOut) {
        if (delta.dataType != x_.dataType || xOut.dataType != x_.dataType)
            throw Error::unsupportedDataTypeCombination("GatedMLP residual tensors must have x's dtype.");
        if (wPost.dataType != DataType::f32) throw Error::unsupportedDataTypeCombination("post-norm weight must be f32.");
        requireElements(delta, H_, "GatedMLP delta");
        requireElements(wPost, H_, "GatedMLP post-norm weight");
        requireElements(xOut, H_, "GatedMLP x_out");
        if (xOut.data == x_.data) throw Error::invalidArgument("GatedMLP x_out must not alias x (blocks read x while block 0 writes x_out)");
        delta_ = delta;
        wPost_ = wPost;
        xOut_ = xOut;
        residual_ = true;
    }

    std::vector<Binding> tensors() const override {
        std::vector<Binding> b = {{x_, kRead}, {wg_, kRead}, {wu_, kRead}, {wd_, kRead}, {out_, kWrite}};
        if (hasNorm_) b.push_back({nw_, kRead});
        if (hasHidden_) b.push_back({h_, kWrite});
        if (residual_) {
            b.push_back({delta_, kRead});
            b.push_back({wPost_, kRead});
            b.push_back({xOut_, kWrite});
        }
        return b;
    }

    std::string describe() const override { return gateUpName() + "," + down_->describe(); }

    std::string gateUpName() const {
        return std::string("gated_mlp_gate_up_") + tag(x_.dataType) + (R_ == 1 ? "_r1" : "") + (residual_ ? "_res" : "");
    }

    void encode(KernelCommandEncoder &enc) const override {
        auto run = [&](const Tensor &h) {
            GatedMLPConstants gc{(uint32_t)H_, (uint32_t)F_, hasNorm_ ? 1u : 0u, addOne_ ? 1u : 0u, eps_,
                                 (uint32_t)x_.dataType, residual_ ? 1u : 0u};
            const Tensor normOrDummy = hasNorm_ ? nw_ : x_;
            // delta, w_post and x_out are touched only in the residual form
            const Tensor d = residual_ ? delta_ : x_, w = residual_ ? wPost_ : x_, xo = residual_ ? xOut_ : x_;
            FixedDispatch gu(gateUpName(),
                             {{x_, kRead}, {normOrDummy, kRead}, {wg_, kRead}, {wu_, kRead}, {h, kWrite}, {d, kRead},
                              {w, kRead}, {xo, residual_ ? kWrite : kRead}},
                             {bytesOf(gc)}, grid1(streamBlocks(cdiv(F_, R_)), kBlock, (size_t)H_ * 4));
            enc.dispatch(gu);
            auto down = makeMatmul(h, wd_, out_, 1, F_, H_, true);
            down->encode(enc);
        };
        if (hasHidden_) {
            run(h_);
        } else {
            enc.withTemporaryTensor(ScratchSpec{{F_}, x_.dataType}, [&](Tensor h) { run(h); });
        }
    }

private:
    Tensor x_, nw_, wg_, wu_, wd_, out_, h_, delta_, wPost_, xOut_;
    float eps_;
    bool addOne_, hasNorm_ = false, hasHidden_ = false, residual_ = false;
    int64_t H_ = 0, F_ = 0, R_ = 2;
    std::unique_ptr<Kernel> down_;
};

// The gated MLP with block-affine 4-bit gate, up and down weights: the fused
// front half (q4_gate_up_*) then the 4-bit down matvec (aq_qmv_fast_*).
// bf16 activations; the post-attention residual in front when delta is given.
class GatedMLPQ4Kernel : public Kernel {
public:
    GatedMLPQ4Kernel(const Tensor &x, const Tensor &nw, const AffineQuantizedTensor &wg, const AffineQuantizedTensor &wu,
                     const AffineQuantizedTensor &wd, const Tensor &out, float eps, const Tensor *hidden)
        : x_(x), nw_(nw), wg_(wg), wu_(wu), wd_(wd), out_(out), eps_(eps) {
        for (const AffineQuantizedTensor *q : {&wg, &wu, &wd}) {
            q->validate();
            if (q->bits != 4 || q->groupSize != 64 || q->scales.dataType != DataType::bf16 || q->shape.rank() != 2)
                throw Error::unsupportedDataTypeCombination("GatedMLP quantized weights are 2-D, 4-bit, group 64, bf16-scaled.");
            if (!aligned16(q->packedValues.data) || (reinterpret_cast<uintptr_t>(q->scales.data) & 3) ||
                (q->hasBiases && (reinterpret_cast<uintptr_t>(q->biases.data) & 3)))
                throw Error::invalidArgument("GatedMLP packed values must be 16-byte aligned, scales and biases 4-byte aligned");
        }
        F_ = wg.outFeatures();
        H_ = wg.inFeatures();
        if (wu.shape != wg.shape) throw Error::tensorShapeMismatch("GatedMLP up weight shape must match gate weight " + wg.shape.str() + ".");
        if (wd.shape != Shape({H_, F_}))
            throw Error::tensorShapeMismatch("GatedMLP down weight must be [" + std::to_string(H_) + ", " + std::to_string(F_) + "].");
        if (wg.hasBiases != wu.hasBiases) throw Error::invalidArgument("GatedMLP gate and up weights both have biases or neither");
        if (x.dataType != DataType::bf16 || out.dataType != DataType::bf16 || nw.dataType != DataType::f32)
            throw Error::unsupportedDataTypeCombination("GatedMLP with quantized weights takes bf16 x and out, an f32 norm weight.");
        if (H_ % 128 != 0 || F_ % 128 != 0 || H_ > 8192 || F_ > 16384)
            throw Error::tensorShapeMismatch("GatedMLP quantized: H, F multiples of 128, H <= 8192, F <= 16384.");
        if (x.shape.elementCount() != H_ || out.shape.elementCount() != H_)
            throw Error::tensorShapeMismatch("GatedMLP decodes one row: x and out hold [" + std::to_string(H_) + "].");
        requireElements(x, H_, "x");
        requireElements(nw, H_, "GatedMLP norm weight");
        for (const AffineQuantizedTensor *q : {&wg, &wu, &wd}) {
            const int64_t n = q->outFeatures(), k = q->inFeatures();
            requireElements(q->packedValues, n * (k / 8), "GatedMLP packed values");
            requireElements(q->scales, n * (k / 64), "GatedMLP scales");
            if (q->hasBiases) requireElements(q->biases, n * (k / 64), "GatedMLP biases");
        }
        if (hidden) {
            if (hidden->dataType != DataType::bf16) throw Error::unsupportedDataTypeCombination("GatedMLP hidden must be bf16.");
            requireElements(*hidden, F_, "GatedMLP hidden");
            h_ = *hidden;
            hasHidden_ = true;
        }
        lpr_ = q4Shape(F_, H_, false).lpr;
    }

    void setResidual(const Tensor &delta, const Tensor &wPost, const Tensor &xOut) {
        if (delta.dataType != DataType::bf16 || xOut.dataType != DataType::bf16 || wPost.dataType != DataType::f32)
            throw Error::unsupportedDataTypeCombination("GatedMLP residual: delta and x_out bf16, post-norm weight f32.");
        requireElements(delta, H_, "GatedMLP delta");
        requireElements(wPost, H_, "GatedMLP post-norm weight");
        requireElements(xOut, H_, "GatedMLP x_out");
        if (xOut.data == x_.data) throw Error::invalidArgument("GatedMLP x_out must not alias x (blocks read x while block 0 writes x_out)");
        delta_ = delta;
        wPost_ = wPost;
        xOut_ = xOut;
        residual_ = true;
    }

    std::vector<Binding> tensors() const override {
        std::vector<Binding> b = {{x_, kRead}, {nw_, kRead}, {out_, kWrite}};
        for (const AffineQuantizedTensor *q : {&wg_, &wu_, &wd_}) {
            b.push_back({q->packedValues, kRead});
            b.push_back({q->scales, kRead});
            if (q->hasBiases) b.push_back({q->biases, kRead});
        }
        if (hasHidden_) b.push_back({h_, kWrite});
        if (residual_) {
            b.push_back({delta_, kRead});
            b.push_back({wPost_, kRead});
            b.push_back({xOut_, kWrite});
        }
        return b;
    }

    std::string gateUpName() const {
        return "q4_gate_up_bf16_l" + std::to_string(lpr_) + (residual_ ? "_res" : "");
    }

    std::string describe() const override {
        // the down matvec reads the hidden tensor, or a 256-byte aligned scratch buffer
        void *hp = hasHidden_ ? h_.data : reinterpret_cast<void *>(uintptr_t{256});
        Tensor h(hp, Shape({1, F_}), DataType::bf16), o(out_.data, Shape({1, H_}), DataType::bf16);
        return gateUpName() + "," + Kernels::Matmul(h, wd_, o)->describe();
    }

    void encode(KernelCommandEncoder &enc) const override {
        auto run = [&](const Tensor &h) {
            GatedMLPConstants gc{(uint32_t)H_, (uint32_t)F_, 1u, 0u, eps_, (uint32_t)DataType::bf16, residual_ ? 1u : 0u};
            AffineQMatmulConstants qc{1u, (uint32_t)F_, (uint32_t)H_, (uint32_t)(H_ / 64), (uint32_t)(H_ / 8),
                                      wg_.hasBiases ? 1u : 0u};
            const Tensor d = residual_ ? delta_ : x_, w = residual_ ? wPost_ : x_, xo = residual_ ? xOut_ : x_;
            const size_t lds = (size_t)H_ * 4 + (size_t)(H_ / 64) * 36 * 4 + (size_t)(H_ / 64) * 4;
            FixedDispatch gu(gateUpName(),
                             {{x_, kRead}, {nw_, kRead}, {wg_.packedValues, kRead}, {wg_.scales, kRead},
                              {wg_.hasBiases ? wg_.biases : wg_.scales, kRead}, {wu_.packedValues, kRead}, {wu_.scales, kRead},
                              {wu_.hasBiases ? wu_.biases : wu_.scales, kRead}, {h, kWrite}, {d, kRead}, {w, kRead},
                              {xo, residual_ ? kWrite : kRead}},
                             {bytesOf(gc), bytesOf(qc)}, grid1(streamBlocks(cdiv(F_, 64 / lpr_)), kBlock, lds));
            enc.dispatch(gu);
            Tensor hv(h.data, Shape({1, F_}), DataType::bf16), ov(out_.data, Shape({1, H_}), DataType::bf16);
            Kernels::Matmul(hv, wd_, ov)->encode(enc);
        };
        if (hasHidden_) {
            run(h_);
        } else {
            enc.withTemporaryTensor(ScratchSpec{{F_}, DataType::bf16}, [&](Tensor h) { run(h); });
        }
    }

private:
    Tensor x_, nw_;
    AffineQuantizedTensor wg_, wu_, wd_;
    Tensor out_, h_, delta_, wPost_, xOut_;
    float eps_;
    bool hasHidden_ = false, residual_ = false;
    int64_t H_ = 0, F_ = 0;
    int lpr_ = 8;
};

// ---------------------------------------------------------------------------
// Argmax (Argmax.swift) as two stages over row slices
// ---------------------------------------------------------------------------

class ArgmaxKernel : public Kernel {
public:
    ArgmaxKernel(const Tensor &x, const Tensor &indices, int64_t rows, int64_t n) : x_(x), idx_(indices), rows_(rows), n_(n) {
        if (x.dataType != DataType::f32) throw Error::unsupportedDataTypeCombination("Argmax reads f32 values.");
        if (indices.dataType != DataType::i32) throw Error::unsupportedDataTypeCombination("Argmax indices are i32.");
        if (n <= 0) throw Error::tensorShapeMismatch("Argmax needs a non-empty axis.");
        requireElements(x, rows * n, "Argmax x");
        requireElements(indices, rows, "Argmax indices");
        slices_ = std::clamp<int64_t>(cdiv(n, 4096), 1, 256);
    }
    std::vector<Binding> tensors() const override { return {{x_, kRead}, {idx_, kWrite}}; }
    std::string describe() const override { return "argmax_partial,argmax_finish"; }
    void encode(KernelCommandEncoder &enc) const override {
        if (rows_ == 0) return;
        ArgmaxSliceConstants ac{(uint32_t)rows_, (uint32_t)n_, (uint32_t)slices_};
        enc.withTemporaryTensor(ScratchSpec{{rows_ * slices_}, DataType::f32}, [&](Tensor pv) {
            enc.withTemporaryTensor(ScratchSpec{{rows_ * slices_}, DataType::i32}, [&](Tensor pi) {
                DispatchSize ds;
                ds.grid = dim3((unsigned)slices_, (unsigned)rows_, 1);
                ds.block = dim3(kBlock, 1, 1);
                FixedDispatch s1("argmax_partial", {{x_, kRead}, {pv, kWrite}, {pi, kWrite}}, {bytesOf(ac)}, ds);
                enc.dispatch(s1);
                FixedDispatch s2("argmax_finish", {{x_, kRead}, {pv, kRead}, {pi, kRead}, {idx_, kWrite}}, {bytesOf(ac)},
                                 grid1(rows_, kBlock));
                enc.dispatch(s2);
            });
        });
    }

private:
    Tensor x_, idx_;
    int64_t rows_, n_, slices_ = 1;
};

std::unique_ptr<Kernel> elementwise(const char *base, const Tensor &a, const Tensor *b, const Tensor &out,
                                    std::vector<uint8_t> consts) {
    if (!isFloat(a.dataType)) throw Error::unsupportedDataTypeCombination(std::string("Unsupported ") + base + " data type: " + tag(a.dataType) + ".");
    if (out.dataType != a.dataType || (b && b->dataType != a.dataType))
        throw Error::unsupportedDataTypeCombination(std::string(base) + " needs one dtype for inputs and output.");
    const int64_t count = a.shape.elementCount();
    requireElements(a, count, base);
    requireElements(out, count, base);
    if (b) requireElements(*b, count, base);
    std::string fn = base;
    if (a.dataType != DataType::f32) fn += std::string("_") + tag(a.dataType);
    std::vector<Binding> binds = {{a, kRead}};
    if (b) binds.push_back({*b, kRead});
    binds.push_back({out, kWrite});
    const int64_t blocks = std::clamp<int64_t>(cdiv(cdiv(count, 16 / stride(a.dataType)), kBlock), 1, 8 * deviceCUs());
    return std::make_unique<FixedDispatch>(fn, binds, std::vector<std::vector<uint8_t>>{std::move(consts)}, grid1(blocks, kBlock));
}

}  // namespace

// AffineQuantizedTensor.swift:29-48, plus the format's own consistency (bits
// dividing the 32-bit word, a positive group size).
void AffineQuantizedTensor::validate() const {
    if (shape.rank() < 2) throw Error::tensorInvalidRank(2, shape.rank());
    if (hasBiases) {
        if (biases.dataType != scales.dataType)
            throw Error::unsupportedDataTypeCombination(std::string("AffineQuantizedTensor scales and biases must share a data type; got ") +
                                                        name(scales.dataType) + " and " + name(biases.dataType) + ".");
        if (biases.shape != scales.shape)
            throw Error::tensorShapeMismatch("AffineQuantizedTensor scales and biases must share a shape; got " + scales.shape.str() +
                                             " and " + biases.shape.str() + ".");
    }
    if (packedValues.dataType != DataType::u32)
        throw Error::unsupportedDataTypeCombination(
            std::string("AffineQuantizedTensor packed values must use u32 for packing uint32LittleEndian; got ") +
            name(packedValues.dataType) + ".");
    if (bits <= 0 || bits > 32 || 32 % bits != 0 || groupSize <= 0)
        throw Error::invalidArgument("AffineQuantizedTensor format needs bits dividing 32 and a positive group size.");
}

namespace Kernels {

// FlashAttention.swift:109-113: one query row -> split-KV decoding; 32 rows
// or more with a head dim up to 512 -> the tiled kernel on the matrix cores
// (where the reference takes MPP); otherwise the plain per-row kernel.
AttentionPath route(int64_t queryLen, int64_t headDim, DataType qType) {
    if (queryLen == 1) return AttentionPath::decoding;
    const bool sixteen = qType == DataType::f16 || qType == DataType::bf16;
    // the matrix-core kernels take any head dim up to 512 in 16-byte rows,
    // padded to 64, 128, 256 or 512 inside (MPPFlashAttention's hd256 and
    // hd512 buckets, FlashAttention.swift:305-311), in f16, bf16 and f32
    const int64_t perChunk = sixteen ? 8 : 4;
    if (queryLen >= 32 && (sixteen || qType == DataType::f32) && headDim <= 512 && headDim % perChunk == 0)
        return AttentionPath::tiled;
    return AttentionPath::plain;
}

// FlashAttention.swift:51-90
std::unique_ptr<Kernel> FlashAttention(const Tensor &q, const Tensor &k, const Tensor &v, const Tensor &out, float scale,
                                       AttentionMask mask) {
    if (q.shape.rank() != 4) throw Error::tensorInvalidRank(4, q.shape.rank());
    if (k.shape.rank() != 4) throw Error::tensorInvalidRank(4, k.shape.rank());
    if (v.shape.rank() != 4) throw Error::tensorInvalidRank(4, v.shape.rank());
    const int64_t B = q.shape[0], Nq = q.shape[1], Sq = q.shape[2], Hd = q.shape[3];
    const int64_t Nkv = k.shape[1], Sk = k.shape[2];
    if (k.shape[0] != B || k.shape[3] != Hd)
        throw Error::tensorShapeMismatch("FlashAttention K shape must match Q batch/headDim; q " + q.shape.str() + ", k " + k.shape.str() + ".");
    if (v.shape != k.shape)
        throw Error::tensorShapeMismatch("FlashAttention V shape must match K; v " + v.shape.str() + ", k " + k.shape.str() + ".");
    if (out.shape != Shape({B, Nq, Sq, Hd}))
        throw Error::tensorShapeMismatch("FlashAttention output shape must be " + Shape({B, Nq, Sq, Hd}).str() + "; got " + out.shape.str() + ".");
    return std::make_unique<FlashAttentionKernel>(q, k, v, out, AttnDims{B, Nq, Nkv, Sq, Sk, Hd, Sk}, scale, mask, nullptr);
}

// FlashAttention.swift:13-49, plus key capacity and position
std::unique_ptr<Kernel> FlashAttention(const Tensor &q, const Tensor &k, const Tensor &v, const Tensor &out, int64_t batch,
                                       int64_t queryHeads, int64_t kvHeads, int64_t queryLen, int64_t keyLen, int64_t headDim,
                                       float scale, AttentionMask mask, int64_t keyCapacity, const Tensor *position) {
    const int64_t cap = keyCapacity > 0 ? keyCapacity : keyLen;
    return std::make_unique<FlashAttentionKernel>(q, k, v, out, AttnDims{batch, queryHeads, kvHeads, queryLen, keyLen, headDim, cap},
                                                  scale, mask, position);
}

// The split-KV attention with its partials in the static scratch
// (static_scratch.hip) instead of a borrowed buffer: validation and kernels
// as for FlashAttention with the same dims; no device memory is allocated.
void FlashDecodingNoAlloc(KernelLibrary &library, hipStream_t stream, const Tensor &q, const Tensor &k, const Tensor &v,
                          const Tensor &out, int64_t batch, int64_t queryHeads, int64_t kvHeads, int64_t queryLen,
                          int64_t keyLen, int64_t headDim, float scale, AttentionMask mask, int64_t keyCapacity,
                          const Tensor *position) {
    struct NoScratch : KernelScratchAllocator {
        KernelTemporaryBuffer borrowTemporaryBuffer(size_t) override {
            throw Error(POPCORN_ERR_WORKSPACE_EXHAUSTED, "the allocation-free attention borrows no scratch");
        }
    } none;
    const int64_t cap = keyCapacity > 0 ? keyCapacity : keyLen;
    FlashAttentionKernel fa(q, k, v, out, AttnDims{batch, queryHeads, kvHeads, queryLen, keyLen, headDim, cap}, scale,
                            mask, position);
    fa.useSplitPath();
    size_t bytes = 0;
    void *scratch = staticScratch(&bytes);
    KernelCommandEncoder enc(library, stream, none);
    fa.encodeSplitInto(enc, scratch, bytes);
}

// Matmul.swift:68-93
std::unique_ptr<Kernel> Matmul(const Tensor &a, const Tensor &b, const Tensor &c, bool transposeB) {
    if (a.shape.rank() != 2) throw Error::tensorInvalidRank(2, a.shape.rank());
    if (b.shape.rank() != 2) throw Error::tensorInvalidRank(2, b.shape.rank());
    if (c.shape.rank() != 2) throw Error::tensorInvalidRank(2, c.shape.rank());
    const int64_t m = a.shape[0], k = a.shape[1];
    const int64_t n = transposeB ? b.shape[0] : b.shape[1];
    const Shape expectedB = transposeB ? Shape({n, k}) : Shape({k, n});
    if (b.shape != expectedB)
        throw Error::tensorShapeMismatch("Matmul RHS shape mismatch: expected " + expectedB.str() + ", got " + b.shape.str() + ".");
    if (c.shape != Shape({m, n}))
        throw Error::tensorShapeMismatch("Matmul output shape mismatch: expected " + Shape({m, n}).str() + ", got " + c.shape.str() + ".");
    return makeMatmul(a, b, c, m, k, n, transposeB);
}

std::unique_ptr<Kernel> Matmul(const Tensor &a, const Tensor &b, const Tensor &c, int64_t m, int64_t k, int64_t n, bool transposeB) {
    return makeMatmul(a, b, c, m, k, n, transposeB);
}

// RMSNorm.swift:10-37
std::unique_ptr<Kernel> RMSNorm(const Tensor &x, const Tensor *weight, const Tensor &out, int64_t rowCount, int64_t hiddenSize,
                                float eps, bool addOneToWeight) {
    const char *fn = nullptr;
    switch (x.dataType) {
    case DataType::f32: fn = "rmsnorm"; break;
    case DataType::f16: fn = "rmsnorm_f16"; break;
    case DataType::bf16: fn = "rmsnorm_bf16"; break;
    default: throw Error::unsupportedDataTypeCombination(std::string("Unsupported RMSNorm data type: ") + tag(x.dataType) + ".");
    }
    if (out.dataType != x.dataType) throw Error::unsupportedDataTypeCombination("RMSNorm output must have the input's dtype.");
    if (weight && weight->dataType != DataType::f32)
        throw Error::unsupportedDataTypeCombination("RMSNorm weight must be f32 (RMSNorm.metal:42-46 reads it as float).");
    if (hiddenSize <= 0 || rowCount < 0) throw Error::tensorShapeMismatch("RMSNorm needs a positive hidden size.");
    requireElements(x, rowCount * hiddenSize, "RMSNorm x");
    requireElements(out, rowCount * hiddenSize, "RMSNorm out");
    if (weight) requireElements(*weight, hiddenSize, "RMSNorm weight");
    RMSNormConstants rc{(uint32_t)hiddenSize, weight ? 1u : 0u, addOneToWeight ? 1u : 0u, eps};
    // One block per row; a lone row spreads over more lanes (latency), many
    // rows use 256 threads.
    const int64_t nvec = cdiv(hiddenSize, 16 / stride(x.dataType));
    int threads = kBlock;
    if (rowCount < deviceCUs()) threads = (int)std::clamp<int64_t>(cdiv(nvec, 64) * 64, 64, 1024);
    const Tensor &w = weight ? *weight : x;  // RMSNorm.swift:21: x bound as the absent weight
    return std::make_unique<FixedDispatch>(fn, std::vector<Binding>{{x, kRead}, {w, kRead}, {out, kWrite}},
                                           std::vector<std::vector<uint8_t>>{bytesOf(rc)}, grid1(rowCount, threads));
}

// RMSNorm.swift:39-70
std::unique_ptr<Kernel> RMSNorm(const Tensor &x, const Tensor *weight, const Tensor &out, int axis, float eps, bool addOneToWeight) {
    const int rank = x.shape.rank();
    const int norm = axis < 0 ? rank + axis : axis;
    if (norm != rank - 1 || rank <= 0) throw Error::tensorInvalidAxis(axis, rank);
    if (x.shape != out.shape)
        throw Error::tensorShapeMismatch("RMSNorm output shape must match input; got " + out.shape.str() + ", expected " + x.shape.str() + ".");
    const int64_t H = x.shape[norm];
    const int64_t rows = H ? x.shape.elementCount() / H : 0;
    if (weight && !(weight->shape == Shape({H}) || weight->shape == x.shape))
        throw Error::tensorShapeMismatch("RMSNorm weight shape must be [" + std::to_string(H) + "] or " + x.shape.str() + "; got " +
                                         weight->shape.str() + ".");
    return RMSNorm(x, weight, out, rows, H, eps, addOneToWeight);
}

// KVCacheWrite.swift:7-35, plus f16 and a run-time position
std::unique_ptr<Kernel> KVCacheWrite(const Tensor &source, const Tensor &cache, int64_t batch, int64_t kvHeads, int64_t newLen,
                                     int64_t maxLen, int64_t headDim, int64_t offset, const Tensor *position) {
    using D = DataType;
    const D s = source.dataType, c = cache.dataType;
    const char *fn = nullptr;
    if (s == D::f32 && c == D::f32) fn = "kv_cache_write";
    else if (s == D::bf16 && c == D::bf16) fn = "kv_cache_write_bf16";
    else if (s == D::f32 && c == D::bf16) fn = "kv_cache_write_f32_to_bf16";
    else if (s == D::f16 && c == D::f16) fn = "kv_cache_write_f16";
    else
        throw Error::unsupportedDataTypeCombination(std::string("Unsupported KV cache data type combination: ") + tag(s) + ", " + tag(c) + ".");
    if (batch < 0 || kvHeads < 0 || newLen < 0 || headDim <= 0 || maxLen < 0)
        throw Error::tensorShapeMismatch("KV cache write dimensions must be non-negative.");
    if (!position && (offset < 0 || offset + newLen > maxLen))
        throw Error::tensorShapeMismatch("KV cache write range " + std::to_string(offset) + "..<" + std::to_string(offset + newLen) +
                                         " exceeds cache length " + std::to_string(maxLen) + ".");
    requireElements(source, batch * kvHeads * newLen * headDim, "KV cache source");
    requireElements(cache, batch * kvHeads * maxLen * headDim, "KV cache");
    if (position) {
        if (position->dataType != D::i32) throw Error::unsupportedDataTypeCombination("position tensor must be i32");
        requireElements(*position, 1, "position");
    }
    const int64_t run = 16 / stride(s);
    const int64_t runs = batch * kvHeads * newLen * cdiv(headDim, run);
    const int64_t blocks = std::clamp<int64_t>(cdiv(runs, kBlock), 1, 4096);
    if (!position) {
        // the reference's kernel and constants (KVCacheWrite.metal:6-11)
        KVCacheWriteConstants kc{(uint32_t)batch, (uint32_t)kvHeads, (uint32_t)newLen, (uint32_t)maxLen,
                                 (uint32_t)headDim, (uint32_t)offset};
        return std::make_unique<FixedDispatch>(fn, std::vector<Binding>{{source, kRead}, {cache, kWrite}},
                                               std::vector<std::vector<uint8_t>>{bytesOf(kc)},
                                               grid1(runs ? blocks : 0, kBlock));
    }
    KVCacheWriteExtConstants kc{(uint32_t)batch, (uint32_t)kvHeads, (uint32_t)newLen, (uint32_t)maxLen, (uint32_t)headDim,
                                (uint32_t)std::max<int64_t>(offset, 0), 1u};
    return std::make_unique<FixedDispatch>(std::string(fn) + "_ext",
                                           std::vector<Binding>{{source, kRead}, {cache, kWrite}, {*position, kRead}},
                                           std::vector<std::vector<uint8_t>>{bytesOf(kc)}, grid1(runs ? blocks : 0, kBlock));
}

// KVCacheWrite.swift:37-48
std::unique_ptr<Kernel> KVCacheWrite(const Tensor &source, const Tensor &cache, int64_t offset) {
    if (source.shape.rank() != 4) throw Error::tensorInvalidRank(4, source.shape.rank());
    if (cache.shape.rank() != 4) throw Error::tensorInvalidRank(4, cache.shape.rank());
    const int64_t B = source.shape[0], Nkv = source.shape[1], Snew = source.shape[2], Hd = source.shape[3];
    if (cache.shape[0] != B || cache.shape[1] != Nkv || cache.shape[3] != Hd)
        throw Error::tensorShapeMismatch("KV cache shape must match source batch/heads/headDim; source " + source.shape.str() +
                                         ", cache " + cache.shape.str() + ".");
    if (offset < 0 || offset + Snew > cache.shape[2])
        throw Error::tensorShapeMismatch("KV cache write range " + std::to_string(offset) + "..<" + std::to_string(offset + Snew) +
                                         " exceeds cache length " + std::to_string(cache.shape[2]) + ".");
    return KVCacheWrite(source, cache, B, Nkv, Snew, cache.shape[2], Hd, offset, nullptr);
}

// GeluTanh.swift:28-33
std::unique_ptr<Kernel> GeluTanh(const Tensor &x, const Tensor &out) {
    if (x.shape != out.shape)
        throw Error::tensorShapeMismatch("GeluTanh output shape must match input; got " + out.shape.str() + ", expected " + x.shape.str() + ".");
    return elementwise("gelu_tanh", x, nullptr, out, bytesOf(GeluTanhConstants{(uint32_t)x.shape.elementCount()}));
}

// Mul.swift:28-37
std::unique_ptr<Kernel> Mul(const Tensor &a, const Tensor &b, const Tensor &out) {
    if (a.shape != b.shape) throw Error::tensorShapeMismatch("Mul requires matching input shapes; got " + a.shape.str() + " and " + b.shape.str() + ".");
    if (a.shape != out.shape) throw Error::tensorShapeMismatch("Mul output shape must match inputs; got " + out.shape.str() + ", expected " + a.shape.str() + ".");
    return elementwise("mul", a, &b, out, bytesOf(MulConstants{(uint32_t)a.shape.elementCount()}));
}

// Add.swift
std::unique_ptr<Kernel> Add(const Tensor &a, const Tensor &b, const Tensor &out) {
    if (a.shape != b.shape) throw Error::tensorShapeMismatch("Add requires matching input shapes; got " + a.shape.str() + " and " + b.shape.str() + ".");
    if (a.shape != out.shape) throw Error::tensorShapeMismatch("Add output shape must match inputs; got " + out.shape.str() + ", expected " + a.shape.str() + ".");
    return elementwise("add", a, &b, out, bytesOf(AddConstants{(uint32_t)a.shape.elementCount()}));
}

// ScalarMul.swift
std::unique_ptr<Kernel> ScalarMul(const Tensor &x, float scalar, const Tensor &out) {
    if (x.shape != out.shape)
        throw Error::tensorShapeMismatch("ScalarMul output shape must match input; got " + out.shape.str() + ", expected " + x.shape.str() + ".");
    return elementwise("scalar_mul", x, nullptr, out, bytesOf(ScalarMulConstants{(uint32_t)x.shape.elementCount(), scalar}));
}

// RopeBuildCosSin.swift:8-28: positions i32 [T], inv_freq f32 [Hd2] -> cos,
// sin f32 [T, Hd2] (the Metal kernel's buffer types, checked here).
std::unique_ptr<Kernel> RopeBuildCosSin(const Tensor &positions, const Tensor &invFreq, const Tensor &cosOut,
                                        const Tensor &sinOut, int64_t seqLen, int64_t halfHeadDim, float scaling) {
    if (positions.dataType != DataType::i32) throw Error::unsupportedDataTypeCombination("RoPE positions must be i32.");
    if (invFreq.dataType != DataType::f32 || cosOut.dataType != DataType::f32 || sinOut.dataType != DataType::f32)
        throw Error::unsupportedDataTypeCombination("RoPE invFreq and the cos/sin tables are f32.");
    if (seqLen < 0 || halfHeadDim < 0 || seqLen > UINT32_MAX || halfHeadDim > UINT32_MAX)
        throw Error::tensorShapeMismatch("RoPE table dimensions out of range.");
    requireElements(positions, seqLen, "RoPE positions");
    requireElements(invFreq, halfHeadDim, "RoPE invFreq");
    requireElements(cosOut, seqLen * halfHeadDim, "RoPE cos");
    requireElements(sinOut, seqLen * halfHeadDim, "RoPE sin");
    RopeBuildCosSinConstants c{(uint32_t)seqLen, (uint32_t)halfHeadDim, scaling};
    const int64_t n = seqLen * halfHeadDim;
    const int64_t blocks = n ? std::clamp<int64_t>(cdiv(n, kBlock), 1, 8 * deviceCUs()) : 0;
    return std::make_unique<FixedDispatch>(
        "rope_build_cos_sin",
        std::vector<Binding>{{positions, kRead}, {invFreq, kRead}, {cosOut, kWrite}, {sinOut, kWrite}},
        std::vector<std::vector<uint8_t>>{bytesOf(c)}, grid1(blocks, kBlock));
}

// RopeBuildCosSin.swift:30-50
std::unique_ptr<Kernel> RopeBuildCosSin(const Tensor &positions, const Tensor &invFreq, const Tensor &cosOut,
                                        const Tensor &sinOut, float scaling) {
    if (cosOut.shape != sinOut.shape)
        throw Error::tensorShapeMismatch("RoPE cos and sin output shapes must match; got " + cosOut.shape.str() + " and " +
                                         sinOut.shape.str() + ".");
    if (cosOut.shape.rank() != 2) throw Error::tensorInvalidRank(2, cosOut.shape.rank());
    const int64_t seqLen = cosOut.shape[0], halfHeadDim = cosOut.shape[1];
    if (positions.shape.elementCount() != seqLen)
        throw Error::tensorShapeMismatch("RoPE positions count must equal seqLen " + std::to_string(seqLen) + "; got " +
                                         std::to_string(positions.shape.elementCount()) + ".");
    if (invFreq.shape.elementCount() != halfHeadDim)
        throw Error::tensorShapeMismatch("RoPE invFreq count must equal halfHeadDim " + std::to_string(halfHeadDim) +
                                         "; got " + std::to_string(invFreq.shape.elementCount()) + ".");
    return RopeBuildCosSin(positions, invFreq, cosOut, sinOut, seqLen, halfHeadDim, scaling);
}

// RopeApply.swift:8-44: x [B, T, Nh, Hd] with tables [T, Hd/2]; the function
// is chosen by (x, table) dtypes as the reference does (:25-30); out has x's
// dtype.
std::unique_ptr<Kernel> RopeApply(const Tensor &x, const Tensor &cosT, const Tensor &sinT, const Tensor &out,
                                  int64_t batch, int64_t seqLen, int64_t headCount, int64_t headDim) {
    if (headDim % 2 != 0)
        throw Error::tensorShapeMismatch("RoPE head dimension must be even; got " + std::to_string(headDim) + ".");
    const char *fn = nullptr;
    if (x.dataType == DataType::f32 && cosT.dataType == DataType::f32) fn = "rope_apply";
    else if (x.dataType == DataType::bf16 && cosT.dataType == DataType::bf16) fn = "rope_apply_bf16";
    else if (x.dataType == DataType::bf16 && cosT.dataType == DataType::f32) fn = "rope_apply_f32_tables_bf16";
    else
        throw Error::unsupportedDataTypeCombination(std::string("Unsupported RoPE data type combination: ") + tag(x.dataType) +
                                                    ", " + tag(cosT.dataType) + ".");
    if (sinT.dataType != cosT.dataType || out.dataType != x.dataType)
        throw Error::unsupportedDataTypeCombination("RoPE sin table must match cos, and out must match x.");
    if (batch < 0 || seqLen < 0 || headCount < 0 || headDim < 0 || batch > UINT32_MAX || seqLen > UINT32_MAX ||
        headCount > UINT32_MAX || headDim > UINT32_MAX)
        throw Error::tensorShapeMismatch("RoPE dimensions out of range.");
    const int64_t n = batch * seqLen * headCount * headDim;
    requireElements(x, n, "RoPE x");
    requireElements(out, n, "RoPE out");
    requireElements(cosT, seqLen * (headDim / 2), "RoPE cos");
    requireElements(sinT, seqLen * (headDim / 2), "RoPE sin");
    RopeApplyConstants c{(uint32_t)batch, (uint32_t)seqLen, (uint32_t)headCount, (uint32_t)(headDim / 2)};
    const int64_t items = batch * seqLen * headCount * cdiv(headDim / 2, 8);
    const int64_t blocks = items ? std::clamp<int64_t>(cdiv(items, kBlock), 1, 8 * deviceCUs()) : 0;
    return std::make_unique<FixedDispatch>(
        fn, std::vector<Binding>{{x, kRead}, {cosT, kRead}, {sinT, kRead}, {out, kWrite}},
        std::vector<std::vector<uint8_t>>{bytesOf(c)}, grid1(blocks, kBlock));
}

// RopeApply.swift:46-60
std::unique_ptr<Kernel> RopeApply(const Tensor &x, const Tensor &cosT, const Tensor &sinT, const Tensor &out) {
    if (x.shape.rank() != 4) throw Error::tensorInvalidRank(4, x.shape.rank());
    if (x.shape != out.shape)
        throw Error::tensorShapeMismatch("RoPE output shape must match input; got " + out.shape.str() + ", expected " +
                                         x.shape.str() + ".");
    const int64_t batch = x.shape[0], seqLen = x.shape[1], headCount = x.shape[2], headDim = x.shape[3];
    if (headDim % 2 != 0)
        throw Error::tensorShapeMismatch("RoPE head dimension must be even; got " + std::to_string(headDim) + ".");
    const Shape table{seqLen, headDim / 2};
    if (cosT.shape != table || sinT.shape != table)
        throw Error::tensorShapeMismatch("RoPE tables must have shape " + table.str() + "; got cos " + cosT.shape.str() +
                                         ", sin " + sinT.shape.str() + ".");
    return RopeApply(x, cosT, sinT, out, batch, seqLen, headCount, headDim);
}

// Transpose12.swift:8-25: [D0, D1, D2, D3] -> [D0, D2, D1, D3].
std::unique_ptr<Kernel> Transpose12(const Tensor &src, const Tensor &out, int64_t d0, int64_t d1, int64_t d2, int64_t d3) {
    const char *fn = nullptr;
    switch (src.dataType) {
    case DataType::f32: fn = "transpose12"; break;
    case DataType::f16: fn = "transpose12_f16"; break;
    case DataType::bf16: fn = "transpose12_bf16"; break;
    default:
        throw Error::unsupportedDataTypeCombination(std::string("Unsupported transpose12 data type: ") + tag(src.dataType) + ".");
    }
    if (out.dataType != src.dataType) throw Error::unsupportedDataTypeCombination("Transpose12 output must match the source dtype.");
    for (int64_t d : {d0, d1, d2, d3})
        if (d < 0 || d > UINT32_MAX) throw Error::tensorShapeMismatch("Transpose12 dimensions out of range.");
    const int64_t n = d0 * d1 * d2 * d3;
    requireElements(src, n, "Transpose12 src");
    requireElements(out, n, "Transpose12 out");
    Transpose12Constants c{(uint32_t)d0, (uint32_t)d1, (uint32_t)d2, (uint32_t)d3};
    const int64_t runs = (d3 % (16 / stride(src.dataType)) == 0) ? n / (16 / stride(src.dataType)) : n;
    const int64_t blocks = runs ? std::clamp<int64_t>(cdiv(runs, kBlock), 1, 8 * deviceCUs()) : 0;
    return std::make_unique<FixedDispatch>(fn, std::vector<Binding>{{src, kRead}, {out, kWrite}},
                                           std::vector<std::vector<uint8_t>>{bytesOf(c)}, grid1(blocks, kBlock));
}

// Transpose12.swift:27-35
std::unique_ptr<Kernel> Transpose12(const Tensor &src, const Tensor &out) {
    if (src.shape.rank() != 4) throw Error::tensorInvalidRank(4, src.shape.rank());
    const int64_t d0 = src.shape[0], d1 = src.shape[1], d2 = src.shape[2], d3 = src.shape[3];
    const Shape expected{d0, d2, d1, d3};
    if (out.shape != expected)
        throw Error::tensorShapeMismatch("Transpose12 output shape must be " + expected.str() + "; got " + out.shape.str() + ".");
    return Transpose12(src, out, d0, d1, d2, d3);
}

std::unique_ptr<Kernel> GatedMLP(const Tensor &x, const Tensor *normWeight, const Tensor &wGate, const Tensor &wUp,
                                 const Tensor &wDown, const Tensor &out, float eps, bool addOneToWeight, const Tensor *hidden) {
    return std::make_unique<GatedMLPKernel>(x, normWeight, wGate, wUp, wDown, out, eps, addOneToWeight, hidden);
}

std::unique_ptr<Kernel> GatedMLPResidual(const Tensor &xIn, const Tensor &delta, const Tensor &wPost, const Tensor &xOut,
                                         const Tensor *normWeight, const Tensor &wGate, const Tensor &wUp,
                                         const Tensor &wDown, const Tensor &out, float eps, bool addOneToWeight,
                                         const Tensor *hidden) {
    auto k = std::make_unique<GatedMLPKernel>(xIn, normWeight, wGate, wUp, wDown, out, eps, addOneToWeight, hidden);
    k->setResidual(delta, wPost, xOut);
    return k;
}

std::unique_ptr<Kernel> DecodeAttention(const DecodeAttentionArgs &a) { return std::make_unique<DecodeAttentionKernel>(a); }

std::unique_ptr<Kernel> GatedMLPResidual(const Tensor &xIn, const Tensor *delta, const Tensor *wPost, const Tensor *xOut,
                                         const Tensor &normWeight, const AffineQuantizedTensor &wGate,
                                         const AffineQuantizedTensor &wUp, const AffineQuantizedTensor &wDown, const Tensor &out,
                                         float eps, const Tensor *hidden) {
    auto k = std::make_unique<GatedMLPQ4Kernel>(xIn, normWeight, wGate, wUp, wDown, out, eps, hidden);
    if (delta || wPost || xOut) {
        if (!delta || !wPost || !xOut) throw Error::invalidArgument("the residual form needs delta, w_post and x_out");
        k->setResidual(*delta, *wPost, *xOut);
    }
    return k;
}

std::unique_ptr<Kernel> DecodeMatvec(const DecodeMatvecArgs &a) {
    if (!a.x || !(a.weight || a.qweight) || !a.out) throw Error::invalidArgument("DecodeMatvec needs x, a weight and out");
    if (a.weight && a.qweight) throw Error::invalidArgument("DecodeMatvec takes a dense or a quantized weight, not both");
    const bool q4 = a.qweight != nullptr;
    int64_t N = 0, K = 0;
    DataType t;
    if (q4) {
        const AffineQuantizedTensor &Q = *a.qweight;
        Q.validate();
        N = Q.outFeatures();
        K = Q.inFeatures();
        t = a.x->dataType;
        if (t != DataType::bf16 || Q.bits != 4 || Q.groupSize != 64 || Q.scales.dataType != DataType::bf16)
            throw Error::unsupportedDataTypeCombination("DecodeMatvec with a quantized weight takes bf16 x and a 4-bit, group-64, "
                                                        "bf16-scaled weight.");
        if (K <= 0 || N <= 0 || K % 128 != 0 || K > 8192)
            throw Error::tensorShapeMismatch("DecodeMatvec with a quantized weight needs K a multiple of 128, 0 < K <= 8192.");
        requireElements(Q.packedValues, N * (K / 8), "DecodeMatvec packed values");
        requireElements(Q.scales, N * (K / 64), "DecodeMatvec scales");
        if (Q.hasBiases) requireElements(Q.biases, N * (K / 64), "DecodeMatvec biases");
        if (!aligned16(Q.packedValues.data) || (reinterpret_cast<uintptr_t>(Q.scales.data) & 3) ||
            (Q.hasBiases && (reinterpret_cast<uintptr_t>(Q.biases.data) & 3)))
            throw Error::invalidArgument("DecodeMatvec packed values must be 16-byte aligned, scales and biases 4-byte aligned");
    } else {
        const Tensor &W = *a.weight;
        if (W.shape.rank() != 2) throw Error::tensorInvalidRank(2, W.shape.rank());
        N = W.shape[0];
        K = W.shape[1];
        t = W.dataType;
        if (!isFloat(t) || a.x->dataType != t)
            throw Error::unsupportedDataTypeCombination("DecodeMatvec needs x and weight of one float dtype.");
        if (K <= 0 || N <= 0 || K > kMaxStagedK) throw Error::tensorShapeMismatch("DecodeMatvec needs 0 < K <= 16384 and N > 0.");
        requireElements(W, N * K, "DecodeMatvec weight");
    }
    const DataType o = a.out->dataType;
    if (!(o == t || o == DataType::f32)) throw Error::unsupportedDataTypeCombination("DecodeMatvec output is the weight dtype or f32.");
    requireElements(*a.x, K, "DecodeMatvec x");
    uint32_t flags = 0;
    if (a.delta) {
        if (!a.wPost || !a.xOut) throw Error::invalidArgument("DecodeMatvec with delta needs wPost and xOut");
        if (a.delta->dataType != t || a.xOut->dataType != t || a.wPost->dataType != DataType::f32)
            throw Error::unsupportedDataTypeCombination("DecodeMatvec residual: delta and xOut of x's dtype, wPost f32.");
        requireElements(*a.delta, K, "DecodeMatvec delta");
        requireElements(*a.wPost, K, "DecodeMatvec wPost");
        requireElements(*a.xOut, K, "DecodeMatvec xOut");
        if (a.xOut->data == a.x->data) throw Error::invalidArgument("DecodeMatvec xOut must not alias x");
        flags |= 1u;
    }
    if (a.wPre) {
        if (a.wPre->dataType != DataType::f32) throw Error::unsupportedDataTypeCombination("DecodeMatvec wPre must be f32.");
        requireElements(*a.wPre, K, "DecodeMatvec wPre");
        flags |= 2u;
    }
    DecodeMatvecConstants dc{(uint32_t)K, (uint32_t)N, a.eps, 0u, (uint32_t)t, (uint32_t)N, 0u, 1u, 1u};
    if (a.kCache || a.vCache) {
        if (!a.kCache || !a.vCache || !a.position) throw Error::invalidArgument("KV scatter needs both caches and a position");
        const Tensor &kc = *a.kCache;
        if (kc.shape != a.vCache->shape) throw Error::tensorShapeMismatch("K and V caches must have one shape.");
        const int r = kc.shape.rank();
        if (r < 3 || (r == 4 && kc.shape[0] != 1) || r > 4) throw Error::tensorShapeMismatch("caches must be [1?, Nkv, Smax, Hd].");
        const int64_t Nkv = kc.shape[r - 3], Smax = kc.shape[r - 2], Hd = kc.shape[r - 1];
        if (kc.dataType != o || a.vCache->dataType != o || o != t)
            throw Error::unsupportedDataTypeCombination("KV scatter writes caches of the weight dtype.");
        if (a.position->dataType != DataType::i32) throw Error::unsupportedDataTypeCombination("position tensor must be i32");
        requireElements(*a.position, 1, "position");
        if (a.qRows < 0 || a.qRows + 2 * Nkv * Hd != N)
            throw Error::tensorShapeMismatch("weight rows must be qRows + 2 * Nkv * Hd for the KV scatter.");
        requireElements(*a.out, a.qRows, "DecodeMatvec out");
        flags |= 4u;
        dc.qRows = (uint32_t)a.qRows;
        dc.kvRows = (uint32_t)(Nkv * Hd);
        dc.headDim = (uint32_t)Hd;
        dc.kvStride = (uint32_t)Smax;
    } else {
        requireElements(*a.out, N, "DecodeMatvec out");
    }
    dc.flags = flags;
    const Tensor &x = *a.x;
    if (q4) {
        const AffineQuantizedTensor &Q = *a.qweight;
        const int lpr = q4Shape(N, K, false).lpr;
        const std::string fn = std::string("q4_decode_matvec_bf16_") + tag(o) + "_l" + std::to_string(lpr) + "_f" +
                               std::to_string(flags & 3u);
        AffineQMatmulConstants qc{1u, (uint32_t)N, (uint32_t)K, (uint32_t)(K / 64), (uint32_t)(K / 8), Q.hasBiases ? 1u : 0u};
        std::vector<Binding> b = {
            {x, kRead},
            {a.delta ? *a.delta : x, kRead},
            {a.wPost ? *a.wPost : x, kRead},
            {a.wPre ? *a.wPre : x, kRead},
            {Q.packedValues, kRead},
            {Q.scales, kRead},
            {Q.hasBiases ? Q.biases : Q.scales, kRead},
            {*a.out, kWrite},
            {a.xOut ? *a.xOut : x, a.xOut ? kWrite : kRead},
            {a.kCache ? *a.kCache : *a.out, kWrite},
            {a.vCache ? *a.vCache : *a.out, kWrite},
            {a.position ? *a.position : x, kRead},
        };
        // LDS: x as f32, its bf16 pair words (36 words per group of 64), the group sums
        const size_t lds = (size_t)K * 4 + (size_t)(K / 64) * 36 * 4 + (size_t)(K / 64) * 4;
        return std::make_unique<FixedDispatch>(fn, std::move(b), std::vector<std::vector<uint8_t>>{bytesOf(dc), bytesOf(qc)},
                                               grid1(streamBlocks(cdiv(N, 64 / lpr)), kBlock, lds));
    }
    const int R = matvecRows(N);
    const std::string fn = std::string("decode_matvec_") + tag(t) + "_" + tag(o) + "_r" + std::to_string(R) + "_f" +
                           std::to_string(flags & 3u);
    const Tensor &W = *a.weight;
    std::vector<Binding> b = {
        {x, kRead},
        {a.delta ? *a.delta : x, kRead},
        {a.wPost ? *a.wPost : x, kRead},
        {a.wPre ? *a.wPre : x, kRead},
        {W, kRead},
        {*a.out, kWrite},
        {a.xOut ? *a.xOut : x, a.xOut ? kWrite : kRead},
        {a.kCache ? *a.kCache : *a.out, kWrite},
        {a.vCache ? *a.vCache : *a.out, kWrite},
        {a.position ? *a.position : x, kRead},
    };
    return std::make_unique<FixedDispatch>(fn, std::move(b), std::vector<std::vector<uint8_t>>{bytesOf(dc)},
                                           grid1(streamBlocks(cdiv(N, R)), kBlock, (size_t)K * 4));
}

// EmbeddingGather.swift: ids [N] i32, table [V, H], out [N, H]
std::unique_ptr<Kernel> EmbeddingGather(const Tensor &ids, const Tensor &table, const Tensor &out) {
    using D = DataType;
    if (ids.dataType != D::i32) throw Error::unsupportedDataTypeCombination("EmbeddingGather ids must be i32.");
    if (table.shape.rank() != 2) throw Error::tensorInvalidRank(2, table.shape.rank());
    const int64_t V = table.shape[0], H = table.shape[1], N = ids.shape.elementCount();
    const char *fn = nullptr;
    if (table.dataType == D::f32 && out.dataType == D::f32) fn = "embedding_gather";
    else if (table.dataType == D::f16 && out.dataType == D::f16) fn = "embedding_gather_f16";
    else if (table.dataType == D::bf16 && out.dataType == D::bf16) fn = "embedding_gather_bf16";
    else if (table.dataType == D::bf16 && out.dataType == D::f32) fn = "embedding_gather_bf16_to_f32";
    else throw Error::unsupportedDataTypeCombination("Unsupported EmbeddingGather data type combination.");
    requireElements(out, N * H, "EmbeddingGather out");
    EmbeddingGatherExtConstants ec{(uint32_t)N, (uint32_t)H, (uint32_t)V};
    const int64_t runs = N * cdiv(H, 16 / stride(table.dataType));
    return std::make_unique<FixedDispatch>(std::string(fn) + "_ext",
                                           std::vector<Binding>{{ids, kRead}, {table, kRead}, {out, kWrite}},
                                           std::vector<std::vector<uint8_t>>{bytesOf(ec)},
                                           grid1(runs ? std::clamp<int64_t>(cdiv(runs, kBlock), 1, 4096) : 0, kBlock));
}


// The 4-bit Matmul on the matrix cores for bf16 rows (aq_gemm.hip): x's
// group sums and a pair-ordered copy of x in scratch, then 128 x 128 tiles
// of C, with the K groups split over blocks (and a reduction) when the tiles
// leave CUs idle. Its three launches take ~25-35 us at small m, while the
// streaming matvec per row costs about N K / 2 bytes / 4.5 TB/s per row, so
// the GEMM wins once the rows' weight reads pass ~2^27 bytes (measured at
// N K = 9216 x 2304 both ways: 26 against 43 us at m 16-29, 35 against
// 210 us at m 128).
constexpr int64_t kQ4GemmMinRows = 16;
constexpr int64_t kQ4GemmMinBytes = int64_t{1} << 27;  // m * N * K / 2

class AffineQGemmKernel : public Kernel {
public:
    AffineQGemmKernel(const Tensor &a, const AffineQuantizedTensor &b, const Tensor &c, const AffineQMatmulConstants &qc)
        : a_(a), b_(b), c_(c), qc_(qc) {}
    std::vector<Binding> tensors() const override {
        std::vector<Binding> t = {{b_.packedValues, kRead}, {b_.scales, kRead}, {a_, kRead}, {c_, kWrite}};
        if (b_.hasBiases) t.push_back({b_.biases, kRead});
        return t;
    }
    std::string describe() const override {
        return splits() > 1 ? std::string("aq_gemm_prep_bf16,aq_gemm_mfma_bf16_bf16_splitk_b4_g64,") + reduceName()
                            : std::string("aq_gemm_prep_bf16,") + mainName();
    }
    void encode(KernelCommandEncoder &enc) const override {
        const int64_t m = qc_.M, k = qc_.K, g = qc_.kGroups, n = qc_.N, tiles = cdiv(m, 128) * cdiv(n, 128);
        const int64_t s = splits();
        enc.withTemporaryTensor(ScratchSpec{{m, k}, DataType::bf16}, [&](Tensor xp) {
            enc.withTemporaryTensor(ScratchSpec{{m, g}, DataType::f32}, [&](Tensor xs) {
                FixedDispatch prep("aq_gemm_prep_bf16", {{a_, kRead}, {xp, kWrite}, {xs, kWrite}}, {bytesOf(qc_)},
                                   grid1(cdiv(m * (k / 8), kBlock), kBlock));
                enc.dispatch(prep);
                const Tensor &bias = b_.hasBiases ? b_.biases : b_.scales;
                if (s <= 1) {
                    FixedDispatch gemm(mainName(),
                                       {{b_.packedValues, kRead}, {b_.scales, kRead}, {bias, kRead}, {xp, kRead},
                                        {xs, kRead}, {c_, kWrite}},
                                       {bytesOf(qc_)}, grid1(tiles, kBlock));
                    enc.dispatch(gemm);
                    return;
                }
                enc.withTemporaryTensor(ScratchSpec{{s * m, n}, DataType::f32}, [&](Tensor part) {
                    DispatchSize ds;
                    ds.grid = dim3((unsigned)tiles, (unsigned)s, 1);
                    ds.block = dim3(kBlock, 1, 1);
                    FixedDispatch gemm("aq_gemm_mfma_bf16_bf16_splitk_b4_g64",
                                       {{b_.packedValues, kRead}, {b_.scales, kRead}, {bias, kRead}, {xp, kRead},
                                        {xs, kRead}, {part, kWrite}},
                                       {bytesOf(qc_)}, ds);
                    enc.dispatch(gemm);
                    MatmulConstants mc{(uint32_t)m, (uint32_t)k, (uint32_t)n, 1u};
                    const uint32_t splits = (uint32_t)s;
                    const int64_t blocks = std::clamp<int64_t>(cdiv(m * n / 4, kBlock), 1, 8 * deviceCUs());
                    FixedDispatch reduce(reduceName(), {{part, kRead}, {c_, kWrite}}, {bytesOf(mc), bytesOf(splits)},
                                         grid1(blocks, kBlock));
                    enc.dispatch(reduce);
                });
            });
        });
    }

private:
    // K splits (groups per block) when the tiles leave CUs idle: about two
    // blocks per CU, at least 4 groups each; the reduction takes M N % 4 == 0
    // and 16-byte-aligned C
    int64_t splits() const {
        const int64_t tiles = cdiv((int64_t)qc_.M, 128) * cdiv((int64_t)qc_.N, 128);
        const int64_t want = 2 * (int64_t)deviceCUs() / std::max<int64_t>(tiles, 1);
        const int64_t s = std::min<int64_t>(want, (int64_t)qc_.kGroups / 4);
        const bool reducible = ((int64_t)qc_.M * qc_.N) % 4 == 0 && aligned16(c_.data);
        return reducible && s >= 2 ? s : 1;
    }
    std::string mainName() const { return std::string("aq_gemm_mfma_bf16_bf16_") + tag(c_.dataType) + "_b4_g64"; }
    std::string reduceName() const { return std::string("matmul_splitk_reduce_") + tag(c_.dataType); }
    Tensor a_;
    AffineQuantizedTensor b_;
    Tensor c_;
    AffineQMatmulConstants qc_;
};

// Matmul.swift:99-130 and :279-332
std::unique_ptr<Kernel> Matmul(const Tensor &a, const AffineQuantizedTensor &b, const Tensor &c) {
    using D = DataType;
    b.validate();
    if (a.shape.rank() != 2) throw Error::tensorInvalidRank(2, a.shape.rank());
    if (c.shape.rank() != 2) throw Error::tensorInvalidRank(2, c.shape.rank());
    const int64_t m = a.shape[0], k = a.shape[1], n = b.outFeatures();
    if (b.inFeatures() != k)
        throw Error::tensorShapeMismatch("Matmul quantized RHS shape mismatch: a.shape=[" + std::to_string(m) + "," +
                                         std::to_string(k) + "] but b.inFeatures=" + std::to_string(b.inFeatures()) + ".");
    if (c.shape != Shape{m, n})
        throw Error::tensorShapeMismatch("Matmul output shape mismatch: expected [" + std::to_string(m) + "," + std::to_string(n) +
                                         "], got " + c.shape.str() + ".");
    if (b.groupSize <= 0 || k % b.groupSize != 0)
        throw Error::tensorShapeMismatch("Matmul quantized RHS: K=" + std::to_string(k) + " is not divisible by groupSize=" +
                                         std::to_string(b.groupSize) + ".");
    const D x = a.dataType, sd = b.scales.dataType, o = c.dataType;
    const bool combo = (x == D::bf16 && sd == D::bf16 && (o == D::bf16 || o == D::f32)) ||
                       (x == D::f32 && sd == D::bf16 && o == D::f32);
    if (b.bits != 4 || b.groupSize != 64 || !combo)
        throw Error::unsupportedDataTypeCombination(
            "Unsupported affine quantized matmul combination: format=(bits: " + std::to_string(b.bits) + ", groupSize: " +
            std::to_string(b.groupSize) + "), x=" + tag(x) + ", scales=" + tag(sd) + ", out=" + tag(o) + ".");
    if (m > UINT32_MAX || n > UINT32_MAX || k > UINT32_MAX) throw Error::tensorShapeMismatch("Matmul dimensions out of range.");
    requireElements(a, m * k, "Matmul a");
    requireElements(c, m * n, "Matmul c");
    requireElements(b.packedValues, n * (k / 8), "Matmul quantized packed values");
    requireElements(b.scales, n * (k / 64), "Matmul quantized scales");
    if (b.hasBiases) requireElements(b.biases, n * (k / 64), "Matmul quantized biases");
    AffineQMatmulConstants qc{(uint32_t)m, (uint32_t)n, (uint32_t)k, (uint32_t)(k / 64), (uint32_t)(k / 8), b.hasBiases ? 1u : 0u};
    const Tensor &bias = b.hasBiases ? b.biases : b.scales;
    std::vector<Binding> binds = {{b.packedValues, kRead}, {b.scales, kRead}, {bias, kRead}, {a, kRead}, {c, kWrite}};
    const std::string combo3 = std::string(tag(x)) + "_bf16_" + tag(o) + "_b4_g64";
    const Q4Shape q = q4Shape(n, k, x == D::f32);
    const bool aligned = aligned16(b.packedValues.data) && aligned16(a.data) &&
                         (reinterpret_cast<uintptr_t>(b.scales.data) & 3) == 0 && (reinterpret_cast<uintptr_t>(bias.data) & 3) == 0;
    // a prompt's rows of bf16 activations: the matrix-core GEMM (one pass
    // over the weights for all rows instead of one matvec per row)
    // (buffer copies: every operand under 2^31 bytes; an even number of
    // groups per row, so a group's scale and bias share a 32-bit word with
    // a neighbour of the same row)
    const int64_t lim = int64_t{1} << 31;
    if (x == D::bf16 && m >= kQ4GemmMinRows && m * n * (k / 2) >= kQ4GemmMinBytes && aligned && k % 128 == 0 &&
        m * k * 2 < lim && n * (k / 2) < lim && m * (k / 64) * 4 < lim && cdiv(m, 128) * cdiv(n, 128) <= (int64_t)UINT32_MAX)
        return std::make_unique<AffineQGemmKernel>(a, b, c, qc);
    DispatchSize ds;
    ds.block = dim3(kBlock, 1, 1);
    std::string fn;
    if (q.lpr && aligned && m <= 65535) {
        fn = std::string(m == 1 ? "aq_qmv_fast_" : "aq_matvec_simd4_") + combo3 + "_l" + std::to_string(q.lpr) + "_j" +
             std::to_string(q.j);
        const int64_t units = cdiv(n, 64 / q.lpr);
        ds.grid = dim3((unsigned)streamBlocks(units), (unsigned)m, 1);
    } else {
        if (m > 65535) throw Error::tensorShapeMismatch("quantized Matmul supports at most 65535 rows of a.");
        // the reference's kernel: a 32-lane half-wave per 4 rows, 8 per block
        fn = "aq_matvec_simd4_" + combo3;
        ds.grid = dim3((unsigned)cdiv(cdiv(n, 4), kBlock / 32), (unsigned)m, 1);
    }
    if (m == 0 || n == 0) ds.grid = dim3(0, 1, 1);
    return std::make_unique<FixedDispatch>(fn, binds, std::vector<std::vector<uint8_t>>{bytesOf(qc)}, ds);
}

// EmbeddingGather.swift:45-88
std::unique_ptr<Kernel> EmbeddingGather(const Tensor &ids, const AffineQuantizedTensor &table, const Tensor &out) {
    using D = DataType;
    table.validate();
    if (ids.shape.rank() != 1) throw Error::tensorInvalidRank(1, ids.shape.rank());
    if (ids.dataType != D::i32)
        throw Error::unsupportedDataTypeCombination(std::string("EmbeddingGather with quantized table requires i32 ids; got ") +
                                                    tag(ids.dataType) + ".");
    if (out.shape.rank() != 2) throw Error::tensorInvalidRank(2, out.shape.rank());
    const int64_t T = ids.shape[0], H = table.inFeatures(), V = table.outFeatures();
    if (out.shape != Shape{T, H})
        throw Error::tensorShapeMismatch("EmbeddingGather output shape mismatch: expected [" + std::to_string(T) + "," +
                                         std::to_string(H) + "], got " + out.shape.str() + ".");
    if (table.groupSize <= 0 || H % table.groupSize != 0)
        throw Error::tensorShapeMismatch("EmbeddingGather quantized table hiddenSize=" + std::to_string(H) +
                                         " is not divisible by groupSize=" + std::to_string(table.groupSize) + ".");
    if (table.bits != 4 || table.groupSize != 64)
        throw Error::unsupportedDataTypeCombination(
            "EmbeddingGather currently only supports affine quantized tables with bits=4, groupSize=64, "
            "packing=.uint32LittleEndian.");
    if (table.scales.dataType != D::bf16 || !(out.dataType == D::bf16 || out.dataType == D::f32))
        throw Error::unsupportedDataTypeCombination(std::string("Unsupported quantized EmbeddingGather combination: scales ") +
                                                    tag(table.scales.dataType) + ", out " + tag(out.dataType) + ".");
    if (V > UINT32_MAX || H > UINT32_MAX || T > UINT32_MAX) throw Error::tensorShapeMismatch("EmbeddingGather dimensions out of range.");
    requireElements(table.packedValues, V * (H / 8), "EmbeddingGather quantized packed values");
    requireElements(table.scales, V * (H / 64), "EmbeddingGather quantized scales");
    if (table.hasBiases) requireElements(table.biases, V * (H / 64), "EmbeddingGather quantized biases");
    requireElements(out, T * H, "EmbeddingGather out");
    AffineQEmbeddingGatherExtConstants gc{(uint32_t)T, (uint32_t)H, (uint32_t)(H / 64), (uint32_t)(H / 8),
                                          table.hasBiases ? 1u : 0u, (uint32_t)V};
    const Tensor &bias = table.hasBiases ? table.biases : table.scales;
    const std::string fn = std::string("aq_embedding_gather_bf16_") + tag(out.dataType) + "_b4_g64_ext";
    const int64_t words = T * (H / 8);
    return std::make_unique<FixedDispatch>(
        fn, std::vector<Binding>{{ids, kRead}, {table.packedValues, kRead}, {table.scales, kRead}, {bias, kRead}, {out, kWrite}},
        std::vector<std::vector<uint8_t>>{bytesOf(gc)}, grid1(words ? std::clamp<int64_t>(cdiv(words, kBlock), 1, 4096) : 0, kBlock));
}

// Argmax.swift:24-37
std::unique_ptr<Kernel> Argmax(const Tensor &x, const Tensor &indices) {
    const int rank = x.shape.rank();
    if (rank <= 0) throw Error::tensorInvalidAxis(-1, rank);
    const int64_t n = x.shape[rank - 1];
    const int64_t rows = n ? x.shape.elementCount() / n : 0;
    if (indices.shape.elementCount() != rows)
        throw Error::tensorShapeMismatch("Argmax indices must contain " + std::to_string(rows) + " elements; got " +
                                         std::to_string(indices.shape.elementCount()) + ".");
    return std::make_unique<ArgmaxKernel>(x, indices, rows, n);
}

std::unique_ptr<Kernel> Custom(const std::string &functionName, std::vector<Binding> tensors,
                               std::vector<std::vector<uint8_t>> constants, dim3 grid, dim3 block) {
    return Custom(functionName, std::move(tensors), std::move(constants), grid, block, 0);
}

std::unique_ptr<Kernel> Custom(const std::string &functionName, std::vector<Binding> tensors,
                               std::vector<std::vector<uint8_t>> constants, dim3 grid, dim3 block, size_t dynamicLds) {
    DispatchSize ds;
    ds.grid = grid;
    ds.block = block;
    ds.dynamicLds = dynamicLds;
    return std::make_unique<FixedDispatch>(functionName, std::move(tensors), std::move(constants), ds);
}

std::unique_ptr<Kernel> FillNormal(void *data, DataType dtype, uint64_t count, uint64_t seed, float mean, float stddev) {
    if (!isFloat(dtype)) throw Error::unsupportedDataTypeCombination("fill_normal writes f32, f16 or bf16.");
    if (count && !data) throw Error::invalidArgument("fill_normal: null data pointer");
    FillNormalConstants fc{seed, count, mean, stddev};
    Tensor t(data, Shape({(int64_t)count}), dtype);
    const int64_t blocks = std::clamp<int64_t>(cdiv((int64_t)count, kBlock), 1, 16 * deviceCUs());
    return std::make_unique<FixedDispatch>(std::string("fill_normal_") + tag(dtype), std::vector<Binding>{{t, kWrite}},
                                           std::vector<std::vector<uint8_t>>{bytesOf(fc)}, grid1(count ? blocks : 0, kBlock));
}

}  // namespace Kernels
}  // namespace popcorn

// ---------------------------------------------------------------------------
// The merged-pair exchange of the tiled prefill attention, per stream
// ---------------------------------------------------------------------------

namespace popcorn {
namespace {

struct PairExchangeRegistry {
    std::mutex mu;
    std::map<std::pair<int, hipStream_t>, PairExchange> byStream;
};
PairExchangeRegistry &pairRegistry() {
    static auto *r = new PairExchangeRegistry();  // lives to process exit, as the memory does
    return *r;
}

size_t roundUpPow2(size_t n) {
    size_t p = 1 << 20;
    while (p < n) p <<= 1;
    return p;
}

// Reads the abort word; when set, clears every flag and throws -1019.
void checkOne(const PairExchange &x) {
    uint64_t abortWord = 0;
    checkHip(hipMemcpy(&abortWord, x.flags, 8, hipMemcpyDeviceToHost), "read the pair exchange's abort word");
    if (abortWord == 0) return;
    checkHip(hipMemset(x.flags, 0, PairExchange::kFlags * 8), "clear the pair exchange's flags");
    throw Error(POPCORN_ERR_GPU_INTERNAL,
                "FlashAttention: a merged causal tile pair's ready-flag wait gave up (0.2 s, or a flag left by a "
                "launch that gave up before); the affected output rows hold NaN. The flags have been cleared.");
}

}  // namespace

PairExchange &pairExchange(hipStream_t stream, size_t dataBytes) {
    int dev = 0;
    checkHip(hipGetDevice(&dev), "hipGetDevice");
    auto &r = pairRegistry();
    std::lock_guard<std::mutex> g(r.mu);
    PairExchange &x = r.byStream[{dev, stream}];
    if (!x.flags) {
        x.flags = static_cast<uint64_t *>(UncachedPool::take(PairExchange::kFlags * 8));
        x.dev = dev;
        checkHip(hipMemset(x.flags, 0, PairExchange::kFlags * 8), "zero the pair exchange's flags");
    }
    if (x.dataBytes < dataBytes) {
        // the old block stays reserved: a graph captured with it still uses it
        const size_t n = roundUpPow2(dataBytes);
        x.data = UncachedPool::take(n);
        x.dataBytes = n;
    }
    return x;
}

void checkPairExchange(hipStream_t stream, bool allStreams) {
    int dev = 0;
    checkHip(hipGetDevice(&dev), "hipGetDevice");
    auto &r = pairRegistry();
    std::vector<PairExchange> todo;
    {
        std::lock_guard<std::mutex> g(r.mu);
        for (auto &kv : r.byStream)
            if (kv.first.first == dev && (allStreams || kv.first.second == stream)) todo.push_back(kv.second);
    }
    for (const PairExchange &x : todo) checkOne(x);
}

}  // namespace popcorn
