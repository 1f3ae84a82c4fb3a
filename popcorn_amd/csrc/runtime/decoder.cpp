// The batch-1 greedy decode loop (include/popcorn_decoder.h): device state,
// the per-step kernel list built once from Kernels.* descriptors, and HIP
// graph capture/replay of whole steps.
#include <cmath>
#include <cstring>
#include <map>
#include <mutex>
#include <set>

#include "handles.hpp"
#include "popcorn_decoder.h"

using namespace popcorn;

namespace {

struct Buffer {
    void *p = nullptr;
    size_t bytes = 0;
    Buffer() = default;
    explicit Buffer(size_t n) : bytes(n) {
        if (hipMalloc(&p, n ? n : 1) != hipSuccess) {
            (void)hipGetLastError();
            p = nullptr;
            throw Error::tensorAllocationFailed(n);
        }
    }
    Buffer(const Buffer &) = delete;
    Buffer &operator=(const Buffer &) = delete;
    Buffer(Buffer &&o) noexcept : p(o.p), bytes(o.bytes) { o.p = nullptr; }
    Buffer &operator=(Buffer &&o) noexcept {
        std::swap(p, o.p);
        std::swap(bytes, o.bytes);
        return *this;
    }
    ~Buffer() {
        if (p) (void)hipFree(p);
    }
    template <typename T = uint8_t>
    T *at(size_t byteOffset) const { return reinterpret_cast<T *>(static_cast<uint8_t *>(p) + byteOffset); }
};

// `count` stacked [N, K] block-affine 4-bit matrices (group 64, bf16 scales
// and biases): packed u32 [count][N][K / 8], scales and biases [count][N][K / 64].
struct QMat {
    Buffer packed, scales, biases;
    int64_t N = 0, K = 0;
    void alloc(int64_t n, int64_t k, int64_t count) {
        N = n;
        K = k;
        packed = Buffer((size_t)(count * n * k / 2));
        scales = Buffer((size_t)(count * n * (k / 64) * 2));
        biases = Buffer((size_t)(count * n * (k / 64) * 2));
    }
    Tensor packedAt(int64_t l) const {
        return Tensor(packed.at((size_t)(l * N * K / 2)), Shape({N, K / 8}), DataType::u32);
    }
    Tensor scalesAt(int64_t l) const {
        return Tensor(scales.at((size_t)(l * N * (K / 64) * 2)), Shape({N, K / 64}), DataType::bf16);
    }
    Tensor biasesAt(int64_t l) const {
        return Tensor(biases.at((size_t)(l * N * (K / 64) * 2)), Shape({N, K / 64}), DataType::bf16);
    }
    AffineQuantizedTensor at(int64_t l) const {
        AffineQuantizedTensor q;
        q.packedValues = packedAt(l);
        q.scales = scalesAt(l);
        q.biases = biasesAt(l);
        q.hasBiases = true;
        q.shape = Shape({N, K});
        return q;
    }
};

}  // namespace

struct popcorn_decoder_s {
    popcorn_decoder_config_t cfg{};
    KernelLibrary *lib = nullptr;
    hipStream_t stream = nullptr;
    ScratchPool pool;
    std::unique_ptr<KernelCommandEncoder> enc;

    // sizes
    int64_t L = 0, H = 0, Nq = 0, Nkv = 0, Hd = 0, F = 0, V = 0, S = 0, QW = 0, KW = 0, QKV = 0;

    // weights (bf16 unless noted) and state
    Buffer embedding, finalNorm /*f32*/, wqkv, wo, wg, wu, wd, norms /*f32 [L][4][H]*/;
    Buffer headNorms /*f32 [L][2][Hd], attention_block*/, invFreq /*f32 [Hd/2]*/;
    bool q4 = false;  // weight_bits 4: the matrices below replace the bf16 ones
    QMat qqkv, qo, qg, qu, qd, qemb;
    Buffer kcache, vcache;
    Buffer x, x2, e, qkv, attn, o, mlp, hidden, logits /*f32*/, token /*i32*/, position /*i32*/, history /*i32*/;
    Buffer argValues /*f32 [argSlices]*/, argIndices /*i32 [argSlices]*/;
    int64_t argSlices = 1;

    // prime: the input row of the token in `token` (embedding gather, then
    // x sqrt(H)); every later step's tail writes the next one itself
    std::vector<std::unique_ptr<Kernel>> prime, step;
    std::vector<std::string> names;

    hipGraphExec_t graph = nullptr;
    hipGraph_t graphDef = nullptr;
    int graphSteps = 1;
    // The position the next enqueued step decodes at, tracked on the host
    // (reset sets it, every enqueued step adds one, read resynchronises it
    // with device memory) so that run() refuses steps past the KV cache.
    int64_t hostPos = 0;

    ~popcorn_decoder_s() {
        if (graph) (void)hipGraphExecDestroy(graph);
        if (graphDef) (void)hipGraphDestroy(graphDef);
    }

    Tensor bf(void *p, Shape s) const { return Tensor(p, std::move(s), DataType::bf16); }

    size_t layerOffset(int64_t elemsPerLayer, int64_t l, int es = 2) const { return (size_t)(elemsPerLayer * l) * (size_t)es; }

    const QMat *qmat(const std::string &base) const {
        if (!q4) return nullptr;
        if (base == "w_qkv") return &qqkv;
        if (base == "w_o") return &qo;
        if (base == "w_gate") return &qg;
        if (base == "w_up") return &qu;
        if (base == "w_down") return &qd;
        if (base == "embedding") return &qemb;
        return nullptr;
    }

    // "<matrix>", "<matrix>.scales", "<matrix>.biases" of a 4-bit decoder.
    bool quantizedView(const std::string &name, int64_t l, Tensor &t) const {
        const size_t dot = name.find('.');
        const std::string base = name.substr(0, dot), part = dot == std::string::npos ? "" : name.substr(dot + 1);
        const QMat *m = qmat(base);
        if (!m) return false;
        if (part.empty()) t = m->packedAt(l);
        else if (part == "scales") t = m->scalesAt(l);
        else if (part == "biases") t = m->biasesAt(l);
        else return false;
        return true;
    }

    Tensor weight(const char *which, int64_t l) const {
        Tensor qt;
        if (quantizedView(which, l, qt)) return qt;
        if (!strcmp(which, "w_qkv")) return bf(wqkv.at(layerOffset(QKV * H, l)), {QKV, H});
        if (!strcmp(which, "w_o")) return bf(wo.at(layerOffset(H * QW, l)), {H, QW});
        if (!strcmp(which, "w_gate")) return bf(wg.at(layerOffset(F * H, l)), {F, H});
        if (!strcmp(which, "w_up")) return bf(wu.at(layerOffset(F * H, l)), {F, H});
        if (!strcmp(which, "w_down")) return bf(wd.at(layerOffset(H * F, l)), {H, F});
        if (!strcmp(which, "k_cache")) return bf(kcache.at(layerOffset(Nkv * S * Hd, l)), {1, Nkv, S, Hd});
        if (!strcmp(which, "v_cache")) return bf(vcache.at(layerOffset(Nkv * S * Hd, l)), {1, Nkv, S, Hd});
        int slot = !strcmp(which, "norm_in") ? 0 : !strcmp(which, "norm_post_attn") ? 1 : !strcmp(which, "norm_pre_ffn") ? 2
                 : !strcmp(which, "norm_post_ffn") ? 3 : -1;
        if (slot >= 0) return Tensor(norms.at(layerOffset(H, l * 4 + slot, 4)), Shape({H}), DataType::f32);
        const int head = !strcmp(which, "q_norm") ? 0 : !strcmp(which, "k_norm") ? 1 : -1;
        if (head >= 0 && headNorms.p) return Tensor(headNorms.at(layerOffset(Hd, l * 2 + head, 4)), Shape({Hd}), DataType::f32);
        throw Error::invalidArgument(std::string("unknown decoder tensor ") + which);
    }

    // Six dispatches per layer: the QKV matvec (previous layer's post-FFN
    // norm + residual, this layer's input norm, K/V scattered into the caches),
    // split-KV attention with its combine, the O projection, the gate/up
    // matvec (post-attention norm + residual, pre-FFN norm), the down matvec.
    // With attention_block the QKV matvec stores the raw projections and the
    // attention partial kernel applies the per-head norms and RoPE and writes
    // the K/V row (DecodeAttention). The residual stream alternates between x
    // and x2 (blocks of one kernel read one while block 0 writes the other).
    void build() {
        const float eps = cfg.eps;
        const bool block = cfg.attention_block != 0;
        Tensor tx = bf(x.p, {1, H}), tx2 = bf(x2.p, {1, H}), te = bf(e.p, {1, H});
        Tensor tq = bf(qkv.p, {1, QW}), tqkv = bf(qkv.p, {1, QKV});
        Tensor tinv(invFreq.p, Shape({Hd / 2}), DataType::f32);
        Tensor tq4 = bf(qkv.p, {1, Nq, 1, Hd});
        Tensor tattn4 = bf(attn.p, {1, Nq, 1, Hd}), tattn = bf(attn.p, {1, QW});
        Tensor to = bf(o.p, {1, H}), tmlp = bf(mlp.p, {1, H}), th = bf(hidden.p, {F});
        Tensor tpos(position.p, Shape({1}), DataType::i32);
        Tensor ttok(token.p, Shape({1}), DataType::i32);
        Tensor temb = bf(embedding.p, {V, H});
        Tensor tlog(logits.p, Shape({1, V}), DataType::f32);
        Tensor tfin(finalNorm.p, Shape({H}), DataType::f32);

        auto add = [&](std::unique_ptr<Kernel> k) { step.push_back(std::move(k)); };
        // Gemma4TextInference.swift:184-185: gather, then scale by sqrt(H);
        // run before the first step of each run(), the steps' tails after
        if (q4) prime.push_back(Kernels::EmbeddingGather(ttok, qemb.at(0), te));
        else prime.push_back(Kernels::EmbeddingGather(ttok, temb, te));
        prime.push_back(Kernels::ScalarMul(te, std::sqrt((float)H), tx));
        const AttentionMask causal{0, -1};
        Tensor prevPostFfn;
        for (int64_t l = 0; l < L; ++l) {
            Tensor nin = weight("norm_in", l), npa = weight("norm_post_attn", l);
            Tensor npf = weight("norm_pre_ffn", l), npo = weight("norm_post_ffn", l);
            Tensor kc = weight("k_cache", l), vc = weight("v_cache", l);
            Tensor wqkv_l = q4 ? Tensor() : weight("w_qkv", l), wo_l = q4 ? Tensor() : weight("w_o", l);
            const AffineQuantizedTensor qqkv_l = q4 ? qqkv.at(l) : AffineQuantizedTensor(),
                                        qo_l = q4 ? qo.at(l) : AffineQuantizedTensor();
            Kernels::DecodeMatvecArgs qkvArgs;
            if (l == 0) {
                qkvArgs.x = &tx;
            } else {
                qkvArgs.x = &tx2;
                qkvArgs.delta = &tmlp;
                qkvArgs.wPost = &prevPostFfn;
                qkvArgs.xOut = &tx;
            }
            qkvArgs.wPre = &nin;
            if (q4) qkvArgs.qweight = &qqkv_l;
            else qkvArgs.weight = &wqkv_l;
            qkvArgs.eps = eps;
            if (block) {
                qkvArgs.out = &tqkv;
                add(Kernels::DecodeMatvec(qkvArgs));
                Tensor wqn = weight("q_norm", l), wkn = weight("k_norm", l);
                Kernels::DecodeAttentionArgs at;
                at.qkv = &tqkv;
                at.kCache = &kc;
                at.vCache = &vc;
                at.out = &tattn4;
                at.position = &tpos;
                at.qNorm = &wqn;
                at.kNorm = &wkn;
                at.invFreq = &tinv;
                at.vNorm = true;
                at.queryHeads = Nq;
                at.kvHeads = Nkv;
                at.eps = eps;
                at.scale = cfg.attn_scale;
                at.mask = causal;
                add(Kernels::DecodeAttention(at));
            } else {
                qkvArgs.out = &tq;
                qkvArgs.kCache = &kc;
                qkvArgs.vCache = &vc;
                qkvArgs.position = &tpos;
                qkvArgs.qRows = QW;
                add(Kernels::DecodeMatvec(qkvArgs));
                add(Kernels::FlashAttention(tq4, kc, vc, tattn4, 1, Nq, Nkv, 1, 1, Hd, cfg.attn_scale, causal, S, &tpos));
            }
            Kernels::DecodeMatvecArgs oArgs;
            oArgs.x = &tattn;
            if (q4) oArgs.qweight = &qo_l;
            else oArgs.weight = &wo_l;
            oArgs.out = &to;
            add(Kernels::DecodeMatvec(oArgs));
            if (q4)
                add(Kernels::GatedMLPResidual(tx, &to, &npa, &tx2, npf, qg.at(l), qu.at(l), qd.at(l), tmlp, eps, &th));
            else
                add(Kernels::GatedMLPResidual(tx, to, npa, tx2, &npf, weight("w_gate", l), weight("w_up", l),
                                              weight("w_down", l), tmlp, eps, false, &th));
            prevPostFfn = npo;
        }
        // Gemma4TextInference.swift:201-206: the last post-FFN norm + residual,
        // the final norm and the tied LM head in one matvec, then argmax
        Kernels::DecodeMatvecArgs head;
        head.x = &tx2;
        head.delta = &tmlp;
        head.wPost = &prevPostFfn;
        head.xOut = &tx;
        head.wPre = &tfin;
        const AffineQuantizedTensor qemb0 = q4 ? qemb.at(0) : AffineQuantizedTensor();
        if (q4) head.qweight = &qemb0;
        else head.weight = &temb;
        head.out = &tlog;
        head.eps = eps;
        add(Kernels::DecodeMatvec(head));
        // Argmax (Argmax.metal) in two stages: the slices' candidates, then
        // one block that picks the token, records it, advances the position
        // and writes the next step's input row (gather, x sqrt(H))
        Tensor tpv(argValues.p, Shape({argSlices}), DataType::f32);
        Tensor tpi(argIndices.p, Shape({argSlices}), DataType::i32);
        ArgmaxSliceConstants ac{1u, (uint32_t)V, (uint32_t)argSlices};
        add(Kernels::Custom("argmax_partial", {{tlog, kRead}, {tpv, kWrite}, {tpi, kWrite}}, {bytesOf(ac)},
                            dim3((unsigned)argSlices, 1, 1), dim3(256, 1, 1)));
        Tensor thist(history.p, Shape({std::max<int64_t>(cfg.history_len, 1)}), DataType::i32);
        DecodeNextTokenConstants nc{(uint32_t)V, (uint32_t)argSlices, (uint32_t)H,
                                    (uint32_t)std::max(cfg.history_len, 0), 1, std::sqrt((float)H), 1u};
        if (q4)
            add(Kernels::Custom("decode_next_token_q4_bf16",
                                {{tlog, kRead}, {tpv, kRead}, {tpi, kRead}, {ttok, kWrite}, {tpos, kReadWrite},
                                 {thist, kWrite}, {qemb.packedAt(0), kRead}, {qemb.scalesAt(0), kRead},
                                 {qemb.biasesAt(0), kRead}, {tx, kWrite}},
                                {bytesOf(nc)}, dim3(1, 1, 1), dim3(256, 1, 1)));
        else
            add(Kernels::Custom("decode_next_token_bf16",
                                {{tlog, kRead}, {tpv, kRead}, {tpi, kRead}, {ttok, kWrite}, {tpos, kReadWrite},
                                 {thist, kWrite}, {temb, kRead}, {tx, kWrite}},
                                {bytesOf(nc)}, dim3(1, 1, 1), dim3(256, 1, 1)));
        for (const auto &k : step) {
            std::string d = k->describe();
            size_t s = 0;
            while (s <= d.size()) {
                size_t c = d.find(',', s);
                if (c == std::string::npos) c = d.size();
                names.push_back(d.substr(s, c - s));
                s = c + 1;
            }
        }
    }

    void encodeStep() {
        for (const auto &k : step) enc->encode(*k);
    }

    void capture() {
        if (graph) return;
        // One eager step caches every function and fills the scratch pool, so
        // the capture allocates nothing; token and position are restored (the
        // KV row it wrote is rewritten by the first real step).
        int32_t tok = 0, pos = 0;
        checkHip(hipMemcpyAsync(&tok, token.p, 4, hipMemcpyDeviceToHost, stream), "read token");
        checkHip(hipMemcpyAsync(&pos, position.p, 4, hipMemcpyDeviceToHost, stream), "read position");
        checkHip(hipStreamSynchronize(stream), "sync");
        encodeStep();
        checkHip(hipMemcpyAsync(token.p, &tok, 4, hipMemcpyHostToDevice, stream), "restore token");
        checkHip(hipMemcpyAsync(position.p, &pos, 4, hipMemcpyHostToDevice, stream), "restore position");
        checkHip(hipStreamSynchronize(stream), "sync");
        checkHip(hipStreamBeginCapture(stream, hipStreamCaptureModeThreadLocal), "hipStreamBeginCapture");
        try {
            for (int i = 0; i < graphSteps; ++i) encodeStep();
        } catch (...) {
            hipGraph_t g = nullptr;
            (void)hipStreamEndCapture(stream, &g);
            if (g) (void)hipGraphDestroy(g);
            throw;
        }
        checkHip(hipStreamEndCapture(stream, &graphDef), "hipStreamEndCapture");
        checkHip(hipGraphInstantiate(&graph, graphDef, nullptr, nullptr, 0), "hipGraphInstantiate");
    }

    void encodePrime() {
        for (const auto &k : prime) enc->encode(*k);
    }

    void run(int32_t steps, bool useGraph) {
        if (steps < 0) throw Error::invalidArgument("steps must be >= 0");
        if (steps == 0) return;
        // a step at position p writes KV row p and attends rows 0..p
        if (hostPos < 0 || hostPos + steps > S)
            throw Error::tensorShapeMismatch("decode steps at positions " + std::to_string(hostPos) + "..<" +
                                             std::to_string(hostPos + steps) + " exceed the KV cache length " +
                                             std::to_string(S) + ".");
        hostPos += steps;
        if (!useGraph) {
            encodePrime();
            for (int32_t i = 0; i < steps; ++i) encodeStep();
            return;
        }
        capture();
        encodePrime();
        int32_t i = 0;
        for (; i + graphSteps <= steps; i += graphSteps) checkHip(hipGraphLaunch(graph, stream), "hipGraphLaunch");
        for (; i < steps; ++i) encodeStep();
    }

    int64_t stepBytes(int32_t pos) const {
        // bytes per weight: 2 (bf16), or 1/2 + 2 x 2 / 64 (4-bit values, bf16 scale and bias per 64)
        auto wbytes = [&](int64_t elems) { return q4 ? elems / 2 + elems / 16 : elems * 2; };
        const int64_t layerW = wbytes(QKV * H + H * QW + 3 * F * H) + 4 * H * 4;
        const int64_t kv = 2 * Nkv * (int64_t)(pos + 1) * Hd * 2;  // K and V rows read
        return L * (layerW + kv) + wbytes(V * H) + H * 4 + V * 4;
    }
};

static popcorn_status_t guardedDec(const std::function<void()> &f) {
    try {
        f();
        setLastError("");
        return POPCORN_OK;
    } catch (const Error &e) {
        setLastError(e.what());
        return e.code();
    } catch (const std::exception &e) {
        setLastError(e.what());
        return POPCORN_ERR_GPU_INTERNAL;
    }
}

extern "C" {

popcorn_status_t popcorn_decoder_create(popcorn_library_t library, popcorn_stream_t stream,
                                        const popcorn_decoder_config_t *config, popcorn_decoder_t *decoder) {
    return guardedDec([&] {
        if (!library || !config || !decoder) throw Error::invalidArgument("library, config and decoder must not be NULL");
        const popcorn_decoder_config_t &c = *config;
        if (c.layers <= 0 || c.hidden <= 0 || c.query_heads <= 0 || c.kv_heads <= 0 || c.head_dim <= 0 || c.ffn <= 0 ||
            c.vocab <= 0 || c.max_seq <= 0)
            throw Error::tensorShapeMismatch("decoder dimensions must be positive");
        auto d = std::make_unique<popcorn_decoder_s>();
        d->cfg = c;
        d->lib = library->lib.get();
        d->stream = reinterpret_cast<hipStream_t>(stream);
        d->graphSteps = std::max(1, c.graph_steps);
        d->L = c.layers;
        d->H = c.hidden;
        d->Nq = c.query_heads;
        d->Nkv = c.kv_heads;
        d->Hd = c.head_dim;
        d->F = c.ffn;
        d->V = c.vocab;
        d->S = c.max_seq;
        d->QW = d->Nq * d->Hd;
        d->KW = d->Nkv * d->Hd;
        d->QKV = d->QW + 2 * d->KW;
        const int64_t L = d->L, H = d->H, F = d->F;
        if (c.weight_bits != 0 && c.weight_bits != 16 && c.weight_bits != 4)
            throw Error::invalidArgument("weight_bits is 16 (bf16) or 4 (block-affine, group 64)");
        d->q4 = c.weight_bits == 4;
        d->finalNorm = Buffer((size_t)(H * 4));
        if (d->q4) {
            if (H % 128 || F % 128 || d->QW % 128)
                throw Error::tensorShapeMismatch("4-bit weights need hidden, ffn and query width multiples of 128");
            d->qemb.alloc(d->V, H, 1);
            d->qqkv.alloc(d->QKV, H, L);
            d->qo.alloc(H, d->QW, L);
            d->qg.alloc(F, H, L);
            d->qu.alloc(F, H, L);
            d->qd.alloc(H, F, L);
        } else {
            d->embedding = Buffer((size_t)(d->V * H * 2));
            d->wqkv = Buffer((size_t)(L * d->QKV * H * 2));
            d->wo = Buffer((size_t)(L * H * d->QW * 2));
            d->wg = Buffer((size_t)(L * F * H * 2));
            d->wu = Buffer((size_t)(L * F * H * 2));
            d->wd = Buffer((size_t)(L * H * F * 2));
        }
        d->norms = Buffer((size_t)(L * 4 * H * 4));
        d->kcache = Buffer((size_t)(L * d->Nkv * d->S * d->Hd * 2));
        d->vcache = Buffer((size_t)(L * d->Nkv * d->S * d->Hd * 2));
        d->x = Buffer((size_t)(H * 2));
        d->x2 = Buffer((size_t)(H * 2));
        d->e = Buffer((size_t)(H * 2));
        d->qkv = Buffer((size_t)(d->QKV * 2));
        if (c.attention_block) {
            if (d->Hd % 2 != 0) throw Error::tensorShapeMismatch("attention_block needs an even head dim");
            if (!(c.rope_theta > 0.0f)) throw Error::invalidArgument("attention_block needs rope_theta > 0");
            d->headNorms = Buffer((size_t)(L * 2 * d->Hd * 4));
            // Gemma4Workspace.swift:195-197: inv_freq[i] = 1 / theta^(2i / Hd), in double, stored f32
            std::vector<float> inv((size_t)(d->Hd / 2));
            for (size_t i = 0; i < inv.size(); ++i)
                inv[i] = (float)(1.0 / std::pow((double)c.rope_theta, (double)(2 * i) / (double)d->Hd));
            d->invFreq = Buffer(inv.size() * 4);
            checkHip(hipMemcpy(d->invFreq.p, inv.data(), inv.size() * 4, hipMemcpyHostToDevice), "upload inv_freq");
        }
        d->attn = Buffer((size_t)(d->QW * 2));
        d->o = Buffer((size_t)(H * 2));
        d->mlp = Buffer((size_t)(H * 2));
        d->hidden = Buffer((size_t)(F * 2));
        d->logits = Buffer((size_t)(d->V * 4));
        d->token = Buffer(4);
        d->position = Buffer(4);
        d->history = Buffer((size_t)(std::max(c.history_len, 1) * 4));
        d->argSlices = std::clamp<int64_t>((d->V + 4095) / 4096, 1, 256);  // as Kernels::Argmax slices a row
        d->argValues = Buffer((size_t)(d->argSlices * 4));
        d->argIndices = Buffer((size_t)(d->argSlices * 4));
        checkHip(hipMemsetAsync(d->token.p, 0, 4, d->stream), "memset");
        checkHip(hipMemsetAsync(d->position.p, 0, 4, d->stream), "memset");
        checkHip(hipMemsetAsync(d->history.p, 0xff, d->history.bytes, d->stream), "memset");
        d->enc = std::make_unique<KernelCommandEncoder>(*d->lib, d->stream, d->pool);
        d->build();
        *decoder = d.release();
    });
}

popcorn_status_t popcorn_decoder_destroy(popcorn_decoder_t decoder) {
    return guardedDec([&] {
        if (!decoder) return;
        (void)hipStreamSynchronize(decoder->stream);
        delete decoder;
    });
}

popcorn_status_t popcorn_decoder_randomize(popcorn_decoder_t d, uint64_t seed) {
    return guardedDec([&] {
        if (!d) throw Error::invalidArgument("decoder must not be NULL");
        uint64_t s = seed * 1000;
        auto fill = [&](Buffer &b, DataType t, float mean, float std) {
            d->enc->encode(*Kernels::FillNormal(b.p, t, b.bytes / (size_t)stride(t), ++s, mean, std));
        };
        fill(d->finalNorm, DataType::f32, 1.0f, 0.1f);
        if (d->q4) {
            // values: the bits of N(0, 1) f32 draws; scale ~ 0.02 / 4.6 (the spread
            // of a 4-bit value), bias ~ -7.5 scale: weights of order N(0, 0.02)
            for (QMat *m : {&d->qemb, &d->qqkv, &d->qo, &d->qg, &d->qu, &d->qd}) {
                fill(m->packed, DataType::f32, 0.0f, 1.0f);
                fill(m->scales, DataType::bf16, 0.0043f, 0.0005f);
                fill(m->biases, DataType::bf16, -0.032f, 0.003f);
            }
        } else {
            fill(d->embedding, DataType::bf16, 0.0f, 0.02f);
            fill(d->wqkv, DataType::bf16, 0.0f, 0.02f);
            fill(d->wo, DataType::bf16, 0.0f, 0.02f);
            fill(d->wg, DataType::bf16, 0.0f, 0.02f);
            fill(d->wu, DataType::bf16, 0.0f, 0.02f);
            fill(d->wd, DataType::bf16, 0.0f, 0.02f);
        }
        fill(d->norms, DataType::f32, 1.0f, 0.1f);
        if (d->headNorms.p) fill(d->headNorms, DataType::f32, 1.0f, 0.1f);
        fill(d->kcache, DataType::bf16, 0.0f, 1.0f);
        fill(d->vcache, DataType::bf16, 0.0f, 1.0f);
        checkHip(hipStreamSynchronize(d->stream), "sync");
    });
}

popcorn_status_t popcorn_decoder_tensor(popcorn_decoder_t d, const char *name, int32_t layer, popcorn_tensor_t *out) {
    return guardedDec([&] {
        if (!d || !name || !out) throw Error::invalidArgument("decoder, name and tensor must not be NULL");
        Tensor t;
        std::string n = name;
        if (d->quantizedView(n, 0, t) && n.rfind("embedding", 0) == 0) {
        } else if (n == "embedding") t = d->bf(d->embedding.p, {d->V, d->H});
        else if (n == "final_norm") t = Tensor(d->finalNorm.p, Shape({d->H}), DataType::f32);
        else if (n == "x") t = d->bf(d->x.p, {d->H});
        else if (n == "x2") t = d->bf(d->x2.p, {d->H});
        else if (n == "q") t = d->bf(d->qkv.p, {d->QW});
        else if (n == "qkv") t = d->bf(d->qkv.p, {d->QKV});
        else if (n == "inv_freq" && d->invFreq.p) t = Tensor(d->invFreq.p, Shape({d->Hd / 2}), DataType::f32);
        else if (n == "attn") t = d->bf(d->attn.p, {d->QW});
        else if (n == "o") t = d->bf(d->o.p, {d->H});
        else if (n == "mlp") t = d->bf(d->mlp.p, {d->H});
        else if (n == "hidden") t = d->bf(d->hidden.p, {d->F});
        else if (n == "logits") t = Tensor(d->logits.p, Shape({d->V}), DataType::f32);
        else if (n == "token") t = Tensor(d->token.p, Shape({1}), DataType::i32);
        else if (n == "position") t = Tensor(d->position.p, Shape({1}), DataType::i32);
        else if (n == "history") t = Tensor(d->history.p, Shape({std::max(d->cfg.history_len, 1)}), DataType::i32);
        else {
            if (layer < 0 || layer >= d->L) throw Error::invalidArgument("layer out of range");
            t = d->weight(name, layer);
        }
        std::memset(out, 0, sizeof(*out));
        out->data = t.data;
        out->dtype = (int32_t)t.dataType;
        out->rank = t.shape.rank();
        for (int i = 0; i < t.shape.rank(); ++i) out->shape[i] = t.shape[i];
    });
}

popcorn_status_t popcorn_decoder_reset(popcorn_decoder_t d, int32_t token, int32_t position) {
    return guardedDec([&] {
        if (!d) throw Error::invalidArgument("decoder must not be NULL");
        if (token < 0 || token >= d->V) throw Error::invalidArgument("token outside the vocabulary");
        if (position < 0 || position >= d->S) throw Error::invalidArgument("position outside the KV cache");
        checkHip(hipMemcpyAsync(d->token.p, &token, 4, hipMemcpyHostToDevice, d->stream), "write token");
        checkHip(hipMemcpyAsync(d->position.p, &position, 4, hipMemcpyHostToDevice, d->stream), "write position");
        checkHip(hipStreamSynchronize(d->stream), "sync");
        d->hostPos = position;
    });
}

popcorn_status_t popcorn_decoder_step(popcorn_decoder_t d, int32_t steps, int32_t use_graph) {
    return guardedDec([&] {
        if (!d) throw Error::invalidArgument("decoder must not be NULL");
        d->run(steps, use_graph != 0);
    });
}

popcorn_status_t popcorn_decoder_read(popcorn_decoder_t d, int32_t *token, int32_t *position) {
    return guardedDec([&] {
        if (!d) throw Error::invalidArgument("decoder must not be NULL");
        int32_t v[2] = {0, 0};
        checkHip(hipMemcpyAsync(&v[0], d->token.p, 4, hipMemcpyDeviceToHost, d->stream), "read token");
        checkHip(hipMemcpyAsync(&v[1], d->position.p, 4, hipMemcpyDeviceToHost, d->stream), "read position");
        checkHip(hipStreamSynchronize(d->stream), "sync");
        if (token) *token = v[0];
        if (position) *position = v[1];
        d->hostPos = v[1];
    });
}

popcorn_status_t popcorn_decoder_describe(popcorn_decoder_t d, char *buffer, size_t capacity, int32_t *dispatches) {
    return guardedDec([&] {
        if (!d) throw Error::invalidArgument("decoder must not be NULL");
        std::string s;
        for (size_t i = 0; i < d->names.size(); ++i) s += (i ? "," : "") + d->names[i];
        if (dispatches) *dispatches = (int32_t)d->names.size();
        if (buffer && capacity) {
            std::strncpy(buffer, s.c_str(), capacity - 1);
            buffer[capacity - 1] = '\0';
        }
    });
}

int64_t popcorn_decoder_step_bytes(popcorn_decoder_t d, int32_t position) { return d ? d->stepBytes(position) : 0; }

popcorn_status_t popcorn_decoder_time_kernel(popcorn_decoder_t d, const char *function_name, int32_t reps,
                                             float *mean_ms, int32_t *launches) {
    return guardedDec([&] {
        if (!d || !function_name || !mean_ms) throw Error::invalidArgument("decoder, name and mean_ms must not be NULL");
        if (reps <= 0) throw Error::invalidArgument("reps must be positive");
        int32_t per = 0;
        for (const std::string &n : d->names) per += (n == function_name) ? 1 : 0;
        if (per == 0) throw Error::kernelFunctionNotFound(std::string(function_name) + " (not dispatched by a decode step)");
        hipEvent_t a = nullptr, b = nullptr;
        checkHip(hipEventCreate(&a), "hipEventCreate");
        checkHip(hipEventCreate(&b), "hipEventCreate");
        struct Cleanup {
            popcorn_decoder_s *d;
            hipEvent_t a, b;
            ~Cleanup() {
                d->enc->setDispatchFilter("");
                (void)hipEventDestroy(a);
                (void)hipEventDestroy(b);
            }
        } cleanup{d, a, b};
        // the step's tail kernel advances the position and rewrites the
        // token; both are restored afterwards
        int32_t saved[2] = {0, 0};
        checkHip(hipMemcpyAsync(&saved[0], d->token.p, 4, hipMemcpyDeviceToHost, d->stream), "read token");
        checkHip(hipMemcpyAsync(&saved[1], d->position.p, 4, hipMemcpyDeviceToHost, d->stream), "read position");
        checkHip(hipStreamSynchronize(d->stream), "sync");
        struct Restore {
            popcorn_decoder_s *d;
            int32_t *v;
            ~Restore() {
                (void)hipStreamSynchronize(d->stream);
                (void)hipMemcpy(d->token.p, &v[0], 4, hipMemcpyHostToDevice);
                (void)hipMemcpy(d->position.p, &v[1], 4, hipMemcpyHostToDevice);
            }
        } restore{d, saved};
        d->enc->setDispatchFilter(function_name);
        d->encodeStep();  // warm: first launch of each
        // the filtered launches of `reps` steps captured as one graph and
        // replayed, so the timing holds GPU time only (no host walk of the
        // other dispatches between lone launches)
        hipGraph_t g = nullptr;
        hipGraphExec_t ge = nullptr;
        checkHip(hipStreamBeginCapture(d->stream, hipStreamCaptureModeThreadLocal), "hipStreamBeginCapture");
        try {
            for (int32_t r = 0; r < reps; ++r) d->encodeStep();
        } catch (...) {
            (void)hipStreamEndCapture(d->stream, &g);
            if (g) (void)hipGraphDestroy(g);
            throw;
        }
        checkHip(hipStreamEndCapture(d->stream, &g), "hipStreamEndCapture");
        struct GraphGuard {
            hipGraph_t &g;
            hipGraphExec_t &e;
            ~GraphGuard() {
                if (e) (void)hipGraphExecDestroy(e);
                if (g) (void)hipGraphDestroy(g);
            }
        } graphGuard{g, ge};
        checkHip(hipGraphInstantiate(&ge, g, nullptr, nullptr, 0), "hipGraphInstantiate");
        checkHip(hipGraphLaunch(ge, d->stream), "hipGraphLaunch");  // warm
        checkHip(hipEventRecord(a, d->stream), "hipEventRecord");
        checkHip(hipGraphLaunch(ge, d->stream), "hipGraphLaunch");
        checkHip(hipEventRecord(b, d->stream), "hipEventRecord");
        checkHip(hipEventSynchronize(b), "hipEventSynchronize");
        float ms = 0;
        checkHip(hipEventElapsedTime(&ms, a, b), "hipEventElapsedTime");
        *mean_ms = ms / (float)(per * reps);
        if (launches) *launches = per * reps;
    });
}

popcorn_status_t popcorn_decoder_time_kernel_in_step(popcorn_decoder_t d, const char *function_name, int32_t steps,
                                                     float *mean_ms, int32_t *launches) {
    return guardedDec([&] {
        if (!d || !function_name || !mean_ms) throw Error::invalidArgument("decoder, name and mean_ms must not be NULL");
        if (steps <= 0 || steps > 16) throw Error::invalidArgument("steps must be in 1..16");
        int32_t per = 0;
        for (const std::string &n : d->names) per += (n == function_name) ? 1 : 0;
        if (per == 0) throw Error::kernelFunctionNotFound(std::string(function_name) + " (not dispatched by a decode step)");
        if (d->hostPos < 0 || d->hostPos + steps > d->S)
            throw Error::tensorShapeMismatch("timed steps would leave the KV cache");
        // A stop event on every launch of the kernel and on every launch of
        // the kernels that come just before it in the step: each event takes
        // its launch's end of execution, so the kernel's time in the step is
        // end(kernel) - end(the launch before it) (its dispatch and its run,
        // as a kernel trace adds up to the step).
        std::set<std::string> before;
        const size_t perStep = d->names.size();
        for (size_t i = 0; i < perStep; ++i)
            if (d->names[(i + 1) % perStep] == function_name) before.insert(d->names[i]);
        size_t marked = 0;  // launches per step that carry an event
        for (const std::string &n : d->names) marked += (n == function_name || before.count(n)) ? 1 : 0;
        const size_t maxEvents = marked * (size_t)steps + 2;
        std::vector<hipEvent_t> ev(maxEvents, nullptr);
        std::vector<size_t> at(maxEvents, 0);
        std::vector<char> self(maxEvents, 0);
        struct Events {
            std::vector<hipEvent_t> &ev;
            popcorn_decoder_s *d;
            ~Events() {
                d->enc->setDispatchHook(nullptr);
                for (hipEvent_t e : ev)
                    if (e) (void)hipEventDestroy(e);
            }
        } guard{ev, d};
        for (hipEvent_t &e : ev) checkHip(hipEventCreateWithFlags(&e, hipEventDisableSystemFence), "hipEventCreate");
        size_t next = 0, dispatch = 0;
        KernelCommandEncoder::TimingHook hook = [&](const std::string &name) -> std::pair<hipEvent_t, hipEvent_t> {
            const size_t i = dispatch++;
            const bool isSelf = name == function_name;
            if ((!isSelf && !before.count(name)) || next >= maxEvents) return {nullptr, nullptr};
            at[next] = i;
            self[next] = isSelf;
            return {nullptr, ev[next++]};
        };
        // the stream waits (about 4 ms per step) while the host enqueues the
        // steps, so they then run back to back with no host gaps between
        // launches
        {
            const Function &hold = d->lib->function("hold_stream");
            uint64_t ticks = (uint64_t)steps * 400000u;
            void *args[] = {&ticks};
            checkHip(hipModuleLaunchKernel(hold.fn, 1, 1, 1, 64, 1, 1, 0, d->stream, args, nullptr), "launch hold_stream");
        }
        d->enc->setDispatchHook(&hook);
        d->run(steps, false);
        d->enc->setDispatchHook(nullptr);
        checkHip(hipStreamSynchronize(d->stream), "sync");
        double total = 0;
        int32_t timed = 0;
        for (size_t j = 1; j < next; ++j) {
            if (!self[j] || at[j] != at[j - 1] + 1) continue;
            float ms = 0;
            checkHip(hipEventElapsedTime(&ms, ev[j - 1], ev[j]), "hipEventElapsedTime");
            total += ms;
            ++timed;
        }
        *mean_ms = timed ? (float)(total / timed) : 0.0f;
        if (launches) *launches = timed;
    });
}

}  // extern "C"
