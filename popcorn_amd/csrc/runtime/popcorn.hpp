// C++ host runtime of the gfx950 build: the reference's Swift API surface
// (Sources/Popcorn/{Tensor,Kernel,KernelCommandEncoder,KernelLibrary,
// KernelResources,ScratchSpec,PopcornError}.swift) restated over HIP.
//
//   Swift (reference)                      here
//   Tensor{MTLBuffer, shape, dataType}     Tensor{device pointer, Shape, DataType}
//   KernelLibrary (metallib, PSO cache)    KernelLibrary (gfx950 code objects,
//                                          hipFunction_t cache)
//   KernelCommandEncoder (compute encoder, KernelCommandEncoder over one
//     barriers from a hazard map)            in-order hipStream_t
//   KernelScratchAllocator                 KernelScratchAllocator
//   PopcornError                           popcorn::Error (same codes)
//   Kernel / DispatchKernel                Kernel / DispatchKernel
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <functional>
#include <map>
#include <memory>
#include <mutex>
#include <string>
#include <vector>

#include "popcorn_hip.h"

namespace popcorn {

// ---- errors (PopcornError.swift:23-42) -----------------------------------

class Error : public std::exception {
public:
    Error(int32_t code, std::string message) : code_(code), message_(std::move(message)) {}
    int32_t code() const { return code_; }
    const char *what() const noexcept override { return message_.c_str(); }

    static Error kernelFunctionNotFound(const std::string &name);
    static Error tensorShapeMismatch(const std::string &message);
    static Error tensorInvalidRank(int expected, int actual);
    static Error tensorInvalidAxis(int axis, int rank);
    static Error unsupportedDataTypeCombination(const std::string &message);
    static Error tensorAllocationFailed(size_t bytes);
    static Error invalidArgument(const std::string &message);
    static Error fromHip(hipError_t err, const std::string &where);

private:
    int32_t code_;
    std::string message_;
};

void checkHip(hipError_t err, const char *where);

// ---- tensors (Tensor.swift) ---------------------------------------------

enum class DataType : int32_t {
    u8 = POPCORN_DTYPE_U8,
    u16 = POPCORN_DTYPE_U16,
    u32 = POPCORN_DTYPE_U32,
    u64 = POPCORN_DTYPE_U64,
    i8 = POPCORN_DTYPE_I8,
    i16 = POPCORN_DTYPE_I16,
    i32 = POPCORN_DTYPE_I32,
    i64 = POPCORN_DTYPE_I64,
    f32 = POPCORN_DTYPE_F32,
    f16 = POPCORN_DTYPE_F16,
    bf16 = POPCORN_DTYPE_BF16,
};

int stride(DataType t);
const char *name(DataType t);  // "f32", "bf16", ...

struct Shape {
    std::vector<int64_t> dims;
    Shape() = default;
    Shape(std::initializer_list<int64_t> d) : dims(d) {}
    explicit Shape(std::vector<int64_t> d) : dims(std::move(d)) {}
    int rank() const { return (int)dims.size(); }
    int64_t elementCount() const;
    int64_t operator[](int i) const { return dims[(size_t)i]; }
    bool operator==(const Shape &o) const { return dims == o.dims; }
    bool operator!=(const Shape &o) const { return dims != o.dims; }
    std::string str() const;
};

struct Tensor {
    void *data = nullptr;
    Shape shape;
    DataType dataType = DataType::f32;

    Tensor() = default;
    Tensor(void *d, Shape s, DataType t = DataType::f32) : data(d), shape(std::move(s)), dataType(t) {}
    static Tensor fromC(const popcorn_tensor_t &t);
    size_t byteCount() const { return (size_t)shape.elementCount() * (size_t)stride(dataType); }
};

enum Access : uint8_t { kRead = 1, kWrite = 2, kReadWrite = 3 };

struct Binding {
    Tensor tensor;
    uint8_t access;
};

// ScratchSpec.swift:10-26
struct ScratchSpec {
    std::vector<int64_t> shape;
    DataType dataType;
    size_t byteCount() const;
};

// ---- scratch (KernelResources.swift:5-36) --------------------------------

struct KernelTemporaryBuffer {
    void *buffer = nullptr;
    size_t length = 0;
    bool wasReused = false;
};

class KernelScratchAllocator {
public:
    virtual ~KernelScratchAllocator() = default;
    virtual KernelTemporaryBuffer borrowTemporaryBuffer(size_t length) = 0;
    virtual void releaseTemporaryBuffer(const KernelTemporaryBuffer &) {}
};

// Best-fit pool over hipMalloc'd buffers for one stream (the GemmaCLI
// ScratchPool, ScratchPool.swift:42-71).
class ScratchPool : public KernelScratchAllocator {
public:
    ~ScratchPool() override;
    KernelTemporaryBuffer borrowTemporaryBuffer(size_t length) override;
    void releaseTemporaryBuffer(const KernelTemporaryBuffer &t) override;
    size_t bytes() const;

private:
    mutable std::mutex mu_;
    std::multimap<size_t, void *> free_;
    std::map<void *, size_t> all_;
    size_t bytes_ = 0;
};

// Adapts the C allocator struct.
class CScratchAllocator : public KernelScratchAllocator {
public:
    explicit CScratchAllocator(popcorn_scratch_allocator_t a) : a_(a) {}
    KernelTemporaryBuffer borrowTemporaryBuffer(size_t length) override;
    void releaseTemporaryBuffer(const KernelTemporaryBuffer &t) override;

private:
    popcorn_scratch_allocator_t a_;
};

// ---- kernel library (KernelLibrary.swift) ---------------------------------

struct FunctionAttributes {
    int maxThreadsPerBlock = 1024;
    int waveSize = 64;
    int staticLds = 0;
    int numVgprs = 0;
    int numSgprs = 0;
    int privateBytes = 0;
};

// A kernel's explicit parameters as its code object's metadata lists them
// (code_object.cpp): device pointers and by-value constants blocks.
struct KernelArg {
    bool pointer = false;
    uint32_t size = 0;
    uint32_t offset = 0;
};

struct KernelLayout {
    std::vector<KernelArg> args;
    uint32_t kernargBytes = 0;
    uint32_t maxThreads = 0;
    uint32_t staticLds = 0;
    std::string str() const;
    // Throws invalidArgument unless the launch binds exactly `nbuffers`
    // pointers then one block of each of `constantSizes`, as the kernel takes.
    void check(const std::string &name, size_t nbuffers, const std::vector<size_t> &constantSizes) const;
};

// Every kernel's layout in a code object (ELF or clang offload bundle);
// throws invalidArgument for a malformed file.
std::map<std::string, KernelLayout> readKernelLayouts(const std::vector<uint8_t> &file);
std::map<std::string, KernelLayout> readKernelLayouts(const std::string &path);

struct Function {
    hipFunction_t fn = nullptr;
    std::string name;
    FunctionAttributes attrs;
    const KernelLayout *layout = nullptr;  // null when the code object's metadata was not readable
};

class KernelLibrary {
public:
    // `path`: a code-object file or a directory of *.hsaco; "" = the kernels
    // shipped next to the shared library.
    explicit KernelLibrary(const std::string &path);
    ~KernelLibrary();
    KernelLibrary(const KernelLibrary &) = delete;
    KernelLibrary &operator=(const KernelLibrary &) = delete;

    const Function &function(const std::string &name);  // throws -1006
    size_t cachedCount() const;
    int device() const { return device_; }
    int computeUnits() const { return cus_; }
    static std::string defaultPath();

private:
    std::vector<hipModule_t> modules_;
    std::map<std::string, KernelLayout> layouts_;
    std::map<std::string, std::unique_ptr<Function>> cache_;
    mutable std::mutex mu_;
    int device_ = 0;
    int cus_ = 256;
};

// ---- kernels (Kernel.swift) ----------------------------------------------

class KernelCommandEncoder;

struct DispatchSize {
    dim3 grid;
    dim3 block;
    size_t dynamicLds = 0;
};

class Kernel {
public:
    virtual ~Kernel() = default;
    virtual std::vector<Binding> tensors() const = 0;
    virtual void encode(KernelCommandEncoder &encoder) const = 0;
    // Function names this kernel dispatches, in order ("a,b").
    virtual std::string describe() const = 0;
};

class DispatchKernel : public Kernel {
public:
    virtual std::string functionName() const = 0;
    // Each constants block as bytes, passed by value after the tensors.
    virtual std::vector<std::vector<uint8_t>> constants() const = 0;
    virtual DispatchSize dispatchSize(const FunctionAttributes &attrs) const = 0;
    void encode(KernelCommandEncoder &encoder) const override;
    std::string describe() const override { return functionName(); }
};

template <typename T>
std::vector<uint8_t> bytesOf(const T &v) {
    const uint8_t *p = reinterpret_cast<const uint8_t *>(&v);
    return std::vector<uint8_t>(p, p + sizeof(T));
}

// ---- command encoder (KernelCommandEncoder.swift) -------------------------

class KernelCommandEncoder {
public:
    KernelCommandEncoder(KernelLibrary &library, hipStream_t stream, KernelScratchAllocator &scratch);

    void encode(const Kernel &kernel) { kernel.encode(*this); }
    // The result-builder form: encode { k1; k2; ... } in order.
    void encode(const std::vector<const Kernel *> &kernels) {
        for (const Kernel *k : kernels) k->encode(*this);
    }
    void dispatch(const DispatchKernel &kernel);
    void barrier();

    template <typename F>
    void withTemporaryTensor(const ScratchSpec &spec, F &&body) {
        KernelTemporaryBuffer t = scratch_.borrowTemporaryBuffer(spec.byteCount());
        ++scratchBorrows_;
        if (t.wasReused) accessByBuffer_[t.buffer] |= kWrite;
        struct Release {
            KernelScratchAllocator &s;
            KernelTemporaryBuffer t;
            ~Release() { s.releaseTemporaryBuffer(t); }
        } release{scratch_, t};
        body(Tensor(t.buffer, Shape(spec.shape), spec.dataType));
    }

    KernelLibrary &library() { return library_; }
    hipStream_t stream() const { return stream_; }
    popcorn_encoder_stats_t stats() const;
    // When set, dispatch() launches only kernels with this function name and
    // skips the rest (used to time one kernel of a composite sequence).
    void setDispatchFilter(const std::string &functionName) { filter_ = functionName; }
    // When set, called with each launch's function name; the events it
    // returns (start, stop; either may be null) are attached to that launch
    // (hipExtModuleLaunchKernel), a pair of nulls launches it plainly.
    using TimingHook = std::function<std::pair<hipEvent_t, hipEvent_t>(const std::string &)>;
    void setDispatchHook(const TimingHook *hook) { hook_ = hook; }


private:
    bool needsBarrier(const std::vector<Binding> &bindings) const;
    void recordAccesses(const std::vector<Binding> &bindings);

    KernelLibrary &library_;
    hipStream_t stream_;
    KernelScratchAllocator &scratch_;
    std::map<const void *, uint8_t> accessByBuffer_;
    int64_t dispatches_ = 0, hazards_ = 0, scratchBorrows_ = 0;
    std::string filter_;
    const TimingHook *hook_ = nullptr;
};

// ---- Kernels.* descriptors --------------------------------------------------

struct AttentionMask {
    uint32_t kind = 0;  // 0 causal, 1 causal + sliding window, 2 bidirectional
    int32_t window = -1;
};

// AffineQuantizedTensor (AffineQuantizedTensor.swift:19-84): packed u32
// values, scales and optional biases [..., out, in / groupSize], logical shape
// [..., out, in]; MLX-style little-endian packing (the only packing the
// reference defines, AffineQuantizationFormat.swift:24-30).
struct AffineQuantizedTensor {
    Tensor packedValues, scales, biases;
    bool hasBiases = false;
    Shape shape;
    int bits = 4, groupSize = 64;
    int64_t outFeatures() const { return shape[shape.rank() - 2]; }
    int64_t inFeatures() const { return shape[shape.rank() - 1]; }
    // The checks of AffineQuantizedTensor.init (AffineQuantizedTensor.swift:22-54).
    void validate() const;
};

namespace Kernels {

enum class AttentionPath { plain = POPCORN_ATTENTION_PLAIN, tiled = POPCORN_ATTENTION_TILED, decoding = POPCORN_ATTENTION_DECODING };

std::unique_ptr<Kernel> FlashAttention(const Tensor &q, const Tensor &k, const Tensor &v, const Tensor &out,
                                       float scale, AttentionMask mask);
std::unique_ptr<Kernel> FlashAttention(const Tensor &q, const Tensor &k, const Tensor &v, const Tensor &out,
                                       int64_t batch, int64_t queryHeads, int64_t kvHeads, int64_t queryLen,
                                       int64_t keyLen, int64_t headDim, float scale, AttentionMask mask,
                                       int64_t keyCapacity = 0, const Tensor *position = nullptr);
AttentionPath route(int64_t queryLen, int64_t headDim, DataType qType);

std::unique_ptr<Kernel> Matmul(const Tensor &a, const Tensor &b, const Tensor &c, bool transposeB);
std::unique_ptr<Kernel> Matmul(const Tensor &a, const Tensor &b, const Tensor &c, int64_t m, int64_t k, int64_t n,
                               bool transposeB);

std::unique_ptr<Kernel> RMSNorm(const Tensor &x, const Tensor *weight, const Tensor &out, int axis, float eps,
                                bool addOneToWeight);
std::unique_ptr<Kernel> RMSNorm(const Tensor &x, const Tensor *weight, const Tensor &out, int64_t rowCount,
                                int64_t hiddenSize, float eps, bool addOneToWeight);

std::unique_ptr<Kernel> KVCacheWrite(const Tensor &source, const Tensor &cache, int64_t offset);
std::unique_ptr<Kernel> KVCacheWrite(const Tensor &source, const Tensor &cache, int64_t batch, int64_t kvHeads,
                                     int64_t newLen, int64_t maxLen, int64_t headDim, int64_t offset,
                                     const Tensor *position = nullptr);

std::unique_ptr<Kernel> GeluTanh(const Tensor &x, const Tensor &out);
std::unique_ptr<Kernel> Mul(const Tensor &a, const Tensor &b, const Tensor &out);
std::unique_ptr<Kernel> Add(const Tensor &a, const Tensor &b, const Tensor &out);
std::unique_ptr<Kernel> ScalarMul(const Tensor &x, float scalar, const Tensor &out);

std::unique_ptr<Kernel> RopeBuildCosSin(const Tensor &positions, const Tensor &invFreq, const Tensor &cosOut,
                                        const Tensor &sinOut, int64_t seqLen, int64_t halfHeadDim, float scaling);
std::unique_ptr<Kernel> RopeBuildCosSin(const Tensor &positions, const Tensor &invFreq, const Tensor &cosOut,
                                        const Tensor &sinOut, float scaling);
std::unique_ptr<Kernel> RopeApply(const Tensor &x, const Tensor &cosT, const Tensor &sinT, const Tensor &out,
                                  int64_t batch, int64_t seqLen, int64_t headCount, int64_t headDim);
std::unique_ptr<Kernel> RopeApply(const Tensor &x, const Tensor &cosT, const Tensor &sinT, const Tensor &out);
std::unique_ptr<Kernel> Transpose12(const Tensor &src, const Tensor &out, int64_t d0, int64_t d1, int64_t d2, int64_t d3);
std::unique_ptr<Kernel> Transpose12(const Tensor &src, const Tensor &out);

std::unique_ptr<Kernel> GatedMLP(const Tensor &x, const Tensor *normWeight, const Tensor &wGate, const Tensor &wUp,
                                 const Tensor &wDown, const Tensor &out, float eps, bool addOneToWeight,
                                 const Tensor *hidden = nullptr);

// The residual form: x = round(xIn + round(RMSNorm(delta) * wPost)) is
// stored to xOut (the attention block's post-norm and residual Add), then
// the gated MLP runs on x.
std::unique_ptr<Kernel> GatedMLPResidual(const Tensor &xIn, const Tensor &delta, const Tensor &wPost, const Tensor &xOut,
                                         const Tensor *normWeight, const Tensor &wGate, const Tensor &wUp,
                                         const Tensor &wDown, const Tensor &out, float eps, bool addOneToWeight,
                                         const Tensor *hidden = nullptr);

// The gated MLP with block-affine 4-bit weights (bf16 activations, an f32
// pre-FFN norm weight); with delta/wPost/xOut the residual form as above.
std::unique_ptr<Kernel> GatedMLPResidual(const Tensor &xIn, const Tensor *delta, const Tensor *wPost, const Tensor *xOut,
                                         const Tensor &normWeight, const AffineQuantizedTensor &wGate,
                                         const AffineQuantizedTensor &wUp, const AffineQuantizedTensor &wDown, const Tensor &out,
                                         float eps, const Tensor *hidden = nullptr);

// Decode matvec with the decoder-layer glue folded in (DecodeMatvecConstants).
struct DecodeMatvecArgs {
    const Tensor *x = nullptr;       // [K] the vector, or the residual stream with delta
    const Tensor *delta = nullptr;   // [K] sub-layer output: x = x + RMSNorm(delta) * wPost
    const Tensor *wPost = nullptr;   // [K] f32
    const Tensor *xOut = nullptr;    // [K] receives the new residual stream
    const Tensor *wPre = nullptr;    // [K] f32: multiply RMSNorm(x) * wPre
    const Tensor *weight = nullptr;  // [N, K]
    const Tensor *out = nullptr;     // [N], or [qRows] with the caches
    const Tensor *kCache = nullptr;  // [1?, Nkv, Smax, Hd]: rows past qRows scatter here...
    const Tensor *vCache = nullptr;  // ...and here, at row position[0]
    const Tensor *position = nullptr;
    int64_t qRows = 0;
    float eps = 1e-6f;
    const AffineQuantizedTensor *qweight = nullptr;  // in place of weight: block-affine 4-bit [N, K]
};
std::unique_ptr<Kernel> DecodeMatvec(const DecodeMatvecArgs &args);

// The attention block of one decode token (DecodeAttentionConstants): raw
// projections in, per-head norms and RoPE, the new K/V row written to the
// caches at position[0], split-KV attention over keys 0..position[0].
struct DecodeAttentionArgs {
    const Tensor *qkv = nullptr;      // [B, (Nq + 2 Nkv) * Hd]
    const Tensor *kCache = nullptr;   // [B, Nkv, S, Hd]
    const Tensor *vCache = nullptr;
    const Tensor *out = nullptr;      // [B, Nq, 1, Hd]
    const Tensor *position = nullptr; // i32 [1]
    const Tensor *qNorm = nullptr;    // f32 [Hd] or absent
    const Tensor *kNorm = nullptr;    // f32 [Hd] or absent
    const Tensor *invFreq = nullptr;  // f32 [Hd/2] or absent (no RoPE)
    bool vNorm = false;
    int64_t queryHeads = 0, kvHeads = 0;
    float eps = 1e-6f, scale = 1.0f, ropeScaling = 1.0f;
    AttentionMask mask{0, -1};
};
std::unique_ptr<Kernel> DecodeAttention(const DecodeAttentionArgs &args);

std::unique_ptr<Kernel> EmbeddingGather(const Tensor &ids, const Tensor &table, const Tensor &out);
// Matmul(_:_:into:) with a quantized RHS (Matmul.swift:99-130) and
// EmbeddingGather(ids:table:into:) with a quantized table (EmbeddingGather.swift:45-88).
std::unique_ptr<Kernel> Matmul(const Tensor &a, const AffineQuantizedTensor &b, const Tensor &c);
std::unique_ptr<Kernel> EmbeddingGather(const Tensor &ids, const AffineQuantizedTensor &table, const Tensor &out);
std::unique_ptr<Kernel> Argmax(const Tensor &x, const Tensor &indices);

std::unique_ptr<Kernel> Custom(const std::string &functionName, std::vector<Binding> tensors,
                               std::vector<std::vector<uint8_t>> constants, dim3 grid, dim3 block);
// The same with `dynamicLds` bytes of dynamic LDS per block.
std::unique_ptr<Kernel> Custom(const std::string &functionName, std::vector<Binding> tensors,
                               std::vector<std::vector<uint8_t>> constants, dim3 grid, dim3 block, size_t dynamicLds);

std::unique_ptr<Kernel> FillNormal(void *data, DataType dtype, uint64_t count, uint64_t seed, float mean,
                                   float stddev);

// FlashAttention's split-KV kernels with the partials in the static scratch:
// enqueues on `stream`, allocates no device memory (popcorn_flash_decoding_no_alloc).
void FlashDecodingNoAlloc(KernelLibrary &library, hipStream_t stream, const Tensor &q, const Tensor &k, const Tensor &v,
                          const Tensor &out, int64_t batch, int64_t queryHeads, int64_t kvHeads, int64_t queryLen,
                          int64_t keyLen, int64_t headDim, float scale, AttentionMask mask, int64_t keyCapacity,
                          const Tensor *position);

}  // namespace Kernels

// The current device's copy of the static scratch array (static_scratch.hip)
// and its size in bytes; looked up once per device.
void *staticScratch(size_t *bytes);

// The exchange of the tiled prefill attention's merged pairs on one stream
// (flash_attention_tiled.hip, pairTiles 2), in uncached device memory that
// is never freed: `data` holds the published partial O and (m, l) rows
// (grown on demand; a grown-out block stays reserved for graphs captured
// with it), `flags` the abort word and one ready flag per split tile, zeroed
// once at creation.
struct PairExchange {
    static constexpr size_t kFlags = 4097;  // abort word + 4096 tiles
    void *data = nullptr;
    size_t dataBytes = 0;
    uint64_t *flags = nullptr;
    int dev = 0;
};
// The exchange of `stream` on the current device with at least `dataBytes`
// of data.
PairExchange &pairExchange(hipStream_t stream, size_t dataBytes);
// After `stream` has drained (or, with stream == nullptr and allStreams,
// every stream of the current device): throws -1019 when a merged pair's
// wait gave up since the last check, clearing that exchange's flags first.
void checkPairExchange(hipStream_t stream, bool allStreams = false);

// Thread-local message of the last failure reported through the C ABI.
void setLastError(const std::string &message);
const char *lastError();

}  // namespace popcorn
