// Runtime core: errors, tensors, scratch, kernel library, command encoder.
#include <dirent.h>
#include <dlfcn.h>

#include <algorithm>
#include <cstdlib>
#include <cstring>
#include <sstream>

#include "popcorn.hpp"

// hip/hip_ext.h's C entry point (its header's C++ part needs the HIP
// compiler): a module launch whose dispatch packet carries start and stop
// events.
extern "C" hipError_t hipExtModuleLaunchKernel(hipFunction_t f, uint32_t globalWorkSizeX, uint32_t globalWorkSizeY,
                                               uint32_t globalWorkSizeZ, uint32_t localWorkSizeX,
                                               uint32_t localWorkSizeY, uint32_t localWorkSizeZ, size_t sharedMemBytes,
                                               hipStream_t hStream, void **kernelParams, void **extra,
                                               hipEvent_t startEvent, hipEvent_t stopEvent, uint32_t flags);

namespace popcorn {

// ---- errors ------------------------------------------------------------------

Error Error::kernelFunctionNotFound(const std::string &name) {
    return Error(POPCORN_ERR_KERNEL_FUNCTION_NOT_FOUND, "kernel function was not found in the library: " + name);
}
Error Error::tensorShapeMismatch(const std::string &message) {
    return Error(POPCORN_ERR_TENSOR_SHAPE_MISMATCH, message);
}
Error Error::tensorInvalidRank(int expected, int actual) {
    return Error(POPCORN_ERR_TENSOR_INVALID_RANK,
                 "Tensor rank mismatch: expected " + std::to_string(expected) + ", got " + std::to_string(actual) + ".");
}
Error Error::tensorInvalidAxis(int axis, int rank) {
    return Error(POPCORN_ERR_TENSOR_INVALID_AXIS,
                 "Tensor axis " + std::to_string(axis) + " is invalid for rank " + std::to_string(rank) + ".");
}
Error Error::unsupportedDataTypeCombination(const std::string &message) {
    return Error(POPCORN_ERR_UNSUPPORTED_DATA_TYPE_COMBINATION, message);
}
Error Error::tensorAllocationFailed(size_t bytes) {
    return Error(POPCORN_ERR_TENSOR_ALLOCATION_FAILED, "Failed to allocate a tensor buffer of " + std::to_string(bytes) + " bytes.");
}
Error Error::invalidArgument(const std::string &message) { return Error(POPCORN_ERR_INVALID_ARGUMENT, message); }

Error Error::fromHip(hipError_t err, const std::string &where) {
    return Error(popcorn_status_from_hip_error((int)err), where + ": " + hipGetErrorString(err));
}

void checkHip(hipError_t err, const char *where) {
    if (err != hipSuccess) throw Error::fromHip(err, where);
}

static thread_local std::string tl_last_error;
void setLastError(const std::string &message) { tl_last_error = message; }
const char *lastError() { return tl_last_error.c_str(); }

// ---- tensors -----------------------------------------------------------------

int stride(DataType t) { return popcorn_dtype_stride((int32_t)t); }

const char *name(DataType t) {
    switch (t) {
    case DataType::u8: return "u8";
    case DataType::u16: return "u16";
    case DataType::u32: return "u32";
    case DataType::u64: return "u64";
    case DataType::i8: return "i8";
    case DataType::i16: return "i16";
    case DataType::i32: return "i32";
    case DataType::i64: return "i64";
    case DataType::f32: return "f32";
    case DataType::f16: return "f16";
    case DataType::bf16: return "bf16";
    }
    return "?";
}

int64_t Shape::elementCount() const {
    int64_t n = 1;
    for (int64_t d : dims) n *= d;
    return n;
}

std::string Shape::str() const {
    std::ostringstream s;
    s << "[";
    for (size_t i = 0; i < dims.size(); ++i) s << (i ? ", " : "") << dims[i];
    s << "]";
    return s.str();
}

Tensor Tensor::fromC(const popcorn_tensor_t &t) {
    if (t.rank < 0 || t.rank > POPCORN_MAX_RANK) throw Error::invalidArgument("tensor rank out of range");
    if (popcorn_dtype_stride(t.dtype) == 0) throw Error::invalidArgument("unknown tensor dtype tag " + std::to_string(t.dtype));
    std::vector<int64_t> dims(t.shape, t.shape + t.rank);
    for (int64_t d : dims)
        if (d < 0) throw Error::invalidArgument("negative tensor dimension");
    return Tensor(t.data, Shape(std::move(dims)), (DataType)t.dtype);
}

size_t ScratchSpec::byteCount() const {
    int64_t n = 1;
    for (int64_t d : shape) n *= d;
    return std::max<size_t>(1, (size_t)n * (size_t)stride(dataType));
}

// ---- scratch -------------------------------------------------------------------

ScratchPool::~ScratchPool() {
    for (auto &kv : all_) (void)hipFree(kv.first);
}

KernelTemporaryBuffer ScratchPool::borrowTemporaryBuffer(size_t length) {
    std::lock_guard<std::mutex> g(mu_);
    length = std::max<size_t>(length, 1);
    auto it = free_.lower_bound(length);
    if (it != free_.end()) {
        KernelTemporaryBuffer t{it->second, it->first, true};
        free_.erase(it);
        return t;
    }
    size_t rounded = (length + 255) & ~(size_t)255;
    void *p = nullptr;
    if (hipMalloc(&p, rounded) != hipSuccess) {
        (void)hipGetLastError();
        throw Error::tensorAllocationFailed(rounded);
    }
    all_[p] = rounded;
    bytes_ += rounded;
    return KernelTemporaryBuffer{p, rounded, false};
}

void ScratchPool::releaseTemporaryBuffer(const KernelTemporaryBuffer &t) {
    std::lock_guard<std::mutex> g(mu_);
    auto it = all_.find(t.buffer);
    if (it != all_.end()) free_.emplace(it->second, t.buffer);
}

size_t ScratchPool::bytes() const {
    std::lock_guard<std::mutex> g(mu_);
    return bytes_;
}

KernelTemporaryBuffer CScratchAllocator::borrowTemporaryBuffer(size_t length) {
    void *p = nullptr;
    int32_t reused = 0;
    popcorn_status_t st = a_.borrow(a_.context, std::max<size_t>(length, 1), &p, &reused);
    if (st != POPCORN_OK || !p) throw Error(st ? st : POPCORN_ERR_TENSOR_ALLOCATION_FAILED, "scratch allocator failed to borrow " + std::to_string(length) + " bytes");
    return KernelTemporaryBuffer{p, length, reused != 0};
}

void CScratchAllocator::releaseTemporaryBuffer(const KernelTemporaryBuffer &t) {
    if (a_.release) a_.release(a_.context, t.buffer);
}

// ---- kernel library ----------------------------------------------------------------

// POPCORN_KERNEL_DIR, else the kernels/ directory next to this library.
std::string KernelLibrary::defaultPath() {
    if (const char *env = std::getenv("POPCORN_KERNEL_DIR"); env && *env) return env;
    Dl_info info;
    if (dladdr((void *)&popcorn_last_error_message, &info) && info.dli_fname) {
        std::string so = info.dli_fname;
        size_t slash = so.find_last_of('/');
        std::string dir = slash == std::string::npos ? "." : so.substr(0, slash);
        return dir + "/kernels";
    }
    return "kernels";
}

static bool endsWith(const std::string &s, const std::string &suffix) {
    return s.size() >= suffix.size() && s.compare(s.size() - suffix.size(), suffix.size(), suffix) == 0;
}

KernelLibrary::KernelLibrary(const std::string &pathIn) {
    std::string path = pathIn.empty() ? defaultPath() : pathIn;
    checkHip(hipGetDevice(&device_), "hipGetDevice");
    hipDeviceProp_t prop;
    checkHip(hipGetDeviceProperties(&prop, device_), "hipGetDeviceProperties");
    cus_ = prop.multiProcessorCount > 0 ? prop.multiProcessorCount : 256;

    std::vector<std::string> files;
    if (DIR *d = opendir(path.c_str())) {
        while (dirent *e = readdir(d)) {
            std::string n = e->d_name;
            if (endsWith(n, ".hsaco")) files.push_back(path + "/" + n);
        }
        closedir(d);
        std::sort(files.begin(), files.end());
    } else {
        files.push_back(path);
    }
    if (files.empty()) throw Error(POPCORN_ERR_KERNEL_FUNCTION_NOT_FOUND, "no code objects in " + path);
    for (const std::string &f : files) {
        // parameter layouts for launch checks; a code object whose metadata
        // cannot be read still loads, its launches go unchecked
        try {
            for (auto &kv : readKernelLayouts(f)) layouts_.emplace(kv.first, std::move(kv.second));
        } catch (const Error &) {
        }
        hipModule_t m = nullptr;
        hipError_t err = hipModuleLoad(&m, f.c_str());
        if (err != hipSuccess) {
            for (hipModule_t mm : modules_) (void)hipModuleUnload(mm);
            modules_.clear();
            throw Error::fromHip(err, "hipModuleLoad(" + f + ")");
        }
        modules_.push_back(m);
    }
}

KernelLibrary::~KernelLibrary() {
    for (hipModule_t m : modules_) (void)hipModuleUnload(m);
}

const Function &KernelLibrary::function(const std::string &fname) {
    std::lock_guard<std::mutex> g(mu_);
    auto it = cache_.find(fname);
    if (it != cache_.end()) return *it->second;
    for (hipModule_t m : modules_) {
        hipFunction_t fn = nullptr;
        if (hipModuleGetFunction(&fn, m, fname.c_str()) == hipSuccess && fn) {
            auto f = std::make_unique<Function>();
            f->fn = fn;
            f->name = fname;
            int v = 0;
            if (hipFuncGetAttribute(&v, HIP_FUNC_ATTRIBUTE_MAX_THREADS_PER_BLOCK, fn) == hipSuccess) f->attrs.maxThreadsPerBlock = v;
            if (hipFuncGetAttribute(&v, HIP_FUNC_ATTRIBUTE_SHARED_SIZE_BYTES, fn) == hipSuccess) f->attrs.staticLds = v;
            if (hipFuncGetAttribute(&v, HIP_FUNC_ATTRIBUTE_NUM_REGS, fn) == hipSuccess) f->attrs.numVgprs = v;
            if (hipFuncGetAttribute(&v, HIP_FUNC_ATTRIBUTE_LOCAL_SIZE_BYTES, fn) == hipSuccess) f->attrs.privateBytes = v;
            (void)hipGetLastError();
            f->attrs.waveSize = 64;
            if (auto it = layouts_.find(fname); it != layouts_.end()) f->layout = &it->second;
            const Function &ref = *f;
            cache_[fname] = std::move(f);
            return ref;
        }
        (void)hipGetLastError();  // a miss in one module is not an error
    }
    throw Error::kernelFunctionNotFound(fname);
}

size_t KernelLibrary::cachedCount() const {
    std::lock_guard<std::mutex> g(mu_);
    return cache_.size();
}

// ---- command encoder -------------------------------------------------------------

void DispatchKernel::encode(KernelCommandEncoder &encoder) const { encoder.dispatch(*this); }

KernelCommandEncoder::KernelCommandEncoder(KernelLibrary &library, hipStream_t stream, KernelScratchAllocator &scratch)
    : library_(library), stream_(stream), scratch_(scratch) {}

// KernelCommandEncoder.swift:155-162: a binding conflicts with an earlier
// access when either side writes.
bool KernelCommandEncoder::needsBarrier(const std::vector<Binding> &bindings) const {
    for (const Binding &b : bindings) {
        auto it = accessByBuffer_.find(b.tensor.data);
        if (it == accessByBuffer_.end()) continue;
        if ((it->second & kWrite) && (b.access & kReadWrite)) return true;
        if ((b.access & kWrite) && (it->second & kReadWrite)) return true;
    }
    return false;
}

void KernelCommandEncoder::recordAccesses(const std::vector<Binding> &bindings) {
    for (const Binding &b : bindings) accessByBuffer_[b.tensor.data] |= b.access;
}

void KernelCommandEncoder::barrier() { accessByBuffer_.clear(); }

void KernelCommandEncoder::dispatch(const DispatchKernel &kernel) {
    if (!filter_.empty() && kernel.functionName() != filter_) return;
    const std::vector<Binding> bindings = kernel.tensors();
    if (needsBarrier(bindings)) {
        // One in-order stream: the previous dispatch's writes are visible to
        // this one without an explicit barrier; count the hazard only.
        ++hazards_;
        barrier();
    }
    const Function &fn = library_.function(kernel.functionName());
    const DispatchSize ds = kernel.dispatchSize(fn.attrs);
    if (ds.grid.x == 0 || ds.grid.y == 0 || ds.grid.z == 0) {
        recordAccesses(bindings);
        return;  // empty launch
    }
    if ((int)(ds.block.x * ds.block.y * ds.block.z) > fn.attrs.maxThreadsPerBlock)
        throw Error::invalidArgument("block of " + std::to_string(ds.block.x * ds.block.y * ds.block.z) +
                                     " threads exceeds the limit of " + kernel.functionName());
    const std::vector<std::vector<uint8_t>> consts = kernel.constants();
    if (fn.layout) {
        std::vector<size_t> sizes;
        for (const auto &c : consts) sizes.push_back(c.size());
        fn.layout->check(kernel.functionName(), bindings.size(), sizes);
    }
    std::vector<void *> ptrs(bindings.size());
    std::vector<void *> params;
    params.reserve(bindings.size() + consts.size());
    for (size_t i = 0; i < bindings.size(); ++i) {
        ptrs[i] = bindings[i].tensor.data;
        params.push_back(&ptrs[i]);
    }
    for (const auto &c : consts) params.push_back(const_cast<uint8_t *>(c.data()));
    std::pair<hipEvent_t, hipEvent_t> timing{nullptr, nullptr};
    if (hook_) timing = (*hook_)(kernel.functionName());
    hipError_t err;
    if (timing.first || timing.second) {
        // hipExtModuleLaunchKernel takes the global size in threads as
        // 32-bit values: a grid whose thread count does not fit is refused
        const uint64_t gx = (uint64_t)ds.grid.x * ds.block.x, gy = (uint64_t)ds.grid.y * ds.block.y,
                       gz = (uint64_t)ds.grid.z * ds.block.z;
        if (gx > UINT32_MAX || gy > UINT32_MAX || gz > UINT32_MAX)
            throw Error::invalidArgument("timed launch of " + kernel.functionName() +
                                         ": the grid holds more than 2^32 - 1 threads in one dimension");
        err = hipExtModuleLaunchKernel(fn.fn, ds.grid.x * ds.block.x, ds.grid.y * ds.block.y, ds.grid.z * ds.block.z,
                                       ds.block.x, ds.block.y, ds.block.z, ds.dynamicLds, stream_, params.data(),
                                       nullptr, timing.first, timing.second, 0);
    } else {
        err = hipModuleLaunchKernel(fn.fn, ds.grid.x, ds.grid.y, ds.grid.z, ds.block.x, ds.block.y, ds.block.z,
                                    (unsigned)ds.dynamicLds, stream_, params.data(), nullptr);
    }
    if (err != hipSuccess) throw Error::fromHip(err, "launch " + kernel.functionName());
    ++dispatches_;
    recordAccesses(bindings);
}

popcorn_encoder_stats_t KernelCommandEncoder::stats() const {
    popcorn_encoder_stats_t s;
    s.dispatches = dispatches_;
    s.hazards = hazards_;
    s.scratch_borrows = scratchBorrows_;
    return s;
}

}  // namespace popcorn
