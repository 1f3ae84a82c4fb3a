// The device scratch of the allocation-free entry point
// (popcorn_flash_decoding_no_alloc): one file-scope array per GPU, part of
// this library's device image, so a call needs no hipMalloc. Its device
// address is looked up once per device with hipGetSymbolAddress and kept;
// host code uses only that address (the array's name in host code is a
// host-side stand-in, not device memory). The array lives until the process
// ends. Calls that overlap on one GPU share it and race.
#include <hip/hip_runtime.h>

#include <map>
#include <mutex>

#include "popcorn.hpp"

namespace {

constexpr size_t kScratchBytes = POPCORN_NO_ALLOC_SCRATCH_BYTES;

__device__ __align__(256) unsigned char scratch[kScratchBytes];

}  // namespace

namespace popcorn {

// The device address of this GPU's copy of the array (the current device's).
void *staticScratch(size_t *bytes) {
    static std::mutex mu;
    static std::map<int, void *> byDevice;
    int dev = 0;
    checkHip(hipGetDevice(&dev), "hipGetDevice");
    std::lock_guard<std::mutex> g(mu);
    auto it = byDevice.find(dev);
    if (it == byDevice.end()) {
        void *ptr = nullptr;
        checkHip(hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)), "hipGetSymbolAddress(scratch)");
        if (!ptr) throw Error(POPCORN_ERR_GPU_INTERNAL, "hipGetSymbolAddress returned no address for the scratch array");
        it = byDevice.emplace(dev, ptr).first;
    }
    if (bytes) *bytes = kScratchBytes;
    return it->second;
}

}  // namespace popcorn
