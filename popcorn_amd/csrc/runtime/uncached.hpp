// Uncached device memory (hipDeviceMallocUncached: every access goes to
// memory, past the per-XCD L2 caches, whatever the instruction's cache
// policy). Blocks of one launch that run on different XCDs exchange data
// through it, since those L2s are not coherent with each other. Such memory
// is never freed once a kernel has read it: a block given back goes to a
// process-wide pool keyed by device and size, and the next request of that
// size on that device reuses it.
#pragma once

#include <map>
#include <mutex>
#include <utility>
#include <vector>

#include "popcorn.hpp"

namespace popcorn {

class UncachedPool {
public:
    // A block of `bytes` on the current device: reused from the pool, or
    // newly allocated (-1003 when the allocation fails).
    static void *take(size_t bytes, int *devOut = nullptr) {
        int dev = 0;
        checkHip(hipGetDevice(&dev), "hipGetDevice");
        if (devOut) *devOut = dev;
        {
            std::lock_guard<std::mutex> g(mu());
            auto &pool = free_()[{dev, bytes}];
            if (!pool.empty()) {
                void *p = pool.back();
                pool.pop_back();
                return p;
            }
        }
        void *p = nullptr;
        if (hipExtMallocWithFlags(&p, bytes ? bytes : 1, hipDeviceMallocUncached) != hipSuccess) {
            (void)hipGetLastError();
            throw Error::tensorAllocationFailed(bytes);
        }
        std::lock_guard<std::mutex> g(mu());
        sizes()[p] = {dev, bytes};
        return p;
    }
    // Gives a block back to the pool (never to hipFree). False when `p` was
    // not taken from this pool.
    static bool give(void *p) {
        std::lock_guard<std::mutex> g(mu());
        auto it = sizes().find(p);
        if (it == sizes().end()) return false;
        free_()[it->second].push_back(p);
        return true;
    }

private:
    using Key = std::pair<int, size_t>;
    static std::mutex &mu() {
        static std::mutex m;
        return m;
    }
    static std::map<Key, std::vector<void *>> &free_() {
        static auto *pool = new std::map<Key, std::vector<void *>>();  // lives to process exit
        return *pool;
    }
    static std::map<void *, Key> &sizes() {
        static auto *s = new std::map<void *, Key>();
        return *s;
    }
};

}  // namespace popcorn
