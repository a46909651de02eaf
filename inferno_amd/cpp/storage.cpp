// storage.cpp -- CPUStorage, HIPStorage (include/inferno/core/storage.h).
//
// HIPStorage keeps a per-device cache of freed blocks, by size class: a
// training step frees and re-allocates the same activation and gradient sizes
// every step, and returning each block to the runtime (hipFreeAsync) costs
// ~0.1 ms of host time per call, more than the kernels of many ops.  Reuse is
// safe without any synchronisation because every tensor on a device is used
// in order on that device's library stream: work on a reused block is always
// enqueued after the previous owner's work.  A miss allocates with
// hipMallocAsync on that stream; if the device is out of memory the cache is
// released to the runtime and the allocation retried.
#include "inferno/core/storage.h"

#include <map>
#include <mutex>

#include "hipctx.h"

namespace Inferno {

namespace {

struct BlockCache {
    std::mutex mu;
    std::multimap<size_t, void*> free_blocks;  // size class -> block
    size_t held = 0;                           // bytes in free_blocks
};

BlockCache& cache_for(int device) {
    static std::mutex mu;
    static auto* caches = new std::vector<BlockCache*>();  // process lifetime: no teardown-order frees
    std::lock_guard<std::mutex> lk(mu);
    if ((size_t)device >= caches->size()) caches->resize((size_t)device + 1, nullptr);
    BlockCache*& c = (*caches)[(size_t)device];
    if (!c) c = new BlockCache();
    return *c;
}

// 512-byte granules up to 1 MiB, 1 MiB granules above (at most ~0.2% waste on
// the large activation buffers).
size_t size_class(size_t n) {
    const size_t g = n <= (size_t(1) << 20) ? 512 : (size_t(1) << 20);
    return (n + g - 1) / g * g;
}

void release_cache(BlockCache& c, int device) {
    hipStream_t s = detail::stream_for(device);
    for (auto& [sz, p] : c.free_blocks) (void)hipFreeAsync(p, s);
    c.free_blocks.clear();
    c.held = 0;
    (void)hipStreamSynchronize(s);
}

}  // namespace

CPUStorage::CPUStorage(size_t nbytes) : m_data(nbytes) {}

HIPStorage::HIPStorage(size_t nbytes, int device_index) : m_nbytes(nbytes), m_device(device_index) {
    if (nbytes == 0) return;
    const size_t cls = size_class(nbytes);
    BlockCache& c = cache_for(device_index);
    {
        std::lock_guard<std::mutex> lk(c.mu);
        auto it = c.free_blocks.find(cls);
        if (it != c.free_blocks.end()) {
            m_ptr = it->second;
            c.free_blocks.erase(it);
            c.held -= cls;
            return;
        }
    }
    // An error that an earlier HIP call left pending is raised here, named,
    // instead of being cleared with this allocation's own out-of-memory status.
    detail::hip_check(hipGetLastError(), "HIP error pending from an earlier call (before hipMallocAsync)");
    detail::DeviceGuard g(device_index);
    hipError_t e = hipMallocAsync(&m_ptr, cls, detail::stream_for(device_index));
    if (e == hipErrorOutOfMemory) {
        (void)hipGetLastError();  // this allocation's own failure: release the cache and retry once
        {
            std::lock_guard<std::mutex> lk(c.mu);
            release_cache(c, device_index);
        }
        e = hipMallocAsync(&m_ptr, cls, detail::stream_for(device_index));
    }
    detail::hip_check(e, "hipMallocAsync");
}

HIPStorage::~HIPStorage() {
    if (!m_ptr) return;
    BlockCache& c = cache_for(m_device);
    std::lock_guard<std::mutex> lk(c.mu);
    const size_t cls = size_class(m_nbytes);
    c.free_blocks.emplace(cls, m_ptr);
    c.held += cls;
}

std::shared_ptr<Storage> make_storage(size_t nbytes, const Device& device) {
    if (device.is_cpu()) return std::make_shared<CPUStorage>(nbytes);
    return std::make_shared<HIPStorage>(nbytes, device.index);
}

}  // namespace Inferno
