// storage.cpp -- CPUStorage, HIPStorage (include/inferno/core/storage.h).
#include "inferno/core/storage.h"

#include "hipctx.h"

namespace Inferno {

CPUStorage::CPUStorage(size_t nbytes) : m_data(nbytes) {}

HIPStorage::HIPStorage(size_t nbytes, int device_index) : m_nbytes(nbytes), m_device(device_index) {
    if (nbytes == 0) return;
    detail::DeviceGuard g(device_index);
    detail::hip_check(hipMallocAsync(&m_ptr, nbytes, detail::stream_for(device_index)), "hipMallocAsync");
}

HIPStorage::~HIPStorage() {
    if (!m_ptr) return;
    // Stream-ordered free: work already queued on the stream that reads this
    // buffer completes first.  Errors at process teardown are ignored.
    int prev = -1;
    if (hipGetDevice(&prev) != hipSuccess) return;
    if (prev != m_device) (void)hipSetDevice(m_device);
    (void)hipFreeAsync(m_ptr, detail::stream_for(m_device));
    if (prev != m_device) (void)hipSetDevice(prev);
}

std::shared_ptr<Storage> make_storage(size_t nbytes, const Device& device) {
    if (device.is_cpu()) return std::make_shared<CPUStorage>(nbytes);
    return std::make_shared<HIPStorage>(nbytes, device.index);
}

}  // namespace Inferno
