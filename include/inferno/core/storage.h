// storage.h -- raw byte buffers behind tensors.
//
// Storage / CPUStorage follow the reference (src/inferno/storage/storage.h:19-64,
// cpustorage.h:19-33).  HIPStorage replaces CUDAStorage (cudastorage.cpp:16-23):
// freed blocks go to a per-device cache and are handed to the next allocation
// of the same size class (every tensor on a device is used in order on that
// device's library stream, so reuse needs no synchronisation); a miss allocates
// with hipMallocAsync on that stream.  The reference pays a cudaMalloc per op
// output instead.  Allocation failures throw instead of being ignored.
#pragma once

#include <cstddef>
#include <memory>
#include <vector>

#include "inferno/core/device.h"

namespace Inferno {

class Storage {
public:
    virtual ~Storage() = default;
    virtual void* raw_ptr() = 0;
    virtual size_t nbytes() const = 0;
    virtual Device device() const = 0;
};

class CPUStorage final : public Storage {
public:
    explicit CPUStorage(size_t nbytes);
    void* raw_ptr() override { return m_data.data(); }
    size_t nbytes() const override { return m_data.size(); }
    Device device() const override { return Device::cpu(); }

private:
    std::vector<std::byte> m_data;
};

class HIPStorage final : public Storage {
public:
    HIPStorage(size_t nbytes, int device_index);
    ~HIPStorage() override;
    HIPStorage(const HIPStorage&) = delete;
    HIPStorage& operator=(const HIPStorage&) = delete;
    void* raw_ptr() override { return m_ptr; }
    size_t nbytes() const override { return m_nbytes; }
    Device device() const override { return Device::hip(m_device); }

private:
    void* m_ptr = nullptr;
    size_t m_nbytes = 0;
    int m_device = 0;
};

std::shared_ptr<Storage> make_storage(size_t nbytes, const Device& device);

}  // namespace Inferno
