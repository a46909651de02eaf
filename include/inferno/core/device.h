// device.h -- where a tensor's storage lives.
//
// Mirrors the reference's Device (include/inferno/core/device.h:6-51) with the
// CUDA case replaced by HIP: Device::hip(i) is GPU i of this process
// (hipSetDevice is applied before every allocation, copy and launch, which the
// reference never does with its index).
#pragma once

namespace Inferno {

enum class DeviceType { CPU, HIP };

class Device {
public:
    DeviceType m_type;
    int index;

    Device(DeviceType t = DeviceType::CPU, int idx = 0) : m_type(t), index(idx) {}

    bool operator==(const Device& o) const { return m_type == o.m_type && index == o.index; }
    bool operator!=(const Device& o) const { return !(*this == o); }

    static Device cpu() { return Device(DeviceType::CPU, 0); }
    static Device hip(int idx = 0) { return Device(DeviceType::HIP, idx); }

    bool is_cpu() const { return m_type == DeviceType::CPU; }
    bool is_hip() const { return m_type == DeviceType::HIP; }
};

}  // namespace Inferno
