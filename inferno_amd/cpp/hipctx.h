// hipctx.h -- per-device HIP stream and error helpers of the Tensor layer (internal).
#pragma once

#include <hip/hip_runtime_api.h>

#include "inferno/core/tensor.h"

namespace Inferno::detail {

// The library's stream on `device`: created on first use with
// hipStreamNonBlocking at the default priority; its memory pool keeps freed
// blocks cached (release threshold = max), so steady-state allocations are
// pool hits.  All Tensor-layer work on a device is ordered on this stream.
hipStream_t stream_for(int device);

// Throws Inferno::Error naming `what` when a HIP call fails.
void hip_check(hipError_t e, const char* what);
// Throws Inferno::Error naming `what` when a C-ABI call returns non-zero.
void status_check(int status, const char* what);

class DeviceGuard {
public:
    explicit DeviceGuard(int device);
    ~DeviceGuard();
    DeviceGuard(const DeviceGuard&) = delete;
    DeviceGuard& operator=(const DeviceGuard&) = delete;

private:
    int m_prev = -1;
};

}  // namespace Inferno::detail
