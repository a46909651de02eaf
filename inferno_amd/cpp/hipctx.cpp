#include "hipctx.h"

#include <cstdint>
#include <mutex>
#include <string>
#include <vector>

#include "inferno_hip.h"

namespace Inferno::detail {

namespace {
std::mutex g_mu;
std::vector<hipStream_t> g_streams;
}  // namespace

void hip_check(hipError_t e, const char* what) {
    if (e != hipSuccess) throw Error(std::string(what) + ": " + hipGetErrorString(e));
}

void status_check(int status, const char* what) {
    if (status == INF_OK) return;
    const std::string detail = inf_last_error_detail();
    throw Error(std::string(what) + ": " + inf_status_string(status) + (detail.empty() ? "" : " [" + detail + "]"));
}

DeviceGuard::DeviceGuard(int device) {
    hip_check(hipGetDevice(&m_prev), "hipGetDevice");
    if (m_prev != device) hip_check(hipSetDevice(device), "hipSetDevice");
}

DeviceGuard::~DeviceGuard() {
    int cur = -1;
    if (hipGetDevice(&cur) == hipSuccess && cur != m_prev && m_prev >= 0) (void)hipSetDevice(m_prev);
}

hipStream_t stream_for(int device) {
    std::lock_guard<std::mutex> lk(g_mu);
    if (device < 0) throw Error("stream_for: negative device index");
    if ((size_t)device >= g_streams.size()) g_streams.resize((size_t)device + 1, nullptr);
    if (!g_streams[(size_t)device]) {
        DeviceGuard g(device);
        hipStream_t s = nullptr;
        hip_check(hipStreamCreateWithFlags(&s, hipStreamNonBlocking), "hipStreamCreateWithFlags");
        hipMemPool_t pool = nullptr;
        if (hipDeviceGetDefaultMemPool(&pool, device) == hipSuccess && pool) {
            uint64_t keep = UINT64_MAX;
            (void)hipMemPoolSetAttribute(pool, hipMemPoolAttrReleaseThreshold, &keep);
        }
        g_streams[(size_t)device] = s;
    }
    return g_streams[(size_t)device];
}

}  // namespace Inferno::detail
