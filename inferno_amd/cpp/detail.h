// detail.h -- helpers shared by the Tensor-layer translation units (internal).
#pragma once

#include <cstdint>
#include <cstring>
#include <string>
#include <vector>

#include "hipctx.h"
#include "inferno/core/tensor.h"
#include "inferno/core/tensorimpl.h"
#include "inferno_hip.h"

namespace Inferno::detail {

inline double load_elem(const void* p, DType dt) {
    switch (dt) {
        case DType::Float32: { float v; std::memcpy(&v, p, 4); return v; }
        case DType::Float64: { double v; std::memcpy(&v, p, 8); return v; }
        case DType::Int32: { int32_t v; std::memcpy(&v, p, 4); return v; }
        case DType::Int8: { int8_t v; std::memcpy(&v, p, 1); return v; }
        case DType::Bool: { uint8_t v; std::memcpy(&v, p, 1); return v ? 1.0 : 0.0; }
        case DType::BFloat16: { bfloat16 v; std::memcpy(&v.bits, p, 2); return (float)v; }
        default: throw Error("load_elem: invalid dtype");
    }
}

inline void store_elem(void* p, DType dt, double x) {
    switch (dt) {
        case DType::Float32: { float v = (float)x; std::memcpy(p, &v, 4); return; }
        case DType::Float64: { std::memcpy(p, &x, 8); return; }
        case DType::Int32: { int32_t v = (int32_t)x; std::memcpy(p, &v, 4); return; }
        case DType::Int8: { int8_t v = (int8_t)x; std::memcpy(p, &v, 1); return; }
        case DType::Bool: { uint8_t v = x != 0.0; std::memcpy(p, &v, 1); return; }
        case DType::BFloat16: { bfloat16 v((float)x); std::memcpy(p, &v.bits, 2); return; }
        default: throw Error("store_elem: invalid dtype");
    }
}

// Element-by-element strided copy on the host (element strides).
inline void copy_strided_host(const char* src, const std::vector<size_t>& sst, char* dst,
                              const std::vector<size_t>& dst_strides, const std::vector<size_t>& shape,
                              size_t esz) {
    size_t n = 1;
    for (size_t s : shape) n *= s;
    const int nd = (int)shape.size();
    std::vector<size_t> idx(shape.size(), 0);
    for (size_t lin = 0; lin < n; ++lin) {
        size_t so = 0, doff = 0;
        for (int d = 0; d < nd; ++d) {
            so += idx[d] * sst[d];
            doff += idx[d] * dst_strides[d];
        }
        std::memcpy(dst + doff * esz, src + so * esz, esz);
        for (int d = nd - 1; d >= 0; --d) {
            if (++idx[d] < shape[d]) break;
            idx[d] = 0;
        }
    }
}

inline inf_dtype inf_dt(DType dt, const char* what) {
    if (dt == DType::Float32) return INF_F32;
    if (dt == DType::BFloat16) return INF_BF16;
    throw Error(std::string(what) + ": HIP path supports Float32 and BFloat16, got " + dtype_name(dt));
}

inline hipStream_t stream_of(const Tensor& t) { return stream_for(t.device().index); }

inline void same_device(const Tensor& a, const Tensor& b, const char* what) {
    if (a.device() != b.device()) throw Error(std::string(what) + ": tensors are on different devices");
}

// A dense copy of any view on its own device (fresh allocation, no grad link).
Tensor dense_copy(const Tensor& src);

inline std::vector<int64_t> to_i64(const std::vector<size_t>& v) { return {v.begin(), v.end()}; }

}  // namespace Inferno::detail
