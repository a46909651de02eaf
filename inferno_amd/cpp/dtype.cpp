#include "inferno/core/dtype.h"

#include <cstring>
#include <stdexcept>

namespace Inferno {

size_t dtype_size(DType dt) {
    switch (dt) {
        case DType::Float32: return 4;
        case DType::Float64: return 8;
        case DType::Int32: return 4;
        case DType::Int8: return 1;
        case DType::Bool: return 1;
        case DType::BFloat16: return 2;
        default: throw std::invalid_argument("dtype_size: invalid dtype");
    }
}

const char* dtype_name(DType dt) {
    switch (dt) {
        case DType::Float32: return "Float32";
        case DType::Float64: return "Float64";
        case DType::Int32: return "Int32";
        case DType::Int8: return "Int8";
        case DType::Bool: return "Bool";
        case DType::BFloat16: return "BFloat16";
        default: return "Invalid";
    }
}

bool is_floating(DType dt) { return dt == DType::Float32 || dt == DType::Float64 || dt == DType::BFloat16; }

bfloat16::bfloat16(float f) {
    uint32_t b;
    std::memcpy(&b, &f, 4);
    if ((b & 0x7F800000u) == 0x7F800000u && (b & 0x007FFFFFu)) {
        bits = (uint16_t)((b >> 16) | 0x40u);
        return;
    }
    b += 0x7FFFu + ((b >> 16) & 1u);
    bits = (uint16_t)(b >> 16);
}

bfloat16::operator float() const {
    const uint32_t b = (uint32_t)bits << 16;
    float f;
    std::memcpy(&f, &b, 4);
    return f;
}

}  // namespace Inferno
