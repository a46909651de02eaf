// dtype.h -- element types of Inferno tensors.
//
// Keeps the reference's enumerator order (include/inferno/core/dtype.h:17-26):
// checkpoints store static_cast<uint32_t>(dtype) (src/inferno/checkpoint/
// checkpoint.cpp:54), so BFloat16 is appended after Invalid instead of being
// inserted.
#pragma once

#include <cstddef>
#include <cstdint>

namespace Inferno {

enum class DType { Float32, Float64, Int32, Int8, Bool, Invalid, BFloat16 };

// Bytes per element; throws std::invalid_argument for DType::Invalid.
// (The reference's dtype_size throws for Int8 too, tensorimpl.cpp:321-329; here it is 1.)
size_t dtype_size(DType dt);
const char* dtype_name(DType dt);
bool is_floating(DType dt);

// bfloat16 storage type: the upper half of an IEEE fp32, rounded to nearest even.
struct bfloat16 {
    uint16_t bits = 0;
    bfloat16() = default;
    explicit bfloat16(float f);
    explicit operator float() const;
};

}  // namespace Inferno
