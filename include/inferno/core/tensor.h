// tensor.h -- the Tensor value type (a shared handle to a TensorImpl).
//
// Same surface as the reference's Tensor (include/inferno/core/tensor.h:52-224)
// for everything the attention path touches: construction, device transfer,
// shape / stride / offset views over shared Storage, grad access, backward,
// item(), and the scalar operators.  Errors throw Inferno::Error (the reference
// logs and calls exit(1), which a caller cannot recover from).
#pragma once

#include <cstring>
#include <initializer_list>
#include <memory>
#include <stdexcept>
#include <string>
#include <type_traits>
#include <vector>

#include "inferno/core/device.h"
#include "inferno/core/dtype.h"

namespace Inferno {

class TensorImpl;
class Storage;

struct Error : std::runtime_error {
    using std::runtime_error::runtime_error;
};

class Tensor {
public:
    Tensor() = default;
    Tensor(DType dtype, std::vector<size_t> shape, std::string name, Device device, bool requires_grad = false);
    Tensor(DType dtype, std::initializer_list<size_t> shape, std::string name, Device device,
           bool requires_grad = false);

    // From host data (converted element-wise to `dtype`), then moved to `device`.
    template <typename T>
    Tensor(DType dtype, const std::vector<T>& data, std::vector<size_t> shape, std::string name,
           Device device = Device::cpu(), bool requires_grad = false) {
        init_from_host(dtype, data.data(), data.size(), host_kind<T>(), std::move(shape), std::move(name), device,
                       requires_grad);
    }
    template <typename T>
    Tensor(DType dtype, const std::vector<T>& data, std::initializer_list<size_t> shape, std::string name,
           Device device = Device::cpu(), bool requires_grad = false)
        : Tensor(dtype, data, std::vector<size_t>(shape), std::move(name), device, requires_grad) {}

    const Device& device() const;
    Tensor to(const Device& dst) const;

    Tensor operator+(const Tensor& other) const;
    Tensor operator*(const Tensor& other) const;

    DType dtype() const;
    std::shared_ptr<Storage>& data() const;
    std::shared_ptr<Tensor>& grad() const;
    Tensor Getgrad() const;
    std::vector<size_t>& shape() const;
    std::vector<size_t>& strides() const;
    size_t& offset() const;
    std::string name() const;
    size_t ndim() const;
    bool requires_grad() const;
    void set_requires_grad(bool flag);
    size_t size() const;   // bytes of the elements the view covers (numel * dtype_size)
    size_t numel() const;
    bool is_contiguous() const;
    bool defined() const { return static_cast<bool>(m_impl); }
    void* data_ptr() const;  // address of element 0 of the view

    static std::vector<size_t> calculate_strides(const std::vector<size_t>& shape);
    static Tensor ones_like(const Tensor& t);
    static Tensor zeros_like(const Tensor& t);
    static Tensor ones(const std::vector<size_t>& shape, DType dtype, Device device, const std::string& name = "ones");
    static Tensor zeros(const std::vector<size_t>& shape, DType dtype, Device device, const std::string& name = "zeros");
    static Tensor full(const std::vector<size_t>& shape, double value, DType dtype, Device device,
                       const std::string& name = "full");

    Tensor transpose(int dima, int dimb) const;
    // Inclusive `end`, as the reference's slice (src/inferno/core/ops.cpp:897-900).
    Tensor slice(int axis, size_t start, size_t end, size_t step = 1) const;
    Tensor reshape(const std::vector<size_t>& newshape) const;
    // Zero-copy split of dimension `dim` into `sizes` (their product must equal
    // shape()[dim]); valid for any strides.  No reference counterpart: it lets
    // [B, T, C] slices be viewed as [B, T, H, D] without the reference's
    // .contiguous() copies (InfernoApp/main.cpp:721-728).
    Tensor unflatten(int dim, const std::vector<size_t>& sizes) const;
    Tensor contiguous() const;

    // Seeds the root with ones (src/inferno/gradengine/engine.cpp:59) ...
    void backward() const;
    // ... or with an explicit upstream gradient of the root's shape (no reference
    // counterpart: the reference injects one through (root * g).backward()).
    void backward(const Tensor& gradient) const;

    double item_double_impl() const;
    int64_t item_int64_impl() const;
    template <typename T>
    T item() const {
        if constexpr (std::is_integral_v<T>)
            return static_cast<T>(item_int64_impl());
        else
            return static_cast<T>(item_double_impl());
    }
    // Copies the view out to host memory in row-major order, converted to double.
    std::vector<double> to_host_double() const;
    std::vector<float> to_host_float() const;

private:
    enum class HostKind { F32, F64, I32, I64, U8, I8, BF16 };
    template <typename T>
    static constexpr HostKind host_kind() {
        if constexpr (std::is_same_v<T, float>) return HostKind::F32;
        else if constexpr (std::is_same_v<T, double>) return HostKind::F64;
        else if constexpr (std::is_same_v<T, int32_t>) return HostKind::I32;
        else if constexpr (std::is_same_v<T, int64_t>) return HostKind::I64;
        else if constexpr (std::is_same_v<T, uint8_t> || std::is_same_v<T, bool>) return HostKind::U8;
        else if constexpr (std::is_same_v<T, int8_t>) return HostKind::I8;
        else if constexpr (std::is_same_v<T, bfloat16>) return HostKind::BF16;
        else static_assert(sizeof(T) == 0, "unsupported host element type");
    }
    void init_from_host(DType dtype, const void* data, size_t count, HostKind kind, std::vector<size_t> shape,
                        std::string name, Device device, bool requires_grad);

    friend std::shared_ptr<TensorImpl> GetImpl(const Tensor& t);
    friend void SetImpl(Tensor& t, std::shared_ptr<TensorImpl> impl);
    std::shared_ptr<TensorImpl> m_impl;
};

std::shared_ptr<TensorImpl> GetImpl(const Tensor& t);
void SetImpl(Tensor& t, std::shared_ptr<TensorImpl> impl);

// Element-wise ops (same shape, or one side a single element).
Tensor add(const Tensor& A, const Tensor& B);
Tensor multiply(const Tensor& A, const Tensor& B);

// A one-element tensor of `like`'s dtype and device holding `value`.
Tensor scalar_like(const Tensor& like, double value);

template <typename T>
    requires std::is_arithmetic_v<T>
Tensor operator*(const Tensor& A, T other) {
    return multiply(A, scalar_like(A, static_cast<double>(other)));
}
template <typename T>
    requires std::is_arithmetic_v<T>
Tensor operator*(T other, const Tensor& A) {
    return multiply(scalar_like(A, static_cast<double>(other)), A);
}

}  // namespace Inferno
