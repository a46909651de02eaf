// tensorimpl.h -- shape / strides / offset view over shared Storage, plus the
// autograd links (grad, grad_fn, the leaf's AccumulateGrad).  Mirrors the role
// of the reference's TensorImpl (src/inferno/core/tensorimpl.h:35-136,
// grad_edge at tensorimpl.cpp:389-470).
#pragma once

#include <memory>
#include <string>
#include <vector>

#include "inferno/core/device.h"
#include "inferno/core/dtype.h"
#include "inferno/core/storage.h"

namespace Inferno {

class Node;
class Tensor;

class TensorImpl : public std::enable_shared_from_this<TensorImpl> {
public:
    // Fresh contiguous tensor with uninitialised storage on `device`.
    TensorImpl(DType dtype, std::vector<size_t> shape, std::string name, Device device, bool requires_grad);
    // View over existing storage.
    TensorImpl(std::shared_ptr<Storage> storage, DType dtype, std::vector<size_t> shape,
               std::vector<size_t> strides, size_t offset, std::string name, Device device, bool requires_grad);

    DType dtype() const { return m_dtype; }
    std::vector<size_t>& shape() { return m_shape; }
    std::vector<size_t>& strides() { return m_strides; }
    size_t& offset() { return m_offset; }
    std::shared_ptr<Storage>& storage() { return m_storage; }
    const Device& device() const { return m_device; }
    const std::string& name() const { return m_name; }
    bool requires_grad() const { return m_requires_grad; }
    void set_requires_grad(bool f) { m_requires_grad = f; }
    std::shared_ptr<Tensor>& grad() { return m_grad; }
    std::shared_ptr<Node>& gradfn() { return m_gradfn; }

    size_t numel() const;
    bool is_contiguous() const;
    void* data_ptr() const;

    // The node that receives this tensor's gradient: its grad_fn, else (for a
    // leaf that requires grad) its AccumulateGrad, else null.
    std::shared_ptr<Node> grad_edge();

private:
    DType m_dtype;
    std::vector<size_t> m_shape;
    std::vector<size_t> m_strides;
    size_t m_offset = 0;
    std::shared_ptr<Storage> m_storage;
    Device m_device;
    std::string m_name;
    bool m_requires_grad = false;
    std::shared_ptr<Tensor> m_grad;
    std::shared_ptr<Node> m_gradfn;
    std::shared_ptr<Node> m_accumulate;
};

// A view of `base`'s storage (ops.cpp:824-848): shares storage, no grad link.
Tensor make_view(const Tensor& base, std::vector<size_t> shape, std::vector<size_t> strides, size_t offset,
                 const std::string& name);

}  // namespace Inferno
