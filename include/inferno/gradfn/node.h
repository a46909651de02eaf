// node.h -- autograd graph nodes (the reference's Node, src/inferno/gradfn/node.h:23-45).
//
// A node keeps what its backward needs, implements backward() (read the
// upstream gradient with Engine::grad_in, compute under NoGradGuard, pass
// results to each input's grad_edge with Engine::accumulate), release() (drop
// saved tensors after the pass) and get_inputs() (the tensors whose edges the
// engine follows to order the graph).
#pragma once

#include <memory>
#include <string>
#include <vector>

#include "inferno/core/tensor.h"

namespace Inferno {

class TensorImpl;

class Node {
public:
    virtual ~Node() = default;
    virtual void backward() = 0;
    virtual void release() {}
    virtual void get_inputs(std::vector<Tensor>& out) const = 0;
    const std::string& name() const { return m_name; }
    void set_name(std::string n) { m_name = std::move(n); }

private:
    std::string m_name;
};

// Sink of a leaf that requires grad: sums incoming gradients into leaf.grad()
// (accumulategrad.cpp:17-31).
class AccumulateGrad final : public Node {
public:
    explicit AccumulateGrad(std::weak_ptr<TensorImpl> leaf);
    void backward() override;
    void get_inputs(std::vector<Tensor>&) const override {}

private:
    std::weak_ptr<TensorImpl> m_leaf;
};

// y = a * b (same shape or one side scalar): da = g * b, db = g * a (multiplybackward.cpp:34-57).
class MultiplyBackward final : public Node {
public:
    MultiplyBackward(const Tensor& a, const Tensor& b);
    void backward() override;
    void release() override;
    void get_inputs(std::vector<Tensor>& out) const override;

private:
    Tensor m_a, m_b;
};

// y = a + b: da = g, db = g (reduced to one element for a scalar side).
class AddBackward final : public Node {
public:
    AddBackward(const Tensor& a, const Tensor& b);
    void backward() override;
    void release() override;
    void get_inputs(std::vector<Tensor>& out) const override;

private:
    Tensor m_a, m_b;
};

// View nodes: the gradient of a view is the inverse view of the upstream gradient.
class TransposeBackward final : public Node {
public:
    TransposeBackward(const Tensor& a, int dima, int dimb);
    void backward() override;
    void release() override;
    void get_inputs(std::vector<Tensor>& out) const override;

private:
    Tensor m_a;
    int m_dima, m_dimb;
};

class ReshapeBackward final : public Node {
public:
    explicit ReshapeBackward(const Tensor& a);
    void backward() override;
    void release() override;
    void get_inputs(std::vector<Tensor>& out) const override;

private:
    Tensor m_a;
    std::vector<size_t> m_shape;
};

class ContiguousBackward final : public Node {
public:
    explicit ContiguousBackward(const Tensor& a);
    void backward() override;
    void release() override;
    void get_inputs(std::vector<Tensor>& out) const override;

private:
    Tensor m_a;
};

class SliceBackward final : public Node {
public:
    SliceBackward(const Tensor& a, int axis, size_t start, size_t step);
    void backward() override;
    void release() override;
    void get_inputs(std::vector<Tensor>& out) const override;

private:
    Tensor m_a;
    int m_axis;
    size_t m_start, m_step;
};

}  // namespace Inferno
