// softmax.h -- Softmax over one axis with its backward node.
//
// Same signature and output conventions as the reference (softmax.h:9,
// softmax.cpp:22-79): the result is a new tensor with requires_grad = true, and
// a SoftmaxBackward is attached when grad is enabled and A requires grad.
// HIP tensors run inf_softmax_fwd / inf_softmax_bwd (one wave per row).
#pragma once

#include "inferno/core/tensor.h"
#include "inferno/gradfn/node.h"

namespace Inferno {

Tensor Softmax(Tensor& A, int axis = -1);

// dx = y * (g - sum_axis(g * y)) (softmaxbackward.h:64-131, softmaxbackward.cpp:36-128)
class SoftmaxBackward final : public Node {
public:
    SoftmaxBackward(const Tensor& A, const Tensor& out, int axis);
    void backward() override;
    void release() override;
    void get_inputs(std::vector<Tensor>& out) const override;

private:
    Tensor m_A, m_out;
    int m_axis;
};

}  // namespace Inferno
