// linear.h -- y = x W + b with W [in, out], b [out] (include/inferno/modules/linear.h,
// linear.cpp of the reference).  Initialised like the reference: Xavier-uniform
// in +-sqrt(6 / (in + out)) for both W and b (linear.cpp:9-46).
#pragma once
#include "inferno/modules/module.h"

namespace Inferno {

class Linear : public Module {
public:
    Linear(size_t in_features, size_t out_features, Device device = Device::cpu(), DType dtype = DType::Float32);
    Tensor forward(const Tensor& input);
    Tensor forward(Tensor& input) override { return forward(static_cast<const Tensor&>(input)); }
    Tensor operator()(Tensor& input) { return forward(input); }

    Tensor m_weights;
    Tensor m_biases;

private:
    size_t m_in_features;
    size_t m_out_features;
};

}  // namespace Inferno
