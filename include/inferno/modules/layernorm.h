// layernorm.h -- LayerNorm over the last dimension with learnable gamma (ones)
// and beta (zeros), fp32 parameters (include/inferno/modules/layernorm.h,
// layernorm.cpp of the reference).
#pragma once
#include "inferno/modules/module.h"

namespace Inferno {

class LayerNorm : public Module {
public:
    LayerNorm(size_t normalized_dim, float eps = 1e-5f, Device device = Device::cpu(), DType dtype = DType::Float32);
    Tensor forward(Tensor& input) override;
    Tensor operator()(Tensor& input) { return forward(input); }
    // Parameter access (no reference counterpart; the reference's are private).
    Tensor& gamma() { return m_gamma; }
    Tensor& beta() { return m_beta; }
    float eps() const { return m_eps; }

private:
    Tensor m_beta;
    Tensor m_gamma;
    size_t m_dim;
    float m_eps;
};

}  // namespace Inferno
