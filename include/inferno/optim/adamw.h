// adamw.h -- AdamW over a parameter list (include/inferno/optim/adamw.h,
// src/inferno/optim/adamw.cpp of the reference): same defaults, bias
// corrections 1 - beta^step in float, decoupled weight decay added to the
// update, state created as zeros on the first step of each parameter,
// parameters without a gradient skipped.  Moments are fp32 (the reference
// keeps them in the parameter's dtype; identical for Float32 parameters).
#pragma once
#include <unordered_map>
#include <vector>
#include "inferno/core/tensor.h"

namespace Inferno {

class OptimizerAdamW {
public:
    OptimizerAdamW(std::vector<Tensor*> parameters, float lr = 3e-4f, float beta1 = 0.9f, float beta2 = 0.95f,
                   float eps = 1e-8f, float weight_decay = 0.1f)
        : m_parameters(std::move(parameters)),
          m_lr(lr),
          m_beta1(beta1),
          m_beta2(beta2),
          m_eps(eps),
          m_weight_decay(weight_decay),
          m_step(0) {}
    void step();
    void zero_grad();
    size_t step_count() const { return m_step; }

private:
    struct AdamWState {
        Tensor m;
        Tensor v;
        bool initialized = false;
    };
    std::vector<Tensor*> m_parameters;
    std::unordered_map<Tensor*, AdamWState> m_state;
    float m_lr;
    float m_beta1;
    float m_beta2;
    float m_eps;
    float m_weight_decay;
    size_t m_step;
};

}  // namespace Inferno
