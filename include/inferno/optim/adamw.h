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
        : params_(std::move(parameters)), lr_(lr), beta1_(beta1), beta2_(beta2), eps_(eps), decay_(weight_decay) {}
    void step();
    void zero_grad();
    size_t step_count() const { return steps_; }

private:
    // fp32 first and second moments of one parameter, allocated on its first step
    struct Moments {
        Tensor first;
        Tensor second;
    };
    std::vector<Tensor*> params_;
    std::unordered_map<Tensor*, Moments> moments_;
    float lr_, beta1_, beta2_, eps_, decay_;
    size_t steps_ = 0;
};

}  // namespace Inferno
