// crossentropyloss.h -- mean cross-entropy of logits [..., V] against Int32
// targets [...] (include/inferno/loss/crossentropyloss.h of the reference).
#pragma once
#include "inferno/core/tensor.h"

namespace Inferno {

class CrossEntropyLoss {
public:
    Tensor forward(Tensor& logits, Tensor& target);
    Tensor operator()(Tensor& logits, Tensor& target) { return forward(logits, target); }
};

}  // namespace Inferno
