// gelu.h -- tanh-approximation GELU (include/inferno/functional/gelu.h of the
// reference; gelu.cpp, gelu_kernels.h:9-16).  As in the reference the output
// always reports requires_grad (gelu.cpp:29); the GeluBackward node is attached
// only when grad is enabled and the input requires grad.
#pragma once
#include "inferno/core/tensor.h"

namespace Inferno {
Tensor gelu(const Tensor& A);
}  // namespace Inferno
