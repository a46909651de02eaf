// ops.h -- the tensor ops of the GPT training step around the attention path.
//
// Same conventions as the reference's ops (src/inferno/core/ops.cpp): free
// functions returning a new Tensor, outputs allocated by the op on the inputs'
// device, a backward node attached when grad is enabled and an input requires
// grad.  HIP tensors run on the gfx950 kernels and hipBLASLt through the C-ABI
// (include/inferno_hip.h); CPU tensors run plain loops in the reference's
// accumulation order.
#pragma once
#include <cmath>
#include <string>
#include <vector>
#include "inferno/core/tensor.h"

namespace Inferno {

// Batched matrix product [..., M, K] x [..., K, N] -> [..., M, N] with the
// leading (batch) dimensions broadcast as in matmul (ops.cpp:437-735).  The
// output is contiguous.  Unlike the reference, view offsets are honoured
// (ops.cpp:443-444 drops them).
Tensor matmul(const Tensor& A, const Tensor& B, const std::string& name = "matmul");

// x [..., in] @ W [in, out] + b [out] as one GEMM with a bias epilogue: the
// composition matmul(x, W) + b of Linear::forward (linear.cpp:49-54) with one
// LinearBackward node (dx = g W^T, dW = x^T g, db = column sums of g) in place
// of MMBackward + AddBackward.  b may be undefined.
Tensor linear(const Tensor& x, const Tensor& W, const Tensor& b);

// LayerNorm over the last dimension (layernorm.cpp:33-80, layernorm_kernels.h:48-87).
Tensor layer_norm(const Tensor& x, const Tensor& gamma, const Tensor& beta, float eps);

// LayerNorm(x + r) with the sum returned through *sum: the residual add and the
// next LayerNorm of a transformer block.  Equals layer_norm(x + r, ...) (which
// it runs when a gradient is needed or on the CPU); on HIP without gradients it
// is one pass (inf_add_layernorm_fwd).  No reference counterpart.
Tensor add_layer_norm(const Tensor& x, const Tensor& r, const Tensor& gamma, const Tensor& beta, float eps,
                      Tensor* sum);

// table[ids] for Int32 ids [...] -> [..., dim] (embedding.cpp:52-104).
Tensor embedding(const Tensor& ids, const Tensor& table);

// Mean cross-entropy of logits [..., V] against Int32 targets [...]
// (crossentropyloss.cpp, cpuops.h:707-749); returns a one-element tensor.
Tensor cross_entropy(const Tensor& logits, const Tensor& target);

// Causal multi-head attention straight out of a fused projection:
// qkv [B, T, 3C] holds q | k | v along the last dimension (the layout of
// InfernoApp/main.cpp:712-718); returns y [B, T, C] with head h in columns
// [h*D, (h+1)*D).  No copies: q, k, v are read through strides and y is
// written in [B, T, C] directly; the backward writes dq | dk | dv into one
// [B, T, 3C] gradient.  Replaces the slice / contiguous / reshape / transpose /
// matmul / masked_fill / Softmax / matmul / transpose / contiguous chain of
// MultiHeadAttentionFast4::forward (main.cpp:712-764).
Tensor qkv_attention(const Tensor& qkv, size_t num_heads, bool causal = true, float scale = NAN);

// Upper triangle of the last two dimensions: element (..., r, c) kept when
// c - r >= diagonal, else zero; any dtype, dense output, no gradient
// (ops.cpp:1355-1398, cpu_triu cpuops.h:617-656).  Rank < 2 throws (the
// reference logs an error and exits).
Tensor triu(const Tensor& A, int diagonal);

// value where mask != 0, input elsewhere; the integer mask (Int32, Int8 or Bool)
// broadcasts from the right, size-1 dimensions repeating; value converted to
// the input dtype as static_cast<AT>(value); dense output, no gradient
// (ops.cpp:1235-1289, cpu_masked_fill cpuops.h:659-705).  A mask that does not
// broadcast throws (the reference does not check it).
Tensor masked_fill(const Tensor& input, const Tensor& mask, float value);

// Index of the largest element along the last dimension -- the first one on
// ties, as std::max_element picks -- as Int32 [...] for x [..., n]; no
// gradient.  No counterpart in the reference (it has no generation loop): the
// greedy next-token pick, so only the indices leave the device.
Tensor argmax(const Tensor& x);

// Sums g over the dimensions that broadcasting expanded, to `shape`
// (sum_to_shape, src/inferno/core/broadcastops.cpp:19-106).  HIP tensors: the
// expanded dimensions must be leading ones.
Tensor sum_to_shape(const Tensor& g, const std::vector<size_t>& shape);

}  // namespace Inferno
