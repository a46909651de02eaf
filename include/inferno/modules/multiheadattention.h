// multiheadattention.h -- causal multi-head self-attention module, the drop-in
// for MultiHeadAttentionFast4 (InfernoApp/main.cpp:675-811): a fused
// [C -> 3C] projection "Wqkv", fused causal attention read straight out of the
// projection, and the [C -> C] output projection "W_out" (same parameter names
// and shapes, so state dicts line up).
//
// Behavioural difference, on purpose: the reference's .contiguous() calls
// return tensors without grad (ops.cpp:1308), which cuts the graph so Wqkv and
// everything before the attention never receive gradients.  Here gradients
// flow into Wqkv, the input and (through it) the LayerNorm before it.
#pragma once
#include "inferno/modules/linear.h"

namespace Inferno {

class MultiHeadAttention : public Module {
public:
    MultiHeadAttention(size_t embed_dim, size_t num_heads, Device device = Device::cpu(),
                       DType dtype = DType::Float32);
    Tensor forward(Tensor& x) override;  // x [B, T, C] -> [B, T, C]
    Linear& qkv_proj() { return Wqkv_layer; }
    Linear& out_proj() { return W_out; }

private:
    size_t m_embed_dim;
    size_t m_num_heads;
    size_t m_head_dim;
    Linear Wqkv_layer;  // constructed first, as in the reference (main.cpp:805-806)
    Linear W_out;
};

}  // namespace Inferno
