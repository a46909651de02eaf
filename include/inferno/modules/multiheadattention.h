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

// Keys and values of one attention layer for incremental decoding: [B, H,
// capacity, D] device buffers and the number of positions filled.  No
// reference counterpart (the reference has no generation loop; see the
// commented-out last-position select, InfernoApp/main.cpp:1173-1177).
struct KVCache {
    // k and v are the two halves of one [2, B, H, capacity, D] buffer `kv`, so
    // appending a step's keys and values is one strided copy.  A cache built
    // from separate k / v tensors (kv undefined) is appended with two copies.
    Tensor kv, k, v;
    size_t length = 0;
    KVCache() = default;
    KVCache(size_t B, size_t H, size_t capacity, size_t D, Device device, DType dtype = DType::Float32);
    size_t capacity() const { return k.defined() ? k.shape()[2] : 0; }
};

class MultiHeadAttention : public Module {
public:
    MultiHeadAttention(size_t embed_dim, size_t num_heads, Device device = Device::cpu(),
                       DType dtype = DType::Float32);
    Tensor forward(Tensor& x) override;  // x [B, T, C] -> [B, T, C]
    // Inference with a cache: x [B, t, C] holds the next t positions; their keys
    // and values are appended to `cache` and each attends causally to every
    // cached position before it (t == 1: the single-query decode kernel; t > 1:
    // the causal kernel with Tq = t < Tk).  No graph is recorded.
    Tensor forward_cached(const Tensor& x, KVCache& cache);
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
