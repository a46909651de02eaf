// attention.h -- fused scaled-dot-product attention and its backward node.
//
// New API surface: the reference composes attention from ~10 generic ops in
// MultiHeadAttentionFast4::forward (InfernoApp/main.cpp:692-768) and lists a
// fused op as roadmap work (README.md:855).  The op follows the reference's op
// conventions: returns a new tensor, attaches AttentionBackward when grad is
// enabled and any input requires grad.
//
//   q: [B, H, Tq, D], k, v: [B, H, Tk, D] -- any strides with a unit stride on D,
//   same dtype (Float32 or BFloat16) and device.  On HIP the fused kernels take
//   D in {32, 64, 128}; any other D <= 128 runs them on copies zero-padded along
//   D (exact: the padding adds zero terms), and D > 128 (Float32) runs the
//   reference's composed chain on the HIP ops.
//   causal: key j visible to query i iff j <= i + (Tk - Tq), bit-identical to
//   triu(ones, 1) + masked_fill(-1e9f) (main.cpp:747-748).
//   scale: NaN means 1.0f / sqrt((float)D) (main.cpp:743).
#pragma once

#include <cmath>

#include "inferno/core/tensor.h"
#include "inferno/gradfn/node.h"

namespace Inferno {

Tensor scaled_dot_product_attention(const Tensor& q, const Tensor& k, const Tensor& v, bool causal = true,
                                    float scale = NAN);

// Forward that also returns the per-row log-sum-exp (fp32 [B, H, Tq]).
Tensor scaled_dot_product_attention_lse(const Tensor& q, const Tensor& k, const Tensor& v, bool causal,
                                        float scale, Tensor* lse_out);

// One query per (b, h) against a KV cache: q [B, H, 1, D], caches [B, H, Tk, D].
// Inference only (no graph node); equals the last row of a causal prefill.
Tensor attention_decode(const Tensor& q, const Tensor& kcache, const Tensor& vcache, float scale = NAN);

// Saves q, k, v, O and LSE (never P); produces dQ, dK, dV in one fused pass.
// With a padded head dim it also keeps the padded q, k, v and O the forward ran
// on, and sends the first D columns of the padded gradients to q, k, v.
class AttentionBackward final : public Node {
public:
    AttentionBackward(const Tensor& q, const Tensor& k, const Tensor& v, const Tensor& out, const Tensor& lse,
                      bool causal, float scale);
    AttentionBackward(const Tensor& q, const Tensor& k, const Tensor& v, const Tensor& lse, bool causal, float scale,
                      const Tensor& q_padded, const Tensor& k_padded, const Tensor& v_padded,
                      const Tensor& out_padded);
    void backward() override;
    void release() override;
    void get_inputs(std::vector<Tensor>& out) const override;

private:
    Tensor m_q, m_k, m_v, m_out, m_lse;
    Tensor m_qp, m_kp, m_vp, m_op;  // padded copies (defined only for a padded head dim)
    bool m_causal;
    float m_scale;
};

}  // namespace Inferno
