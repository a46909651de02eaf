// nnbackward.h -- backward nodes of the ops in inferno/core/ops.h and gelu.
// Each follows the reference node's contract (node.h:23-45): backward() reads
// Engine::grad_in(this, 0) under a NoGradGuard and accumulates into each input
// that has a grad edge; release() drops the saved tensors.
#pragma once
#include <cmath>
#include "inferno/gradfn/node.h"

namespace Inferno {

// C = A @ B: dA = G B^T, dB = A^T G, each summed to its input's shape (mmbackward.cpp:36-98).
class MMBackward final : public Node {
public:
    MMBackward(const Tensor& a, const Tensor& b);
    void backward() override;
    void release() override;
    void get_inputs(std::vector<Tensor>& out) const override;
private:
    Tensor m_a, m_b;
};

// y = x W + b (x flattened to rows): dx = g W^T, dW = x^T g, db = column sums of g.
class LinearBackward final : public Node {
public:
    LinearBackward(const Tensor& x, const Tensor& w, const Tensor& b);
    void backward() override;
    void release() override;
    void get_inputs(std::vector<Tensor>& out) const override;
private:
    Tensor m_x, m_w, m_b;
};

// layernormbackward.cpp:29-110; saves the fp32 per-row mean and invstd.
class LayerNormBackward final : public Node {
public:
    LayerNormBackward(const Tensor& x, const Tensor& gamma, const Tensor& beta, const Tensor& mean,
                      const Tensor& invstd);
    void backward() override;
    void release() override;
    void get_inputs(std::vector<Tensor>& out) const override;
private:
    Tensor m_x, m_gamma, m_beta, m_mean, m_invstd;
};

// gelubackward.cpp: dx = g * gelu'(x).
class GeluBackward final : public Node {
public:
    explicit GeluBackward(const Tensor& x);
    void backward() override;
    void release() override;
    void get_inputs(std::vector<Tensor>& out) const override;
private:
    Tensor m_x;
};

// embeddingbackward.cpp:35-45: dtable[ids[t]] += g[t].
class EmbeddingBackward final : public Node {
public:
    EmbeddingBackward(const Tensor& table, const Tensor& ids);
    void backward() override;
    void release() override;
    void get_inputs(std::vector<Tensor>& out) const override;
private:
    Tensor m_table, m_ids;
};

// crossentropylossbackward.cpp: dlogits = (softmax - onehot) * g / rows; keeps
// the forward's per-row log-sum-exp so the backward is one pass.
class CrossEntropyLossBackward final : public Node {
public:
    CrossEntropyLossBackward(const Tensor& logits, const Tensor& target, const Tensor& lse);
    void backward() override;
    void release() override;
    void get_inputs(std::vector<Tensor>& out) const override;
private:
    Tensor m_logits, m_target, m_lse;
};

// qkv_attention: saves qkv, y and the per-row LSE (never P); writes dq | dk | dv
// into one [B, T, 3C] gradient with the fused attention backward.
class QKVAttentionBackward final : public Node {
public:
    QKVAttentionBackward(const Tensor& qkv, const Tensor& y, const Tensor& lse, size_t num_heads, bool causal,
                         float scale);
    void backward() override;
    void release() override;
    void get_inputs(std::vector<Tensor>& out) const override;
private:
    Tensor m_qkv, m_y, m_lse;
    size_t m_heads;
    bool m_causal;
    float m_scale;
};

}  // namespace Inferno
