// embedding.h -- token embedding table [vocab, dim] (include/inferno/modules/
// embedding.h, embedding.cpp of the reference).  The reference initialises it
// with Tensor::randn, which is uniform in [-1, 1] for Float32
// (tensor.cpp:1057-1062); so does this one.
#pragma once
#include "inferno/modules/module.h"

namespace Inferno {

class Embedding : public Module {
public:
    Embedding(size_t vocab_size, size_t embed_dim, Device device = Device::cpu(), DType dtype = DType::Float32);
    Tensor forward(Tensor& token_ids) override;
    Tensor operator()(Tensor& input) { return forward(input); }
    // The table itself (no reference counterpart): lets a model tie its output
    // projection to the embedding (logits = x @ weight^T).
    Tensor& weight() { return m_embeddings; }

private:
    Tensor m_embeddings;  // [vocab_size, embedding_dim]
};

}  // namespace Inferno
