// modules.cpp -- Module, Linear, LayerNorm, Embedding, MultiHeadAttention,
// CrossEntropyLoss, OptimizerAdamW and RandomGenerator
// (include/inferno/modules/*.h, loss/crossentropyloss.h, optim/adamw.h,
// util/random.h).  Same constructors, parameter names, defaults and
// registration as the reference's (module.cpp, linear.cpp, layernorm.cpp,
// embedding.cpp, crossentropyloss.cpp, adamw.cpp, random.cpp,
// InfernoApp/main.cpp:675-811); the compute goes through the ops of
// inferno/core/ops.h.
#include <cmath>
#include <map>
#include <random>
#include <vector>

#include "detail.h"
#include "inferno/gradengine/engine.h"
#include "inferno/loss/crossentropyloss.h"
#include "inferno/modules/embedding.h"
#include "inferno/modules/layernorm.h"
#include "inferno/modules/linear.h"
#include "inferno/modules/module.h"
#include "inferno/modules/multiheadattention.h"
#include "inferno/optim/adamw.h"
#include "inferno/util/random.h"
#include "inferno/functional/attention.h"

namespace Inferno {

// ------------------------------------------------------------- RandomGenerator
namespace {
std::mt19937& engine_ref() {
    static std::mt19937 gen(5489u);
    return gen;
}
}  // namespace

void RandomGenerator::initialize() { engine_ref().seed(std::random_device{}()); }
void RandomGenerator::initializeWithSeed(unsigned int seed) { engine_ref().seed(seed); }

std::vector<float> RandomGenerator::generateRandomFloatVector(size_t size, float minValue, float maxValue) {
    std::uniform_real_distribution<float> d(minValue, maxValue);
    std::vector<float> v(size);
    for (auto& x : v) x = d(engine_ref());
    return v;
}
std::vector<double> RandomGenerator::generateRandomDoubleVector(size_t size, double minValue, double maxValue) {
    std::uniform_real_distribution<double> d(minValue, maxValue);
    std::vector<double> v(size);
    for (auto& x : v) x = d(engine_ref());
    return v;
}
std::vector<int> RandomGenerator::generateRandomIntVector(size_t size, int minValue, int maxValue) {
    std::uniform_int_distribution<int> d(minValue, maxValue);
    std::vector<int> v(size);
    for (auto& x : v) x = d(engine_ref());
    return v;
}
float RandomGenerator::generateRandomFloat(float minValue, float maxValue) {
    return std::uniform_real_distribution<float>(minValue, maxValue)(engine_ref());
}
double RandomGenerator::generateRandomDouble(double minValue, double maxValue) {
    return std::uniform_real_distribution<double>(minValue, maxValue)(engine_ref());
}
int RandomGenerator::generateRandomInt(int minValue, int maxValue) {
    return std::uniform_int_distribution<int>(minValue, maxValue)(engine_ref());
}
std::vector<float> RandomGenerator::generateNormalFloatVector(size_t size, float mean, float stddev) {
    std::normal_distribution<float> d(mean, stddev);
    std::vector<float> v(size);
    for (auto& x : v) x = d(engine_ref());
    return v;
}

// ---------------------------------------------------------------------- Module
Tensor Module::forward(Tensor&) { throw Error("forward(input) not implemented!"); }

std::vector<Tensor*> Module::parameters() const {
    std::vector<Tensor*> all;
    for (const auto& [name, t] : _parameters) all.push_back(t);
    for (const auto& [name, child] : _children) {
        auto c = child->parameters();
        all.insert(all.end(), c.begin(), c.end());
    }
    return all;
}

static void check_free(const std::string& name, bool p, bool b, bool c) {
    if (p) throw std::runtime_error("Parameter already registered: " + name);
    if (b) throw std::runtime_error("Name already used by buffer: " + name);
    if (c) throw std::runtime_error("Name already used by submodule: " + name);
}

void Module::register_parameter(const std::string& name, Tensor* tensor) {
    check_free(name, _parameters.count(name), _buffers.count(name), _children.count(name));
    _parameters[name] = tensor;
}
void Module::register_module(const std::string& name, Module* module) {
    check_free(name, _parameters.count(name), _buffers.count(name), _children.count(name));
    _children[name] = module;
}
void Module::register_buffer(const std::string& name, Tensor* tensor) {
    check_free(name, _parameters.count(name), _buffers.count(name), _children.count(name));
    _buffers[name] = tensor;
}

void Module::to(const Device& device) {
    for (auto& [name, p] : _parameters)
        if (p) *p = p->to(device);
    for (auto& [name, b] : _buffers)
        if (b) *b = b->to(device);
    for (auto& [name, c] : _children)
        if (c) c->to(device);
}

StateDict Module::state_dict() const {
    StateDict out;
    collect_state_dict(out, "");
    return out;
}

void Module::collect_state_dict(StateDict& out, const std::string& prefix) const {
    const auto full = [&](const std::string& n) { return prefix.empty() ? n : prefix + "." + n; };
    for (const auto& [name, t] : _parameters) out[full(name)] = *t;
    for (const auto& [name, t] : _buffers) out[full(name)] = *t;
    for (const auto& [name, c] : _children) c->collect_state_dict(out, full(name));
}

// ---------------------------------------------------------------------- Linear
Linear::Linear(size_t in_features, size_t out_features, Device device, DType dtype)
    : m_in_features(in_features), m_out_features(out_features) {
    if (dtype != DType::Float32 && dtype != DType::BFloat16) throw Error("Unsupported dtype in Linear");
    const float limit = std::sqrt(6.0f / static_cast<float>(in_features + out_features));
    auto w = RandomGenerator::generateRandomFloatVector(in_features * out_features, -limit, limit);
    m_weights = Tensor(dtype, w, std::vector<size_t>{in_features, out_features}, "weights", device, true);
    auto b = RandomGenerator::generateRandomFloatVector(out_features, -limit, limit);
    m_biases = Tensor(dtype, b, std::vector<size_t>{out_features}, "biases", device, true);
    register_parameter("weights", &m_weights);
    register_parameter("bias", &m_biases);
}

Tensor Linear::forward(const Tensor& input) { return linear(input, m_weights, m_biases); }

// ------------------------------------------------------------------- LayerNorm
LayerNorm::LayerNorm(size_t normalized_dim, float eps, Device device, DType dtype)
    : m_dim(normalized_dim), m_eps(eps) {
    if (dtype != DType::Float32 && dtype != DType::BFloat16) throw Error("LayerNorm: floating dtype expected");
    NoGradGuard guard;
    m_beta = Tensor(DType::Float32, std::vector<float>(normalized_dim, 0.0f), std::vector<size_t>{normalized_dim},
                    "ln_beta", device, true);
    m_gamma = Tensor(DType::Float32, std::vector<float>(normalized_dim, 1.0f), std::vector<size_t>{normalized_dim},
                     "ln_gamma", device, true);
    register_parameter("beta", &m_beta);
    register_parameter("gamma", &m_gamma);
}

Tensor LayerNorm::forward(Tensor& input) {
    if (input.ndim() == 0 || input.shape().back() != m_dim) throw Error("LayerNorm: last dimension mismatch");
    return layer_norm(input, m_gamma, m_beta, m_eps);
}

// ------------------------------------------------------------------- Embedding
Embedding::Embedding(size_t vocab_size, size_t embed_dim, Device device, DType dtype) {
    if (dtype != DType::Float32 && dtype != DType::BFloat16) throw Error("Embedding: floating dtype expected");
    NoGradGuard guard;
    auto v = RandomGenerator::generateRandomFloatVector(vocab_size * embed_dim, -1.0f, 1.0f);
    m_embeddings = Tensor(dtype, v, std::vector<size_t>{vocab_size, embed_dim}, "embedding", device, true);
    register_parameter("weight", &m_embeddings);
}

Tensor Embedding::forward(Tensor& token_ids) { return embedding(token_ids, m_embeddings); }

// ---------------------------------------------------------- MultiHeadAttention
MultiHeadAttention::MultiHeadAttention(size_t embed_dim, size_t num_heads, Device device, DType dtype)
    : m_embed_dim(embed_dim),
      m_num_heads(num_heads),
      m_head_dim(num_heads ? embed_dim / num_heads : 0),
      Wqkv_layer(embed_dim, embed_dim * 3, device, dtype),
      W_out(embed_dim, embed_dim, device, dtype) {
    if (num_heads == 0 || embed_dim % num_heads != 0)
        throw Error("MultiHeadAttention: embed_dim must be divisible by num_heads");
    register_module("Wqkv", &Wqkv_layer);
    register_module("W_out", &W_out);
}

Tensor MultiHeadAttention::forward(Tensor& x) {
    if (x.ndim() != 3) throw Error("MultiHeadAttention expects [B, T, C]");
    if (x.shape()[2] != m_embed_dim) throw Error("MultiHeadAttention: embed_dim mismatch");
    Tensor qkv = Wqkv_layer.forward(static_cast<const Tensor&>(x));  // [B, T, 3C]
    Tensor y = qkv_attention(qkv, m_num_heads, true);                  // [B, T, C]
    return W_out.forward(static_cast<const Tensor&>(y));
}

KVCache::KVCache(size_t B, size_t H, size_t capacity, size_t D, Device device, DType dtype)
    : kv(dtype, std::vector<size_t>{2, B, H, capacity, D}, "kv_cache", device, false) {
    const std::vector<size_t> shape{B, H, capacity, D};
    const auto st = Tensor::calculate_strides(shape);
    k = make_view(kv, shape, st, kv.offset(), "kv_cache_k");
    v = make_view(kv, shape, st, kv.offset() + B * H * capacity * D, "kv_cache_v");
}

namespace {
// dst (a view) = src (a view of the same shape), element-wise through strides.
void copy_view(const Tensor& src, Tensor& dst) {
    if (src.shape() != dst.shape() || src.dtype() != dst.dtype()) throw Error("copy_view: shape or dtype mismatch");
    const size_t esz = dtype_size(src.dtype());
    if (src.device().is_cpu()) {
        detail::copy_strided_host(static_cast<const char*>(src.data_ptr()), src.strides(),
                                  static_cast<char*>(dst.data_ptr()), dst.strides(), src.shape(), esz);
        return;
    }
    auto shape = detail::to_i64(src.shape());
    auto ss = detail::to_i64(src.strides());
    auto ds = detail::to_i64(dst.strides());
    detail::DeviceGuard g(src.device().index);
    detail::status_check(inf_copy_strided(src.data_ptr(), ss.data(), dst.data_ptr(), ds.data(), (int)src.ndim(),
                                          shape.data(), (int)esz, detail::stream_of(src)),
                         "inf_copy_strided");
}
}  // namespace

Tensor MultiHeadAttention::forward_cached(const Tensor& x, KVCache& cache) {
    NoGradGuard ng;
    if (x.ndim() != 3 || x.shape()[2] != m_embed_dim) throw Error("MultiHeadAttention: expects [B, t, C]");
    const size_t B = x.shape()[0], t = x.shape()[1], C = m_embed_dim, H = m_num_heads, D = m_head_dim;
    if (!cache.k.defined() || cache.k.shape()[0] != B || cache.k.shape()[1] != H || cache.k.shape()[3] != D)
        throw Error("MultiHeadAttention: KV cache shape does not match [B, H, capacity, D]");
    if (cache.length + t > cache.capacity()) throw Error("MultiHeadAttention: KV cache is full");
    if (cache.k.device() != x.device()) throw Error("MultiHeadAttention: KV cache is on another device");
    Tensor qkv = Wqkv_layer.forward(x).contiguous();  // [B, t, 3C]
    const std::vector<size_t> hs{B, H, t, D};
    const std::vector<size_t> hst{t * 3 * C, D, 3 * C, 1};
    Tensor q = make_view(qkv, hs, hst, qkv.offset(), "q");
    Tensor knew = make_view(qkv, hs, hst, qkv.offset() + C, "k_new");
    Tensor vnew = make_view(qkv, hs, hst, qkv.offset() + 2 * C, "v_new");
    const bool joint = cache.kv.defined() && cache.kv.ndim() == 5 && cache.kv.strides()[0] > 0 &&
                       GetImpl(cache.k)->storage() == GetImpl(cache.kv)->storage() &&
                       GetImpl(cache.v)->storage() == GetImpl(cache.kv)->storage() &&
                       cache.k.offset() == cache.kv.offset() &&
                       cache.v.offset() == cache.kv.offset() + cache.kv.strides()[0] &&
                       cache.k.strides() == std::vector<size_t>(cache.kv.strides().begin() + 1, cache.kv.strides().end());
    if (joint) {
        // keys and values of the step in one copy: source [2, B, H, t, D] out of
        // qkv (k at column C, v at 2C), destination slots of both cache halves
        Tensor kvnew = make_view(qkv, {2, B, H, t, D}, {C, t * 3 * C, D, 3 * C, 1}, qkv.offset() + C, "kv_new");
        Tensor kvdst = make_view(cache.kv, {2, B, H, t, D}, cache.kv.strides(), cache.kv.offset() + cache.length * D,
                                 "kv_slot");
        copy_view(kvnew, kvdst);
    } else {
        Tensor kdst = make_view(cache.k, hs, cache.k.strides(), cache.k.offset() + cache.length * D, "k_slot");
        Tensor vdst = make_view(cache.v, hs, cache.v.strides(), cache.v.offset() + cache.length * D, "v_slot");
        copy_view(knew, kdst);
        copy_view(vnew, vdst);
    }
    // The cache advances only when the whole step succeeds: a throw below
    // leaves its length as it was (the slots just written lie past it).
    const size_t len0 = cache.length;
    try {
        const size_t len = len0 + t;
        const std::vector<size_t> all{B, H, len, D};
        Tensor kall = make_view(cache.k, all, cache.k.strides(), cache.k.offset(), "k_cache");
        Tensor vall = make_view(cache.v, all, cache.v.strides(), cache.v.offset(), "v_cache");
        Tensor y4 = t == 1 ? attention_decode(q, kall, vall) : scaled_dot_product_attention(q, kall, vall, true);
        // [B, H, t, D] -> [B, t, C]; at t = 1 the dense [B, H, 1, D] already has that layout
        Tensor y = t == 1 ? y4.reshape({B, 1, C}) : y4.transpose(1, 2).contiguous().reshape({B, t, C});
        Tensor out = W_out.forward(static_cast<const Tensor&>(y));
        cache.length = len;
        return out;
    } catch (...) {
        cache.length = len0;
        throw;
    }
}

// ------------------------------------------------------------ CrossEntropyLoss
Tensor CrossEntropyLoss::forward(Tensor& logits, Tensor& target) { return cross_entropy(logits, target); }

// -------------------------------------------------------------- OptimizerAdamW
void OptimizerAdamW::step() {
    NoGradGuard guard;
    steps_++;
    const float bc1 = 1.0f - std::pow(beta1_, static_cast<float>(steps_));
    const float bc2 = 1.0f - std::pow(beta2_, static_cast<float>(steps_));
    // HIP parameters are updated together, one multi-tensor call per (device,
    // dtype); `keep` holds the contiguous gradient copies until the calls are
    // enqueued (later reuse of their blocks is stream-ordered after them).
    std::map<std::pair<int, int>, std::vector<inf_adamw_tensor>> groups;
    std::vector<Tensor> keep;
    for (Tensor* p : params_) {
        if (p == nullptr || !p->grad()) continue;
        Tensor* grad = p->grad().get();
        if (grad->dtype() != p->dtype() || grad->shape() != p->shape())
            throw Error("OptimizerAdamW: gradient dtype / shape differs from the parameter's");
        if (!p->is_contiguous()) throw Error("OptimizerAdamW: parameters must be contiguous");
        Tensor g = grad->contiguous();
        Moments& st = moments_[p];
        if (!st.first.defined()) {
            st.first = Tensor::zeros(p->shape(), DType::Float32, p->device(), "adamw_m");
            st.second = Tensor::zeros(p->shape(), DType::Float32, p->device(), "adamw_v");
        }
        const size_t n = p->numel();
        if (p->device().is_cpu()) {
            // cpu_adamw_step_impl (adamw.h:67-111)
            char* pp = static_cast<char*>(p->data_ptr());
            const char* gp = static_cast<const char*>(g.data_ptr());
            float* mp = static_cast<float*>(st.first.data_ptr());
            float* vp = static_cast<float*>(st.second.data_ptr());
            const size_t esz = dtype_size(p->dtype());
            for (size_t i = 0; i < n; ++i) {
                const float gr = (float)detail::load_elem(gp + i * esz, p->dtype());
                float mi = mp[i], vi = vp[i], pi = (float)detail::load_elem(pp + i * esz, p->dtype());
                mi = beta1_ * mi + (1.0f - beta1_) * gr;
                vi = beta2_ * vi + (1.0f - beta2_) * gr * gr;
                const float m_hat = mi / bc1;
                const float v_hat = vi / bc2;
                float update = m_hat / (std::sqrt(v_hat) + eps_);
                if (decay_ != 0.0f) update += decay_ * pi;
                pi -= lr_ * update;
                detail::store_elem(pp + i * esz, p->dtype(), pi);
                mp[i] = mi;
                vp[i] = vi;
            }
        } else {
            const int dt = (int)detail::inf_dt(p->dtype(), "OptimizerAdamW");
            groups[{p->device().index, dt}].push_back(inf_adamw_tensor{p->data_ptr(), g.data_ptr(),
                                                                       static_cast<float*>(st.first.data_ptr()),
                                                                       static_cast<float*>(st.second.data_ptr()),
                                                                       (int64_t)n});
            keep.push_back(g);
        }
    }
    for (auto& [key, list] : groups) {
        detail::DeviceGuard dg(key.first);
        detail::status_check(inf_adamw_step_multi(list.data(), (int)list.size(), lr_, beta1_, beta2_, eps_,
                                                  decay_, bc1, bc2, (inf_dtype)key.second,
                                                  detail::stream_for(key.first)),
                             "inf_adamw_step_multi");
    }
}

void OptimizerAdamW::zero_grad() {
    for (auto& p : params_)
        if (p != nullptr) p->grad() = nullptr;
}

}  // namespace Inferno
