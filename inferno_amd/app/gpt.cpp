// gpt.cpp -- the GPT training step around the attention path, on the C++
// drop-in (libinferno.so).  Mirrors the application classes of
// InfernoApp/main.cpp: PositionalEncoding (:20-64), TransformerBlock
// (:817-926, LayerNorm -> attention -> residual -> LayerNorm -> Linear ->
// GELU -> Linear -> residual) and GPTModel (:940-1033), with the attention
// block replaced by the fused MultiHeadAttention module.  The output
// projection is tied to the token embedding (logits = x @ E^T) unless --untied
// is given, in which case it is the reference's separate Linear "linear1".
//
//   gpt bench [--layers L] [--dmodel C] [--heads H] [--ctx T] [--vocab V]
//             [--batch B] [--steps K] [--warmup W] [--untied] [--deterministic]
//       random-init weights N(0, 0.02) (biases 0, LayerNorm gamma 1 / beta 0),
//       tokens uniform in [0, V), targets = tokens shifted by one, AdamW
//       lr 3e-4; times K training steps (forward, cross-entropy, backward,
//       AdamW, zero_grad) on hip:0 and prints one JSON line with tokens/s and
//       the attention share of the step time.  --deterministic (any command)
//       takes the attention backward's dQ from the query-major pass
//       (inf_set_deterministic), the same bits on every run.
//   gpt generate [--layers L] [--dmodel C] [--heads H] [--vocab V] [--ctx T]
//                [--batch B] [--prompt P] [--new N]
//       greedy generation with one KV cache per layer on hip:0 (prefill of a
//       random P-token prompt, then N tokens one at a time through the
//       single-query decode kernel); prints one JSON line with the prefill
//       time and the per-token decode time.
//   gpt decode-check <dir> <cpu|hip> [--prefill P]
//       full causal forward of tokens.bin vs incremental decoding (prefill of P
//       tokens, then one at a time); writes logits_full.bin and logits_inc.bin.
//   gpt step <dir> <cpu|hip> [--untied]
//       reads config.txt ("L C H T V B"), tokens.bin / targets.bin (int32 [B, T])
//       and one <state-dict name>.bin (fp32) per parameter from <dir>; runs one
//       training step; writes loss.bin, grad_<name>.bin (before the update) and
//       param_<name>.bin (after it).
#include <hip/hip_runtime_api.h>

#include "inferno_hip.h"

#include <algorithm>
#include <chrono>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <fstream>
#include <iostream>
#include <memory>
#include <random>
#include <string>
#include <vector>

#include "inferno/inferno.h"

using namespace Inferno;

// ------------------------------------------------------------------- model
class PositionalEncoding : public Module {
public:
    PositionalEncoding(size_t context_size, size_t embed_dim, Device device) {
        std::vector<float> pe_data(context_size * embed_dim);
        for (size_t pos = 0; pos < context_size; ++pos)
            for (size_t i = 0; i < embed_dim; ++i) {
                const float exponent = 2.0f * float(i / 2) / float(embed_dim);
                const float angle = float(pos) / std::pow(10000.0f, exponent);
                pe_data[pos * embed_dim + i] = (i % 2 == 0) ? std::sin(angle) : std::cos(angle);
            }
        pe = Tensor(DType::Float32, pe_data, std::vector<size_t>{context_size, embed_dim}, "positional-encoding",
                    device);
        register_buffer("pe", &pe);
    }
    Tensor forward(Tensor& x) override { return forward_at(x, 0); }
    // x [B, t, C] holding positions pos0 .. pos0 + t - 1
    Tensor forward_at(const Tensor& x, size_t pos0) {
        const size_t T = x.shape()[1];
        if (pos0 + T > pe.shape()[0]) throw Error("PositionalEncoding: position beyond the context size");
        Tensor p = (pos0 == 0 && T == pe.shape()[0]) ? pe : pe.slice(0, pos0, pos0 + T - 1);
        return x + p;
    }
    Tensor pe;
};

class TransformerBlock : public Module {
public:
    TransformerBlock(size_t embed_dim, size_t nheads, Device device, DType dtype)
        : attn(embed_dim, nheads, device, dtype),
          layernorm1(embed_dim, 1e-5f, device, dtype),
          layernorm2(embed_dim, 1e-5f, device, dtype),
          feedforward1(embed_dim, 4 * embed_dim, device, dtype),
          feedforward2(4 * embed_dim, embed_dim, device, dtype) {
        register_module("attn", &attn);
        register_module("ln1", &layernorm1);
        register_module("ln2", &layernorm2);
        register_module("ff1", &feedforward1);
        register_module("ff2", &feedforward2);
    }
    Tensor forward(Tensor& x) override {
        Tensor normed = layernorm1.forward(x);
        Tensor attn_out = attn.forward(normed);
        Tensor h = x + attn_out;
        Tensor normed2 = layernorm2.forward(h);
        Tensor n = feedforward1.forward(static_cast<const Tensor&>(normed2));
        n = gelu(n);
        Tensor ff = feedforward2.forward(static_cast<const Tensor&>(n));
        return h + ff;
    }
    // Inference on the next positions with this layer's KV cache, given x and
    // normed = LayerNorm-1(x): returns the MLP output and sets *h = x +
    // attention.  The block's output h + MLP is left to the caller, which adds
    // it and applies the next LayerNorm in one pass, as this does for h and
    // LayerNorm-2 (add_layer_norm: one launch instead of an add and a norm).
    Tensor forward_cached(const Tensor& x, const Tensor& normed, KVCache& cache, Tensor* h) {
        Tensor a = attn.forward_cached(normed, cache);
        Tensor normed2 = add_layer_norm(x, a, layernorm2.gamma(), layernorm2.beta(), layernorm2.eps(), h);
        Tensor n = gelu(feedforward1.forward(static_cast<const Tensor&>(normed2)));
        return feedforward2.forward(static_cast<const Tensor&>(n));
    }
    MultiHeadAttention attn;
    LayerNorm layernorm1, layernorm2;
    Linear feedforward1, feedforward2;
};

class GPTModel : public Module {
public:
    GPTModel(size_t vocab_size, size_t context_size, size_t embed_dim, size_t nheads, size_t nblocks, bool tied,
             Device device, DType dtype)
        : emb1(vocab_size, embed_dim, device, dtype),
          pos_enc(context_size, embed_dim, device),
          layernorm1(embed_dim, 1e-5f, device, dtype),
          m_tied(tied) {
        m_heads = nheads;
        m_embed = embed_dim;
        register_module("tok_embedding", &emb1);
        register_module("pos_encoding", &pos_enc);
        blocks.reserve(nblocks);
        for (size_t i = 0; i < nblocks; ++i) {
            blocks.push_back(std::make_unique<TransformerBlock>(embed_dim, nheads, device, dtype));
            register_module("block" + std::to_string(i), blocks.back().get());
        }
        if (!tied) {
            linear1 = std::make_unique<Linear>(embed_dim, vocab_size, device, dtype);
            register_module("linear1", linear1.get());
        }
        register_module("ln1", &layernorm1);
    }
    Tensor forward(Tensor& input) override {
        Tensor x = emb1.forward(input);
        x = pos_enc.forward(x);
        for (auto& b : blocks) x = b->forward(x);
        x = layernorm1.forward(x);
        if (m_tied) return matmul(x, emb1.weight().transpose(0, 1), "logits");
        return linear1->forward(static_cast<const Tensor&>(x));
    }
    // One KV cache per block, for up to `capacity` positions.
    std::vector<KVCache> make_caches(size_t B, size_t capacity, const Device& dev) {
        std::vector<KVCache> c;
        for (size_t i = 0; i < blocks.size(); ++i) c.emplace_back(B, m_heads, capacity, m_embed / m_heads, dev);
        return c;
    }
    // Logits [B, t, V] of the next t tokens [B, t], appending to the caches.
    Tensor forward_cached(Tensor& tokens, std::vector<KVCache>& caches) {
        NoGradGuard ng;
        const size_t pos0 = caches.empty() ? 0 : caches[0].length;
        Tensor x = emb1.forward(tokens);
        x = pos_enc.forward_at(x, pos0);
        // normed: the LayerNorm the next block (or the final one) reads
        Tensor normed = (blocks.empty() ? layernorm1 : blocks[0]->layernorm1).forward(x);
        for (size_t i = 0; i < blocks.size(); ++i) {
            Tensor h;
            Tensor mlp = blocks[i]->forward_cached(x, normed, caches[i], &h);
            LayerNorm& next = i + 1 < blocks.size() ? blocks[i + 1]->layernorm1 : layernorm1;
            normed = add_layer_norm(h, mlp, next.gamma(), next.beta(), next.eps(), &x);  // x = h + mlp
        }
        if (m_tied) return matmul(normed, emb1.weight().transpose(0, 1), "logits");
        return linear1->forward(static_cast<const Tensor&>(normed));
    }
    size_t m_heads = 0, m_embed = 0;
    Embedding emb1;
    PositionalEncoding pos_enc;
    std::vector<std::unique_ptr<TransformerBlock>> blocks;
    std::unique_ptr<Linear> linear1;
    LayerNorm layernorm1;
    bool m_tied;
};

// ------------------------------------------------------------------ helpers
static std::vector<char> read_file(const std::string& path) {
    std::ifstream f(path, std::ios::binary);
    if (!f) throw Error("cannot read " + path);
    return std::vector<char>((std::istreambuf_iterator<char>(f)), std::istreambuf_iterator<char>());
}

static void write_f32(const std::string& path, const std::vector<float>& v) {
    std::ofstream f(path, std::ios::binary);
    f.write(reinterpret_cast<const char*>(v.data()), (std::streamsize)(v.size() * 4));
}

static void set_param(Tensor& p, const std::vector<float>& v) {
    if (v.size() != p.numel()) throw Error("parameter size mismatch for " + p.name());
    Tensor h(DType::Float32, v, p.shape(), p.name(), Device::cpu());
    Tensor d = h.to(p.device());
    d.set_requires_grad(p.requires_grad());
    p = d;
}

static void sync(const Device& d) {
    if (!d.is_cpu()) (void)hipDeviceSynchronize();
}

// --------------------------------------------------------------------- step
static int run_step(const std::string& dir, const Device& dev, bool tied) {
    std::ifstream cf(dir + "/config.txt");
    size_t L, C, H, T, V, B;
    if (!(cf >> L >> C >> H >> T >> V >> B)) throw Error("bad config.txt");
    GPTModel model(V, T, C, H, L, tied, dev, DType::Float32);
    // load parameters by state-dict name (pointers from parameters() are stable)
    {
        StateDict sd = model.state_dict();
        std::vector<Tensor*> params = model.parameters();
        for (auto& [name, t] : sd) {
            Tensor* target = nullptr;
            for (Tensor* p : params)
                if (GetImpl(*p) == GetImpl(t)) target = p;
            if (!target) continue;  // buffers (pos_encoding.pe) stay as built
            auto raw = read_file(dir + "/" + name + ".bin");
            std::vector<float> v(raw.size() / 4);
            std::memcpy(v.data(), raw.data(), v.size() * 4);
            set_param(*target, v);
        }
    }
    auto tok = read_file(dir + "/tokens.bin"), tgt = read_file(dir + "/targets.bin");
    std::vector<int32_t> tv(B * T), gv(B * T);
    std::memcpy(tv.data(), tok.data(), tv.size() * 4);
    std::memcpy(gv.data(), tgt.data(), gv.size() * 4);
    Tensor x(DType::Int32, tv, std::vector<size_t>{B, T}, "tokens", dev);
    Tensor y(DType::Int32, gv, std::vector<size_t>{B, T}, "targets", dev);

    CrossEntropyLoss loss_fn;
    OptimizerAdamW opt(model.parameters());
    Tensor logits = model.forward(x);
    Tensor loss = loss_fn(logits, y);
    loss.backward();
    write_f32(dir + "/loss.bin", loss.to_host_float());
    StateDict sd = model.state_dict();
    for (auto& [name, t] : sd) {
        if (!t.grad()) continue;
        write_f32(dir + "/grad_" + name + ".bin", t.grad()->to_host_float());
    }
    opt.step();
    opt.zero_grad();
    sd = model.state_dict();
    for (auto& [name, t] : sd) write_f32(dir + "/param_" + name + ".bin", t.to_host_float());
    sync(dev);
    std::cout << "step ok: loss " << loss.to_host_float()[0] << "\n";
    return 0;
}

// ------------------------------------------------------------- decode-check
// Full causal forward of tokens [B, T] vs incremental decoding: prefill of the
// first P tokens, then one token at a time through the KV caches.  Writes
// logits_full.bin and logits_inc.bin ([B, T, V] fp32).
static void load_params(GPTModel& model, const std::string& dir) {
    StateDict sd = model.state_dict();
    std::vector<Tensor*> params = model.parameters();
    for (auto& [name, t] : sd) {
        Tensor* target = nullptr;
        for (Tensor* p : params)
            if (GetImpl(*p) == GetImpl(t)) target = p;
        if (!target) continue;
        auto raw = read_file(dir + "/" + name + ".bin");
        std::vector<float> v(raw.size() / 4);
        std::memcpy(v.data(), raw.data(), v.size() * 4);
        set_param(*target, v);
    }
}

static int run_decode_check(const std::string& dir, const Device& dev, size_t P) {
    std::ifstream cf(dir + "/config.txt");
    size_t L, C, H, T, V, B;
    if (!(cf >> L >> C >> H >> T >> V >> B)) throw Error("bad config.txt");
    GPTModel model(V, T, C, H, L, true, dev, DType::Float32);
    load_params(model, dir);
    auto tok = read_file(dir + "/tokens.bin");
    std::vector<int32_t> tv(B * T);
    std::memcpy(tv.data(), tok.data(), tv.size() * 4);
    Tensor x(DType::Int32, tv, std::vector<size_t>{B, T}, "tokens", dev);
    {
        NoGradGuard ng;
        write_f32(dir + "/logits_full.bin", model.forward(x).to_host_float());
    }
    auto caches = model.make_caches(B, T, dev);
    std::vector<float> inc(B * T * V);
    auto put = [&](const Tensor& logits, size_t pos0) {
        const size_t t = logits.shape()[1];
        auto h = logits.to_host_float();
        for (size_t b = 0; b < B; ++b)
            for (size_t i = 0; i < t; ++i)
                std::memcpy(&inc[(b * T + pos0 + i) * V], &h[(b * t + i) * V], V * 4);
    };
    std::vector<int32_t> chunk(B * P);
    for (size_t b = 0; b < B; ++b)
        for (size_t i = 0; i < P; ++i) chunk[b * P + i] = tv[b * T + i];
    Tensor xp(DType::Int32, chunk, std::vector<size_t>{B, P}, "prompt", dev);
    put(model.forward_cached(xp, caches), 0);
    for (size_t pos = P; pos < T; ++pos) {
        std::vector<int32_t> one(B);
        for (size_t b = 0; b < B; ++b) one[b] = tv[b * T + pos];
        Tensor x1(DType::Int32, one, std::vector<size_t>{B, 1}, "next", dev);
        put(model.forward_cached(x1, caches), pos);
    }
    write_f32(dir + "/logits_inc.bin", inc);
    sync(dev);
    std::cout << "decode-check ok\n";
    return 0;
}

// --------------------------------------------------------- generate-check
// Greedy generation from given parameters and prompt (tokens.bin, [B, P]
// int32): prefill through the KV caches, then N tokens, each the argmax of
// the last position's logits, picked on the device and fed back from there
// (the same loop as `gpt generate`; the picks and logits are also copied out
// for the check).  Writes
// generated.bin ([B, N] int32) and gen_logits.bin ([B, N, V] fp32, the
// logits each pick was made from).
static int run_generate_check(const std::string& dir, const Device& dev, size_t P, size_t N) {
    std::ifstream cf(dir + "/config.txt");
    size_t L, C, H, T, V, B;
    if (!(cf >> L >> C >> H >> T >> V >> B)) throw Error("bad config.txt");
    if (P < 1 || P + N > T) throw Error("generate-check: need 1 <= prompt and prompt + new <= context");
    GPTModel model(V, T, C, H, L, true, dev, DType::Float32);
    load_params(model, dir);
    auto tok = read_file(dir + "/tokens.bin");
    if (tok.size() < B * P * 4) throw Error("generate-check: tokens.bin holds fewer than B * prompt tokens");
    std::vector<int32_t> prompt(B * P);
    std::memcpy(prompt.data(), tok.data(), prompt.size() * 4);
    auto caches = model.make_caches(B, T, dev);
    std::vector<int32_t> gen(B * N);
    std::vector<float> glog(B * N * V);
    Tensor x(DType::Int32, prompt, std::vector<size_t>{B, P}, "prompt", dev);
    for (size_t i = 0; i < N; ++i) {
        Tensor logits = model.forward_cached(x, caches);  // [B, t, V]
        const size_t t = logits.shape()[1];
        Tensor last = logits.slice(1, t - 1, t - 1);      // [B, 1, V]
        Tensor next = argmax(last);                       // [B, 1] Int32 on the device
        const std::vector<double> pick = next.to_host_double();
        const std::vector<float> lh = last.to_host_float();
        for (size_t b = 0; b < B; ++b) {
            gen[b * N + i] = (int32_t)pick[b];
            std::memcpy(&glog[(b * N + i) * V], &lh[b * V], V * 4);
        }
        x = next;
    }
    {
        std::ofstream f(dir + "/generated.bin", std::ios::binary);
        f.write(reinterpret_cast<const char*>(gen.data()), (std::streamsize)(gen.size() * 4));
    }
    write_f32(dir + "/gen_logits.bin", glog);
    sync(dev);
    std::cout << "generate-check ok\n";
    return 0;
}

// ----------------------------------------------------------------- generate
// Greedy generation with KV caches on hip:0: a random prompt of P tokens per
// sequence, then N new tokens.  Each pick stays on the device as the next
// step's input ([B, 1] Int32 from argmax), so the host enqueues step after
// step without waiting for the GPU; the tokens are read back after the loop.
static size_t arg(int argc, char** argv, const char* name, size_t def);
static void init_normal(Module& m, float stddev, const Device& dev);

static int run_generate(int argc, char** argv) {
    const size_t L = arg(argc, argv, "--layers", 12), C = arg(argc, argv, "--dmodel", 768),
                 H = arg(argc, argv, "--heads", 12), V = arg(argc, argv, "--vocab", 8192),
                 B = arg(argc, argv, "--batch", 8), P = arg(argc, argv, "--prompt", 512),
                 N = arg(argc, argv, "--new", 64), T = arg(argc, argv, "--ctx", 1024);
    if (P + N > T) throw Error("generate: prompt + new tokens exceed the context size");
    const Device dev = Device::hip(0);
    RandomGenerator::initializeWithSeed(42);
    GPTModel model(V, T, C, H, L, true, dev, DType::Float32);
    init_normal(model, 0.02f, dev);
    std::mt19937_64 rng(42);
    std::uniform_int_distribution<int> tokd(0, (int)V - 1);
    std::vector<int32_t> prompt(B * P);
    for (auto& t : prompt) t = tokd(rng);
    auto pick_last = [&](const Tensor& logits) {
        // the greedy pick of the last position: [B, 1] Int32 on the device
        const size_t t = logits.shape()[1];
        return argmax(logits.slice(1, t - 1, t - 1));
    };
    auto run_once = [&](double* prefill_ms, double* decode_ms, std::vector<int32_t>* out) {
        auto caches = model.make_caches(B, T, dev);
        Tensor xp(DType::Int32, prompt, std::vector<size_t>{B, P}, "prompt", dev);
        sync(dev);
        const auto t0 = std::chrono::steady_clock::now();
        std::vector<Tensor> picks;
        picks.push_back(pick_last(model.forward_cached(xp, caches)));
        sync(dev);
        const auto t1 = std::chrono::steady_clock::now();
        for (size_t i = 1; i < N; ++i) picks.push_back(pick_last(model.forward_cached(picks.back(), caches)));
        out->assign(B * N, 0);  // step-major: token i of sequence b at i * B + b
        for (size_t i = 0; i < N; ++i) {
            const std::vector<double> h = picks[i].to_host_double();
            for (size_t b = 0; b < B; ++b) (*out)[i * B + b] = (int32_t)h[b];
        }
        const auto t2 = std::chrono::steady_clock::now();
        *prefill_ms = std::chrono::duration<double, std::milli>(t1 - t0).count();
        *decode_ms = std::chrono::duration<double, std::milli>(t2 - t1).count();
    };
    double pm = 0, dm = 0;
    std::vector<int32_t> gen;
    run_once(&pm, &dm, &gen);  // warm-up (plans, caches)
    run_once(&pm, &dm, &gen);
    const double steps = (double)(N - 1);
    std::printf(
        "{\"workload\": \"GPT greedy generation L%zu C%zu H%zu V%zu B%zu prompt %zu new %zu, KV cache\", "
        "\"prefill_ms\": %.3f, \"decode_ms_per_token\": %.4f, \"decode_tokens_per_s\": %.1f, "
        "\"first_tokens\": [%d, %d, %d]}\n",
        L, C, H, V, B, P, N, pm, dm / steps, (double)B * steps / (dm * 1e-3), gen[0], gen.size() > 1 ? gen[1] : 0,
        gen.size() > 2 ? gen[2] : 0);
    return 0;
}

// ---------------------------------------------------------------- fullcheck
// Properties of one full-size training step (config 3 by default) that need
// no oracle run at that size:
//   - params0.bin / grads.bin / params1.bin: every parameter before the step,
//     its gradient and its value after AdamW (fp32, concatenated in the order
//     of params.txt: "name numel" lines), for an elementwise check of the
//     update and of finiteness;
//   - dirderiv.txt: directional derivatives.  For a direction u (N(0, 1) per
//     element, seeded) over a set of parameters and a step h, the loss at
//     P + h u and P - h u (forward only) against the gradient's prediction
//     sum g . (P+ - P-) / 2h over the realised fp32 perturbations.  Sets: all
//     parameters, then each parameter type across the layers.  Lines:
//     "set h L0 Lplus Lminus predicted".
static int run_fullcheck(int argc, char** argv) {
    const std::string dir = argv[2];
    const size_t L = arg(argc, argv, "--layers", 12), C = arg(argc, argv, "--dmodel", 768),
                 H = arg(argc, argv, "--heads", 12), T = arg(argc, argv, "--ctx", 1024),
                 V = arg(argc, argv, "--vocab", 8192), B = arg(argc, argv, "--batch", 8);
    const Device dev = Device::hip(0);
    RandomGenerator::initializeWithSeed(42);
    GPTModel model(V, T, C, H, L, true, dev, DType::Float32);
    init_normal(model, 0.02f, dev);
    std::mt19937_64 rng(42);
    std::uniform_int_distribution<int> tokd(0, (int)V - 1);
    std::vector<int32_t> seq(B * (T + 1));
    for (auto& t : seq) t = tokd(rng);
    std::vector<int32_t> xs(B * T), ys(B * T);
    for (size_t b = 0; b < B; ++b)
        for (size_t t = 0; t < T; ++t) {
            xs[b * T + t] = seq[b * (T + 1) + t];
            ys[b * T + t] = seq[b * (T + 1) + t + 1];
        }
    Tensor x(DType::Int32, xs, std::vector<size_t>{B, T}, "tokens", dev);
    Tensor y(DType::Int32, ys, std::vector<size_t>{B, T}, "targets", dev);

    // parameters by state-dict name
    std::vector<std::pair<std::string, Tensor*>> named;
    {
        StateDict sd = model.state_dict();
        std::vector<Tensor*> params = model.parameters();
        for (auto& [name, t] : sd)
            for (Tensor* p : params)
                if (GetImpl(*p) == GetImpl(t)) named.emplace_back(name, p);
    }
    std::vector<std::vector<float>> p0, g;
    CrossEntropyLoss loss_fn;
    OptimizerAdamW opt(model.parameters());
    Tensor logits = model.forward(x);
    Tensor loss = loss_fn(logits, y);
    loss.backward();
    const double L0 = loss.to_host_float()[0];
    {
        std::ofstream idx(dir + "/params.txt");
        std::ofstream fp(dir + "/params0.bin", std::ios::binary), fg(dir + "/grads.bin", std::ios::binary);
        for (auto& [name, p] : named) {
            if (!p->grad()) throw Error("fullcheck: no gradient for " + name);
            p0.push_back(p->to_host_float());
            g.push_back(p->grad()->to_host_float());
            idx << name << " " << p0.back().size() << "\n";
            fp.write(reinterpret_cast<const char*>(p0.back().data()), (std::streamsize)(p0.back().size() * 4));
            fg.write(reinterpret_cast<const char*>(g.back().data()), (std::streamsize)(g.back().size() * 4));
        }
    }
    opt.step();
    opt.zero_grad();
    {
        std::ofstream fp(dir + "/params1.bin", std::ios::binary);
        for (auto& [name, p] : named) {
            const std::vector<float> v = p->to_host_float();
            fp.write(reinterpret_cast<const char*>(v.data()), (std::streamsize)(v.size() * 4));
        }
    }
    sync(dev);
    std::cout << "step done: loss " << L0 << "\n" << std::flush;

    // directional derivatives (forward only, parameters restored from p0 after each set)
    auto type_of = [](const std::string& name) {
        return name.rfind("block", 0) == 0 ? "block*" + name.substr(name.find('.')) : name;
    };
    std::vector<std::string> sets{"all"};
    for (auto& [name, p] : named) {
        const std::string t = type_of(name);
        if (std::find(sets.begin(), sets.end(), t) == sets.end()) sets.push_back(t);
    }
    auto loss_now = [&]() {
        NoGradGuard ng;
        Tensor lg = model.forward(x);
        return (double)loss_fn(lg, y).to_host_float()[0];
    };
    std::ofstream out(dir + "/dirderiv.txt");
    out.precision(17);
    const double hs[] = {3e-4, 1e-3, 3e-3};
    for (size_t si = 0; si < sets.size(); ++si) {
        std::vector<size_t> members;
        for (size_t i = 0; i < named.size(); ++i)
            if (sets[si] == "all" || type_of(named[i].first) == sets[si]) members.push_back(i);
        std::vector<std::vector<float>> u(members.size());
        for (size_t m = 0; m < members.size(); ++m) {
            std::mt19937_64 ur(1000003ULL * (si + 1) + members[m]);
            std::normal_distribution<float> nd(0.f, 1.f);
            u[m].resize(p0[members[m]].size());
            for (float& e : u[m]) e = nd(ur);
        }
        for (const double h : hs) {
            double pred = 0.0, lp = 0.0, lm = 0.0;
            std::vector<std::vector<float>> plus(members.size());
            for (int sign : {1, -1}) {
                for (size_t m = 0; m < members.size(); ++m) {
                    const std::vector<float>& base = p0[members[m]];
                    std::vector<float> v(base.size());
                    for (size_t e = 0; e < v.size(); ++e) v[e] = base[e] + (float)(sign * h) * u[m][e];
                    if (sign > 0) {
                        plus[m] = v;
                    } else {
                        const std::vector<float>& gm = g[members[m]];
                        for (size_t e = 0; e < v.size(); ++e)
                            pred += (double)gm[e] * ((double)plus[m][e] - (double)v[e]);
                    }
                    set_param(*named[members[m]].second, v);
                }
                (sign > 0 ? lp : lm) = loss_now();
            }
            pred /= 2.0 * h;
            for (size_t m = 0; m < members.size(); ++m) set_param(*named[members[m]].second, p0[members[m]]);
            out << sets[si] << " " << h << " " << L0 << " " << lp << " " << lm << " " << pred << "\n" << std::flush;
        }
        std::cout << "direction " << sets[si] << " done\n" << std::flush;
    }
    std::cout << "fullcheck ok\n";
    return 0;
}

// -------------------------------------------------------------------- bench
static size_t arg(int argc, char** argv, const char* name, size_t def) {
    for (int i = 2; i + 1 < argc; ++i)
        if (std::strcmp(argv[i], name) == 0) return (size_t)std::strtoull(argv[i + 1], nullptr, 10);
    return def;
}
static bool flag(int argc, char** argv, const char* name) {
    for (int i = 2; i < argc; ++i)
        if (std::strcmp(argv[i], name) == 0) return true;
    return false;
}

static void init_normal(Module& m, float stddev, const Device& dev) {
    // Linear weights and the embedding ~ N(0, stddev); biases 0; LayerNorm as built.
    StateDict sd = m.state_dict();
    std::vector<Tensor*> params = m.parameters();
    for (auto& [name, t] : sd) {
        Tensor* p = nullptr;
        for (Tensor* q : params)
            if (GetImpl(*q) == GetImpl(t)) p = q;
        if (!p) continue;
        const auto ends = [&](const char* s) {
            const size_t n = std::strlen(s);
            return name.size() >= n && name.compare(name.size() - n, n, s) == 0;
        };
        std::vector<float> v;
        if (ends(".weights") || ends("tok_embedding.weight"))
            v = RandomGenerator::generateNormalFloatVector(p->numel(), 0.0f, stddev);
        else if (ends(".bias"))
            v.assign(p->numel(), 0.0f);
        else
            continue;
        Tensor h(DType::Float32, v, p->shape(), p->name(), Device::cpu());
        Tensor d = h.to(dev);
        if (p->dtype() != DType::Float32) throw Error("bench init: Float32 parameters only");
        d.set_requires_grad(true);
        *p = d;
    }
}

static int run_bench(int argc, char** argv) {
    const size_t L = arg(argc, argv, "--layers", 12), C = arg(argc, argv, "--dmodel", 768),
                 H = arg(argc, argv, "--heads", 12), T = arg(argc, argv, "--ctx", 1024),
                 V = arg(argc, argv, "--vocab", 8192), B = arg(argc, argv, "--batch", 8),
                 K = arg(argc, argv, "--steps", 5), W = arg(argc, argv, "--warmup", 2);
    const bool tied = !flag(argc, argv, "--untied");
    const Device dev = Device::hip(0);
    RandomGenerator::initializeWithSeed(42);
    GPTModel model(V, T, C, H, L, tied, dev, DType::Float32);
    init_normal(model, 0.02f, dev);
    size_t nparams = 0;
    for (Tensor* p : model.parameters()) nparams += p->numel();

    std::mt19937_64 rng(42);
    std::uniform_int_distribution<int> tokd(0, (int)V - 1);
    std::vector<int32_t> seq(B * (T + 1));
    for (auto& t : seq) t = tokd(rng);
    std::vector<int32_t> xs(B * T), ys(B * T);
    for (size_t b = 0; b < B; ++b)
        for (size_t t = 0; t < T; ++t) {
            xs[b * T + t] = seq[b * (T + 1) + t];
            ys[b * T + t] = seq[b * (T + 1) + t + 1];
        }
    Tensor x(DType::Int32, xs, std::vector<size_t>{B, T}, "tokens", dev);
    Tensor y(DType::Int32, ys, std::vector<size_t>{B, T}, "targets", dev);
    CrossEntropyLoss loss_fn;
    OptimizerAdamW opt(model.parameters(), 3e-4f);
    float first_loss = 0.f, last_loss = 0.f;
    auto step = [&]() {
        Tensor logits = model.forward(x);
        Tensor loss = loss_fn(logits, y);
        loss.backward();
        opt.step();
        opt.zero_grad();
        return loss;
    };
    for (size_t i = 0; i < W; ++i) {
        Tensor l = step();
        if (i == 0) first_loss = l.to_host_float()[0];
    }
    sync(dev);
    const auto t0 = std::chrono::steady_clock::now();
    Tensor l;
    for (size_t i = 0; i < K; ++i) l = step();
    sync(dev);
    const auto t1 = std::chrono::steady_clock::now();
    last_loss = l.to_host_float()[0];
    const double step_ms = std::chrono::duration<double, std::milli>(t1 - t0).count() / (double)K;

    // Attention share: the fused attention forward + backward of one layer at
    // this shape, timed alone (wall clock between device synchronisations), times L.
    double attn_ms = 0.0;
    {
        std::vector<float> qv(B * T * 3 * C);
        std::mt19937 g2(7);
        std::normal_distribution<float> nd(0.f, 1.f);
        for (auto& v : qv) v = nd(g2);
        Tensor qkv = Tensor(DType::Float32, qv, std::vector<size_t>{B, T, 3 * C}, "qkv", dev, true);
        std::vector<float> gv(B * T * C);
        for (auto& v : gv) v = nd(g2);
        Tensor gy(DType::Float32, gv, std::vector<size_t>{B, T, C}, "gy", dev);
        auto once = [&]() {
            Tensor yy = qkv_attention(qkv, H, true);
            yy.backward(gy);
            qkv.grad() = nullptr;
        };
        once();
        sync(dev);
        const int reps = 10;
        const auto a0 = std::chrono::steady_clock::now();
        for (int i = 0; i < reps; ++i) once();
        sync(dev);
        const auto a1 = std::chrono::steady_clock::now();
        attn_ms = std::chrono::duration<double, std::milli>(a1 - a0).count() / reps * (double)L;
    }
    const double tokens = (double)(B * T);
    std::printf(
        "{\"workload\": \"GPT training step L%zu C%zu H%zu T%zu V%zu B%zu %s\", \"tokens_per_step\": %.0f, "
        "\"ms_per_step\": %.4f, \"tokens_per_s\": %.1f, \"attention_ms_per_step\": %.4f, "
        "\"attention_share\": %.4f, \"params\": %zu, \"loss_first\": %.6f, \"loss_last\": %.6f, "
        "\"steps\": %zu, \"warmup\": %zu}\n",
        L, C, H, T, V, B, tied ? "tied" : "untied", tokens, step_ms, tokens / (step_ms * 1e-3), attn_ms,
        attn_ms / step_ms, nparams, first_loss, last_loss, K, W);
    return 0;
}

int main(int argc, char** argv) {
    try {
        if (flag(argc, argv, "--deterministic")) inf_set_deterministic(1);
        if (argc >= 2 && std::strcmp(argv[1], "bench") == 0) return run_bench(argc, argv);
        if (argc >= 2 && std::strcmp(argv[1], "generate") == 0) return run_generate(argc, argv);
        if (argc >= 4 && std::strcmp(argv[1], "decode-check") == 0) {
            const Device dev = std::strcmp(argv[3], "hip") == 0 ? Device::hip(0) : Device::cpu();
            return run_decode_check(argv[2], dev, arg(argc, argv, "--prefill", 4));
        }
        if (argc >= 3 && std::strcmp(argv[1], "fullcheck") == 0) return run_fullcheck(argc, argv);
        if (argc >= 4 && std::strcmp(argv[1], "generate-check") == 0) {
            const Device dev = std::strcmp(argv[3], "hip") == 0 ? Device::hip(0) : Device::cpu();
            return run_generate_check(argv[2], dev, arg(argc, argv, "--prompt", 4), arg(argc, argv, "--new", 8));
        }
        if (argc >= 4 && std::strcmp(argv[1], "step") == 0) {
            const Device dev = std::strcmp(argv[3], "hip") == 0 ? Device::hip(0) : Device::cpu();
            return run_step(argv[2], dev, !flag(argc, argv, "--untied"));
        }
        std::cerr << "usage: gpt bench [options] | gpt step <dir> <cpu|hip> [--untied] | gpt decode-check <dir> "
                     "<cpu|hip> [--prefill P] | gpt generate-check <dir> <cpu|hip> [--prompt P] [--new N] | "
                     "gpt generate [options]\n";
        return 2;
    } catch (const std::exception& e) {
        std::cerr << "error: " << e.what() << "\n";
        return 1;
    }
}
