// engine.cpp -- autograd engine and the generic nodes (include/inferno/gradengine/engine.h,
// include/inferno/gradfn/node.h).  Behaviour follows src/inferno/gradengine/engine.cpp:32-199:
// topological order from the root's grad edge, seed, reverse execution, release.
#include <algorithm>
#include <functional>
#include <map>
#include <unordered_set>

#include "detail.h"
#include "inferno/core/ops.h"
#include "inferno/gradengine/engine.h"
#include "inferno/gradfn/node.h"

namespace Inferno {

bool grad_enabled = true;

namespace {
// Gradients waiting at (node, slot) during one backward pass.
thread_local std::map<std::pair<Node*, int>, Tensor> g_grads;
}  // namespace

void Engine::accumulate(Node* node, int slot, const Tensor& g) {
    if (!node) return;
    NoGradGuard ng;
    auto key = std::make_pair(node, slot);
    auto it = g_grads.find(key);
    if (it == g_grads.end())
        g_grads.emplace(key, g);
    else
        it->second = add(it->second, g);
}

Tensor Engine::grad_in(Node* node, int slot) {
    auto it = g_grads.find(std::make_pair(node, slot));
    if (it == g_grads.end()) throw Error("Engine::grad_in: no gradient reached node '" + node->name() + "'");
    return it->second;
}

void Engine::backward(const Tensor& root) {
    Tensor seed;
    {
        NoGradGuard ng;
        seed = Tensor::ones_like(root);
    }
    backward(root, seed);
}

void Engine::backward(const Tensor& root, const Tensor& seed) {
    auto edge = GetImpl(root)->grad_edge();
    if (!edge) throw Error("backward: '" + root.name() + "' does not require grad");
    if (seed.shape() != root.shape()) throw Error("backward: seed shape does not match the root");
    if (seed.device() != root.device()) throw Error("backward: seed is on another device");

    std::vector<std::shared_ptr<Node>> order;  // post-order: inputs before consumers
    std::unordered_set<Node*> seen;
    std::function<void(const std::shared_ptr<Node>&)> visit = [&](const std::shared_ptr<Node>& n) {
        if (!seen.insert(n.get()).second) return;
        std::vector<Tensor> ins;
        n->get_inputs(ins);
        for (const Tensor& t : ins) {
            if (!t.defined()) continue;
            auto e = GetImpl(t)->grad_edge();
            if (e) visit(e);
        }
        order.push_back(n);
    };
    visit(edge);

    g_grads.clear();
    accumulate(edge.get(), 0, seed);
    for (auto it = order.rbegin(); it != order.rend(); ++it) {
        if (g_grads.count(std::make_pair(it->get(), 0)) == 0) continue;  // nothing flowed here
        (*it)->backward();
    }
    for (auto& n : order) n->release();
    g_grads.clear();
}

// ------------------------------------------------------------------- nodes --
AccumulateGrad::AccumulateGrad(std::weak_ptr<TensorImpl> leaf) : m_leaf(std::move(leaf)) {}

void AccumulateGrad::backward() {
    NoGradGuard ng;
    Tensor g = Engine::grad_in(this, 0);
    auto leaf = m_leaf.lock();
    if (!leaf) return;
    if (!g.is_contiguous()) g = g.contiguous();
    if (leaf->grad())
        *leaf->grad() = add(*leaf->grad(), g);
    else
        leaf->grad() = std::make_shared<Tensor>(g);
}

static void send(const Tensor& input, const Tensor& g) {
    auto e = GetImpl(input)->grad_edge();
    if (e) Engine::accumulate(e.get(), 0, g);
}

static bool wants_grad(const Tensor& t) { return t.defined() && GetImpl(t)->grad_edge() != nullptr; }

// Sum of all elements as a one-element tensor (the gradient of a broadcast scalar).
static Tensor sum_all(const Tensor& g, const Tensor& like) {
    auto v = g.to_host_double();
    double s = 0;
    for (double x : v) s += x;
    return Tensor::full({1}, s, like.dtype(), like.device(), "sum");
}

// The gradient of an operand that broadcasting expanded: summed back to the
// operand's shape (a single element, or the trailing block of a broadcast).
static Tensor reduce_to(const Tensor& g, const Tensor& like) {
    if (g.shape() == like.shape()) return g;
    if (like.numel() == 1 && g.numel() != 1) return sum_all(g, like);
    return sum_to_shape(g, like.shape());
}

MultiplyBackward::MultiplyBackward(const Tensor& a, const Tensor& b) : m_a(a), m_b(b) { set_name("MultiplyBackward"); }
void MultiplyBackward::backward() {
    NoGradGuard ng;
    Tensor g = Engine::grad_in(this, 0);
    if (wants_grad(m_a)) send(m_a, reduce_to(multiply(g, m_b), m_a));
    if (wants_grad(m_b)) send(m_b, reduce_to(multiply(g, m_a), m_b));
}
void MultiplyBackward::release() { m_a = Tensor(); m_b = Tensor(); }
void MultiplyBackward::get_inputs(std::vector<Tensor>& out) const { out.push_back(m_a); out.push_back(m_b); }

AddBackward::AddBackward(const Tensor& a, const Tensor& b) : m_a(a), m_b(b) { set_name("AddBackward"); }
void AddBackward::backward() {
    NoGradGuard ng;
    Tensor g = Engine::grad_in(this, 0);
    if (wants_grad(m_a)) send(m_a, reduce_to(g, m_a));
    if (wants_grad(m_b)) send(m_b, reduce_to(g, m_b));
}
void AddBackward::release() { m_a = Tensor(); m_b = Tensor(); }
void AddBackward::get_inputs(std::vector<Tensor>& out) const { out.push_back(m_a); out.push_back(m_b); }

TransposeBackward::TransposeBackward(const Tensor& a, int dima, int dimb) : m_a(a), m_dima(dima), m_dimb(dimb) {
    set_name("TransposeBackward");
}
void TransposeBackward::backward() {
    NoGradGuard ng;
    send(m_a, Engine::grad_in(this, 0).transpose(m_dima, m_dimb));
}
void TransposeBackward::release() { m_a = Tensor(); }
void TransposeBackward::get_inputs(std::vector<Tensor>& out) const { out.push_back(m_a); }

ReshapeBackward::ReshapeBackward(const Tensor& a) : m_a(a), m_shape(a.shape()) { set_name("ReshapeBackward"); }
void ReshapeBackward::backward() {
    NoGradGuard ng;
    send(m_a, Engine::grad_in(this, 0).contiguous().reshape(m_shape));
}
void ReshapeBackward::release() { m_a = Tensor(); }
void ReshapeBackward::get_inputs(std::vector<Tensor>& out) const { out.push_back(m_a); }

ContiguousBackward::ContiguousBackward(const Tensor& a) : m_a(a) { set_name("ContiguousBackward"); }
void ContiguousBackward::backward() {
    NoGradGuard ng;
    send(m_a, Engine::grad_in(this, 0));
}
void ContiguousBackward::release() { m_a = Tensor(); }
void ContiguousBackward::get_inputs(std::vector<Tensor>& out) const { out.push_back(m_a); }

SliceBackward::SliceBackward(const Tensor& a, int axis, size_t start, size_t step)
    : m_a(a), m_axis(axis), m_start(start), m_step(step) {
    set_name("SliceBackward");
}
void SliceBackward::backward() {
    NoGradGuard ng;
    Tensor g = Engine::grad_in(this, 0);
    Tensor full = Tensor::zeros(m_a.shape(), g.dtype(), g.device(), "slice_grad");
    auto st = full.strides();
    const size_t off = m_start * st[m_axis];
    st[m_axis] *= m_step;
    const size_t esz = dtype_size(g.dtype());
    if (g.device().is_cpu()) {
        detail::copy_strided_host(static_cast<const char*>(g.data_ptr()), g.strides(),
                                  static_cast<char*>(full.data_ptr()) + off * esz, st, g.shape(), esz);
    } else {
        auto shape = detail::to_i64(g.shape());
        auto sst = detail::to_i64(g.strides());
        auto dst = detail::to_i64(st);
        detail::DeviceGuard dg(g.device().index);
        detail::status_check(inf_copy_strided(g.data_ptr(), sst.data(), static_cast<char*>(full.data_ptr()) + off * esz,
                                              dst.data(), (int)g.ndim(), shape.data(), (int)esz, detail::stream_of(g)),
                             "inf_copy_strided");
    }
    send(m_a, full);
}
void SliceBackward::release() { m_a = Tensor(); }
void SliceBackward::get_inputs(std::vector<Tensor>& out) const { out.push_back(m_a); }

// --------------------------------------------------- element-wise add / mul --
static Tensor binary(int op, const Tensor& A, const Tensor& B, const char* what) {
    detail::same_device(A, B, what);
    if (A.dtype() != B.dtype()) throw Error(std::string(what) + ": dtype mismatch");
    const bool a_s = A.numel() == 1, b_s = B.numel() == 1;
    // Trailing broadcast: one operand's shape (leading ones dropped) is a suffix
    // of the other's, e.g. [B, T, C] + [T, C] or [M, N] + [N].
    int bcast = 0;  // 1: B repeats over A's leading dims, 2: A repeats over B's
    if (!a_s && !b_s && A.shape() != B.shape()) {
        const auto suffix = [](const std::vector<size_t>& big, const std::vector<size_t>& small) {
            size_t i = 0;
            while (i < small.size() && small[i] == 1) ++i;
            const size_t k = small.size() - i;
            return k <= big.size() && std::equal(small.begin() + (long)i, small.end(), big.end() - (long)k);
        };
        if (A.ndim() >= B.ndim() && suffix(A.shape(), B.shape()))
            bcast = 1;
        else if (B.ndim() >= A.ndim() && suffix(B.shape(), A.shape()))
            bcast = 2;
        else
            throw Error(std::string(what) + ": shapes must match, broadcast over leading dimensions, "
                                            "or one side be a single element");
    }
    Tensor a = A, b = B;
    {
        NoGradGuard ng;
        if (!a.is_contiguous()) a = a.contiguous();
        if (!b.is_contiguous()) b = b.contiguous();
    }
    const Tensor& big = (bcast == 2 || (a_s && !b_s)) ? b : a;
    Tensor out(A.dtype(), big.shape(), what, A.device(), false);
    const size_t n = out.numel();
    if (bcast) {
        const Tensor& full = bcast == 1 ? a : b;
        const Tensor& rep = bcast == 1 ? b : a;
        const size_t nb = rep.numel();
        if (A.device().is_cpu()) {
            const char* pf = static_cast<const char*>(full.data_ptr());
            const char* pr = static_cast<const char*>(rep.data_ptr());
            char* po = static_cast<char*>(out.data_ptr());
            const size_t esz = dtype_size(A.dtype());
            for (size_t i = 0; i < n; ++i) {
                const double x = detail::load_elem(pf + i * esz, A.dtype());
                const double y = detail::load_elem(pr + (i % nb) * esz, A.dtype());
                detail::store_elem(po + i * esz, A.dtype(), op == INF_BIN_ADD ? (float)x + (float)y : (float)x * (float)y);
            }
        } else if (n) {
            detail::DeviceGuard g(A.device().index);
            detail::status_check(inf_binary_bcast(op, full.data_ptr(), rep.data_ptr(), out.data_ptr(), (int64_t)n,
                                                  (int64_t)nb, detail::inf_dt(A.dtype(), what), detail::stream_of(A)),
                                 "inf_binary_bcast");
        }
    } else if (A.device().is_cpu()) {
        const char* pa = static_cast<const char*>(a.data_ptr());
        const char* pb = static_cast<const char*>(b.data_ptr());
        char* po = static_cast<char*>(out.data_ptr());
        const size_t esz = dtype_size(A.dtype());
        if (A.dtype() == DType::Float32) {
            const float* fa = reinterpret_cast<const float*>(pa);
            const float* fb = reinterpret_cast<const float*>(pb);
            float* fo = reinterpret_cast<float*>(po);
            for (size_t i = 0; i < n; ++i) {
                const float x = fa[a_s ? 0 : i], y = fb[b_s ? 0 : i];
                fo[i] = op == INF_BIN_ADD ? x + y : x * y;
            }
        } else {
            for (size_t i = 0; i < n; ++i) {
                const double x = detail::load_elem(pa + (a_s ? 0 : i) * esz, A.dtype());
                const double y = detail::load_elem(pb + (b_s ? 0 : i) * esz, A.dtype());
                detail::store_elem(po + i * esz, A.dtype(), op == INF_BIN_ADD ? x + y : x * y);
            }
        }
    } else {
        detail::DeviceGuard g(A.device().index);
        detail::status_check(inf_binary(op, a.data_ptr(), b.data_ptr(), out.data_ptr(), (int64_t)n, a_s && !b_s ? 1 : 0,
                                        b_s && !a_s ? 1 : 0, detail::inf_dt(A.dtype(), what), detail::stream_of(A)),
                             "inf_binary");
    }
    if (grad_enabled && (A.requires_grad() || B.requires_grad())) {
        out.set_requires_grad(true);
        if (op == INF_BIN_ADD)
            GetImpl(out)->gradfn() = std::make_shared<AddBackward>(A, B);
        else
            GetImpl(out)->gradfn() = std::make_shared<MultiplyBackward>(A, B);
    }
    return out;
}

Tensor add(const Tensor& A, const Tensor& B) { return binary(INF_BIN_ADD, A, B, "add"); }
Tensor multiply(const Tensor& A, const Tensor& B) { return binary(INF_BIN_MUL, A, B, "multiply"); }

}  // namespace Inferno
