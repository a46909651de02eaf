// attention.cpp -- scaled_dot_product_attention, AttentionBackward, attention_decode
// (include/inferno/functional/attention.h).
//
// HIP tensors go to the fused kernels through the C-ABI (inf_attn_fwd /
// inf_attn_bwd / inf_attn_decode), reading q, k, v, dO in place through their
// strides.  CPU tensors run the reference's own chain per head -- q@k^T with
// fp32 sums in k order (cpuops.h:412-431), a separate * scale rounding,
// masked_fill(triu(ones, 1 + Tk - Tq), -1e9f), softmax with exp in double
// (softmax_kernels.h:77-102), P@V; and for the backward MMBackward /
// SoftmaxBackward / MultiplyBackward / TransposeBackward (mmbackward.cpp:77-80,
// softmaxbackward.h:111-128, multiplybackward.cpp:41) -- so CPU results equal
// what Inferno's CPU path computes.  A HIP tensor never takes the CPU branch.
#include <algorithm>
#include <cfloat>
#include <cmath>
#include <mutex>

#include "detail.h"
#include "inferno/functional/attention.h"
#include "inferno/gradengine/engine.h"

namespace Inferno {

namespace {

struct Shape4 {
    size_t B, H, Tq, Tk, D;
};

Shape4 check_qkv(const Tensor& q, const Tensor& k, const Tensor& v, const char* what) {
    if (!q.defined() || !k.defined() || !v.defined()) throw Error(std::string(what) + ": undefined input");
    if (q.ndim() != 4 || k.ndim() != 4 || v.ndim() != 4)
        throw Error(std::string(what) + ": q, k, v must be 4-D [B, H, T, D]");
    detail::same_device(q, k, what);
    detail::same_device(q, v, what);
    if (q.dtype() != k.dtype() || q.dtype() != v.dtype()) throw Error(std::string(what) + ": dtype mismatch");
    if (q.dtype() != DType::Float32 && q.dtype() != DType::BFloat16)
        throw Error(std::string(what) + ": Float32 or BFloat16 expected");
    const auto &qs = q.shape(), &ks = k.shape(), &vs = v.shape();
    if (ks != vs || qs[0] != ks[0] || qs[1] != ks[1] || qs[3] != ks[3])
        throw Error(std::string(what) + ": shapes must be q [B,H,Tq,D], k = v [B,H,Tk,D]");
    return {qs[0], qs[1], qs[2], ks[2], qs[3]};
}

float resolve_scale(float scale, size_t D) { return std::isnan(scale) ? 1.0f / std::sqrt((float)D) : scale; }

// A view the C-ABI accepts as is (unit d stride, 4-element aligned rows), else a dense copy.
Tensor abi_view(const Tensor& t) {
    const auto& st = t.strides();
    const size_t esz = dtype_size(t.dtype());
    const bool ok = st[3] == 1 && st[0] % 4 == 0 && st[1] % 4 == 0 && st[2] % 4 == 0 &&
                    reinterpret_cast<uintptr_t>(t.data_ptr()) % (4 * esz) == 0;
    if (ok) return t;
    NoGradGuard ng;
    return detail::dense_copy(t);  // fresh allocation: aligned, dense
}

// Workspace of at least `bytes`, 256-byte aligned (the C-ABI's requirement).
struct Workspace {
    Tensor buf;
    void* ptr = nullptr;
    Workspace(size_t bytes, const Device& dev)
        : buf(DType::Float32, std::vector<size_t>{bytes / 4 + 64 + 1}, "attention_ws", dev, false) {
        const uintptr_t p = reinterpret_cast<uintptr_t>(buf.data_ptr());
        ptr = reinterpret_cast<void*>((p + 255) & ~uintptr_t(255));
    }
};

// The decode workspace of each device: grown on demand and reused by every call
// (all calls on a device are ordered on that device's library stream).  Kept for
// the life of the process (never destroyed, so no free runs after HIP teardown).
void* decode_workspace(size_t bytes, const Device& dev) {
    static std::mutex mu;
    static auto* per_device = new std::vector<Tensor>();
    if (bytes == 0) return nullptr;
    std::lock_guard<std::mutex> lk(mu);
    if (per_device->size() <= (size_t)dev.index) per_device->resize((size_t)dev.index + 1);
    Tensor& t = (*per_device)[(size_t)dev.index];
    if (!t.defined() || t.size() < bytes + 256) t = Tensor(DType::Float32, {bytes / 4 + 128}, "decode_ws", dev, false);
    const uintptr_t p = reinterpret_cast<uintptr_t>(t.data_ptr());
    return reinterpret_cast<void*>((p + 255) & ~uintptr_t(255));
}

inf_strides strides_of(const Tensor& t) {
    const auto& s = t.strides();
    return inf_strides{(int64_t)s[0], (int64_t)s[1], (int64_t)s[2], (int64_t)s[3]};
}

// ---- CPU branch: the reference chain, one head at a time -------------------
std::vector<float> gather_head(const Tensor& t, size_t b, size_t h) {
    const auto& sh = t.shape();
    const auto& st = t.strides();
    const size_t T = sh[2], D = sh[3], esz = dtype_size(t.dtype());
    std::vector<float> out(T * D);
    const char* base = static_cast<const char*>(t.data_ptr());
    for (size_t i = 0; i < T; ++i)
        for (size_t d = 0; d < D; ++d)
            out[i * D + d] = (float)detail::load_elem(base + (b * st[0] + h * st[1] + i * st[2] + d * st[3]) * esz, t.dtype());
    return out;
}

void scatter_head(Tensor& t, size_t b, size_t h, const std::vector<float>& x) {
    const auto& sh = t.shape();
    const auto& st = t.strides();
    const size_t T = sh[2], D = sh[3], esz = dtype_size(t.dtype());
    char* base = static_cast<char*>(t.data_ptr());
    for (size_t i = 0; i < T; ++i)
        for (size_t d = 0; d < D; ++d)
            detail::store_elem(base + (b * st[0] + h * st[1] + i * st[2] + d * st[3]) * esz, t.dtype(), x[i * D + d]);
}

// S = (q k^T) * scale, masked; P = softmax(S).  Returns P; S keeps the masked scores.
void cpu_scores_probs(const std::vector<float>& Q, const std::vector<float>& K, size_t Tq, size_t Tk, size_t D,
                      float scale, bool causal, std::vector<float>& S, std::vector<float>& P) {
    S.assign(Tq * Tk, 0.f);
    P.assign(Tq * Tk, 0.f);
    for (size_t i = 0; i < Tq; ++i)
        for (size_t j = 0; j < Tk; ++j) {
            float sum = 0.f;
            for (size_t d = 0; d < D; ++d) sum += Q[i * D + d] * K[j * D + d];
            S[i * Tk + j] = sum;
        }
    for (float& s : S) s = s * scale;
    if (causal) {
        const int diag = 1 + (int)(Tk - Tq);
        for (size_t i = 0; i < Tq; ++i)
            for (size_t j = 0; j < Tk; ++j)
                if ((int)j - (int)i >= diag) S[i * Tk + j] = -1e9f;
    }
    for (size_t i = 0; i < Tq; ++i) {
        const float* s = &S[i * Tk];
        float* p = &P[i * Tk];
        float mx = -FLT_MAX;
        for (size_t j = 0; j < Tk; ++j)
            if (s[j] > mx) mx = s[j];
        float sum = 0.f;
        for (size_t j = 0; j < Tk; ++j) {
            p[j] = (float)std::exp((double)(s[j] - mx));
            sum += p[j];
        }
        for (size_t j = 0; j < Tk; ++j) p[j] /= sum;
    }
}

void cpu_fwd(const Tensor& q, const Tensor& k, const Tensor& v, const Shape4& s, float scale, bool causal, Tensor& out,
             Tensor& lse) {
    float* L = static_cast<float*>(lse.data_ptr());
    std::vector<float> S, P;
    for (size_t b = 0; b < s.B; ++b)
        for (size_t h = 0; h < s.H; ++h) {
            auto Q = gather_head(q, b, h), K = gather_head(k, b, h), V = gather_head(v, b, h);
            cpu_scores_probs(Q, K, s.Tq, s.Tk, s.D, scale, causal, S, P);
            std::vector<float> O(s.Tq * s.D);
            for (size_t i = 0; i < s.Tq; ++i)
                for (size_t d = 0; d < s.D; ++d) {
                    float sum = 0.f;
                    for (size_t j = 0; j < s.Tk; ++j) sum += P[i * s.Tk + j] * V[j * s.D + d];
                    O[i * s.D + d] = sum;
                }
            scatter_head(out, b, h, O);
            for (size_t i = 0; i < s.Tq; ++i) {
                double mx = -INFINITY, acc = 0.0;
                for (size_t j = 0; j < s.Tk; ++j) mx = std::max(mx, (double)S[i * s.Tk + j]);
                for (size_t j = 0; j < s.Tk; ++j) acc += std::exp((double)S[i * s.Tk + j] - mx);
                L[(b * s.H + h) * s.Tq + i] = (float)(mx + std::log(acc));
            }
        }
}

void cpu_bwd(const Tensor& q, const Tensor& k, const Tensor& v, const Tensor& g, const Shape4& s, float scale,
             bool causal, Tensor& dq, Tensor& dk, Tensor& dv) {
    std::vector<float> S, P;
    const size_t Tq = s.Tq, Tk = s.Tk, D = s.D;
    for (size_t b = 0; b < s.B; ++b)
        for (size_t h = 0; h < s.H; ++h) {
            auto Q = gather_head(q, b, h), K = gather_head(k, b, h), V = gather_head(v, b, h), G = gather_head(g, b, h);
            cpu_scores_probs(Q, K, Tq, Tk, D, scale, causal, S, P);
            std::vector<float> dP(Tq * Tk), dS(Tq * Tk), dQ(Tq * D), dK(Tk * D), dV(Tk * D);
            for (size_t i = 0; i < Tq; ++i)
                for (size_t j = 0; j < Tk; ++j) {
                    float sum = 0.f;
                    for (size_t d = 0; d < D; ++d) sum += G[i * D + d] * V[j * D + d];
                    dP[i * Tk + j] = sum;
                }
            for (size_t j = 0; j < Tk; ++j)
                for (size_t d = 0; d < D; ++d) {
                    float sum = 0.f;
                    for (size_t i = 0; i < Tq; ++i) sum += P[i * Tk + j] * G[i * D + d];
                    dV[j * D + d] = sum;
                }
            for (size_t i = 0; i < Tq; ++i) {
                float dot = 0.f;
                for (size_t j = 0; j < Tk; ++j) dot += dP[i * Tk + j] * P[i * Tk + j];
                for (size_t j = 0; j < Tk; ++j) dS[i * Tk + j] = P[i * Tk + j] * (dP[i * Tk + j] - dot);
            }
            for (float& x : dS) x = x * scale;
            for (size_t i = 0; i < Tq; ++i)
                for (size_t d = 0; d < D; ++d) {
                    float sum = 0.f;
                    for (size_t j = 0; j < Tk; ++j) sum += dS[i * Tk + j] * K[j * D + d];
                    dQ[i * D + d] = sum;
                }
            for (size_t d = 0; d < D; ++d)
                for (size_t j = 0; j < Tk; ++j) {
                    float sum = 0.f;
                    for (size_t i = 0; i < Tq; ++i) sum += Q[i * D + d] * dS[i * Tk + j];
                    dK[j * D + d] = sum;
                }
            scatter_head(dq, b, h, dQ);
            scatter_head(dk, b, h, dK);
            scatter_head(dv, b, h, dV);
        }
}

}  // namespace

Tensor scaled_dot_product_attention_lse(const Tensor& q, const Tensor& k, const Tensor& v, bool causal, float scale,
                                        Tensor* lse_out) {
    const Shape4 s = check_qkv(q, k, v, "scaled_dot_product_attention");
    if (causal && s.Tq > s.Tk) throw Error("scaled_dot_product_attention: causal needs Tq <= Tk");
    const float sc = resolve_scale(scale, s.D);
    if (!(sc > 0.f) || !std::isfinite(sc)) throw Error("scaled_dot_product_attention: scale must be finite and > 0");
    Tensor out(q.dtype(), {s.B, s.H, s.Tq, s.D}, "attention", q.device(), false);
    Tensor lse(DType::Float32, {s.B, s.H, s.Tq}, "attention_lse", q.device(), false);
    if (s.B && s.H && s.Tq && s.Tk) {
        if (q.device().is_cpu()) {
            cpu_fwd(q, k, v, s, sc, causal, out, lse);
        } else {
            Tensor qa = abi_view(q), ka = abi_view(k), va = abi_view(v);
            detail::DeviceGuard g(q.device().index);
            const inf_dtype dt = detail::inf_dt(q.dtype(), "scaled_dot_product_attention");
            size_t ws_bytes = 0;
            if (causal)
                detail::status_check(inf_attn_workspace_bytes(INF_OP_ATTN_FWD, (int)s.B, (int)s.H, (int)s.Tq,
                                                              (int)s.Tk, (int)s.D, dt, &ws_bytes),
                                     "inf_attn_workspace_bytes");
            Workspace ws(ws_bytes, q.device());
            detail::status_check(
                inf_attn_fwd(qa.data_ptr(), strides_of(qa), ka.data_ptr(), strides_of(ka), va.data_ptr(), strides_of(va),
                             out.data_ptr(), strides_of(out), static_cast<float*>(lse.data_ptr()), ws.ptr, ws_bytes,
                             (int)s.B, (int)s.H, (int)s.Tq, (int)s.Tk, (int)s.D, sc, causal ? 1 : 0, dt,
                             detail::stream_of(q)),
                "inf_attn_fwd");
        }
    }
    if (grad_enabled && (q.requires_grad() || k.requires_grad() || v.requires_grad())) {
        out.set_requires_grad(true);
        GetImpl(out)->gradfn() = std::make_shared<AttentionBackward>(q, k, v, out, lse, causal, sc);
    }
    if (lse_out) *lse_out = lse;
    return out;
}

Tensor scaled_dot_product_attention(const Tensor& q, const Tensor& k, const Tensor& v, bool causal, float scale) {
    return scaled_dot_product_attention_lse(q, k, v, causal, scale, nullptr);
}

AttentionBackward::AttentionBackward(const Tensor& q, const Tensor& k, const Tensor& v, const Tensor& out,
                                     const Tensor& lse, bool causal, float scale)
    : m_q(q),
      m_k(k),
      m_v(v),
      m_out(make_view(out, out.shape(), out.strides(), out.offset(), "attention_saved")),
      m_lse(lse),
      m_causal(causal),
      m_scale(scale) {
    set_name("AttentionBackward");
}

void AttentionBackward::backward() {
    NoGradGuard ng;
    Tensor g = Engine::grad_in(this, 0);
    const Shape4 s = check_qkv(m_q, m_k, m_v, "AttentionBackward");
    Tensor dq(m_q.dtype(), m_q.shape(), "attention_dq", m_q.device(), false);
    Tensor dk(m_k.dtype(), m_k.shape(), "attention_dk", m_k.device(), false);
    Tensor dv(m_v.dtype(), m_v.shape(), "attention_dv", m_v.device(), false);
    if (m_q.device().is_cpu()) {
        cpu_bwd(m_q, m_k, m_v, g, s, m_scale, m_causal, dq, dk, dv);
    } else {
        const inf_dtype dt = detail::inf_dt(m_q.dtype(), "AttentionBackward");
        size_t ws_bytes = 0;
        detail::status_check(inf_attn_workspace_bytes(INF_OP_ATTN_BWD, (int)s.B, (int)s.H, (int)s.Tq, (int)s.Tk,
                                                      (int)s.D, dt, &ws_bytes),
                             "inf_attn_workspace_bytes");
        Workspace ws(ws_bytes, m_q.device());
        Tensor qa = abi_view(m_q), ka = abi_view(m_k), va = abi_view(m_v), oa = abi_view(m_out), ga = abi_view(g);
        detail::DeviceGuard dg(m_q.device().index);
        detail::status_check(
            inf_attn_bwd(qa.data_ptr(), strides_of(qa), ka.data_ptr(), strides_of(ka), va.data_ptr(), strides_of(va),
                         oa.data_ptr(), strides_of(oa), ga.data_ptr(), strides_of(ga),
                         static_cast<const float*>(m_lse.data_ptr()), dq.data_ptr(), strides_of(dq), dk.data_ptr(),
                         strides_of(dk), dv.data_ptr(), strides_of(dv), ws.ptr, ws_bytes, (int)s.B, (int)s.H,
                         (int)s.Tq, (int)s.Tk, (int)s.D, m_scale, m_causal ? 1 : 0, dt, detail::stream_of(m_q)),
            "inf_attn_bwd");
    }
    if (auto e = GetImpl(m_q)->grad_edge()) Engine::accumulate(e.get(), 0, dq);
    if (auto e = GetImpl(m_k)->grad_edge()) Engine::accumulate(e.get(), 0, dk);
    if (auto e = GetImpl(m_v)->grad_edge()) Engine::accumulate(e.get(), 0, dv);
}

void AttentionBackward::release() {
    m_q = m_k = m_v = m_out = m_lse = Tensor();
}

void AttentionBackward::get_inputs(std::vector<Tensor>& out) const {
    out.push_back(m_q);
    out.push_back(m_k);
    out.push_back(m_v);
}

Tensor attention_decode(const Tensor& q, const Tensor& kcache, const Tensor& vcache, float scale) {
    const Shape4 s = check_qkv(q, kcache, vcache, "attention_decode");
    if (s.Tq != 1) throw Error("attention_decode: q must be [B, H, 1, D]");
    const float sc = resolve_scale(scale, s.D);
    if (q.device().is_cpu()) {
        NoGradGuard ng;
        return scaled_dot_product_attention(q, kcache, vcache, false, sc);
    }
    Tensor out(q.dtype(), {s.B, s.H, 1, s.D}, "attention_decode", q.device(), false);
    const inf_dtype dt = detail::inf_dt(q.dtype(), "attention_decode");
    size_t ws_bytes = 0;
    detail::status_check(inf_attn_workspace_bytes(INF_OP_ATTN_DECODE, (int)s.B, (int)s.H, 1, (int)s.Tk, (int)s.D, dt,
                                                  &ws_bytes),
                         "inf_attn_workspace_bytes");
    void* ws = decode_workspace(ws_bytes, q.device());
    Tensor qa = abi_view(q), ka = abi_view(kcache), va = abi_view(vcache);
    detail::DeviceGuard g(q.device().index);
    detail::status_check(inf_attn_decode(qa.data_ptr(), strides_of(qa), ka.data_ptr(), strides_of(ka), va.data_ptr(),
                                         strides_of(va), out.data_ptr(), strides_of(out), (int)s.B, (int)s.H, (int)s.Tk,
                                         (int)s.D, sc, dt, ws, ws_bytes, detail::stream_of(q)),
                         "inf_attn_decode");
    return out;
}

}  // namespace Inferno
