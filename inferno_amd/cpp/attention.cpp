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
//
// Head dims on HIP: the fused kernels are built for D in {32, 64, 128}.  Any
// other D up to 128 runs them on copies zero-padded along D to the next of
// those sizes: the zero columns add exact zeros to q k^T and leave zero
// columns in O, dQ, dK and dV, so the first D columns (and the LSE) are the
// unpadded results; the scale stays that of the real D.  D above 128 (Float32)
// runs the reference's composed chain (main.cpp:732-754: q k^T, * scale, the
// causal mask, Softmax, P v) on the library's HIP ops, its backward through
// their nodes; the mask enters as an added -1e9 bias (masked_fill's output
// carries no graph node, as in the reference, which would cut dQ and dK).
#include <algorithm>
#include <cfloat>
#include <cmath>
#include <mutex>

#include "detail.h"
#include "inferno/core/ops.h"
#include "inferno/functional/attention.h"
#include "inferno/functional/softmax.h"
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

// ---- head dims the fused kernels do not take -------------------------------
bool fused_head_dim(size_t D) { return D == 32 || D == 64 || D == 128; }
size_t padded_head_dim(size_t D) { return D <= 32 ? 32 : D <= 64 ? 64 : 128; }

// dst = src, two HIP views of one shape.
void copy_into(const Tensor& src, Tensor& dst) {
    const auto shape = detail::to_i64(src.shape());
    const auto ss = detail::to_i64(src.strides());
    const auto ds = detail::to_i64(dst.strides());
    detail::DeviceGuard g(src.device().index);
    detail::status_check(inf_copy_strided(src.data_ptr(), ss.data(), dst.data_ptr(), ds.data(), (int)src.ndim(),
                                          shape.data(), (int)dtype_size(src.dtype()), detail::stream_of(src)),
                         "inf_copy_strided");
}

// [B, H, T, D] -> a dense zero-filled [B, H, T, Dp] holding it in columns [0, D).
Tensor pad_head_dim(const Tensor& t, size_t Dp) {
    NoGradGuard ng;
    std::vector<size_t> shape = t.shape();
    shape[3] = Dp;
    Tensor out = Tensor::zeros(shape, t.dtype(), t.device(), "attention_padded");
    if (t.numel()) {
        Tensor dst = make_view(out, t.shape(), out.strides(), out.offset(), "attention_pad_dst");
        copy_into(t, dst);
    }
    return out;
}

// The first D columns of [B, H, T, Dp], dense.
Tensor unpad_head_dim(const Tensor& t, size_t D) {
    NoGradGuard ng;
    std::vector<size_t> shape = t.shape();
    shape[3] = D;
    return detail::dense_copy(make_view(t, shape, t.strides(), t.offset(), "attention_unpad_src"));
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

// The fused forward on HIP views (D in {32, 64, 128}) into out / lse.
void hip_fwd(const Tensor& q, const Tensor& k, const Tensor& v, Tensor& out, Tensor& lse, const Shape4& s, float sc,
             bool causal) {
    Tensor qa = abi_view(q), ka = abi_view(k), va = abi_view(v);
    detail::DeviceGuard g(q.device().index);
    const inf_dtype dt = detail::inf_dt(q.dtype(), "scaled_dot_product_attention");
    size_t ws_bytes = 0;
    if (causal)
        detail::status_check(inf_attn_workspace_bytes(INF_OP_ATTN_FWD, (int)s.B, (int)s.H, (int)s.Tq, (int)s.Tk,
                                                      (int)s.D, dt, &ws_bytes),
                             "inf_attn_workspace_bytes");
    Workspace ws(ws_bytes, q.device());
    detail::status_check(
        inf_attn_fwd(qa.data_ptr(), strides_of(qa), ka.data_ptr(), strides_of(ka), va.data_ptr(), strides_of(va),
                     out.data_ptr(), strides_of(out), static_cast<float*>(lse.data_ptr()), ws.ptr, ws_bytes, (int)s.B,
                     (int)s.H, (int)s.Tq, (int)s.Tk, (int)s.D, sc, causal ? 1 : 0, dt, detail::stream_of(q)),
        "inf_attn_fwd");
}

// The fused backward on HIP views into dq / dk / dv.
void hip_bwd(const Tensor& q, const Tensor& k, const Tensor& v, const Tensor& o, const Tensor& g, const Tensor& lse,
             Tensor& dq, Tensor& dk, Tensor& dv, const Shape4& s, float sc, bool causal) {
    const inf_dtype dt = detail::inf_dt(q.dtype(), "AttentionBackward");
    size_t ws_bytes = 0;
    detail::status_check(inf_attn_workspace_bytes(INF_OP_ATTN_BWD, (int)s.B, (int)s.H, (int)s.Tq, (int)s.Tk,
                                                  (int)s.D, dt, &ws_bytes),
                         "inf_attn_workspace_bytes");
    Workspace ws(ws_bytes, q.device());
    Tensor qa = abi_view(q), ka = abi_view(k), va = abi_view(v), oa = abi_view(o), ga = abi_view(g);
    detail::DeviceGuard dg(q.device().index);
    detail::status_check(
        inf_attn_bwd(qa.data_ptr(), strides_of(qa), ka.data_ptr(), strides_of(ka), va.data_ptr(), strides_of(va),
                     oa.data_ptr(), strides_of(oa), ga.data_ptr(), strides_of(ga),
                     static_cast<const float*>(lse.data_ptr()), dq.data_ptr(), strides_of(dq), dk.data_ptr(),
                     strides_of(dk), dv.data_ptr(), strides_of(dv), ws.ptr, ws_bytes, (int)s.B, (int)s.H, (int)s.Tq,
                     (int)s.Tk, (int)s.D, sc, causal ? 1 : 0, dt, detail::stream_of(q)),
        "inf_attn_bwd");
}

// Per-row log-sum-exp of dense fp32 scores [B, H, Tq, Tk] on HIP: the
// cross-entropy kernel's row LSE (its loss against target 0 is discarded).
Tensor rows_lse(const Tensor& S, const Shape4& s) {
    NoGradGuard ng;
    const int64_t rows = (int64_t)(s.B * s.H * s.Tq), cols = (int64_t)s.Tk;
    Tensor lse(DType::Float32, {s.B, s.H, s.Tq}, "attention_lse", S.device(), false);
    Tensor targets = Tensor::zeros({(size_t)rows}, DType::Int32, S.device(), "lse_targets");
    Tensor loss(DType::Float32, {1}, "lse_loss", S.device(), false);
    size_t ws_bytes = 0;
    detail::status_check(inf_nn_workspace_bytes(INF_OP_CROSS_ENTROPY, rows, cols, &ws_bytes), "inf_nn_workspace_bytes");
    Workspace ws(ws_bytes, S.device());
    detail::DeviceGuard g(S.device().index);
    detail::status_check(inf_cross_entropy_fwd(S.data_ptr(), cols, static_cast<const int32_t*>(targets.data_ptr()),
                                               static_cast<float*>(loss.data_ptr()),
                                               static_cast<float*>(lse.data_ptr()), rows, cols, INF_F32, ws.ptr,
                                               ws_bytes, detail::stream_of(S)),
                         "inf_cross_entropy_fwd");
    return lse;
}

// D > 128 on HIP: the reference's composed chain, fp32, with autograd through
// matmul / multiply / add / Softmax.
Tensor composed_attention(const Tensor& q, const Tensor& k, const Tensor& v, const Shape4& s, bool causal, float sc,
                          Tensor* lse_out) {
    if (q.dtype() != DType::Float32)
        throw Error("scaled_dot_product_attention: a head dim above 128 runs the composed Float32 chain on HIP "
                    "(BFloat16 inputs need D <= 128)");
    Tensor S = matmul(q, k.transpose(-1, -2), "QK ^ T") * sc;
    if (causal) {
        Tensor bias;
        {
            NoGradGuard ng;
            const Tensor ones = Tensor::ones({1, 1, s.Tq, s.Tk}, DType::Int32, q.device(), "causal_mask_ones");
            bias = masked_fill(Tensor::zeros({1, 1, s.Tq, s.Tk}, DType::Float32, q.device(), "causal_bias"),
                               triu(ones, (int)(1 + s.Tk - s.Tq)), -1e9f);
        }
        S = S + bias;
    }
    if (lse_out) *lse_out = rows_lse(S.contiguous(), s);
    Tensor P = Softmax(S, -1);
    return matmul(P, v, "attn@V");
}

}  // namespace

Tensor scaled_dot_product_attention_lse(const Tensor& q, const Tensor& k, const Tensor& v, bool causal, float scale,
                                        Tensor* lse_out) {
    const Shape4 s = check_qkv(q, k, v, "scaled_dot_product_attention");
    if (causal && s.Tq > s.Tk) throw Error("scaled_dot_product_attention: causal needs Tq <= Tk");
    const float sc = resolve_scale(scale, s.D);
    if (!(sc > 0.f) || !std::isfinite(sc)) throw Error("scaled_dot_product_attention: scale must be finite and > 0");
    const bool hip = !q.device().is_cpu();
    if (hip && s.D > 128 && s.B && s.H && s.Tq && s.Tk) return composed_attention(q, k, v, s, causal, sc, lse_out);
    Tensor lse(DType::Float32, {s.B, s.H, s.Tq}, "attention_lse", q.device(), false);
    if (hip && !fused_head_dim(s.D)) {
        const size_t Dp = padded_head_dim(s.D);
        Shape4 sp = s;
        sp.D = Dp;
        Tensor qp = pad_head_dim(q, Dp), kp = pad_head_dim(k, Dp), vp = pad_head_dim(v, Dp);
        Tensor op(q.dtype(), {s.B, s.H, s.Tq, Dp}, "attention_padded", q.device(), false);
        if (s.B && s.H && s.Tq && s.Tk) hip_fwd(qp, kp, vp, op, lse, sp, sc, causal);
        Tensor out = unpad_head_dim(op, s.D);
        if (grad_enabled && (q.requires_grad() || k.requires_grad() || v.requires_grad())) {
            out.set_requires_grad(true);
            GetImpl(out)->gradfn() = std::make_shared<AttentionBackward>(q, k, v, lse, causal, sc, qp, kp, vp, op);
        }
        if (lse_out) *lse_out = lse;
        return out;
    }
    Tensor out(q.dtype(), {s.B, s.H, s.Tq, s.D}, "attention", q.device(), false);
    if (s.B && s.H && s.Tq && s.Tk) {
        if (!hip)
            cpu_fwd(q, k, v, s, sc, causal, out, lse);
        else
            hip_fwd(q, k, v, out, lse, s, sc, causal);
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

AttentionBackward::AttentionBackward(const Tensor& q, const Tensor& k, const Tensor& v, const Tensor& lse,
                                     bool causal, float scale, const Tensor& q_padded, const Tensor& k_padded,
                                     const Tensor& v_padded, const Tensor& out_padded)
    : m_q(q),
      m_k(k),
      m_v(v),
      m_lse(lse),
      m_qp(q_padded),
      m_kp(k_padded),
      m_vp(v_padded),
      m_op(out_padded),
      m_causal(causal),
      m_scale(scale) {
    set_name("AttentionBackward");
}

void AttentionBackward::backward() {
    NoGradGuard ng;
    Tensor g = Engine::grad_in(this, 0);
    const Shape4 s = check_qkv(m_q, m_k, m_v, "AttentionBackward");
    Tensor dq, dk, dv;
    if (m_qp.defined()) {
        // padded head dim: the fused backward on the padded copies, then the first D columns
        const size_t Dp = m_qp.shape()[3];
        Shape4 sp = s;
        sp.D = Dp;
        Tensor dqp(m_qp.dtype(), m_qp.shape(), "attention_dq_padded", m_qp.device(), false);
        Tensor dkp(m_kp.dtype(), m_kp.shape(), "attention_dk_padded", m_kp.device(), false);
        Tensor dvp(m_vp.dtype(), m_vp.shape(), "attention_dv_padded", m_vp.device(), false);
        if (s.B && s.H && s.Tq && s.Tk)
            hip_bwd(m_qp, m_kp, m_vp, m_op, pad_head_dim(g, Dp), m_lse, dqp, dkp, dvp, sp, m_scale, m_causal);
        dq = unpad_head_dim(dqp, s.D);
        dk = unpad_head_dim(dkp, s.D);
        dv = unpad_head_dim(dvp, s.D);
    } else {
        dq = Tensor(m_q.dtype(), m_q.shape(), "attention_dq", m_q.device(), false);
        dk = Tensor(m_k.dtype(), m_k.shape(), "attention_dk", m_k.device(), false);
        dv = Tensor(m_v.dtype(), m_v.shape(), "attention_dv", m_v.device(), false);
        if (m_q.device().is_cpu())
            cpu_bwd(m_q, m_k, m_v, g, s, m_scale, m_causal, dq, dk, dv);
        else
            hip_bwd(m_q, m_k, m_v, m_out, g, m_lse, dq, dk, dv, s, m_scale, m_causal);
    }
    if (auto e = GetImpl(m_q)->grad_edge()) Engine::accumulate(e.get(), 0, dq);
    if (auto e = GetImpl(m_k)->grad_edge()) Engine::accumulate(e.get(), 0, dk);
    if (auto e = GetImpl(m_v)->grad_edge()) Engine::accumulate(e.get(), 0, dv);
}

void AttentionBackward::release() {
    m_q = m_k = m_v = m_out = m_lse = Tensor();
    m_qp = m_kp = m_vp = m_op = Tensor();
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
    if (q.device().is_cpu() || s.D > 128) {
        NoGradGuard ng;
        return scaled_dot_product_attention(q, kcache, vcache, false, sc);
    }
    if (!fused_head_dim(s.D)) {
        // a padded copy of the cache prefix per call: correct, not fast
        const size_t Dp = padded_head_dim(s.D);
        return unpad_head_dim(attention_decode(pad_head_dim(q, Dp), pad_head_dim(kcache, Dp),
                                               pad_head_dim(vcache, Dp), sc),
                              s.D);
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
