// ref_shim.cpp -- C entry points over Inferno's own header-only CPU kernels.
//
// TEST INFRASTRUCTURE ONLY.  This file is compiled by oracle/Makefile (target
// `ref`) against the reference tree at /root/reference, and the result goes to
// oracle/_ref/libinferno_ref.so.  It contains no reference code: it includes
// the reference's headers where they lie and instantiates their templates, so
// tests can check the restated oracle (oracle.c) against the reference's own
// arithmetic, bit for bit.
//
// What is reachable here: cpu_matmul, cpu_multiply, cpu_triu, cpu_masked_fill,
// cpu_contiguous_copy, cpu_cross_entropy_loss (src/inferno/core/cpuops.h),
// cpu_softmax (src/inferno/functional/softmax_kernels.h), cpu_gelu
// (gelu_kernels.h), cpu_gelu_backward (src/inferno/gradfn/gelubackward.h),
// cpu_embedding (src/inferno/modules/embedding_kernels.h),
// cpu_layer_normalization (layernorm_kernels.h) and cpu_adamw_step_impl
// (include/inferno/optim/adamw.h).  cpu_layernorm_backward and
// cpu_cross_entropy_loss_backward are not (their headers pull broadcastops.h).  cpu_softmax_backward
// (src/inferno/gradfn/softmaxbackward.h) is not: that header pulls
// tensorimpl.h -> cudastorage.h -> <cuda_runtime.h>.  Logger::Append is
// referenced only on cpu_matmul's rank<2 error path; its definition
// (src/inferno/util/logger.cpp) cannot compile on a case-sensitive file system
// (it includes "Logger.h"), so the library is linked without it and must be
// loaded with RTLD_LAZY; the error path is never taken with rank-4 inputs.
#include <cmath>
#include <cstddef>
#include <cstdint>
#include <functional>
#include <limits>
#include <numeric>
#include <stdexcept>
#include <string>
#include <vector>

#include "inferno/util/logger.h"
#include "inferno/core/cpuops.h"
#include "inferno/functional/softmax_kernels.h"
#include "inferno/functional/gelu_kernels.h"
#include "inferno/gradfn/gelubackward.h"
#include "inferno/modules/embedding_kernels.h"
#include "inferno/modules/layernorm_kernels.h"
#include "inferno/optim/adamw.h"

using Shape = std::vector<size_t>;

static Shape dense_strides(const Shape& s) {
    Shape st(s.size(), 1);
    for (int i = (int)s.size() - 2; i >= 0; --i) st[i] = st[i + 1] * s[i + 1];
    return st;
}

extern "C" {

// Batched [B,H,M,K] x [B,H,K,N] -> dense [B,H,M,N] through cpu_matmul, with
// explicit element strides for both operands (rank 4, no offsets).
void ref_matmul4_f32(const float* a, const int64_t* a_strides, const float* b,
                     const int64_t* b_strides, float* out, int64_t B, int64_t H, int64_t M,
                     int64_t K, int64_t N) {
    Shape as{(size_t)B, (size_t)H, (size_t)M, (size_t)K};
    Shape bs{(size_t)B, (size_t)H, (size_t)K, (size_t)N};
    Shape os{(size_t)B, (size_t)H, (size_t)M, (size_t)N};
    Shape ast(a_strides, a_strides + 4), bst(b_strides, b_strides + 4);
    Inferno::cpu_matmul<float, float, float>(a, b, out, as, ast, bs, bst, os);
}

// x * s with s a one-element tensor (Tensor * float, tensor.h:288-293).
void ref_scale_f32(const float* a, int64_t n, float s, float* out) {
    Shape as{(size_t)n}, bs{1};
    Shape ast{1}, bst{1};
    Inferno::cpu_multiply<float, float, float>(a, &s, out, as, ast, 0, bs, bst, 0, as, (size_t)n);
}

// triu(ones[1,1,rows,cols], diagonal) as Int32 (main.cpp:794-806).
void ref_triu_ones_i32(int64_t rows, int64_t cols, int diagonal, int32_t* out) {
    Shape s{1, 1, (size_t)rows, (size_t)cols};
    std::vector<int> ones((size_t)(rows * cols), 1);
    Inferno::cpu_triu<int>(ones.data(), out, s, dense_strides(s), 0, (size_t)(rows * cols), diagonal);
}

// masked_fill of a dense [B,H,rows,cols] input with a [1,1,rows,cols] mask.
void ref_masked_fill_f32(const float* in, int64_t B, int64_t H, int64_t rows, int64_t cols,
                         const int32_t* mask, float fill, float* out) {
    Shape is{(size_t)B, (size_t)H, (size_t)rows, (size_t)cols};
    Shape ms{1, 1, (size_t)rows, (size_t)cols};
    size_t n = (size_t)(B * H * rows * cols);
    Inferno::cpu_masked_fill<float, int>(in, mask, out, is, dense_strides(is), 0, ms,
                                         dense_strides(ms), 0, n, fill);
}

// Row softmax over the last axis of a dense [rows, cols] tensor.
void ref_softmax_f32(const float* x, int64_t rows, int64_t cols, float* y) {
    Shape s{(size_t)rows, (size_t)cols};
    Shape st = dense_strides(s);
    Inferno::cpu_softmax<float, float>(x, y, s, st, st, 0, 0, 1);
}

// The other two instantiations Softmax dispatches (dispatchAny with
// promote_t<AT, float>, dtype_dispatch.h:8-52): Float64 -> Float64 and
// Int32 -> Float32.
void ref_softmax_f64(const double* x, int64_t rows, int64_t cols, double* y) {
    Shape s{(size_t)rows, (size_t)cols};
    Shape st = dense_strides(s);
    Inferno::cpu_softmax<double, double>(x, y, s, st, st, 0, 0, 1);
}
void ref_softmax_i32(const int32_t* x, int64_t rows, int64_t cols, float* y) {
    Shape s{(size_t)rows, (size_t)cols};
    Shape st = dense_strides(s);
    Inferno::cpu_softmax<int, float>(x, y, s, st, st, 0, 0, 1);
}

// transpose(-1,-2).contiguous() of a dense [B,H,R,C] tensor -> [B,H,C,R].
void ref_transpose_contig_f32(const float* x, int64_t B, int64_t H, int64_t R, int64_t C,
                              float* out) {
    Shape vs{(size_t)B, (size_t)H, (size_t)C, (size_t)R};
    Shape vst{(size_t)(H * R * C), (size_t)(R * C), 1, (size_t)C};
    Inferno::cpu_contiguous_copy<float>(x, out, vs, vst, 0, (size_t)(B * H * R * C));
}

// InfernoApp/main.cpp:737-754 on dense [B,H,T,D] q, k, v: o = softmax(mask(q@kt*scale)) @ v.
// p (optional) receives the [B,H,T,T] attention probabilities.
void ref_attn_fwd_f32(const float* q, const float* k, const float* v, int64_t B, int64_t H,
                      int64_t T, int64_t D, float scale, int causal, float* o, float* p) {
    const size_t TT = (size_t)(B * H * T * T);
    std::vector<float> kt((size_t)(B * H * T * D)), s(TT), s2(TT), attn(TT);
    ref_transpose_contig_f32(k, B, H, T, D, kt.data());
    const int64_t qs[4] = {H * T * D, T * D, D, 1};
    const int64_t kts[4] = {H * D * T, D * T, T, 1};
    ref_matmul4_f32(q, qs, kt.data(), kts, s.data(), B, H, T, D, T);
    ref_scale_f32(s.data(), (int64_t)TT, scale, s2.data());
    if (causal) {
        std::vector<int32_t> mask((size_t)(T * T));
        ref_triu_ones_i32(T, T, 1, mask.data());
        ref_masked_fill_f32(s2.data(), B, H, T, T, mask.data(), -1e9f, s.data());
    } else {
        s = s2;
    }
    ref_softmax_f32(s.data(), B * H * T, T, attn.data());
    const int64_t ps[4] = {H * T * T, T * T, T, 1};
    const int64_t vs[4] = {H * T * D, T * D, D, 1};
    ref_matmul4_f32(attn.data(), ps, v, vs, o, B, H, T, T, D);
    if (p)
        for (size_t i = 0; i < TT; ++i) p[i] = attn[i];
}

// The MMBackward / MultiplyBackward / TransposeBackward stages of the backward
// chain with dS supplied by the caller (SoftmaxBackward is not compilable here):
//   dP = dO @ v^T, dV = P^T @ dO          (mmbackward.cpp:77,80)
//   dS' = dS * scale                      (multiplybackward.cpp:41)
//   dQ = dS' @ k, dKt = q^T @ dS', dK = dKt^T (mmbackward.cpp:77,80; transposebackward.cpp:41)
void ref_attn_bwd_stages_f32(const float* q, const float* k, const float* v, const float* p,
                             const float* dout, const float* ds, int64_t B, int64_t H, int64_t T,
                             int64_t D, float scale, float* dp, float* dv, float* dq, float* dk) {
    const size_t TT = (size_t)(B * H * T * T), TD = (size_t)(B * H * T * D);
    std::vector<float> vt(TD), pt(TT), dss(TT), qt(TD), dkt(TD);
    const int64_t td[4] = {H * T * D, T * D, D, 1};
    const int64_t dt[4] = {H * D * T, D * T, T, 1};
    const int64_t tt[4] = {H * T * T, T * T, T, 1};
    ref_transpose_contig_f32(v, B, H, T, D, vt.data());
    ref_matmul4_f32(dout, td, vt.data(), dt, dp, B, H, T, D, T);
    ref_transpose_contig_f32(p, B, H, T, T, pt.data());
    ref_matmul4_f32(pt.data(), tt, dout, td, dv, B, H, T, T, D);
    ref_scale_f32(ds, (int64_t)TT, scale, dss.data());
    // B^T of kt is k itself (kt = k^T, contiguous), so dQ = dS' @ k.
    ref_matmul4_f32(dss.data(), tt, k, td, dq, B, H, T, T, D);
    ref_transpose_contig_f32(q, B, H, T, D, qt.data());
    ref_matmul4_f32(qt.data(), dt, dss.data(), tt, dkt.data(), B, H, D, T, T);
    ref_transpose_contig_f32(dkt.data(), B, H, D, T, dk);
}

// ---- model ops around the path ----------------------------------------------

void ref_layernorm_f32(const float* x, const float* gamma, const float* beta, float* y, float* mean, float* invstd,
                       int64_t rows, int64_t dim, float eps) {
    Inferno::cpu_layer_normalization<float>(x, y, gamma, beta, mean, invstd, (size_t)rows, (size_t)dim, eps);
}

void ref_gelu_f32(const float* x, float* y, int64_t n) { Inferno::cpu_gelu<float, float>(x, y, (size_t)n, 0); }

void ref_gelu_bwd_f32(const float* x, const float* g, float* dx, int64_t n) {
    Inferno::cpu_gelu_backward<float, float, float>(x, g, dx, (size_t)n, 0);
}

void ref_cross_entropy_f32(const float* logits, const int32_t* targets, float* out, int64_t rows, int64_t vocab) {
    Inferno::cpu_cross_entropy_loss<float>(logits, targets, out, (size_t)rows, (size_t)vocab);
}

void ref_embedding_f32(const int32_t* ids, const float* table, float* out, int64_t n_tokens, int64_t dim) {
    Inferno::cpu_embedding<float, int>(ids, table, out, 1, (size_t)n_tokens, (size_t)dim);
}

void ref_adamw_f32(float* p, const float* g, float* m, float* v, int64_t n, float lr, float beta1, float beta2,
                   float eps, float weight_decay, float bc1, float bc2) {
    Inferno::cpu_adamw_step_impl<float, float>(p, g, m, v, (size_t)n, lr, beta1, beta2, eps, weight_decay, bc1, bc2);
}

}  // extern "C"
