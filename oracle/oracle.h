/*
 * oracle.h -- CPU restatement of Inferno's causal-attention arithmetic.
 *
 * TEST INFRASTRUCTURE ONLY.  Only tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py may load this library, and only as the checker
 * (or as the timed CPU baseline).  The product path (inferno_amd, libinferno_hip)
 * never links, loads or calls it.
 *
 * Every function restates a reference routine literally (same loop order, same
 * fp32 rounding points, exp evaluated in double) so that its outputs equal what
 * Inferno's own CPU path would produce on the same inputs.  Citations are
 * relative to the reference tree (K9Megahertz/Inferno).
 *
 * Layout convention: every tensor is dense row-major; attention tensors are
 * [B, H, T, D] and scores are [T, T] per (b, h).
 */
#ifndef INFERNO_ORACLE_H
#define INFERNO_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- input generator (the reference has none: it is uniform-only) ------- */
/* MT19937-64 (Matsumoto & Nishimura, ACM TOMACS 2000), the engine the C++
 * standard calls std::mt19937_64. */
typedef struct {
    uint64_t mt[312];
    int idx;
} orc_mt64;

void orc_mt64_seed(orc_mt64* g, uint64_t seed);
uint64_t orc_mt64_next(orc_mt64* g);
/* n draws of N(0, sigma^2): 53-bit uniforms -> Box-Muller in double -> float */
void orc_randn_f32(uint64_t seed, double sigma, float* out, size_t n);
/* fp32 -> bf16 bits, round-to-nearest-even (NaN kept quiet) */
void orc_round_bf16(const float* in, uint16_t* out, size_t n);
void orc_bf16_to_f32(const uint16_t* in, float* out, size_t n);

/* ---- reference kernels, restated ---------------------------------------- */
/* cpu_matmul (src/inferno/core/cpuops.h:336-434) for one dense matrix pair:
 * out[m][n] = sum_k a[m*sa0 + k*sa1] * b[k*sb0 + n*sb1], fp32 sum in k order. */
void orc_matmul_f32(const float* a, int64_t sa0, int64_t sa1,
                    const float* b, int64_t sb0, int64_t sb1,
                    float* out, int64_t M, int64_t K, int64_t N);
/* cpu_multiply by a broadcast scalar (src/inferno/core/cpuops.h:165-226) */
void orc_scale_f32(const float* a, float s, float* out, int64_t n);
/* cpu_triu on ones (src/inferno/core/cpuops.h:617-656): (col-row >= diag) */
void orc_triu_ones_i32(int32_t* out, int64_t rows, int64_t cols, int diagonal);
/* cpu_masked_fill (src/inferno/core/cpuops.h:659-705), mask broadcast [rows, cols] */
void orc_masked_fill_f32(const float* in, const int32_t* mask, float fill,
                         float* out, int64_t rows, int64_t cols);
/* cpu_softmax over the last axis (src/inferno/functional/softmax_kernels.h:40-104) */
void orc_softmax_f32(const float* x, float* y, int64_t rows, int64_t cols);
/* cpu_softmax_backward over the last axis (src/inferno/gradfn/softmaxbackward.h:64-131) */
void orc_softmax_bwd_f32(const float* y, const float* g, float* dx, int64_t rows, int64_t cols);
/* Softmax's other dtypes (softmax.cpp:25 dispatchAny, RT = promote_t<AT, float>,
 * dtype_dispatch.h:8-52): cpu_softmax<double, double> and cpu_softmax<int, float>. */
void orc_softmax_f64(const double* x, double* y, int64_t rows, int64_t cols);
void orc_softmax_i32(const int32_t* x, float* y, int64_t rows, int64_t cols);
/* cpu_softmax_backward<double, double, double> (RT = promote_t<AT, GT> of
 * dispatchFloatTwo, softmaxbackward.cpp:40-45; a Float32 operand converts exactly). */
void orc_softmax_bwd_f64(const double* y, const double* g, double* dx, int64_t rows, int64_t cols);

/* ---- attention, composed as InfernoApp/main.cpp:737-754 ------------------ */
/* Forward on dense [B,H,Tq,D] q and [B,H,Tk,D] k, v.  Causal masking is
 * triu(ones[Tq,Tk], 1 + (Tk-Tq)) filled with -1e9f (main.cpp:747-748 with
 * the end-aligned offset; Tq == Tk is the reference's own case).
 * o: [B,H,Tq,D]; lse (optional): [B,H,Tq], fp64 closed form over the masked,
 * scaled scores, rounded to fp32; p (optional): [B,H,Tq,Tk]. */
void orc_attn_fwd_f32(const float* q, const float* k, const float* v,
                      int64_t B, int64_t H, int64_t Tq, int64_t Tk, int64_t D,
                      float scale, int causal, float* o, float* lse, float* p);
/* Backward: the chain MMBackward(P,V) -> SoftmaxBackward -> MultiplyBackward
 * -> MMBackward(Q,K^T) -> TransposeBackward, driven by dO.  Writes dq, dk, dv
 * (each dense like its input); ds (optional) receives SoftmaxBackward's dS (before the scale) per head. */
void orc_attn_bwd_f32(const float* q, const float* k, const float* v, const float* dout,
                      int64_t B, int64_t H, int64_t Tq, int64_t Tk, int64_t D,
                      float scale, int causal, float* dq, float* dk, float* dv, float* ds);
/* Decode: one query per (b,h) against the whole cache (no key masked). */
void orc_attn_decode_f32(const float* q, const float* kc, const float* vc,
                         int64_t B, int64_t H, int64_t Tk, int64_t D, float scale, float* o);

/* ---- model ops around the path (oracle_nn.c) ----------------------------- */
/* cpu_layer_normalization (src/inferno/modules/layernorm_kernels.h:48-87):
 * mean and biased variance in fp32 sequential sums, invstd = 1/sqrtf(var+eps);
 * mean_out / invstd_out may be NULL. */
void orc_layernorm_f32(const float* x, const float* gamma, const float* beta, float* y, float* mean_out,
                       float* invstd_out, int64_t rows, int64_t dim, float eps);
/* cpu_layernorm_backward (src/inferno/gradfn/layernormbackward.h:47-97) */
void orc_layernorm_bwd_f32(const float* x, const float* gout, const float* gamma, const float* mean,
                           const float* invstd, float* gx, float* ggamma, float* gbeta, int64_t rows, int64_t dim);
/* cpu_gelu (src/inferno/functional/gelu_kernels.h:9-27): tanh approximation */
void orc_gelu_f32(const float* x, float* y, int64_t n);
/* cpu_gelu_backward (src/inferno/gradfn/gelubackward.h:27-61) */
void orc_gelu_bwd_f32(const float* x, const float* g, float* dx, int64_t n);
/* cpu_cross_entropy_loss (src/inferno/core/cpuops.h:707-749): mean over rows;
 * out[0] = NaN for a target outside [0, vocab) (the reference exits) */
void orc_cross_entropy_f32(const float* logits, const int32_t* targets, float* out, int64_t rows, int64_t vocab);
/* cpu_cross_entropy_loss_backward (src/inferno/gradfn/crossentropylossbackward.h:45-86) */
void orc_cross_entropy_bwd_f32(const float* logits, const int32_t* targets, const float* upstream, float* grad,
                               int64_t rows, int64_t vocab);
/* cpu_embedding (src/inferno/modules/embedding_kernels.h:19-31) */
void orc_embedding_f32(const int32_t* ids, const float* table, float* out, int64_t n_tokens, int64_t dim);
/* scatter_add_embedding / cpu_scatter_add_embedding (src/inferno/core/broadcastops.cpp:120-166,
 * broadcastops.h:61-74) into a zeroed table gradient */
void orc_embedding_bwd_f32(const int32_t* ids, const float* gout, float* dtable, int64_t n_tokens, int64_t vocab,
                           int64_t dim);
/* cpu_adamw_step_impl (include/inferno/optim/adamw.h:67-111) */
void orc_adamw_f32(float* p, const float* g, float* m, float* v, int64_t n, float lr, float beta1, float beta2,
                   float eps, float weight_decay, float bc1, float bc2);
/* OptimizerAdamW::step's bias correction 1 - pow(beta, step) in float (src/inferno/optim/adamw.cpp) */
float orc_adamw_bias_correction(float beta, int64_t step);
/* cpu_sum_to_shape (src/inferno/core/broadcastops.h:22-48) for [rows, cols] -> [cols]:
 * the source is walked in linear order, each element added to its column */
void orc_sum_rows_f32(const float* x, float* out, int64_t rows, int64_t cols);

#ifdef __cplusplus
}
#endif
#endif
