/*
 * oracle_nn.c -- CPU restatement of the reference's model ops around the
 * attention path (the GPT training step): LayerNorm, tanh-GELU, cross-entropy,
 * embedding, AdamW, bias / broadcast reductions.
 *
 * TEST INFRASTRUCTURE ONLY, like oracle.c: the checker for the HIP path.  The
 * product library never links, loads or calls this file.
 *
 * Each function follows the reference routine cited in oracle.h loop for loop
 * (same accumulation order, same fp32 rounding points, float exp / log / tanh
 * / sqrt as the reference's float instantiations call them).  Built with
 * -O2 -ffp-contract=off like oracle.c.
 *
 * Pinning (tests/test_oracle_nn.py):
 *   - orc_layernorm_f32, orc_gelu_f32, orc_gelu_bwd_f32, orc_cross_entropy_f32,
 *     orc_embedding_f32, orc_adamw_f32: bit-exact against the reference's own
 *     header kernels compiled from /root/reference into oracle/_ref.
 *   - orc_layernorm_bwd_f32, orc_cross_entropy_bwd_f32 (their headers pull in
 *     <cuda_runtime.h>): fp64 central differences of the forward, the
 *     closed-form invariants (dx rows sum to 0 and are orthogonal to xhat for
 *     LayerNorm; gradient rows sum to 0 for cross-entropy) and brute force.
 *   - orc_embedding_bwd_f32, orc_sum_rows_f32: brute-force scatter / column
 *     sums in fp64 on integer-valued inputs (exact in fp32).
 */
#include <math.h>
#include <stdint.h>
#include <string.h>

#include "oracle.h"

void orc_layernorm_f32(const float* x, const float* gamma, const float* beta, float* y, float* mean_out,
                       float* invstd_out, int64_t rows, int64_t dim, float eps) {
    for (int64_t b = 0; b < rows; ++b) {
        const float* xr = x + b * dim;
        float mean = 0.0f;
        for (int64_t i = 0; i < dim; ++i) mean += xr[i];
        mean /= (float)dim;
        float var = 0.0f;
        for (int64_t i = 0; i < dim; ++i) {
            const float d = xr[i] - mean;
            var += d * d;
        }
        var /= (float)dim;
        const float invstd = 1.0f / sqrtf(var + eps);
        if (mean_out) mean_out[b] = mean;
        if (invstd_out) invstd_out[b] = invstd;
        for (int64_t i = 0; i < dim; ++i) {
            const float xhat = (xr[i] - mean) * invstd;
            y[b * dim + i] = xhat * gamma[i] + beta[i];
        }
    }
}

void orc_layernorm_bwd_f32(const float* x, const float* gout, const float* gamma, const float* mean,
                           const float* invstd, float* gx, float* ggamma, float* gbeta, int64_t rows, int64_t dim) {
    for (int64_t i = 0; i < dim; ++i) {
        ggamma[i] = 0.0f;
        gbeta[i] = 0.0f;
    }
    for (int64_t b = 0; b < rows; ++b) {
        const int64_t base = b * dim;
        const float m = mean[b], is = invstd[b];
        float sum_dxhat = 0.0f, sum_dxhat_xhat = 0.0f;
        for (int64_t i = 0; i < dim; ++i) {
            const float xhat = (x[base + i] - m) * is;
            const float dxhat = gout[base + i] * gamma[i];
            gbeta[i] += gout[base + i];
            ggamma[i] += gout[base + i] * xhat;
            sum_dxhat += dxhat;
            sum_dxhat_xhat += dxhat * xhat;
        }
        const float dim_f = (float)dim;
        for (int64_t i = 0; i < dim; ++i) {
            const float xhat = (x[base + i] - m) * is;
            const float dxhat = gout[base + i] * gamma[i];
            gx[base + i] = (is / dim_f) * (dim_f * dxhat - sum_dxhat - xhat * sum_dxhat_xhat);
        }
    }
}

static float gelu1(float x) {
    const float a = 0.7978845608028654f, k = 0.044715f;
    const float x3 = x * x * x;
    const float inner = a * (x + k * x3);
    return 0.5f * x * (1.0f + tanhf(inner));
}

static float gelu_grad1(float x) {
    const float a = 0.7978845608028654f, k = 0.044715f;
    const float k3 = 3.0f * k, half = 0.5f, one = 1.0f;
    const float x2 = x * x;
    const float x3 = x2 * x;
    const float u = a * (x + k * x3);
    const float t = tanhf(u);
    const float sech2 = one - t * t;
    return half * (one + t) + half * x * sech2 * a * (one + k3 * x2);
}

void orc_gelu_f32(const float* x, float* y, int64_t n) {
    for (int64_t i = 0; i < n; ++i) y[i] = gelu1(x[i]);
}

void orc_gelu_bwd_f32(const float* x, const float* g, float* dx, int64_t n) {
    for (int64_t i = 0; i < n; ++i) dx[i] = g[i] * gelu_grad1(x[i]);
}

void orc_cross_entropy_f32(const float* logits, const int32_t* targets, float* out, int64_t rows, int64_t vocab) {
    float total = 0.0f;
    for (int64_t r = 0; r < rows; ++r) {
        const float* row = logits + r * vocab;
        const int32_t t = targets[r];
        if (t < 0 || t >= vocab) {
            out[0] = NAN;
            return;
        }
        float mx = row[0];
        for (int64_t v = 1; v < vocab; ++v)
            if (row[v] > mx) mx = row[v];
        float sum = 0.0f;
        for (int64_t v = 0; v < vocab; ++v) sum += expf(row[v] - mx);
        const float lse = logf(sum);
        total += -(row[t] - mx - lse);
    }
    out[0] = total / (float)rows;
}

void orc_cross_entropy_bwd_f32(const float* logits, const int32_t* targets, const float* upstream, float* grad,
                               int64_t rows, int64_t vocab) {
    const float scale = upstream[0] / (float)rows;
    for (int64_t r = 0; r < rows; ++r) {
        const float* row = logits + r * vocab;
        float* g = grad + r * vocab;
        float mx = row[0];
        for (int64_t v = 1; v < vocab; ++v)
            if (row[v] > mx) mx = row[v];
        float sum = 0.0f;
        for (int64_t v = 0; v < vocab; ++v) sum += expf(row[v] - mx);
        for (int64_t v = 0; v < vocab; ++v) g[v] = expf(row[v] - mx) / sum * scale;
        g[targets[r]] -= scale;
    }
}

void orc_embedding_f32(const int32_t* ids, const float* table, float* out, int64_t n_tokens, int64_t dim) {
    for (int64_t t = 0; t < n_tokens; ++t) memcpy(out + t * dim, table + (int64_t)ids[t] * dim, (size_t)dim * 4);
}

void orc_embedding_bwd_f32(const int32_t* ids, const float* gout, float* dtable, int64_t n_tokens, int64_t vocab,
                           int64_t dim) {
    memset(dtable, 0, (size_t)(vocab * dim) * 4);
    for (int64_t t = 0; t < n_tokens; ++t) {
        float* o = dtable + (int64_t)ids[t] * dim;
        const float* g = gout + t * dim;
        for (int64_t e = 0; e < dim; ++e) o[e] += g[e];
    }
}

void orc_adamw_f32(float* p, const float* g, float* m, float* v, int64_t n, float lr, float beta1, float beta2,
                   float eps, float weight_decay, float bc1, float bc2) {
    for (int64_t i = 0; i < n; ++i) {
        const float grad = g[i];
        float mi = m[i], vi = v[i], pi = p[i];
        mi = beta1 * mi + (1.0f - beta1) * grad;
        vi = beta2 * vi + (1.0f - beta2) * grad * grad;
        const float m_hat = mi / bc1;
        const float v_hat = vi / bc2;
        float update = m_hat / (sqrtf(v_hat) + eps);
        if (weight_decay != 0.0f) update += weight_decay * pi;
        pi -= lr * update;
        p[i] = pi;
        m[i] = mi;
        v[i] = vi;
    }
}

void orc_sum_rows_f32(const float* x, float* out, int64_t rows, int64_t cols) {
    for (int64_t c = 0; c < cols; ++c) out[c] = 0.0f;
    for (int64_t r = 0; r < rows; ++r)
        for (int64_t c = 0; c < cols; ++c) out[c] += x[r * cols + c];
}

float orc_adamw_bias_correction(float beta, int64_t step) { return 1.0f - powf(beta, (float)step); }
