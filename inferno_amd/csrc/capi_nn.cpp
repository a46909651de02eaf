// capi_nn.cpp -- the extern "C" entry points of the model ops around the
// attention path (include/inferno_hip.h, "model ops" section): argument
// validation on the host, workspace sizing, launches.  Nothing here allocates.
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdint>

#include "inferno_hip.h"
#include <algorithm>

#include "kernels.h"

namespace {

constexpr size_t kGemmWorkspace = size_t(32) << 20;  // hipBLASLt workspace offered to the heuristic

bool dtype_ok(int dt) { return dt == INF_F32 || dt == INF_BF16; }
int esz(inf_dtype dt) { return dt == INF_F32 ? 4 : 2; }
bool aligned(const void* p, size_t a) { return reinterpret_cast<uintptr_t>(p) % a == 0; }
int hip_status(int e) { return e == 0 ? INF_OK : INF_ERR_HIP; }
hipStream_t S(void* s) { return static_cast<hipStream_t>(s); }

}  // namespace

extern "C" {

int inf_nn_workspace_bytes(int op, int64_t rows, int64_t cols, size_t* out) {
    if (!out) return INF_ERR_NULL_POINTER;
    *out = 0;
    if (rows < 0 || cols < 0) return INF_ERR_BAD_SHAPE;
    switch (op) {
        case INF_OP_GEMM: *out = kGemmWorkspace; return INF_OK;
        case INF_OP_LAYERNORM_BWD: *out = (size_t)2 * inf::ln_bwd_blocks(rows) * (size_t)cols * 4; return INF_OK;
        case INF_OP_COL_SUM: *out = (size_t)inf::col_sum_chunks(rows) * (size_t)cols * 4; return INF_OK;
        case INF_OP_CROSS_ENTROPY: *out = (size_t)rows * 4; return INF_OK;
        default: return INF_ERR_UNSUPPORTED;
    }
}

int inf_gemm(int trans_a, int trans_b, int64_t M, int64_t N, int64_t K, float alpha, const void* A, int64_t lda,
             int64_t stride_a, const void* B, int64_t ldb, int64_t stride_b, float beta, void* C, int64_t ldc,
             int64_t stride_c, int64_t batch, const void* bias, inf_dtype dt, void* workspace, size_t ws_bytes,
             void* stream) {
    if (!dtype_ok(dt)) return INF_ERR_BAD_DTYPE;
    if (M < 0 || N < 0 || K < 0 || batch < 1) return INF_ERR_BAD_SHAPE;
    if (M == 0 || N == 0) return INF_OK;
    if (!A || !B || !C) return INF_ERR_NULL_POINTER;
    // stored (rows x cols) of A and B; leading dimension >= cols
    const int64_t a_cols = trans_a ? M : K, b_cols = trans_b ? K : N;
    if (lda < (a_cols > 1 ? a_cols : 1) || ldb < (b_cols > 1 ? b_cols : 1) || ldc < N) return INF_ERR_BAD_STRIDE;
    if (batch > 1 && (stride_a < 0 || stride_b < 0 || stride_c < 0)) return INF_ERR_BAD_STRIDE;
    if (M > INT32_MAX || N > INT32_MAX || K > INT32_MAX || batch > INT32_MAX) return INF_ERR_BAD_SHAPE;
    if (ws_bytes && !workspace) return INF_ERR_NULL_POINTER;
    if (K == 0) return INF_ERR_BAD_SHAPE;  // no product to form
    inf::GemmArgs g;
    g.ta = trans_a ? 1 : 0;
    g.tb = trans_b ? 1 : 0;
    g.bf16 = dt == INF_BF16;
    g.M = M;
    g.N = N;
    g.K = K;
    g.alpha = alpha;
    g.beta = beta;
    g.A = A;
    g.lda = lda;
    g.sa = stride_a;
    g.B = B;
    g.ldb = ldb;
    g.sb = stride_b;
    g.C = C;
    g.ldc = ldc;
    g.sc = stride_c;
    g.batch = batch;
    g.bias = bias;
    g.ws = workspace;
    g.ws_bytes = workspace ? ws_bytes : 0;
    const int e = inf::launch_gemm(g, S(stream));
    return e == 0 ? INF_OK : (e == 2 ? INF_ERR_UNSUPPORTED : INF_ERR_HIP);
}

int inf_layernorm_fwd(const void* x, int64_t ldx, void* y, int64_t ldy, const float* gamma, const float* beta,
                      float* mean, float* invstd, int64_t rows, int64_t dim, float eps, inf_dtype dt, void* stream) {
    if (!dtype_ok(dt)) return INF_ERR_BAD_DTYPE;
    if (rows < 0 || dim < 1 || dim > INT32_MAX) return INF_ERR_BAD_SHAPE;
    if (rows == 0) return INF_OK;
    if (!x || !y || !gamma || !beta) return INF_ERR_NULL_POINTER;
    if (ldx < dim || ldy < dim) return INF_ERR_BAD_STRIDE;
    if (!(eps >= 0.f) || !std::isfinite(eps)) return INF_ERR_BAD_SCALE;
    // The register kernel needs 16-byte rows and parameters; anything else takes
    // the scalar kernel (same arithmetic).
    const size_t va = 4 * (size_t)esz(dt);
    const int vec = dim % 4 == 0 && ldx % 4 == 0 && ldy % 4 == 0 && aligned(x, va) && aligned(y, va) &&
                    aligned(gamma, 16) && aligned(beta, 16);
    inf::LnParams p{x, y, gamma, beta, mean, invstd, rows, ldx, ldy, (int)dim, eps, vec};
    return hip_status(inf::launch_ln_fwd(p, dt == INF_BF16, S(stream)));
}

int inf_add_layernorm_fwd(const void* x, int64_t ldx, const void* r, int64_t ldr, void* h, int64_t ldh, void* y,
                          int64_t ldy, const float* gamma, const float* beta, float* mean, float* invstd, int64_t rows,
                          int64_t dim, float eps, inf_dtype dt, void* stream) {
    if (!dtype_ok(dt)) return INF_ERR_BAD_DTYPE;
    if (rows < 0 || dim < 1 || dim > INT32_MAX) return INF_ERR_BAD_SHAPE;
    if (rows == 0) return INF_OK;
    if (!x || !r || !h || !y || !gamma || !beta) return INF_ERR_NULL_POINTER;
    if (ldx < dim || ldr < dim || ldh < dim || ldy < dim) return INF_ERR_BAD_STRIDE;
    if (!(eps >= 0.f) || !std::isfinite(eps)) return INF_ERR_BAD_SCALE;
    const size_t va = 4 * (size_t)esz(dt);
    const int vec = dim % 4 == 0 && ldx % 4 == 0 && ldr % 4 == 0 && ldh % 4 == 0 && ldy % 4 == 0 && aligned(x, va) &&
                    aligned(r, va) && aligned(h, va) && aligned(y, va) && aligned(gamma, 16) && aligned(beta, 16);
    inf::LnParams p{x, y, gamma, beta, mean, invstd, rows, ldx, ldy, (int)dim, eps, vec, r, h, ldr, ldh};
    return hip_status(inf::launch_ln_fwd(p, dt == INF_BF16, S(stream)));
}

int inf_layernorm_bwd(const void* x, int64_t ldx, const void* dy, int64_t lddy, const float* gamma, const float* mean,
                      const float* invstd, void* dx, int64_t lddx, float* dgamma, float* dbeta, int accumulate,
                      int64_t rows, int64_t dim, inf_dtype dt, void* workspace, size_t ws_bytes, void* stream) {
    if (!dtype_ok(dt)) return INF_ERR_BAD_DTYPE;
    if (rows < 0 || dim < 1) return INF_ERR_BAD_SHAPE;
    if (dim % 4 != 0 || dim > inf::kLnBwdMaxDim) return INF_ERR_UNSUPPORTED;
    if (!x || !dy || !gamma || !mean || !invstd || !dx || !dgamma || !dbeta) return INF_ERR_NULL_POINTER;
    if (ldx < dim || lddy < dim || lddx < dim) return INF_ERR_BAD_STRIDE;
    const size_t va = 4 * (size_t)esz(dt);
    if (!aligned(x, va) || !aligned(dy, va) || !aligned(dx, va) || !aligned(gamma, 16) || ldx % 4 || lddy % 4 ||
        lddx % 4)
        return INF_ERR_ALIGNMENT;
    size_t need = 0;
    inf_nn_workspace_bytes(INF_OP_LAYERNORM_BWD, rows, dim, &need);
    if (!workspace || ws_bytes < need) return INF_ERR_WORKSPACE;
    if (!aligned(workspace, 16)) return INF_ERR_ALIGNMENT;
    if (rows == 0) {
        if (accumulate) return INF_OK;
        const int e1 = inf::launch_fill(dgamma, dim, 4, 0u, S(stream));
        return hip_status(e1 ? e1 : inf::launch_fill(dbeta, dim, 4, 0u, S(stream)));
    }
    inf::LnBwdParams p{x, dy, dx, gamma, mean, invstd, dgamma, dbeta, static_cast<float*>(workspace),
                       rows, ldx, lddy, lddx, (int)dim, accumulate ? 1 : 0};
    return hip_status(inf::launch_ln_bwd(p, dt == INF_BF16, S(stream)));
}

int inf_gelu_fwd(const void* x, void* y, int64_t n, inf_dtype dt, void* stream) {
    if (!dtype_ok(dt)) return INF_ERR_BAD_DTYPE;
    if (n < 0) return INF_ERR_BAD_SHAPE;
    if (n == 0) return INF_OK;
    if (!x || !y) return INF_ERR_NULL_POINTER;
    const size_t va = 4 * (size_t)esz(dt);
    if (!aligned(x, va) || !aligned(y, va)) return INF_ERR_ALIGNMENT;
    return hip_status(inf::launch_gelu_fwd(x, y, n, dt == INF_BF16, S(stream)));
}

int inf_gelu_bwd(const void* x, const void* dy, void* dx, int64_t n, inf_dtype dt, void* stream) {
    if (!dtype_ok(dt)) return INF_ERR_BAD_DTYPE;
    if (n < 0) return INF_ERR_BAD_SHAPE;
    if (n == 0) return INF_OK;
    if (!x || !dy || !dx) return INF_ERR_NULL_POINTER;
    const size_t va = 4 * (size_t)esz(dt);
    if (!aligned(x, va) || !aligned(dy, va) || !aligned(dx, va)) return INF_ERR_ALIGNMENT;
    return hip_status(inf::launch_gelu_bwd(x, dy, dx, n, dt == INF_BF16, S(stream)));
}

int inf_cross_entropy_fwd(const void* logits, int64_t ld, const int32_t* targets, float* loss, float* lse,
                          int64_t rows, int64_t vocab, inf_dtype dt, void* workspace, size_t ws_bytes, void* stream) {
    if (!dtype_ok(dt)) return INF_ERR_BAD_DTYPE;
    if (rows < 1 || vocab < 1) return INF_ERR_BAD_SHAPE;
    if (!logits || !targets || !loss || !lse) return INF_ERR_NULL_POINTER;
    if (ld < vocab) return INF_ERR_BAD_STRIDE;
    if (!workspace || ws_bytes < (size_t)rows * 4) return INF_ERR_WORKSPACE;
    if (!aligned(workspace, 4)) return INF_ERR_ALIGNMENT;
    if (vocab % 4 == 0 && (ld % 4 || !aligned(logits, 4 * (size_t)esz(dt)))) return INF_ERR_ALIGNMENT;
    inf::CeParams p{logits, targets, static_cast<float*>(workspace), lse, nullptr, nullptr, rows, vocab, ld, 0};
    return hip_status(inf::launch_ce_fwd(p, loss, dt == INF_BF16, S(stream)));
}

int inf_cross_entropy_bwd(const void* logits, int64_t ld, const int32_t* targets, const float* lse,
                          const float* upstream, void* dlogits, int64_t ldg, int64_t rows, int64_t vocab, inf_dtype dt,
                          void* stream) {
    if (!dtype_ok(dt)) return INF_ERR_BAD_DTYPE;
    if (rows < 1 || vocab < 1) return INF_ERR_BAD_SHAPE;
    if (!logits || !targets || !lse || !upstream || !dlogits) return INF_ERR_NULL_POINTER;
    if (ld < vocab || ldg < vocab) return INF_ERR_BAD_STRIDE;
    const size_t va = 4 * (size_t)esz(dt);
    if (vocab % 4 == 0 && (ld % 4 || ldg % 4 || !aligned(logits, va) || !aligned(dlogits, va)))
        return INF_ERR_ALIGNMENT;
    inf::CeParams p{logits, targets, nullptr, const_cast<float*>(lse), upstream, dlogits, rows, vocab, ld, ldg};
    return hip_status(inf::launch_ce_bwd(p, dt == INF_BF16, S(stream)));
}

int inf_embedding_fwd(const int32_t* ids, int64_t n_tokens, const void* table, int64_t vocab, int64_t dim, void* out,
                      inf_dtype dt, void* stream) {
    if (!dtype_ok(dt)) return INF_ERR_BAD_DTYPE;
    if (n_tokens < 0 || vocab < 1 || dim < 1) return INF_ERR_BAD_SHAPE;
    if (dim % 4) return INF_ERR_UNSUPPORTED;
    if (n_tokens == 0) return INF_OK;
    if (!ids || !table || !out) return INF_ERR_NULL_POINTER;
    const size_t va = 4 * (size_t)esz(dt);
    if (!aligned(table, va) || !aligned(out, va)) return INF_ERR_ALIGNMENT;
    inf::EmbParams p{ids, table, nullptr, out, n_tokens, vocab, dim};
    return hip_status(inf::launch_embed_fwd(p, dt == INF_BF16, S(stream)));
}

int inf_embedding_bwd(const int32_t* ids, int64_t n_tokens, const float* dout, int64_t vocab, int64_t dim,
                      float* dtable, int zero_first, void* stream) {
    if (n_tokens < 0 || vocab < 1 || dim < 1) return INF_ERR_BAD_SHAPE;
    if (dim % 4) return INF_ERR_UNSUPPORTED;
    if (!dtable) return INF_ERR_NULL_POINTER;
    if (n_tokens > 0 && (!ids || !dout)) return INF_ERR_NULL_POINTER;
    if (!aligned(dtable, 16) || (dout && !aligned(dout, 16))) return INF_ERR_ALIGNMENT;
    if (inf_get_deterministic() && dim <= 16384) {
        // each row summed in token order by one workgroup (no atomics, no fill)
        inf::EmbParams p{ids, nullptr, dout, dtable, n_tokens, vocab, dim};
        return hip_status(inf::launch_embed_bwd_det(p, zero_first, S(stream)));
    }
    if (zero_first) {
        const int e = inf::launch_fill(dtable, vocab * dim, 4, 0u, S(stream));
        if (e) return INF_ERR_HIP;
    }
    if (n_tokens == 0) return INF_OK;
    inf::EmbParams p{ids, nullptr, dout, dtable, n_tokens, vocab, dim};
    return hip_status(inf::launch_embed_bwd(p, S(stream)));
}

int inf_adamw_step(void* p, const void* g, float* m, float* v, int64_t n, float lr, float beta1, float beta2, float eps,
                   float weight_decay, float bias_correction1, float bias_correction2, inf_dtype dt, void* stream) {
    if (!dtype_ok(dt)) return INF_ERR_BAD_DTYPE;
    if (n < 0) return INF_ERR_BAD_SHAPE;
    if (n == 0) return INF_OK;
    if (!p || !g || !m || !v) return INF_ERR_NULL_POINTER;
    if (!(bias_correction1 > 0.f) || !(bias_correction2 > 0.f)) return INF_ERR_BAD_SCALE;
    inf::AdamWParams a{p, g, m, v, n, lr, beta1, beta2, eps, weight_decay, bias_correction1, bias_correction2};
    return hip_status(inf::launch_adamw(a, dt == INF_BF16, S(stream)));
}

int inf_adamw_step_multi(const inf_adamw_tensor* tensors, int n_tensors, float lr, float beta1, float beta2,
                         float eps, float weight_decay, float bias_correction1, float bias_correction2, inf_dtype dt,
                         void* stream) {
    if (!dtype_ok(dt)) return INF_ERR_BAD_DTYPE;
    if (n_tensors < 0) return INF_ERR_BAD_SHAPE;
    if (n_tensors == 0) return INF_OK;
    if (!tensors) return INF_ERR_NULL_POINTER;
    if (!(bias_correction1 > 0.f) || !(bias_correction2 > 0.f)) return INF_ERR_BAD_SCALE;
    const uintptr_t pa = dt == INF_BF16 ? 8 : 16;  // 4 elements of p / g per access
    for (int i = 0; i < n_tensors; ++i) {
        const inf_adamw_tensor& t = tensors[i];
        if (t.n < 0) return INF_ERR_BAD_SHAPE;
        if (t.n == 0) continue;
        if (!t.p || !t.g || !t.m || !t.v) return INF_ERR_NULL_POINTER;
        if (reinterpret_cast<uintptr_t>(t.p) % pa || reinterpret_cast<uintptr_t>(t.g) % pa ||
            reinterpret_cast<uintptr_t>(t.m) % 16 || reinterpret_cast<uintptr_t>(t.v) % 16)
            return INF_ERR_ALIGNMENT;
        if (t.n > (int64_t)1 << 40) return INF_ERR_BAD_SHAPE;
    }
    // Launches of up to kAdamWMaxTensors tensors and < 2^31 workgroups each.
    inf::AdamWMultiParams a{};
    a.lr = lr; a.beta1 = beta1; a.beta2 = beta2; a.eps = eps; a.weight_decay = weight_decay;
    a.bc1 = bias_correction1; a.bc2 = bias_correction2;
    auto flush = [&]() -> int {
        if (a.n_tensors == 0) return INF_OK;
        const int st = hip_status(inf::launch_adamw_multi(a, dt == INF_BF16, S(stream)));
        a.n_tensors = 0;
        a.block0[0] = 0;
        return st;
    };
    constexpr int64_t kMaxBlocks = (int64_t)1 << 30;
    for (int i = 0; i < n_tensors; ++i) {
        const inf_adamw_tensor& t = tensors[i];
        if (t.n == 0) continue;
        int64_t off = 0;
        while (off < t.n) {  // a tensor larger than one launch's block budget is cut in pieces
            const int64_t room = kMaxBlocks - a.block0[a.n_tensors];
            int64_t take = std::min<int64_t>(t.n - off, room * 1024);
            if (take <= 0 || a.n_tensors == inf::kAdamWMaxTensors) {
                if (const int st = flush()) return st;
                continue;
            }
            const int k = a.n_tensors;
            const size_t esz = dt == INF_BF16 ? 2 : 4;
            a.p[k] = static_cast<char*>(t.p) + off * esz;
            a.g[k] = static_cast<const char*>(t.g) + off * esz;
            a.m[k] = t.m + off;
            a.v[k] = t.v + off;
            a.n[k] = take;
            a.block0[k + 1] = a.block0[k] + (int)((take + 1023) / 1024);
            a.n_tensors = k + 1;
            off += take;
        }
    }
    return flush();
}

int inf_col_sum(const void* x, int64_t rows, int64_t cols, int64_t ldx, float* out, int accumulate, inf_dtype dt,
                void* workspace, size_t ws_bytes, void* stream) {
    if (!dtype_ok(dt)) return INF_ERR_BAD_DTYPE;
    if (rows < 0 || cols < 1) return INF_ERR_BAD_SHAPE;
    if (!out) return INF_ERR_NULL_POINTER;
    if (ldx < cols) return INF_ERR_BAD_STRIDE;
    if (rows == 0) return accumulate ? INF_OK : hip_status(inf::launch_fill(out, cols, 4, 0u, S(stream)));
    if (!x) return INF_ERR_NULL_POINTER;
    size_t need = 0;
    inf_nn_workspace_bytes(INF_OP_COL_SUM, rows, cols, &need);
    if (!workspace || ws_bytes < need) return INF_ERR_WORKSPACE;
    if (!aligned(workspace, 4)) return INF_ERR_ALIGNMENT;
    return hip_status(inf::launch_col_sum(x, out, static_cast<float*>(workspace), rows, cols, ldx, accumulate ? 1 : 0,
                                          dt == INF_BF16, S(stream)));
}

int inf_binary_bcast(int op, const void* a, const void* b, void* out, int64_t n, int64_t nb, inf_dtype dt,
                     void* stream) {
    if (!dtype_ok(dt)) return INF_ERR_BAD_DTYPE;
    if (op != INF_BIN_ADD && op != INF_BIN_MUL) return INF_ERR_UNSUPPORTED;
    if (n < 0 || nb < 1 || (n % nb) != 0) return INF_ERR_BAD_SHAPE;
    if (n == 0) return INF_OK;
    if (!a || !b || !out) return INF_ERR_NULL_POINTER;
    const size_t va = 4 * (size_t)esz(dt);
    const int vec = nb % 4 == 0 && aligned(a, va) && aligned(b, va) && aligned(out, va);
    return hip_status(inf::launch_bcast(op, a, b, out, n, nb, vec, dt == INF_BF16, S(stream)));
}

int inf_argmax_rows(const void* x, int64_t rows, int64_t cols, int64_t ld, int32_t* out, inf_dtype dt, void* stream) {
    if (!dtype_ok(dt)) return INF_ERR_BAD_DTYPE;
    if (rows < 0 || rows > INT32_MAX || cols < 1 || cols > INT32_MAX) return INF_ERR_BAD_SHAPE;
    if (ld < cols) return INF_ERR_BAD_STRIDE;
    if (rows == 0) return INF_OK;
    if (!x || !out) return INF_ERR_NULL_POINTER;
    return hip_status(inf::launch_argmax_rows(x, rows, cols, ld, out, dt == INF_BF16, S(stream)));
}

}  // extern "C"
