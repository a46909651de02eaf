/*
 * inferno_hip.h -- C-ABI launch layer for Inferno's causal-attention path on
 * AMD Instinct MI355X (gfx950).
 *
 * This header replaces, for the attention path, the templated CUDA launcher
 * declarations of the reference (src/inferno/cuda/cudaops.h:102-183) and the
 * per-op metadata cudaMalloc pattern of its launchers (e.g.
 * src/inferno/cuda/cudasoftmax.cu:142-171).  Signatures use C types only:
 * raw device pointers, element strides and sizes passed by value.
 *
 * Conventions shared by every entry point:
 *   - Returns INF_OK (0) on success.  Arguments are validated on the host
 *     before anything touches the GPU, so an invalid call returns an error
 *     code without a device.  HIP failures return INF_ERR_HIP.
 *   - The layer never allocates: outputs and workspaces come from the caller
 *     (query sizes with inf_attn_workspace_bytes).
 *   - Work is enqueued on `stream` (a hipStream_t; NULL = the default stream)
 *     and is asynchronous with respect to the host.
 *   - Attention tensors are 4-D [B, H, T, D] views with arbitrary element
 *     strides for B, H and T and a unit stride for D; rows must be 16-byte
 *     aligned (fp32) or 8-byte aligned (bf16).
 *   - Causal semantics are those of triu(ones[T,T], 1) + masked_fill(-1e9f)
 *     (InfernoApp/main.cpp:747-748, 781-811): key j is visible to query i iff
 *     j <= i + (Tk - Tq).  The reference only has Tq == Tk.
 *   - dtype INF_BF16 means bf16 storage for q, k, v, o, dO, dq, dk, dv with
 *     fp32 arithmetic; lse and the workspace are always fp32.
 */
#ifndef INFERNO_HIP_H
#define INFERNO_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* INF_F64 and INF_I32 are accepted by the softmax entry points only (the
 * other element types of the reference's Softmax dispatch); the attention,
 * decode and nn entry points return INF_ERR_BAD_DTYPE for them. */
typedef enum { INF_F32 = 0, INF_BF16 = 1, INF_F64 = 2, INF_I32 = 3 } inf_dtype;

/* Element strides of a [B, H, T, D] view: d must be 1, all >= 0, and
 * t <= 2^22 (tiles are addressed with 32-bit byte offsets); otherwise the
 * attention entry points return INF_ERR_BAD_STRIDE.  Output views (o, dq,
 * dk, dv) must not overlap themselves: ordering the dims of extent > 1 by
 * stride, each stride must be at least the span of the dims inside it (D for
 * the head dim), else INF_ERR_BAD_STRIDE. */
typedef struct {
    int64_t b, h, t, d;
} inf_strides;

enum {
    INF_OK = 0,
    INF_ERR_NULL_POINTER = 1,
    INF_ERR_BAD_SHAPE = 2,
    INF_ERR_BAD_STRIDE = 3,
    INF_ERR_BAD_DTYPE = 4,
    INF_ERR_UNSUPPORTED = 5, /* e.g. head dim not in {32, 64, 128} */
    INF_ERR_WORKSPACE = 6,
    INF_ERR_ALIGNMENT = 7,
    INF_ERR_BAD_SCALE = 8,
    INF_ERR_HIP = 9
};

/* Workspace ops for inf_attn_workspace_bytes. */
enum { INF_OP_ATTN_FWD = 0, INF_OP_ATTN_BWD = 1, INF_OP_ATTN_DECODE = 2 };

/* Human-readable text for a status code (static storage). */
const char* inf_status_string(int status);

/* Text about the most recent failure inside the library on the calling thread
 * (which library call failed, with its status and the problem shape), or ""
 * (thread-local storage, valid until the thread's next failing call). */
const char* inf_last_error_detail(void);

/* Library ABI version (major*10000 + minor*100 + patch). */
int inf_version(void);

/* Bytes of workspace an op needs for this shape (0 when none) on the current
 * device.  INF_OP_ATTN_FWD reports what a causal call needs (a non-causal
 * forward needs none); the size depends on the device's CU count, so query it
 * with the device that will run the call current. */
int inf_attn_workspace_bytes(int op, int B, int H, int Tq, int Tk, int D, inf_dtype dt,
                             size_t* out_bytes);

/*
 * Fused causal attention forward: o = softmax(mask(q k^T * scale)) v, and the
 * per-row log-sum-exp lse[b,h,i] = ln sum_j exp(s_ij) over the masked, scaled
 * scores (fp32, dense [B, H, Tq]) for the backward pass.
 * Replaces the chain matmul -> multiply -> triu/masked_fill -> Softmax ->
 * matmul of InfernoApp/main.cpp:737-754 (ops.cpp:437, ops.cpp:204,
 * ops.cpp:1235, softmax.cpp:22).  scale must be finite and > 0.
 * workspace: inf_attn_workspace_bytes(INF_OP_ATTN_FWD, ...) bytes, 256-byte
 * aligned, holding the partial results of query tiles whose key range is split
 * across workgroups (may be NULL when that size is 0); its contents on entry
 * do not matter.
 */
int inf_attn_fwd(const void* q, inf_strides sq, const void* k, inf_strides sk, const void* v,
                 inf_strides sv, void* o, inf_strides so, float* lse, void* workspace,
                 size_t ws_bytes, int B, int H, int Tq, int Tk, int D, float scale, int causal,
                 inf_dtype dt, void* stream);

/*
 * Fused causal attention backward (recompute from q, k, v, o, lse): writes
 * dq, dk, dv.  Replaces MMBackward(attn, v) -> SoftmaxBackward ->
 * MultiplyBackward -> MMBackward(q, kt) -> TransposeBackward
 * (mmbackward.cpp:36-98, softmaxbackward.cpp:36-128,
 * multiplybackward.cpp:34-57, transposebackward.cpp:35-51).
 * workspace: at least inf_attn_workspace_bytes(INF_OP_ATTN_BWD, ...) bytes,
 * 256-byte aligned; its contents on entry do not matter.  It holds the row
 * dots dO.O, the fp32 dQ accumulator (bf16, unless dq comes from the
 * query-major pass: inf_set_deterministic), and, for causal shapes whose
 * grid leaves the device unevenly loaded, the partial dK / dV of split key
 * blocks and their arrival counters.  Calls that share one workspace must not
 * overlap.
 */
int inf_attn_bwd(const void* q, inf_strides sq, const void* k, inf_strides sk, const void* v,
                 inf_strides sv, const void* o, inf_strides so, const void* dout,
                 inf_strides sdo, const float* lse, void* dq, inf_strides sdq, void* dk,
                 inf_strides sdk, void* dv, inf_strides sdv, void* workspace, size_t ws_bytes,
                 int B, int H, int Tq, int Tk, int D, float scale, int causal, inf_dtype dt,
                 void* stream);

/*
 * Deterministic dQ (process-wide, off by default; no counterpart in the
 * reference, whose CPU path sums dQ in a fixed order, cpuops.h:412-431).
 * inf_attn_bwd normally adds each key block's dQ contribution with fp32
 * atomics, so the last bits of dq may differ between runs (O, LSE, dK and dV
 * never do).  With enable != 0, every later inf_attn_bwd call takes dq from a
 * query-major pass instead: one workgroup per query tile recomputes the
 * scores and sums its key tiles in key order, the same on every run, at the
 * cost of two more matrix products per score.  The mode is read once per
 * call; the backward's workspace size depends on it (bf16 then needs no dQ
 * accumulator), so query inf_attn_workspace_bytes after setting it.  It also
 * makes inf_embedding_bwd sum each row in token order instead of with fp32
 * atomics, so with both a training step of the GPT model built on these calls
 * is bitwise reproducible.  Returns the previous setting.
 */
int inf_set_deterministic(int enable);
int inf_get_deterministic(void);

/*
 * Row softmax over the last axis: y = softmax(x) per row of `cols` elements
 * (unit stride within a row, row strides in elements).  Replaces cpu_softmax /
 * cuda_softmax behind Softmax(Tensor&, int) (softmax.cpp:22-79,
 * cudasoftmax.cu:110-172) for a contiguous last axis.  dt follows the
 * reference's dispatch (RT = promote_t<AT, float>): INF_F32 and INF_BF16
 * (fp32 arithmetic), INF_F64 (double arithmetic, exp included) and INF_I32
 * (x holds int32, y fp32: the ints enter the fp32 arithmetic converted).
 */
int inf_softmax_fwd(const void* x, void* y, int64_t rows, int64_t cols, int64_t x_row_stride,
                    int64_t y_row_stride, inf_dtype dt, void* stream);

/*
 * Softmax backward: dx = y * (dy - sum(dy * y)) per row.  Replaces
 * cpu_softmax_backward / cuda_softmax_backward behind SoftmaxBackward
 * (softmaxbackward.h:64-131, softmaxbackward.cpp:36-128,
 * cudasoftmax.cu:222-373).  y, dy and dx share dt: INF_F32, INF_BF16 or
 * INF_F64 (INF_I32 returns INF_ERR_BAD_DTYPE: dispatchFloatTwo takes floats).
 */
int inf_softmax_bwd(const void* y, const void* dy, void* dx, int64_t rows, int64_t cols,
                    int64_t y_row_stride, int64_t dy_row_stride, int64_t dx_row_stride,
                    inf_dtype dt, void* stream);

/*
 * Softmax along axis `axis` (negative counts from the end) of strided views
 * of rank 1..8: for every index of the other dims, the line of shape[axis]
 * elements x_strides[axis] apart.  Replaces cuda_softmax's strided walk
 * (src/inferno/cuda/cudasoftmax.cu:16-97, 110-172), one thread per line as
 * there, for an axis that is not the last: no transposed copies.  Strides are
 * in elements, >= 0; y must not overlap itself (else INF_ERR_BAD_STRIDE).
 * dt as inf_softmax_fwd (INF_I32: x int32, y fp32).  Many lines (>= 65536)
 * run one thread per line (an online max / sum pass and a write pass), fewer
 * run one workgroup per line.
 */
int inf_softmax_fwd_axis(const void* x, const int64_t* x_strides, void* y, const int64_t* y_strides, int ndim,
                         const int64_t* shape, int axis, inf_dtype dt, void* stream);

/*
 * Softmax backward along a strided axis: dx = y * (dy - sum(dy * y)) per line,
 * the lines as inf_softmax_fwd_axis's.  Replaces cuda_softmax_backward
 * (src/inferno/cuda/cudasoftmax.cu:222-373).  y, dy and dx share dt: INF_F32,
 * INF_BF16 or INF_F64; dx must not overlap itself.
 */
int inf_softmax_bwd_axis(const void* y, const int64_t* y_strides, const void* dy, const int64_t* dy_strides,
                         void* dx, const int64_t* dx_strides, int ndim, const int64_t* shape, int axis,
                         inf_dtype dt, void* stream);

/*
 * Single-query decode against a KV cache: o[b,h] = softmax(q k^T * scale) v
 * over all Tk cached keys (q, o: [B, H, 1, D]; caches [B, H, Tk, D]).  The
 * reference has no decode path; this equals the last row of a Tk-long causal
 * prefill through the same chain (InfernoApp/main.cpp:737-754 with Tq = 1).
 * workspace: inf_attn_workspace_bytes(INF_OP_ATTN_DECODE, ...) bytes, 256-byte
 * aligned (may be NULL when that size is 0, i.e. when one split covers Tk);
 * its contents on entry do not matter.
 */
int inf_attn_decode(const void* q, inf_strides sq, const void* kcache, inf_strides sk,
                    const void* vcache, inf_strides sv, void* o, inf_strides so, int B, int H,
                    int Tk, int D, float scale, inf_dtype dt, void* workspace, size_t ws_bytes,
                    void* stream);

/*
 * inf_attn_decode without a workspace: no counterpart in the reference.  For
 * callers that cannot allocate device memory (code under HIP graph capture,
 * tight serving loops, harnesses that forbid hipMalloc): the split partials
 * live in a static 4 MiB device array of the library (one per device, held
 * until the process ends), so the call allocates nothing.  Same arguments,
 * kernels and results as inf_attn_decode.  A shape whose partials need more
 * than 4 MiB (inf_attn_workspace_bytes(INF_OP_ATTN_DECODE, ...) > 4 MiB; only
 * some head-dim-128 shapes) returns INF_ERR_WORKSPACE before any HIP call.
 * Every call on a device shares that device's array: calls that overlap on
 * one device (other streams, other threads) race.
 */
int inf_attn_decode_static(const void* q, inf_strides sq, const void* kcache, inf_strides sk,
                           const void* vcache, inf_strides sv, void* o, inf_strides so, int B, int H,
                           int Tk, int D, float scale, inf_dtype dt, void* stream);

/* ---- element-wise support for the Tensor layer around the path ------------- */

/* dst[i] = value for i < n; elem_bytes 1, 2 or 4; `bits` holds the value's bit
 * pattern in the low elem_bytes bytes.  Replaces cuda_fill
 * (src/inferno/cuda/cudafilltensor.cu:16-42), which seeds Engine::backward with
 * ones_like (src/inferno/gradengine/engine.cpp:59). */
int inf_fill(void* dst, int64_t n, int elem_bytes, uint32_t bits, void* stream);

/* out[i] = a[i] (op) b[i], op INF_BIN_ADD or INF_BIN_MUL, dense operands of n
 * elements; a_scalar / b_scalar mark an operand broadcast from one element.
 * Replaces cuda_add / cuda_multiply (src/inferno/cuda/cudaadd.cu:20-142,
 * cudamultiply.cu:16-146) for the same-shape and scalar cases the path uses
 * (scores * scale, main.cpp:744; gradient accumulation, engine.cpp:166). */
enum { INF_BIN_ADD = 0, INF_BIN_MUL = 1 };
int inf_binary(int op, const void* a, const void* b, void* out, int64_t n, int a_scalar, int b_scalar,
               inf_dtype dt, void* stream);

/* triu of a strided view into a dense output of `shape` (rank 2..8, element
 * strides): element (..., r, c) is copied when c - r >= diagonal, else written
 * as all-zero bits; elem_bytes 1, 2, 4 or 8 (the copy is bit-exact for any
 * dtype).  Replaces cuda_triu (src/inferno/cuda/cudatri.cu:8-89) behind
 * triu (src/inferno/core/ops.cpp:1355-1398). */
int inf_triu(const void* a, const int64_t* a_strides, void* out, int rank, const int64_t* shape, int diagonal,
             int elem_bytes, void* stream);

/* out (dense, `shape`) = mask != 0 ? fill : in, for the strided view `in` and an
 * integer mask (mask_bytes 1, 4 or 8) broadcast from the right: mask_rank <=
 * rank and each mask dimension equal to the input's or 1 (size-1 dimensions
 * repeat; anything else is INF_ERR_BAD_SHAPE).  fill_bits holds the fill
 * value's bit pattern in the input's element type (elem_bytes 1, 2, 4 or 8).
 * Replaces cuda_masked_fill (src/inferno/cuda/cudamaskedfill.cu:23-164) behind
 * masked_fill (src/inferno/core/ops.cpp:1235-1289). */
int inf_masked_fill(const void* in, const int64_t* in_strides, const void* mask, const int64_t* mask_shape,
                    const int64_t* mask_strides, int mask_rank, int mask_bytes, void* out, int rank,
                    const int64_t* shape, uint64_t fill_bits, int elem_bytes, void* stream);

/* Strided copy: for every index tuple idx over `shape` (rank <= 8),
 * dst[sum_d idx_d * dst_strides[d]] = src[sum_d idx_d * src_strides[d]]
 * (element strides, elem_bytes 1, 2, 4 or 8).  With dense dst_strides this is
 * cuda_contiguous_copy (src/inferno/cuda/cudacontiguous.cu:16-139) without its
 * per-call metadata cudaMalloc and device synchronisation; with strided dst it
 * writes a gradient back into a view of a larger tensor (SliceBackward,
 * src/inferno/gradfn/slicebackward.cpp:35-53). */
int inf_copy_strided(const void* src, const int64_t* src_strides, void* dst,
                     const int64_t* dst_strides, int ndim, const int64_t* shape, int elem_bytes,
                     void* stream);

/* ---- model ops either side of the path: the GPT training step -------------
 * (embedding -> [LayerNorm -> MultiHeadAttention -> residual
 * -> LayerNorm -> Linear -> GELU -> Linear -> residual] x L -> LayerNorm ->
 * tied logits -> cross-entropy -> AdamW).  Same conventions as above: host-side
 * validation first, no allocation, caller-provided workspaces (sizes from
 * inf_nn_workspace_bytes), asynchronous on `stream`.  Matrices are row-major
 * with a leading dimension in elements; fp32 or bf16 storage, fp32 arithmetic;
 * LayerNorm parameters, statistics, AdamW moments and reductions are fp32. */

enum { INF_OP_GEMM = 3, INF_OP_LAYERNORM_BWD = 4, INF_OP_COL_SUM = 5, INF_OP_CROSS_ENTROPY = 6 };

/* Workspace bytes for a model op: INF_OP_GEMM (any shape; the hipBLASLt
 * workspace), INF_OP_LAYERNORM_BWD (rows, cols = dim), INF_OP_COL_SUM (rows,
 * cols), INF_OP_CROSS_ENTROPY (rows, cols = vocab). */
int inf_nn_workspace_bytes(int op, int64_t rows, int64_t cols, size_t* out_bytes);

/* C[b] = alpha * op(A[b]) op(B[b]) + beta * C[b] (+ bias[n] added to every row)
 * for b < batch, row-major: op(A) is M x K (A stored M x K, or K x M when
 * trans_a), op(B) is K x N (B stored K x N, or N x K when trans_b); batch
 * strides in elements.  Runs on hipBLASLt (fp32 matrix cores for fp32).
 * Replaces cublas_mm_strided_batched_row_major and cuda_matmul
 * (src/inferno/cuda/cudamatmul.cu:120-216, 1114-1179) behind matmul
 * (src/inferno/core/ops.cpp:437-735) and Linear::forward (linear.cpp:49-54). */
int inf_gemm(int trans_a, int trans_b, int64_t M, int64_t N, int64_t K, float alpha, const void* A, int64_t lda,
             int64_t stride_a, const void* B, int64_t ldb, int64_t stride_b, float beta, void* C, int64_t ldc,
             int64_t stride_c, int64_t batch, const void* bias, inf_dtype dt, void* workspace, size_t ws_bytes,
             void* stream);

/* LayerNorm over the last `dim` elements of each of `rows` rows:
 * y = (x - mean) / sqrt(var + eps) * gamma + beta (biased variance), and the
 * per-row mean and 1/sqrt(var + eps) (either may be NULL).  Replaces
 * cuda_layer_normalization (src/inferno/cuda/cudaops.h:78, cudalayernorm.cu)
 * behind LayerNorm::forward (src/inferno/modules/layernorm.cpp:33-80). */
int inf_layernorm_fwd(const void* x, int64_t ldx, void* y, int64_t ldy, const float* gamma, const float* beta,
                      float* mean, float* invstd, int64_t rows, int64_t dim, float eps, inf_dtype dt, void* stream);

/* Residual add and LayerNorm in one pass: h = x + r (rounded to dt, stored),
 * y = LayerNorm(h) as inf_layernorm_fwd computes it -- the same values as an
 * add followed by inf_layernorm_fwd.  h may be x or r (updated in place); y
 * must not overlap x, r or h.  No reference counterpart: the reference runs
 * the transformer block's residual add and the next LayerNorm as two launches
 * (`x = x + attn_out` then `layernorm2.forward(x)`, InfernoApp/main.cpp:868-874);
 * this is for inference loops, where each launch costs more than the row's
 * work. */
int inf_add_layernorm_fwd(const void* x, int64_t ldx, const void* r, int64_t ldr, void* h, int64_t ldh, void* y,
                          int64_t ldy, const float* gamma, const float* beta, float* mean, float* invstd, int64_t rows,
                          int64_t dim, float eps, inf_dtype dt, void* stream);

/* LayerNorm backward from the saved mean / invstd: dx, and dgamma = sum_rows
 * dy * xhat, dbeta = sum_rows dy (overwritten, or added to when accumulate).
 * dim % 4 == 0 and dim <= 2048.  Replaces cuda_layernorm_backward
 * (src/inferno/cuda/cudaops.h:82) behind LayerNormBackward
 * (src/inferno/gradfn/layernormbackward.cpp:29-110). */
int inf_layernorm_bwd(const void* x, int64_t ldx, const void* dy, int64_t lddy, const float* gamma, const float* mean,
                      const float* invstd, void* dx, int64_t lddx, float* dgamma, float* dbeta, int accumulate,
                      int64_t rows, int64_t dim, inf_dtype dt, void* workspace, size_t ws_bytes, void* stream);

/* tanh-approximation GELU, y = 0.5 x (1 + tanh(sqrt(2/pi) (x + 0.044715 x^3))),
 * and its backward dx = dy * gelu'(x), over n dense elements.  Replaces
 * cuda_gelu / cuda_gelu_backward (src/inferno/cuda/cudaops.h:130, 137) behind
 * gelu (src/inferno/functional/gelu.cpp) and GeluBackward. */
int inf_gelu_fwd(const void* x, void* y, int64_t n, inf_dtype dt, void* stream);
int inf_gelu_bwd(const void* x, const void* dy, void* dx, int64_t n, inf_dtype dt, void* stream);

/* Mean cross-entropy over rows of logits [rows, vocab] (row stride ld) with
 * int32 targets: loss[0] = mean_r (lse_r - logits[r, target_r]), and the
 * per-row lse for the backward.  A target outside [0, vocab) makes the loss
 * NaN (the reference exits).  Replaces cuda_cross_entropy_loss
 * (src/inferno/cuda/cudaops.h:186) behind CrossEntropyLoss::forward
 * (src/inferno/loss/crossentropyloss.cpp). */
int inf_cross_entropy_fwd(const void* logits, int64_t ld, const int32_t* targets, float* loss, float* lse,
                          int64_t rows, int64_t vocab, inf_dtype dt, void* workspace, size_t ws_bytes, void* stream);

/* dlogits = (softmax(logits) - onehot(target)) * upstream[0] / rows, from the
 * forward's lse.  Replaces cuda_cross_entropy_loss_backward
 * (src/inferno/cuda/cudaops.h:190) behind CrossEntropyLossBackward. */
int inf_cross_entropy_bwd(const void* logits, int64_t ld, const int32_t* targets, const float* lse,
                          const float* upstream, void* dlogits, int64_t ldg, int64_t rows, int64_t vocab, inf_dtype dt,
                          void* stream);

/* out[t, :] = table[ids[t], :] (dim % 4 == 0; an id outside [0, vocab) gives a
 * NaN row).  Replaces cuda_embedding (src/inferno/cuda/cudaops.h:65). */
int inf_embedding_fwd(const int32_t* ids, int64_t n_tokens, const void* table, int64_t vocab, int64_t dim, void* out,
                      inf_dtype dt, void* stream);

/* dtable[ids[t], :] += dout[t, :] (fp32, atomic); zero_first clears dtable
 * first.  In the deterministic mode (inf_set_deterministic, dim <= 16384) each
 * row of dtable is instead summed in token order by one workgroup, the same
 * bits on every run.  Replaces cuda_scatter_add_embedding
 * (src/inferno/cuda/cudaops.h:68) behind EmbeddingBackward. */
int inf_embedding_bwd(const int32_t* ids, int64_t n_tokens, const float* dout, int64_t vocab, int64_t dim,
                      float* dtable, int zero_first, void* stream);

/* One AdamW update of n elements (p, g in dt; m, v fp32), bias corrections
 * computed by the caller: m = b1 m + (1-b1) g; v = b2 v + (1-b2) g^2;
 * p -= lr * ((m/bc1) / (sqrt(v/bc2) + eps) + wd * p).  Replaces
 * cuda_adamw_step_impl (src/inferno/cuda/cudaops.h:61) behind
 * OptimizerAdamW::step (src/inferno/optim/adamw.cpp). */
int inf_adamw_step(void* p, const void* g, float* m, float* v, int64_t n, float lr, float beta1, float beta2, float eps,
                   float weight_decay, float bias_correction1, float bias_correction2, inf_dtype dt, void* stream);

/* One parameter tensor of a multi-tensor AdamW step: p, g (dt), m, v (fp32),
 * n elements; p and g 16-byte (fp32) / 8-byte (bf16) aligned, m and v 16-byte
 * aligned, tensors disjoint. */
typedef struct {
    void* p;
    const void* g;
    float* m;
    float* v;
    int64_t n;
} inf_adamw_tensor;

/* The same update as inf_adamw_step (bit-identical per element) over a list of
 * tensors in as few launches as the list allows (48 tensors per launch).
 * Replaces the per-parameter loop of OptimizerAdamW::step
 * (src/inferno/optim/adamw.cpp:18-64, one cuda_adamw_step_impl launch per
 * parameter).  The table is read on the host during the call. */
int inf_adamw_step_multi(const inf_adamw_tensor* tensors, int n_tensors, float lr, float beta1, float beta2,
                         float eps, float weight_decay, float bias_correction1, float bias_correction2, inf_dtype dt,
                         void* stream);

/* out[c] = sum_r x[r * ldx + c] (or out[c] += when accumulate), fp32 result:
 * the bias gradient of Linear and the gradient of a broadcast operand.
 * Replaces cuda_sum_to_shape (src/inferno/cuda/cudaops.h:43) for reductions
 * over leading dimensions. */
int inf_col_sum(const void* x, int64_t rows, int64_t cols, int64_t ldx, float* out, int accumulate, inf_dtype dt,
                void* workspace, size_t ws_bytes, void* stream);

/* out[i] = a[i] (op) b[i % nb] for i < n (b repeated over leading dimensions:
 * a bias over rows, a positional table over the batch); op INF_BIN_ADD or
 * INF_BIN_MUL.  Replaces cuda_add / cuda_multiply (cudaadd.cu, cudamultiply.cu)
 * for trailing broadcasts. */
int inf_binary_bcast(int op, const void* a, const void* b, void* out, int64_t n, int64_t nb, inf_dtype dt,
                     void* stream);

/* out[r] = the column index of the largest element of row r of x [rows, cols]
 * (row stride ld elements), the first one on ties -- std::max_element's pick.
 * No counterpart in the reference, which has no generation loop: the greedy
 * next-token choice, so only rows int32 values leave the device. */
int inf_argmax_rows(const void* x, int64_t rows, int64_t cols, int64_t ld, int32_t* out, inf_dtype dt, void* stream);

#ifdef __cplusplus
}
#endif
#endif
