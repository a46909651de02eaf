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

typedef enum { INF_F32 = 0, INF_BF16 = 1 } inf_dtype;

/* Element strides of a [B, H, T, D] view (d must be 1). */
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

/* Library ABI version (major*10000 + minor*100 + patch). */
int inf_version(void);

/* Bytes of workspace an op needs for this shape (0 when none). */
int inf_attn_workspace_bytes(int op, int B, int H, int Tq, int Tk, int D, inf_dtype dt,
                             size_t* out_bytes);

/*
 * Fused causal attention forward: o = softmax(mask(q k^T * scale)) v, and the
 * per-row log-sum-exp lse[b,h,i] = ln sum_j exp(s_ij) over the masked, scaled
 * scores (fp32, dense [B, H, Tq]) for the backward pass.
 * Replaces the chain matmul -> multiply -> triu/masked_fill -> Softmax ->
 * matmul of InfernoApp/main.cpp:737-754 (ops.cpp:437, ops.cpp:204,
 * ops.cpp:1235, softmax.cpp:22).  scale must be finite and > 0.
 */
int inf_attn_fwd(const void* q, inf_strides sq, const void* k, inf_strides sk, const void* v,
                 inf_strides sv, void* o, inf_strides so, float* lse, int B, int H, int Tq,
                 int Tk, int D, float scale, int causal, inf_dtype dt, void* stream);

/*
 * Fused causal attention backward (recompute from q, k, v, o, lse): writes
 * dq, dk, dv.  Replaces MMBackward(attn, v) -> SoftmaxBackward ->
 * MultiplyBackward -> MMBackward(q, kt) -> TransposeBackward
 * (mmbackward.cpp:36-98, softmaxbackward.cpp:36-128,
 * multiplybackward.cpp:34-57, transposebackward.cpp:35-51).
 * workspace: at least inf_attn_workspace_bytes(INF_OP_ATTN_BWD, ...) bytes,
 * 256-byte aligned; its contents on entry do not matter.
 */
int inf_attn_bwd(const void* q, inf_strides sq, const void* k, inf_strides sk, const void* v,
                 inf_strides sv, const void* o, inf_strides so, const void* dout,
                 inf_strides sdo, const float* lse, void* dq, inf_strides sdq, void* dk,
                 inf_strides sdk, void* dv, inf_strides sdv, void* workspace, size_t ws_bytes,
                 int B, int H, int Tq, int Tk, int D, float scale, int causal, inf_dtype dt,
                 void* stream);

/*
 * Row softmax over the last axis: y = softmax(x) per row of `cols` elements
 * (unit stride within a row, row strides in elements).  Replaces cpu_softmax /
 * cuda_softmax behind Softmax(Tensor&, int) (softmax.cpp:22-79,
 * cudasoftmax.cu:110-172) for a contiguous last axis.
 */
int inf_softmax_fwd(const void* x, void* y, int64_t rows, int64_t cols, int64_t x_row_stride,
                    int64_t y_row_stride, inf_dtype dt, void* stream);

/*
 * Softmax backward: dx = y * (dy - sum(dy * y)) per row.  Replaces
 * cpu_softmax_backward / cuda_softmax_backward behind SoftmaxBackward
 * (softmaxbackward.h:64-131, softmaxbackward.cpp:36-128,
 * cudasoftmax.cu:222-373).
 */
int inf_softmax_bwd(const void* y, const void* dy, void* dx, int64_t rows, int64_t cols,
                    int64_t y_row_stride, int64_t dy_row_stride, int64_t dx_row_stride,
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

#ifdef __cplusplus
}
#endif
#endif
