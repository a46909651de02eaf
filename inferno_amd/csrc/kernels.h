// kernels.h -- parameter blocks and host launchers shared by the C-ABI layer
// (capi.cpp) and the kernel translation units.  Internal; not installed.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <string>

namespace inf {

struct View4 {            // element strides of a [B,H,T,D] view, d stride 1
    int64_t b, h, t;
};

// Work split of the forward: dispatch group g (grid blocks [g*B*H, (g+1)*B*H),
// one per head) runs query tile `qt` over key tiles [t0, t1).  slot < 0: the
// group covers the tile's whole key range and writes O / LSE; slot >= 0: it
// writes partials (unnormalised O, row max, row sum) to partial slot `slot`
// and attn_fwd_merge_kernel combines the slots of that query tile.
constexpr int kMaxFwdGroups = 96;
struct FwdGroup {
    int qt, t0, t1, slot;
};

struct FwdParams {
    const void* q;
    const void* k;
    const void* v;
    void* o;
    float* lse;           // dense [B,H,Tq] or null
    View4 sq, sk, sv, so;
    int B, H, Tq, Tk, D;
    int causal;
    int off;              // Tk - Tq: key j visible to query i iff j <= i + off
    float scale;          // softmax scale
    float c;              // scale * log2(e)
    int n_qtiles;
    int n_groups;         // 0: one group per query tile, heaviest first (no split)
    int n_slots;          // partial slots in use
    float* part;          // workspace: n_slots * B*H * kFwdBM * (D + 2) floats
    int n_split;          // query tiles whose key range is split
    int pv_prio;          // bf16 D = 128 unsplit: P.V MFMAs at raised wave priority (see fwd_plan)
    FwdGroup groups[kMaxFwdGroups];
    int split_qt[kMaxFwdGroups / 2], split_slot0[kMaxFwdGroups / 2], split_count[kMaxFwdGroups / 2];
};

// Split plan of the forward for a shape (causal; fp32 and bf16 kernels).
struct FwdPlan {
    int n_groups = 0, n_slots = 0;
    // bf16 D = 128 without a split: the P.V MFMAs at raised wave priority only
    // when the grid exceeds one round of the device's workgroup slots
    int pv_prio = 1;
    FwdGroup groups[kMaxFwdGroups];
    // per split query tile: first slot and number of slots
    int n_split = 0;
    int split_qt[kMaxFwdGroups / 2], split_slot0[kMaxFwdGroups / 2], split_count[kMaxFwdGroups / 2];
};
// Returns 0, or the HIP error an earlier call left pending (see report_pending_error).
int fwd_plan(int B, int H, int Tq, int Tk, int D, int causal, int bf16, FwdPlan* out);
size_t fwd_workspace_bytes(const FwdPlan& plan, int B, int H, int D);

// Backward work split: a group is one key block's query-tile range [t0, t1)
// (in 32-row tiles) for every (b, h).  Groups of a split key block write fp32
// partial dK^T / dV^T accumulators to `part` (slot slot0 + chunk); the last of
// its `n_chunks` groups to finish (per-(split, b, h) counter) adds the others'
// partials to its own and stores dK and dV.
constexpr int kMaxBwdGroups = 48;
struct BwdGroup {
    int kb, t0, t1;
    int split;     // -1: unsplit key block, else index of the split key block
    int chunk, n_chunks, slot0;
};

struct BwdPlan {
    int n_groups = 0, n_split = 0, n_slots = 0;
    int bk = 0;  // keys per workgroup of the kernel the plan is for
    BwdGroup groups[kMaxBwdGroups];
};
// Returns 0, or the HIP error an earlier call left pending (see report_pending_error).
int bwd_plan(int B, int H, int Tq, int Tk, int D, int causal, int bf16, BwdPlan* out);
// Bytes of the split plan's workspace: partials then counters (0 without a split).
size_t bwd_split_workspace_bytes(const BwdPlan& plan, int B, int H, int D);

struct BwdParams {
    const void* q;
    const void* k;
    const void* v;
    const void* o;
    const void* dout;
    const float* lse;     // dense [B,H,Tq]
    float* delta;         // workspace, dense [B,H,Tq]: rowsum(dO * O) (unused where the main kernel forms it)
    float* delta_lo;      // workspace, dense [B,H,Tq]: the short rows' delta is delta + delta_lo (bwd_split.h)
    float* dq_acc;        // fp32 dQ accumulation (dq itself for fp32)
    View4 sacc;           // strides of dq_acc
    void* dq;
    void* dk;
    void* dv;
    View4 sq, sk, sv, so, sdo, sdq, sdk, sdv;
    int B, H, Tq, Tk, D;
    int causal, off;
    float scale, c;
    int n_kblocks;
    int dq_direct;          // bf16: dQ from the query-major pass (no accumulator, no atomics)
    int pre_delta;          // bwd_pre computes delta (set by the launcher: off where no kernel reads it)
    int n_qtiles;           // query tiles of kBwdDqBM rows (dQ pass)
    int n_short;            // rows [0, n_short) see only keys of key block 0 (bwd_short_rows)
    // split plan (n_groups == 0: workgroup w takes key block w / (B*H), all its tiles)
    int n_groups, n_split;
    float* part;            // n_slots * B*H * 2*D*(keys per workgroup) floats (lane-major accumulators)
    unsigned* counters;     // n_split * B*H, zeroed by bwd_pre / bwd_zero
    BwdGroup groups[kMaxBwdGroups];
};

struct DecodeParams {
    const void* q;
    const void* k;
    const void* v;
    void* o;
    float* part;          // workspace [B*H, nsplit, D + 2]
    View4 sq, sk, sv, so;
    int B, H, Tk, D;
    int nsplit;           // key splits per (b, h)
    int chunk;            // keys per split
    float c;              // scale * log2(e)
};

struct SoftmaxParams {
    const void* x;        // fwd: x; bwd: y
    const void* g;        // bwd: dy
    void* y;              // fwd: y; bwd: dx
    int64_t rows;
    int64_t cols;
    int64_t sx, sg, sy;   // row strides (elements)
};

constexpr int kMaxRank = 8;
struct StridedCopy {      // element strides of source and destination
    int ndim;
    int64_t n;
    int64_t shape[kMaxRank];
    int64_t sstride[kMaxRank];
    int64_t dstride[kMaxRank];
};

// ---- model ops around the attention path (nn.hip) ----------------------------
struct LnParams {         // LayerNorm forward over rows of `dim` (unit column stride)
    const void* x;
    void* y;
    const float* gamma;
    const float* beta;
    float* mean;          // [rows] or null
    float* invstd;        // [rows] or null
    int64_t rows, ldx, ldy;
    int dim;
    float eps;
    int vec;              // 16-byte rows and parameters: the register kernel
    const void* r;        // residual added to x first (null: plain LayerNorm) ...
    void* h;              // ... and the sum x + r, stored in the element type
    int64_t ldr, ldh;
};

struct LnBwdParams {
    const void* x;
    const void* dy;
    void* dx;
    const float* gamma;
    const float* mean;
    const float* invstd;
    float* dgamma;
    float* dbeta;
    float* part;          // workspace: 2 * ln_bwd_blocks(rows) * dim floats
    int64_t rows, ldx, lddy, lddx;
    int dim;
    int accumulate;       // add into dgamma / dbeta instead of overwriting
};

struct CeParams {
    const void* logits;   // [rows, vocab], row stride ld
    const int32_t* targets;
    float* row_loss;      // workspace [rows]
    float* lse;           // [rows]: written by the forward, read by the backward
    const float* upstream;  // backward: the loss gradient (one element)
    void* grad;           // backward: dlogits, row stride ldg
    int64_t rows, vocab, ld, ldg;
};

struct EmbParams {
    const int32_t* ids;   // [n_tokens]
    const void* table;    // [vocab, dim]
    const void* dout;     // backward: [n_tokens, dim] fp32
    void* out;            // forward: [n_tokens, dim]; backward: dtable [vocab, dim] fp32 (zeroed)
    int64_t n_tokens, vocab, dim;
};

struct AdamWParams {
    void* p;
    const void* g;
    float* m;
    float* v;
    int64_t n;
    float lr, beta1, beta2, eps, weight_decay, bc1, bc2;
};

// Multi-tensor AdamW: up to kAdamWMaxTensors tensors per launch, the table
// passed by value in the kernel arguments; workgroup w updates elements
// [1024 (w - block0[t]), +1024) of the tensor t with block0[t] <= w < block0[t+1].
constexpr int kAdamWMaxTensors = 48;
struct AdamWMultiParams {
    float lr, beta1, beta2, eps, weight_decay, bc1, bc2;
    int n_tensors;
    void* p[kAdamWMaxTensors];
    const void* g[kAdamWMaxTensors];
    float* m[kAdamWMaxTensors];
    float* v[kAdamWMaxTensors];
    int64_t n[kAdamWMaxTensors];
    int block0[kAdamWMaxTensors + 1];
};

struct GemmArgs {         // row-major C = alpha * op(A) op(B) + beta * C (+ bias[N] per row)
    int ta, tb, bf16;
    int64_t M, N, K;
    float alpha, beta;
    const void* A;
    int64_t lda, sa;
    const void* B;
    int64_t ldb, sb;
    void* C;
    int64_t ldc, sc;
    int64_t batch;
    const void* bias;     // [N] or null
    void* ws;
    size_t ws_bytes;
};
// 0 = ok, 1 = library error, 2 = no algorithm for the problem
int launch_gemm(const GemmArgs& g, hipStream_t s);

// Thread-local text about the last failure inside the library (inf_last_error_detail).
void set_error_detail(const std::string& msg);
// Names a HIP error that an earlier, unrelated call left pending on this
// thread (found before a query of ours would clear it) in the detail text,
// and returns it, so the entry point fails with INF_ERR_HIP and launches nothing.
int report_pending_error(hipError_t e, const char* where);

constexpr int kLnBwdMaxBlocks = 512;  // stage-1 workgroups of the LayerNorm backward
constexpr int kColChunk = 32;         // rows per partial of the column sum
constexpr int kLnBwdMaxDim = 2048;    // register path of the LayerNorm backward
int ln_bwd_blocks(int64_t rows);
int col_sum_chunks(int64_t rows);     // partial rows the column sum needs

int launch_ln_fwd(const LnParams& p, int bf16, hipStream_t s);
int launch_ln_bwd(const LnBwdParams& p, int bf16, hipStream_t s);
int launch_col_sum(const void* x, float* out, float* part, int64_t rows, int64_t cols, int64_t ldx, int accumulate,
                   int bf16, hipStream_t s);
int launch_gelu_fwd(const void* x, void* y, int64_t n, int bf16, hipStream_t s);
int launch_gelu_bwd(const void* x, const void* dy, void* dx, int64_t n, int bf16, hipStream_t s);
int launch_ce_fwd(const CeParams& p, float* loss, int bf16, hipStream_t s);
int launch_ce_bwd(const CeParams& p, int bf16, hipStream_t s);
int launch_embed_fwd(const EmbParams& p, int bf16, hipStream_t s);
int launch_embed_bwd(const EmbParams& p, hipStream_t s);
// Deterministic embedding backward (rows summed in token order); dim <= 16384.
int launch_embed_bwd_det(const EmbParams& p, int zero_first, hipStream_t s);
int launch_adamw(const AdamWParams& a, int bf16, hipStream_t s);
int launch_adamw_multi(const AdamWMultiParams& a, int bf16, hipStream_t s);
int launch_argmax_rows(const void* x, int64_t rows, int64_t cols, int64_t ld, int32_t* out, int bf16, hipStream_t s);
int launch_bcast(int op, const void* a, const void* b, void* out, int64_t n, int64_t nb, int vec, int bf16,
                 hipStream_t s);

// Launchers return a hipError_t value (0 = hipSuccess).
int launch_attn_fwd(const FwdParams& p, int bf16, hipStream_t s);
int launch_attn_fwd_bf16(const FwdParams& p, hipStream_t s);  // bf16-MFMA forward (no merge pass)
int fwd_bf16_occupancy(int D, int* blocks_per_cu);  // hipError_t
int launch_attn_bwd(const BwdParams& p, int bf16, hipStream_t s);
int bwd_main_bf16_occupancy(int D, int* blocks_per_cu);  // hipError_t
int launch_bwd_main_bf16(const BwdParams& p, hipStream_t s);  // bf16-MFMA backward main kernel
int launch_attn_decode(const DecodeParams& p, int bf16, hipStream_t s);
// Decode split plan (number of key splits per row, keys per split) for a shape.
void decode_plan(int B, int H, int Tk, int D, int* nsplit, int* chunk);
// The static scratch of inf_attn_decode_static (4 MiB: every shape whose
// B*H*nsplit*(D+2) floats fit; the plan keeps B*H*nsplit below 8192, so only
// D = 128 shapes with 8066 <= B*H*nsplit <= 8191 need more: 4 MiB holds 8065
// rows of 130 floats), and its
// device address on the current device (looked up once per device).
constexpr size_t kDecodeScratchBytes = (size_t)4 << 20;
int decode_scratch(float** out);
// Element types of the standalone softmax: fp32, bf16 storage (fp32
// arithmetic), int32 input with fp32 output (forward only), fp64.
enum class SmType { F32, BF16, I32, F64 };
int launch_softmax_fwd(const SoftmaxParams& p, SmType t, int vec_ok, hipStream_t s);
int launch_softmax_bwd(const SoftmaxParams& p, SmType t, int vec_ok, hipStream_t s);

// Softmax along one axis of strided views (rank <= kMaxRank), in place of
// moving the axis last: the other dims index `groups` lines (the last dim
// fastest), each of `n` elements `s*[axis]` apart.
struct SoftmaxAxis {
    const void* x;   // fwd: x; bwd: y
    const void* g;   // bwd: dy
    void* y;         // fwd: y; bwd: dx
    int ndim, axis;
    int64_t groups, n;
    int64_t shape[kMaxRank];
    int64_t sx[kMaxRank], sg[kMaxRank], sy[kMaxRank];  // element strides of x, g, y
};
int launch_softmax_axis_fwd(const SoftmaxAxis& p, SmType t, hipStream_t s);
int launch_softmax_axis_bwd(const SoftmaxAxis& p, SmType t, hipStream_t s);
int launch_fill(void* dst, int64_t n, int elem_bytes, uint32_t bits, hipStream_t s);
int launch_binary(int op, const void* a, const void* b, void* out, int64_t n, int a_scalar, int b_scalar,
                  int bf16, hipStream_t s);
int launch_copy_strided(const void* src, void* dst, const StridedCopy& c, int elem_bytes, hipStream_t s);

// triu of a strided view into a dense output: StridedCopy's shape / sstride
// describe the source (dstride unused).
int launch_triu(const void* src, void* dst, const StridedCopy& c, int diagonal, int elem_bytes, hipStream_t s);

struct MaskedFill {       // element strides; mstride is the mask's, padded on the left, 0 where it repeats
    int ndim;
    int64_t n;
    int64_t shape[kMaxRank];
    int64_t istride[kMaxRank];
    int64_t mstride[kMaxRank];
};
int launch_masked_fill(const void* in, const void* mask, void* out, const MaskedFill& m, int elem_bytes,
                       int mask_bytes, uint64_t fill_bits, hipStream_t s);

// Tile shapes the host needs for grids and workspace sizing.
constexpr int kFwdBM = 128;      // query rows per forward workgroup
constexpr int kFwdBf16BN = 64;   // keys per K/V tile of the bf16 forward (every D)
// Backward workgroups: one wave per 32 keys.  bf16 at D = 64: 8 waves = 256
// keys, half the dQ atomics per key (two waves per SIMD, as with two 4-wave
// workgroups); at bf16 speed the atomics are a device-wide limit.  fp32 keeps
// 4 waves (its atomics cost ~2.5%, and 256-key blocks measured 5-10% slower
// under a causal mask: fewer, heavier workgroups).  fp32 at D = 128 needs
// ~430 registers per wave (one wave per SIMD) and D = 32 keeps three 4-wave
// workgroups per CU: both use 4 waves.  bf16 at D = 128 runs its own kernel,
// 8 waves x 16 keys: 128 keys per workgroup, as with 4 x 32.
constexpr int bwd_waves(int bf16, int D) { return bf16 && D == 64 ? 8 : 4; }
constexpr int bwd_bf16_waves(int D) { return bwd_waves(1, D); }
inline int bwd_keys_per_wg(int bf16, int D) { return bf16 && D == 128 ? 128 : 32 * bwd_waves(bf16, D); }
constexpr int kBwdBQ = 32;       // query rows per backward inner step
// Leading query rows whose visible keys all lie in key block 0 (keys_per_wg
// keys): their softmax-backward row dot is formed inside the block-0
// workgroup from its own P and dP (bwd_split.h) -- on problems where those
// rows number at most kBwdShortMaxRows over all heads, else none.  There each
// row's rounding is measured against a scale the row itself sets (few rows),
// and the prologue that forms it costs little; on larger problems the tensor's
// scale comes from many rows, the row dot from rowsum(dO * O) is far within
// the error bars, and the prologue measured +10-70% on short sequences (its S
// and dP on every short row again).  Rows with one visible key need no row
// dot: every kernel sets their dS to 0, as P (dP - dP) is.
constexpr int64_t kBwdShortMaxRows = 4096;
inline int bwd_short_rows(int B, int H, int Tq, int Tk, int causal, int keys_per_wg) {
    int64_t r = causal ? (int64_t)keys_per_wg - ((int64_t)Tk - Tq) : (Tk <= keys_per_wg ? Tq : 0);
    r = r < 0 ? 0 : (r > Tq ? Tq : r);
    return (int64_t)B * H * r <= kBwdShortMaxRows ? (int)r : 0;
}
constexpr int kBwdDqBM = 128;    // query rows per workgroup of the query-major dQ pass
int launch_bwd_dq_bf16(const BwdParams& p, hipStream_t s);
// bf16 at D = 128: dQ from a query-major pass instead of fp32 atomics when a
// query row collects adds from many key blocks (the atomic stream bounds the
// fused kernel there: config 4 -24%, B2 H8 T4096 -14%) and the pass fills
// the device (two workgroups per CU); short ranges, small grids and D = 64
// (whose 256-key blocks halve the adds) keep the atomics.
inline bool bwd_dq_direct(int BH, int Tq, int Tk, int D, int keys_per_wg) {
    return D == 128 && (Tk + keys_per_wg - 1) / keys_per_wg >= 32 &&
           (int64_t)((Tq + kBwdDqBM - 1) / kBwdDqBM) * BH >= 512;
}

}  // namespace inf
