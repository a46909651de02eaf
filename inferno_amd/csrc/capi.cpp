// capi.cpp -- the extern "C" boundary (include/inferno_hip.h): host-side
// argument validation, workspace sizing and kernel launches.
//
// Every check runs before the first HIP call, so invalid arguments return a
// status code on a machine without a GPU.  Nothing here allocates.
#include "inferno_hip.h"

#include <hip/hip_runtime.h>

#include <algorithm>
#include <atomic>
#include <cmath>
#include <cstdint>
#include <cstring>
#include <string>
#include <utility>

#include "kernels.h"

namespace {

constexpr size_t kAlign = 256;

// inf_set_deterministic: every backward takes dQ from the query-major pass.
std::atomic<int> g_deterministic{0};

// Whether a backward of this shape takes dQ from the query-major pass: always
// in the deterministic mode, else bf16 shapes where the atomics bound the
// fused kernel (bwd_dq_direct).
bool dq_from_pass(int det, int B, int H, int Tq, int Tk, int D, inf_dtype dt) {
    return det || (dt == INF_BF16 && inf::bwd_dq_direct(B * H, Tq, Tk, D, inf::bwd_keys_per_wg(1, D)));
}

size_t round_up(size_t x) { return (x + kAlign - 1) / kAlign * kAlign; }

int elem_bytes(inf_dtype dt) { return dt == INF_BF16 ? 2 : (dt == INF_F64 ? 8 : 4); }

bool dtype_ok(int dt) { return dt == INF_F32 || dt == INF_BF16; }

bool head_dim_ok(int D) { return D == 32 || D == 64 || D == 128; }

// Row stride limit: the kernels address a tile of up to 128 rows through a
// buffer resource with 32-bit byte offsets, so 128 * stride * 4 B < 2^31.
constexpr int64_t kMaxRowStride = int64_t(1) << 22;

// A [B,H,T,D] view: unit d stride, non-negative strides at most
// kMaxRowStride along t, rows aligned for 4-element vector access (16 B fp32,
// 8 B bf16).
int check_view(const void* p, const inf_strides& s, inf_dtype dt) {
    if (!p) return INF_ERR_NULL_POINTER;
    if (s.d != 1 || s.b < 0 || s.h < 0 || s.t < 0 || s.t > kMaxRowStride) return INF_ERR_BAD_STRIDE;
    const uintptr_t a = reinterpret_cast<uintptr_t>(p);
    const uintptr_t need = (uintptr_t)(4 * elem_bytes(dt));
    if (a % need) return INF_ERR_ALIGNMENT;
    if ((s.b % 4) || (s.h % 4) || (s.t % 4)) return INF_ERR_ALIGNMENT;
    return INF_OK;
}

// An output [B,H,T,D] view must also give every element its own address:
// workgroups of different heads or rows would otherwise store to (and, for the
// fp32 dQ accumulation, add into) the same words.  Sufficient condition: with
// the dims of extent > 1 in increasing stride order, each stride is at least
// the span of the dims inside it (the head dim's span is D).
int check_out_view(const void* p, const inf_strides& s, inf_dtype dt, int B, int H, int T, int D) {
    const int st = check_view(p, s, dt);
    if (st != INF_OK) return st;
    struct Dim { int64_t n, stride; } d[3] = {{B, s.b}, {H, s.h}, {T, s.t}};
    for (int i = 1; i < 3; ++i)  // insertion sort by stride
        for (int j = i; j > 0 && d[j].stride < d[j - 1].stride; --j) std::swap(d[j], d[j - 1]);
    int64_t span = D;
    for (const Dim& x : d) {
        if (x.n <= 1) continue;
        if (x.stride < span) return INF_ERR_BAD_STRIDE;
        span = x.stride * (x.n - 1) + span;
    }
    return INF_OK;
}

inf::View4 view(const inf_strides& s) { return inf::View4{s.b, s.h, s.t}; }

int hip_status(int e) { return e == 0 ? INF_OK : INF_ERR_HIP; }

int common_shape(int B, int H, int Tq, int Tk, int D, float scale, int dt) {
    if (!dtype_ok(dt)) return INF_ERR_BAD_DTYPE;
    if (B < 1 || H < 1 || Tq < 1 || Tk < 1 || D < 1) return INF_ERR_BAD_SHAPE;
    if (!head_dim_ok(D)) return INF_ERR_UNSUPPORTED;
    if (!(scale > 0.f) || !std::isfinite(scale)) return INF_ERR_BAD_SCALE;
    // grid sizes are 32-bit; keep head counts and lengths well inside them
    if ((int64_t)B * H > (1LL << 24) || Tq > (1 << 24) || Tk > (1 << 24)) return INF_ERR_BAD_SHAPE;
    return INF_OK;
}


thread_local std::string t_detail;

}  // namespace

namespace inf {
void set_error_detail(const std::string& msg) { t_detail = msg; }

int report_pending_error(hipError_t e, const char* where) {
    set_error_detail(std::string(where) + ": HIP error pending from an earlier call: " + hipGetErrorName(e) + " (" +
                     hipGetErrorString(e) + "); nothing launched");
    return (int)e;
}
}  // namespace inf

extern "C" {

const char* inf_last_error_detail(void) { return t_detail.c_str(); }

const char* inf_status_string(int status) {
    switch (status) {
        case INF_OK: return "ok";
        case INF_ERR_NULL_POINTER: return "null pointer argument";
        case INF_ERR_BAD_SHAPE: return "invalid shape";
        case INF_ERR_BAD_STRIDE: return "invalid stride (head-dim stride must be 1, strides >= 0, row stride <= 2^22)";
        case INF_ERR_BAD_DTYPE: return "unsupported dtype";
        case INF_ERR_UNSUPPORTED: return "unsupported configuration (head dim must be 32, 64 or 128)";
        case INF_ERR_WORKSPACE: return "workspace missing or too small";
        case INF_ERR_ALIGNMENT: return "misaligned pointer or stride (rows must allow 4-element vector access)";
        case INF_ERR_BAD_SCALE: return "scale must be finite and > 0";
        case INF_ERR_HIP: return "HIP runtime error";
        default: return "unknown status";
    }
}

int inf_version(void) { return 200; }

int inf_set_deterministic(int enable) { return g_deterministic.exchange(enable ? 1 : 0); }
int inf_get_deterministic(void) { return g_deterministic.load(); }

namespace {

// INF_OK, or INF_ERR_HIP when an earlier call left a HIP error pending.
int bwd_workspace_bytes(int det, int B, int H, int Tq, int Tk, int D, inf_dtype dt, size_t* out) {
    const size_t bh = (size_t)B * H;
    size_t n = 2 * round_up(bh * Tq * sizeof(float));  // delta and its low part (short rows)
    if (dt == INF_BF16 && !dq_from_pass(det, B, H, Tq, Tk, D, dt))
        n += round_up(bh * Tq * (size_t)D * sizeof(float));  // dQ accumulator
    inf::BwdPlan plan;                                        // causal split plan
    if (inf::bwd_plan(B, H, Tq, Tk, D, 1, dt == INF_BF16, &plan)) return INF_ERR_HIP;
    *out = n + round_up(inf::bwd_split_workspace_bytes(plan, B, H, D));
    return INF_OK;
}

}  // namespace

int inf_attn_workspace_bytes(int op, int B, int H, int Tq, int Tk, int D, inf_dtype dt,
                             size_t* out_bytes) {
    if (!out_bytes) return INF_ERR_NULL_POINTER;
    *out_bytes = 0;
    if (op == INF_OP_ATTN_DECODE) Tq = 1;
    const int st = common_shape(B, H, Tq, Tk, D, 1.0f, dt);
    if (st != INF_OK) return st;
    const size_t bh = (size_t)B * H;
    switch (op) {
        case INF_OP_ATTN_FWD: {
            inf::FwdPlan plan;
            if (inf::fwd_plan(B, H, Tq, Tk, D, 1, dt == INF_BF16, &plan)) return INF_ERR_HIP;
            *out_bytes = round_up(inf::fwd_workspace_bytes(plan, B, H, D));
            return INF_OK;
        }
        case INF_OP_ATTN_BWD:
            return bwd_workspace_bytes(g_deterministic.load(), B, H, Tq, Tk, D, dt, out_bytes);
        case INF_OP_ATTN_DECODE: {
            int ns = 1, ch = 0;
            inf::decode_plan(B, H, Tk, D, &ns, &ch);
            *out_bytes = ns > 1 ? round_up(bh * (size_t)ns * (D + 2) * sizeof(float)) : 0;
            return INF_OK;
        }
        default: return INF_ERR_UNSUPPORTED;
    }
}

int inf_attn_fwd(const void* q, inf_strides sq, const void* k, inf_strides sk, const void* v,
                 inf_strides sv, void* o, inf_strides so, float* lse, void* workspace,
                 size_t ws_bytes, int B, int H, int Tq, int Tk, int D, float scale, int causal,
                 inf_dtype dt, void* stream) {
    int st = common_shape(B, H, Tq, Tk, D, scale, dt);
    if (st != INF_OK) return st;
    if (causal && Tq > Tk) return INF_ERR_BAD_SHAPE;
    if ((st = check_view(q, sq, dt)) || (st = check_view(k, sk, dt)) ||
        (st = check_view(v, sv, dt)) || (st = check_out_view(o, so, dt, B, H, Tq, D)))
        return st;
    inf::FwdParams p{};
    p.q = q; p.k = k; p.v = v; p.o = o; p.lse = lse;
    p.sq = view(sq); p.sk = view(sk); p.sv = view(sv); p.so = view(so);
    p.B = B; p.H = H; p.Tq = Tq; p.Tk = Tk; p.D = D;
    p.causal = causal ? 1 : 0;
    p.off = Tk - Tq;
    p.scale = scale;
    p.c = scale * 1.4426950408889634f;
    p.n_qtiles = (Tq + inf::kFwdBM - 1) / inf::kFwdBM;
    inf::FwdPlan plan;
    if (inf::fwd_plan(B, H, Tq, Tk, D, p.causal, dt == INF_BF16, &plan)) return INF_ERR_HIP;
    p.pv_prio = plan.pv_prio;
    const size_t need = inf::fwd_workspace_bytes(plan, B, H, D);
    if (need && (!workspace || ws_bytes < need)) return INF_ERR_WORKSPACE;
    if (need && reinterpret_cast<uintptr_t>(workspace) % kAlign) return INF_ERR_ALIGNMENT;
    if (plan.n_groups) {
        p.n_groups = plan.n_groups;
        p.n_slots = plan.n_slots;
        p.n_split = plan.n_split;
        p.part = static_cast<float*>(workspace);
        std::memcpy(p.groups, plan.groups, sizeof(p.groups));
        std::memcpy(p.split_qt, plan.split_qt, sizeof(p.split_qt));
        std::memcpy(p.split_slot0, plan.split_slot0, sizeof(p.split_slot0));
        std::memcpy(p.split_count, plan.split_count, sizeof(p.split_count));
    }
    return hip_status(inf::launch_attn_fwd(p, dt == INF_BF16, (hipStream_t)stream));
}

int inf_attn_bwd(const void* q, inf_strides sq, const void* k, inf_strides sk, const void* v,
                 inf_strides sv, const void* o, inf_strides so, const void* dout,
                 inf_strides sdo, const float* lse, void* dq, inf_strides sdq, void* dk,
                 inf_strides sdk, void* dv, inf_strides sdv, void* workspace, size_t ws_bytes,
                 int B, int H, int Tq, int Tk, int D, float scale, int causal, inf_dtype dt,
                 void* stream) {
    int st = common_shape(B, H, Tq, Tk, D, scale, dt);
    if (st != INF_OK) return st;
    if (causal && Tq > Tk) return INF_ERR_BAD_SHAPE;
    if (!lse) return INF_ERR_NULL_POINTER;
    if ((st = check_view(q, sq, dt)) || (st = check_view(k, sk, dt)) ||
        (st = check_view(v, sv, dt)) || (st = check_view(o, so, dt)) ||
        (st = check_view(dout, sdo, dt)) || (st = check_out_view(dq, sdq, dt, B, H, Tq, D)) ||
        (st = check_out_view(dk, sdk, dt, B, H, Tk, D)) || (st = check_out_view(dv, sdv, dt, B, H, Tk, D)))
        return st;
    const int det = g_deterministic.load();  // one reading for the whole call
    size_t need = 0;
    if ((st = bwd_workspace_bytes(det, B, H, Tq, Tk, D, dt, &need))) return st;
    if (!workspace || ws_bytes < need) return INF_ERR_WORKSPACE;
    if (reinterpret_cast<uintptr_t>(workspace) % kAlign) return INF_ERR_ALIGNMENT;

    inf::BwdParams p{};
    p.q = q; p.k = k; p.v = v; p.o = o; p.dout = dout; p.lse = lse;
    p.dq = dq; p.dk = dk; p.dv = dv;
    p.sq = view(sq); p.sk = view(sk); p.sv = view(sv); p.so = view(so);
    p.sdo = view(sdo); p.sdq = view(sdq); p.sdk = view(sdk); p.sdv = view(sdv);
    const size_t bh = (size_t)B * H;
    char* ws = static_cast<char*>(workspace);
    p.delta = reinterpret_cast<float*>(ws);
    p.delta_lo = reinterpret_cast<float*>(ws + round_up(bh * Tq * sizeof(float)));
    if (dt == INF_BF16) {
        p.dq_acc = reinterpret_cast<float*>(ws + 2 * round_up(bh * Tq * sizeof(float)));
        p.sacc = inf::View4{(int64_t)H * Tq * D, (int64_t)Tq * D, (int64_t)D};
    } else {
        p.dq_acc = static_cast<float*>(dq);
        p.sacc = view(sdq);
    }
    p.B = B; p.H = H; p.Tq = Tq; p.Tk = Tk; p.D = D;
    p.causal = causal ? 1 : 0;
    p.off = Tk - Tq;
    p.scale = scale;
    p.c = scale * 1.4426950408889634f;
    const int bk = inf::bwd_keys_per_wg(dt == INF_BF16, D);
    p.n_kblocks = (Tk + bk - 1) / bk;
    p.n_short = inf::bwd_short_rows(B, H, Tq, Tk, p.causal, bk);
    p.dq_direct = dq_from_pass(det, B, H, Tq, Tk, D, dt) ? 1 : 0;
    p.n_qtiles = (Tq + inf::kBwdDqBM - 1) / inf::kBwdDqBM;
    if (p.dq_direct) p.dq_acc = nullptr;  // dq is written by the dQ pass
    inf::BwdPlan plan;
    if (inf::bwd_plan(B, H, Tq, Tk, D, p.causal, dt == INF_BF16, &plan)) return INF_ERR_HIP;
    if (plan.n_groups) {
        size_t offset = 2 * round_up(bh * Tq * sizeof(float));
        if (dt == INF_BF16 && !p.dq_direct) offset += round_up(bh * Tq * (size_t)D * sizeof(float));
        const size_t part_bytes = (size_t)plan.n_slots * bh * 2 * (size_t)D * plan.bk * sizeof(float);
        p.part = reinterpret_cast<float*>(ws + offset);
        p.counters = reinterpret_cast<unsigned*>(ws + offset + part_bytes);
        p.n_groups = plan.n_groups;
        p.n_split = plan.n_split;
        std::memcpy(p.groups, plan.groups, sizeof(p.groups));
    }
    return hip_status(inf::launch_attn_bwd(p, dt == INF_BF16, (hipStream_t)stream));
}

// Element types of the softmax entry points: the attention dtypes, plus
// INF_F64 (both directions) and INF_I32 input (forward only, fp32 output).
static inf::SmType sm_type(inf_dtype dt) {
    switch (dt) {
        case INF_BF16: return inf::SmType::BF16;
        case INF_F64: return inf::SmType::F64;
        case INF_I32: return inf::SmType::I32;
        default: return inf::SmType::F32;
    }
}

static int softmax_common(const void* a, const void* b, void* c, int64_t rows, int64_t cols,
                          inf_dtype dt, int* vec_ok, int64_t s1, int64_t s2, int64_t s3) {
    if (!a || !b || !c) return INF_ERR_NULL_POINTER;
    if (rows < 1 || cols < 1 || rows > (1LL << 31)) return INF_ERR_BAD_SHAPE;
    if (s1 < cols || s2 < cols || s3 < cols) return INF_ERR_BAD_STRIDE;
    const uintptr_t need = (uintptr_t)(4 * elem_bytes(dt));
    *vec_ok = (cols % 4 == 0) && (s1 % 4 == 0) && (s2 % 4 == 0) && (s3 % 4 == 0) &&
              (reinterpret_cast<uintptr_t>(a) % need == 0) &&
              (reinterpret_cast<uintptr_t>(b) % need == 0) &&
              (reinterpret_cast<uintptr_t>(c) % need == 0);
    return INF_OK;
}

int inf_softmax_fwd(const void* x, void* y, int64_t rows, int64_t cols, int64_t x_row_stride,
                    int64_t y_row_stride, inf_dtype dt, void* stream) {
    if (!dtype_ok(dt) && dt != INF_F64 && dt != INF_I32) return INF_ERR_BAD_DTYPE;
    int vec_ok = 0;
    const int st = softmax_common(x, x, y, rows, cols, dt, &vec_ok, x_row_stride, y_row_stride,
                                  y_row_stride);
    if (st != INF_OK) return st;
    inf::SoftmaxParams p{x, nullptr, y, rows, cols, x_row_stride, 0, y_row_stride};
    return hip_status(inf::launch_softmax_fwd(p, sm_type(dt), vec_ok, (hipStream_t)stream));
}

int inf_softmax_bwd(const void* y, const void* dy, void* dx, int64_t rows, int64_t cols,
                    int64_t y_row_stride, int64_t dy_row_stride, int64_t dx_row_stride,
                    inf_dtype dt, void* stream) {
    if (!dtype_ok(dt) && dt != INF_F64) return INF_ERR_BAD_DTYPE;
    int vec_ok = 0;
    const int st = softmax_common(y, dy, dx, rows, cols, dt, &vec_ok, y_row_stride, dy_row_stride,
                                  dx_row_stride);
    if (st != INF_OK) return st;
    inf::SoftmaxParams p{y, dy, dx, rows, cols, y_row_stride, dy_row_stride, dx_row_stride};
    return hip_status(inf::launch_softmax_bwd(p, sm_type(dt), vec_ok, (hipStream_t)stream));
}

// Shape / stride checks of the axis entry points, and the launch parameters
// (strides of the operands x, g, y; g may be null for the forward).
static int softmax_axis_common(const void* x, const int64_t* sx, const void* g, const int64_t* sg, void* y,
                               const int64_t* sy, int ndim, const int64_t* shape, int axis, inf::SoftmaxAxis* p) {
    if (ndim < 1) return INF_ERR_BAD_SHAPE;
    if (ndim > inf::kMaxRank) return INF_ERR_UNSUPPORTED;
    if (!shape || !sx || !sy || (g && !sg)) return INF_ERR_NULL_POINTER;
    if (axis < 0) axis += ndim;
    if (axis < 0 || axis >= ndim) return INF_ERR_BAD_SHAPE;
    *p = inf::SoftmaxAxis{};
    p->x = x;
    p->g = g;
    p->y = y;
    p->ndim = ndim;
    p->axis = axis;
    p->groups = 1;
    for (int d = 0; d < ndim; ++d) {
        if (shape[d] < 0) return INF_ERR_BAD_SHAPE;
        if (sx[d] < 0 || sy[d] < 0 || (g && sg[d] < 0)) return INF_ERR_BAD_STRIDE;
        p->shape[d] = shape[d];
        p->sx[d] = sx[d];
        p->sy[d] = sy[d];
        p->sg[d] = g ? sg[d] : 0;
        if (d != axis) p->groups *= shape[d];
    }
    p->n = shape[axis];
    if (p->groups > (1LL << 31) * 256) return INF_ERR_BAD_SHAPE;
    // the output must not overlap itself: ordering its dims of extent > 1 by
    // stride, each stride must exceed the largest offset the dims inside reach
    int order[inf::kMaxRank], m = 0;
    for (int d = 0; d < ndim; ++d)
        if (shape[d] > 1) order[m++] = d;
    std::sort(order, order + m, [&](int a, int b) { return sy[a] < sy[b]; });
    int64_t reach = 0;
    for (int i = 0; i < m; ++i) {
        if (sy[order[i]] <= reach) return INF_ERR_BAD_STRIDE;
        reach += sy[order[i]] * (shape[order[i]] - 1);
    }
    return INF_OK;
}

int inf_softmax_fwd_axis(const void* x, const int64_t* x_strides, void* y, const int64_t* y_strides, int ndim,
                         const int64_t* shape, int axis, inf_dtype dt, void* stream) {
    if (!dtype_ok(dt) && dt != INF_F64 && dt != INF_I32) return INF_ERR_BAD_DTYPE;
    inf::SoftmaxAxis p;
    const int st = softmax_axis_common(x, x_strides, nullptr, nullptr, y, y_strides, ndim, shape, axis, &p);
    if (st != INF_OK) return st;
    if (p.groups == 0 || p.n == 0) return INF_OK;
    if (!x || !y) return INF_ERR_NULL_POINTER;
    return hip_status(inf::launch_softmax_axis_fwd(p, sm_type(dt), (hipStream_t)stream));
}

int inf_softmax_bwd_axis(const void* y, const int64_t* y_strides, const void* dy, const int64_t* dy_strides,
                         void* dx, const int64_t* dx_strides, int ndim, const int64_t* shape, int axis,
                         inf_dtype dt, void* stream) {
    if (!dtype_ok(dt) && dt != INF_F64) return INF_ERR_BAD_DTYPE;
    if (!dy_strides) return INF_ERR_NULL_POINTER;
    inf::SoftmaxAxis p;
    const int st = softmax_axis_common(y, y_strides, dy ? dy : y, dy_strides, dx, dx_strides, ndim, shape, axis, &p);
    if (st != INF_OK) return st;
    if (p.groups == 0 || p.n == 0) return INF_OK;
    if (!y || !dy || !dx) return INF_ERR_NULL_POINTER;
    return hip_status(inf::launch_softmax_axis_bwd(p, sm_type(dt), (hipStream_t)stream));
}

int inf_attn_decode(const void* q, inf_strides sq, const void* kcache, inf_strides sk,
                    const void* vcache, inf_strides sv, void* o, inf_strides so, int B, int H,
                    int Tk, int D, float scale, inf_dtype dt, void* workspace, size_t ws_bytes,
                    void* stream) {
    int st = common_shape(B, H, 1, Tk, D, scale, dt);
    if (st != INF_OK) return st;
    if ((st = check_view(q, sq, dt)) || (st = check_view(kcache, sk, dt)) ||
        (st = check_view(vcache, sv, dt)) || (st = check_out_view(o, so, dt, B, H, 1, D)))
        return st;
    size_t need = 0;
    inf_attn_workspace_bytes(INF_OP_ATTN_DECODE, B, H, 1, Tk, D, dt, &need);
    if (need && (!workspace || ws_bytes < need)) return INF_ERR_WORKSPACE;
    if (need && reinterpret_cast<uintptr_t>(workspace) % kAlign) return INF_ERR_ALIGNMENT;
    inf::DecodeParams p{};
    p.q = q; p.k = kcache; p.v = vcache; p.o = o;
    p.part = static_cast<float*>(workspace);
    inf::decode_plan(B, H, Tk, D, &p.nsplit, &p.chunk);
    p.sq = view(sq); p.sk = view(sk); p.sv = view(sv); p.so = view(so);
    p.B = B; p.H = H; p.Tk = Tk; p.D = D;
    p.c = scale * 1.4426950408889634f;
    return hip_status(inf::launch_attn_decode(p, dt == INF_BF16, (hipStream_t)stream));
}

int inf_attn_decode_static(const void* q, inf_strides sq, const void* kcache, inf_strides sk,
                           const void* vcache, inf_strides sv, void* o, inf_strides so, int B, int H,
                           int Tk, int D, float scale, inf_dtype dt, void* stream) {
    int st = common_shape(B, H, 1, Tk, D, scale, dt);
    if (st != INF_OK) return st;
    if ((st = check_view(q, sq, dt)) || (st = check_view(kcache, sk, dt)) ||
        (st = check_view(vcache, sv, dt)) || (st = check_out_view(o, so, dt, B, H, 1, D)))
        return st;
    size_t need = 0;
    inf_attn_workspace_bytes(INF_OP_ATTN_DECODE, B, H, 1, Tk, D, dt, &need);
    if (need > inf::kDecodeScratchBytes) {
        inf::set_error_detail("inf_attn_decode_static: this shape's split partials need " + std::to_string(need) +
                              " bytes; the static scratch holds " + std::to_string(inf::kDecodeScratchBytes) +
                              " (use inf_attn_decode with a workspace)");
        return INF_ERR_WORKSPACE;
    }
    float* scratch = nullptr;
    const int e = inf::decode_scratch(&scratch);
    if (e != 0) {
        inf::set_error_detail(std::string("inf_attn_decode_static: hipGetSymbolAddress of the scratch failed: ") +
                              hipGetErrorString((hipError_t)e));
        return INF_ERR_HIP;
    }
    inf::DecodeParams p{};
    p.q = q; p.k = kcache; p.v = vcache; p.o = o;
    p.part = scratch;
    inf::decode_plan(B, H, Tk, D, &p.nsplit, &p.chunk);
    p.sq = view(sq); p.sk = view(sk); p.sv = view(sv); p.so = view(so);
    p.B = B; p.H = H; p.Tk = Tk; p.D = D;
    p.c = scale * 1.4426950408889634f;
    return hip_status(inf::launch_attn_decode(p, dt == INF_BF16, (hipStream_t)stream));
}

int inf_fill(void* dst, int64_t n, int elem_bytes, uint32_t bits, void* stream) {
    if (n < 0) return INF_ERR_BAD_SHAPE;
    if (elem_bytes != 1 && elem_bytes != 2 && elem_bytes != 4) return INF_ERR_BAD_DTYPE;
    if (n == 0) return INF_OK;
    if (!dst) return INF_ERR_NULL_POINTER;
    return hip_status(inf::launch_fill(dst, n, elem_bytes, bits, (hipStream_t)stream));
}

int inf_binary(int op, const void* a, const void* b, void* out, int64_t n, int a_scalar, int b_scalar,
               inf_dtype dt, void* stream) {
    if (op != INF_BIN_ADD && op != INF_BIN_MUL) return INF_ERR_UNSUPPORTED;
    if (!dtype_ok(dt)) return INF_ERR_BAD_DTYPE;
    if (n < 0) return INF_ERR_BAD_SHAPE;
    if (n == 0) return INF_OK;
    if (!a || !b || !out) return INF_ERR_NULL_POINTER;
    return hip_status(inf::launch_binary(op, a, b, out, n, a_scalar ? 1 : 0, b_scalar ? 1 : 0,
                                         dt == INF_BF16, (hipStream_t)stream));
}

int inf_triu(const void* a, const int64_t* a_strides, void* out, int rank, const int64_t* shape, int diagonal,
             int elem_bytes, void* stream) {
    if (rank < 2) return INF_ERR_BAD_SHAPE;
    if (rank > inf::kMaxRank) return INF_ERR_UNSUPPORTED;
    if (elem_bytes != 1 && elem_bytes != 2 && elem_bytes != 4 && elem_bytes != 8) return INF_ERR_BAD_DTYPE;
    if (!shape || !a_strides) return INF_ERR_NULL_POINTER;
    inf::StridedCopy c{};
    c.ndim = rank;
    c.n = 1;
    for (int d = 0; d < rank; ++d) {
        if (shape[d] < 0) return INF_ERR_BAD_SHAPE;
        if (a_strides[d] < 0) return INF_ERR_BAD_STRIDE;
        c.shape[d] = shape[d];
        c.sstride[d] = a_strides[d];
        c.n *= shape[d];
    }
    if (c.n == 0) return INF_OK;
    if (!a || !out) return INF_ERR_NULL_POINTER;
    return hip_status(inf::launch_triu(a, out, c, diagonal, elem_bytes, (hipStream_t)stream));
}

int inf_masked_fill(const void* in, const int64_t* in_strides, const void* mask, const int64_t* mask_shape,
                    const int64_t* mask_strides, int mask_rank, int mask_bytes, void* out, int rank,
                    const int64_t* shape, uint64_t fill_bits, int elem_bytes, void* stream) {
    if (rank < 0 || mask_rank < 0 || mask_rank > rank) return INF_ERR_BAD_SHAPE;
    if (rank > inf::kMaxRank) return INF_ERR_UNSUPPORTED;
    if (elem_bytes != 1 && elem_bytes != 2 && elem_bytes != 4 && elem_bytes != 8) return INF_ERR_BAD_DTYPE;
    if (mask_bytes != 1 && mask_bytes != 4 && mask_bytes != 8) return INF_ERR_BAD_DTYPE;
    if ((rank > 0 && (!shape || !in_strides)) || (mask_rank > 0 && (!mask_shape || !mask_strides)))
        return INF_ERR_NULL_POINTER;
    inf::MaskedFill m{};
    m.ndim = rank;
    m.n = 1;
    const int lead = rank - mask_rank;
    for (int d = 0; d < rank; ++d) {
        if (shape[d] < 0) return INF_ERR_BAD_SHAPE;
        if (in_strides[d] < 0) return INF_ERR_BAD_STRIDE;
        m.shape[d] = shape[d];
        m.istride[d] = in_strides[d];
        m.n *= shape[d];
        if (d >= lead) {
            const int64_t md = mask_shape[d - lead];
            if (md != 1 && md != shape[d]) return INF_ERR_BAD_SHAPE;  // not broadcastable
            if (mask_strides[d - lead] < 0) return INF_ERR_BAD_STRIDE;
            m.mstride[d] = md == 1 ? 0 : mask_strides[d - lead];
        }
    }
    if (m.n == 0) return INF_OK;
    if (!in || !mask || !out) return INF_ERR_NULL_POINTER;
    return hip_status(inf::launch_masked_fill(in, mask, out, m, elem_bytes, mask_bytes, fill_bits,
                                              (hipStream_t)stream));
}

int inf_copy_strided(const void* src, const int64_t* src_strides, void* dst,
                     const int64_t* dst_strides, int ndim, const int64_t* shape, int elem_bytes,
                     void* stream) {
    if (ndim < 0 || ndim > inf::kMaxRank) return INF_ERR_UNSUPPORTED;
    if (elem_bytes != 1 && elem_bytes != 2 && elem_bytes != 4 && elem_bytes != 8) return INF_ERR_BAD_DTYPE;
    if (ndim > 0 && (!shape || !src_strides || !dst_strides)) return INF_ERR_NULL_POINTER;
    inf::StridedCopy c{};
    c.ndim = ndim;
    c.n = 1;
    for (int d = 0; d < ndim; ++d) {
        if (shape[d] < 0 || src_strides[d] < 0 || dst_strides[d] < 0) return INF_ERR_BAD_STRIDE;
        c.shape[d] = shape[d];
        c.sstride[d] = src_strides[d];
        c.dstride[d] = dst_strides[d];
        c.n *= shape[d];
    }
    if (c.n == 0) return INF_OK;
    if (!src || !dst) return INF_ERR_NULL_POINTER;
    return hip_status(inf::launch_copy_strided(src, dst, c, elem_bytes, (hipStream_t)stream));
}

}  // extern "C"
