// softmax.hip -- standalone row softmax forward / backward (memory-bound).
//
// Forward follows the reference's three steps per row (softmax_kernels.h:77-102):
// m = max_k x_k; e_k = exp(x_k - m); y_k = e_k / sum_k e_k, with exp evaluated
// as exp2((x - m) * log2(e)) in fp32.  Backward is
// dx_k = y_k * (g_k - sum_j g_j y_j) (softmaxbackward.h:111-128).
//
// Rows of up to 4096 elements (contiguous, 4-element aligned) take one wave
// per row with the row held in VGPRs: one HBM read and one write per
// element, and the reductions are wave-level exchanges.  Other rows take one
// workgroup per row and stream it (max / sum pass, then the write pass).
//
// Element types follow the reference's dispatch (softmax.cpp:25 dispatchAny,
// RT = promote_t<AT, float>, dtype_dispatch.h:8-52): fp32 and bf16 storage
// with fp32 arithmetic; Int32 input with fp32 output (every int enters the
// reference's arithmetic converted to float, so the fp32 kernels run on the
// converted values); Float64 in and out with double arithmetic, exp included
// (softmax_{fwd,bwd}_f64, one workgroup per row).
#include <type_traits>

#include "common.h"
#include "kernels.h"

namespace inf {

// int32 elements, converted to fp32 as they are loaded
__device__ __forceinline__ f32x4 ld4(const int32_t* p) {
    typedef int32_t i32x4 __attribute__((ext_vector_type(4)));
    const i32x4 v = *reinterpret_cast<const i32x4*>(p);
    return f32x4{(float)v[0], (float)v[1], (float)v[2], (float)v[3]};
}
struct I32 {
    static __device__ __forceinline__ float ld(const int32_t* p) { return (float)*p; }
};
template <typename E>
using ElemOf = typename std::conditional<std::is_same<E, float>::value, F32,
                                         typename std::conditional<std::is_same<E, int32_t>::value, I32, BF16>::type>::type;

// EI: input element type; EO: output element type (EI except int32 -> fp32)
template <typename EI, typename EO, int VPT>
__global__ __launch_bounds__(256) void softmax_fwd_wave(SoftmaxParams p) {
    const int lane = threadIdx.x & 63;
    const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (row >= p.rows) return;  // whole wave leaves together; no block barrier below
    const EI* x = (const EI*)p.x + row * p.sx;
    EO* y = (EO*)p.y + row * p.sy;
    const int cols = (int)p.cols;
    f32x4 v[VPT];
    float m = -INFINITY;
#pragma unroll
    for (int i = 0; i < VPT; ++i) {
        const int c = (i * 64 + lane) * 4;
        v[i] = (c < cols) ? ld4(x + c) : f32x4{-INFINITY, -INFINITY, -INFINITY, -INFINITY};
        m = fmaxf(m, fmaxf(fmaxf(v[i][0], v[i][1]), fmaxf(v[i][2], v[i][3])));
    }
    m = wave_max(m);
    const float mc = m * kLog2e;
    float s = 0.f;
#pragma unroll
    for (int i = 0; i < VPT; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            v[i][j] = fast_exp2(fmaf(v[i][j], kLog2e, -mc));
            s += v[i][j];
        }
    s = wave_sum(s);
#pragma unroll
    for (int i = 0; i < VPT; ++i) {
        const int c = (i * 64 + lane) * 4;
        if (c < cols) st4(y + c, v[i] / s);
    }
}

template <typename E>
__device__ __forceinline__ float block_reduce(float v, bool is_max, float* red) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    v = is_max ? wave_max(v) : wave_sum(v);
    __syncthreads();
    if (lane == 0) red[wave] = v;
    __syncthreads();
    return is_max ? fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]))
                  : (red[0] + red[1]) + (red[2] + red[3]);
}

template <typename EI, typename EO>
__global__ __launch_bounds__(256) void softmax_fwd_block(SoftmaxParams p) {
    using Ti = ElemOf<EI>;
    using To = ElemOf<EO>;
    __shared__ float red[4];
    const int64_t row = blockIdx.x;
    const EI* x = (const EI*)p.x + row * p.sx;
    EO* y = (EO*)p.y + row * p.sy;
    float m = -INFINITY;
    for (int64_t c = threadIdx.x; c < p.cols; c += 256) m = fmaxf(m, Ti::ld(x + c));
    m = block_reduce<EI>(m, true, red);
    const float mc = m * kLog2e;
    float s = 0.f;
    for (int64_t c = threadIdx.x; c < p.cols; c += 256) s += fast_exp2(fmaf(Ti::ld(x + c), kLog2e, -mc));
    s = block_reduce<EI>(s, false, red);
    for (int64_t c = threadIdx.x; c < p.cols; c += 256)
        To::st(y + c, fast_exp2(fmaf(Ti::ld(x + c), kLog2e, -mc)) / s);
}

// Float64: the reference's cpu_softmax<double, double> steps in double
// (max, exp(x - max), sum, divide), one workgroup per row.
__device__ __forceinline__ double block_reduce_f64(double v, bool is_max, double* red) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) {
        const double o = __shfl_xor(v, m);
        v = is_max ? fmax(v, o) : v + o;
    }
    __syncthreads();
    if (lane == 0) red[wave] = v;
    __syncthreads();
    return is_max ? fmax(fmax(red[0], red[1]), fmax(red[2], red[3])) : (red[0] + red[1]) + (red[2] + red[3]);
}

__global__ __launch_bounds__(256) void softmax_fwd_f64(SoftmaxParams p) {
    __shared__ double red[4];
    const int64_t row = blockIdx.x;
    const double* x = (const double*)p.x + row * p.sx;
    double* y = (double*)p.y + row * p.sy;
    double m = -INFINITY;
    for (int64_t c = threadIdx.x; c < p.cols; c += 256) m = fmax(m, x[c]);
    m = block_reduce_f64(m, true, red);
    double s = 0.0;
    for (int64_t c = threadIdx.x; c < p.cols; c += 256) s += exp(x[c] - m);
    s = block_reduce_f64(s, false, red);
    for (int64_t c = threadIdx.x; c < p.cols; c += 256) y[c] = exp(x[c] - m) / s;
}

__global__ __launch_bounds__(256) void softmax_bwd_f64(SoftmaxParams p) {
    __shared__ double red[4];
    const int64_t row = blockIdx.x;
    const double* yy = (const double*)p.x + row * p.sx;
    const double* gg = (const double*)p.g + row * p.sg;
    double* dx = (double*)p.y + row * p.sy;
    double dot = 0.0;
    for (int64_t c = threadIdx.x; c < p.cols; c += 256) dot += gg[c] * yy[c];
    dot = block_reduce_f64(dot, false, red);
    for (int64_t c = threadIdx.x; c < p.cols; c += 256) dx[c] = yy[c] * (gg[c] - dot);
}

template <typename E, int VPT>
__global__ __launch_bounds__(256) void softmax_bwd_wave(SoftmaxParams p) {
    const int lane = threadIdx.x & 63;
    const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (row >= p.rows) return;
    const E* yy = (const E*)p.x + row * p.sx;
    const E* gg = (const E*)p.g + row * p.sg;
    E* dx = (E*)p.y + row * p.sy;
    const int cols = (int)p.cols;
    f32x4 yv[VPT], gv[VPT];
    float dot = 0.f;
#pragma unroll
    for (int i = 0; i < VPT; ++i) {
        const int c = (i * 64 + lane) * 4;
        if (c < cols) {
            yv[i] = ld4(yy + c);
            gv[i] = ld4(gg + c);
        } else {
            yv[i] = gv[i] = f32x4{0.f, 0.f, 0.f, 0.f};
        }
        dot += gv[i][0] * yv[i][0] + gv[i][1] * yv[i][1] + gv[i][2] * yv[i][2] + gv[i][3] * yv[i][3];
    }
    dot = wave_sum(dot);
#pragma unroll
    for (int i = 0; i < VPT; ++i) {
        const int c = (i * 64 + lane) * 4;
        if (c < cols) st4(dx + c, yv[i] * (gv[i] - dot));
    }
}

template <typename E>
__global__ __launch_bounds__(256) void softmax_bwd_block(SoftmaxParams p) {
    using Tg = ElemOf<E>;
    __shared__ float red[4];
    const int64_t row = blockIdx.x;
    const E* yy = (const E*)p.x + row * p.sx;
    const E* gg = (const E*)p.g + row * p.sg;
    E* dx = (E*)p.y + row * p.sy;
    float dot = 0.f;
    for (int64_t c = threadIdx.x; c < p.cols; c += 256) dot += Tg::ld(gg + c) * Tg::ld(yy + c);
    dot = block_reduce<E>(dot, false, red);
    for (int64_t c = threadIdx.x; c < p.cols; c += 256) {
        const float yv = Tg::ld(yy + c);
        Tg::st(dx + c, yv * (Tg::ld(gg + c) - dot));
    }
}

// ---- softmax along a strided axis -------------------------------------------
// Each group (an index of the dims other than the axis) is one line of n
// elements.  Many groups: one thread per line, consecutive threads on
// consecutive groups (so the loads coalesce when the last non-axis dim is
// dense), an online max / sum pass and a write pass.  Few groups: one
// workgroup per line, its threads striding the line (max, sum, write passes
// as the row kernels).

// Element offsets of group `grp` in x, g and y.
__device__ __forceinline__ void axis_bases(const SoftmaxAxis& p, int64_t grp, int64_t& bx, int64_t& bg,
                                           int64_t& by) {
    bx = bg = by = 0;
    for (int d = p.ndim - 1; d >= 0; --d) {
        if (d == p.axis) continue;
        const int64_t c = grp % p.shape[d];
        grp /= p.shape[d];
        bx += c * p.sx[d];
        bg += c * p.sg[d];
        by += c * p.sy[d];
    }
}

// Online (max, sum of exp) update with one element; a -inf element against a
// -inf maximum adds nothing, NaN propagates into the sum.
template <typename T>
__device__ __forceinline__ void online_add(T v, T& m, T& s) {
    if (v > m) {
        if constexpr (std::is_same<T, double>::value)
            s = (m == -INFINITY ? 0.0 : s * exp(m - v)) + 1.0;
        else
            s = (m == -INFINITY ? 0.f : s * fast_exp2((m - v) * kLog2e)) + 1.f;
        m = v;
    } else if (!(v == -INFINITY && m == -INFINITY)) {
        if constexpr (std::is_same<T, double>::value)
            s += exp(v - m);
        else
            s += fast_exp2((v - m) * kLog2e);
    }
}

template <typename EI, typename EO>
__global__ __launch_bounds__(256) void softmax_axis_fwd_lines(SoftmaxAxis p) {
    const int64_t grp = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (grp >= p.groups) return;
    int64_t bx, bg, by;
    axis_bases(p, grp, bx, bg, by);
    const EI* x = (const EI*)p.x + bx;
    EO* y = (EO*)p.y + by;
    const int64_t ax = p.sx[p.axis], ay = p.sy[p.axis];
    if constexpr (std::is_same<EI, double>::value) {
        double m = -INFINITY, s = 0.0;
        for (int64_t k = 0; k < p.n; ++k) online_add(x[k * ax], m, s);
        for (int64_t k = 0; k < p.n; ++k) y[k * ay] = exp(x[k * ax] - m) / s;
    } else {
        using Ti = ElemOf<EI>;
        using To = ElemOf<EO>;
        float m = -INFINITY, s = 0.f;
        for (int64_t k = 0; k < p.n; ++k) online_add(Ti::ld(x + k * ax), m, s);
        const float mc = m * kLog2e;
        for (int64_t k = 0; k < p.n; ++k) To::st(y + k * ay, fast_exp2(fmaf(Ti::ld(x + k * ax), kLog2e, -mc)) / s);
    }
}

template <typename E>
__global__ __launch_bounds__(256) void softmax_axis_bwd_lines(SoftmaxAxis p) {
    const int64_t grp = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (grp >= p.groups) return;
    int64_t by, bg, bd;
    axis_bases(p, grp, by, bg, bd);
    const E* yy = (const E*)p.x + by;
    const E* gg = (const E*)p.g + bg;
    E* dx = (E*)p.y + bd;
    const int64_t ay = p.sx[p.axis], ag = p.sg[p.axis], ad = p.sy[p.axis];
    if constexpr (std::is_same<E, double>::value) {
        double dot = 0.0;
        for (int64_t k = 0; k < p.n; ++k) dot += gg[k * ag] * yy[k * ay];
        for (int64_t k = 0; k < p.n; ++k) dx[k * ad] = yy[k * ay] * (gg[k * ag] - dot);
    } else {
        using Te = ElemOf<E>;
        float dot = 0.f;
        for (int64_t k = 0; k < p.n; ++k) dot += Te::ld(gg + k * ag) * Te::ld(yy + k * ay);
        for (int64_t k = 0; k < p.n; ++k) Te::st(dx + k * ad, Te::ld(yy + k * ay) * (Te::ld(gg + k * ag) - dot));
    }
}

template <typename EI, typename EO>
__global__ __launch_bounds__(256) void softmax_axis_fwd_block(SoftmaxAxis p) {
    __shared__ float red[4];
    int64_t bx, bg, by;
    axis_bases(p, blockIdx.x, bx, bg, by);
    using Ti = ElemOf<EI>;
    using To = ElemOf<EO>;
    const EI* x = (const EI*)p.x + bx;
    EO* y = (EO*)p.y + by;
    const int64_t ax = p.sx[p.axis], ay = p.sy[p.axis];
    float m = -INFINITY;
    for (int64_t k = threadIdx.x; k < p.n; k += 256) m = fmaxf(m, Ti::ld(x + k * ax));
    m = block_reduce<EI>(m, true, red);
    const float mc = m * kLog2e;
    float s = 0.f;
    for (int64_t k = threadIdx.x; k < p.n; k += 256) s += fast_exp2(fmaf(Ti::ld(x + k * ax), kLog2e, -mc));
    s = block_reduce<EI>(s, false, red);
    for (int64_t k = threadIdx.x; k < p.n; k += 256) To::st(y + k * ay, fast_exp2(fmaf(Ti::ld(x + k * ax), kLog2e, -mc)) / s);
}

__global__ __launch_bounds__(256) void softmax_axis_fwd_block_f64(SoftmaxAxis p) {
    __shared__ double red[4];
    int64_t bx, bg, by;
    axis_bases(p, blockIdx.x, bx, bg, by);
    const double* x = (const double*)p.x + bx;
    double* y = (double*)p.y + by;
    const int64_t ax = p.sx[p.axis], ay = p.sy[p.axis];
    double m = -INFINITY;
    for (int64_t k = threadIdx.x; k < p.n; k += 256) m = fmax(m, x[k * ax]);
    m = block_reduce_f64(m, true, red);
    double s = 0.0;
    for (int64_t k = threadIdx.x; k < p.n; k += 256) s += exp(x[k * ax] - m);
    s = block_reduce_f64(s, false, red);
    for (int64_t k = threadIdx.x; k < p.n; k += 256) y[k * ay] = exp(x[k * ax] - m) / s;
}

template <typename E>
__global__ __launch_bounds__(256) void softmax_axis_bwd_block(SoftmaxAxis p) {
    using R = typename std::conditional<std::is_same<E, double>::value, double, float>::type;
    __shared__ R red[4];
    int64_t by, bg, bd;
    axis_bases(p, blockIdx.x, by, bg, bd);
    const E* yy = (const E*)p.x + by;
    const E* gg = (const E*)p.g + bg;
    E* dx = (E*)p.y + bd;
    const int64_t ay = p.sx[p.axis], ag = p.sg[p.axis], ad = p.sy[p.axis];
    R dot = 0;
    if constexpr (std::is_same<E, double>::value) {
        for (int64_t k = threadIdx.x; k < p.n; k += 256) dot += gg[k * ag] * yy[k * ay];
        dot = block_reduce_f64(dot, false, red);
        for (int64_t k = threadIdx.x; k < p.n; k += 256) dx[k * ad] = yy[k * ay] * (gg[k * ag] - dot);
    } else {
        using Te = ElemOf<E>;
        for (int64_t k = threadIdx.x; k < p.n; k += 256) dot += Te::ld(gg + k * ag) * Te::ld(yy + k * ay);
        dot = block_reduce<E>(dot, false, red);
        for (int64_t k = threadIdx.x; k < p.n; k += 256)
            Te::st(dx + k * ad, Te::ld(yy + k * ay) * (Te::ld(gg + k * ag) - dot));
    }
}

// Lines per thread when there are enough of them to give every CU a few
// workgroups; a workgroup per line otherwise.
constexpr int64_t kAxisLinesMin = 256 * 256;

template <typename EI, typename EO>
static int launch_axis_fwd(const SoftmaxAxis& p, hipStream_t s) {
    if (p.groups >= kAxisLinesMin)
        hipLaunchKernelGGL((softmax_axis_fwd_lines<EI, EO>), dim3((unsigned)((p.groups + 255) / 256)), dim3(256), 0, s, p);
    else if constexpr (std::is_same<EI, double>::value)
        hipLaunchKernelGGL(softmax_axis_fwd_block_f64, dim3((unsigned)p.groups), dim3(256), 0, s, p);
    else
        hipLaunchKernelGGL((softmax_axis_fwd_block<EI, EO>), dim3((unsigned)p.groups), dim3(256), 0, s, p);
    return (int)hipGetLastError();
}
template <typename E>
static int launch_axis_bwd(const SoftmaxAxis& p, hipStream_t s) {
    if (p.groups >= kAxisLinesMin)
        hipLaunchKernelGGL((softmax_axis_bwd_lines<E>), dim3((unsigned)((p.groups + 255) / 256)), dim3(256), 0, s, p);
    else
        hipLaunchKernelGGL((softmax_axis_bwd_block<E>), dim3((unsigned)p.groups), dim3(256), 0, s, p);
    return (int)hipGetLastError();
}

int launch_softmax_axis_fwd(const SoftmaxAxis& p, SmType t, hipStream_t s) {
    switch (t) {
        case SmType::F32: return launch_axis_fwd<float, float>(p, s);
        case SmType::BF16: return launch_axis_fwd<uint16_t, uint16_t>(p, s);
        case SmType::I32: return launch_axis_fwd<int32_t, float>(p, s);
        case SmType::F64: return launch_axis_fwd<double, double>(p, s);
    }
    return (int)hipErrorInvalidValue;
}
int launch_softmax_axis_bwd(const SoftmaxAxis& p, SmType t, hipStream_t s) {
    switch (t) {
        case SmType::F32: return launch_axis_bwd<float>(p, s);
        case SmType::BF16: return launch_axis_bwd<uint16_t>(p, s);
        case SmType::F64: return launch_axis_bwd<double>(p, s);
        default: return (int)hipErrorInvalidValue;
    }
}

// E: element type of every operand (backward) or of the input (forward; the
// output is EO).
template <typename E, typename EO, bool BWD>
static int launch_sm(const SoftmaxParams& p, int vec_ok, hipStream_t s) {
    const dim3 wgrid((unsigned)((p.rows + 3) / 4));
    if (vec_ok && p.cols <= 4096) {
        const int64_t n4 = (p.cols + 3) / 4;  // 4-element chunks per row
#define INF_SM_CASE(V)                                                                     \
    if (n4 <= 64 * (V)) {                                                                  \
        if constexpr (BWD)                                                                 \
            hipLaunchKernelGGL((softmax_bwd_wave<E, V>), wgrid, dim3(256), 0, s, p);       \
        else                                                                               \
            hipLaunchKernelGGL((softmax_fwd_wave<E, EO, V>), wgrid, dim3(256), 0, s, p);   \
        return (int)hipGetLastError();                                                     \
    }
        INF_SM_CASE(1)
        INF_SM_CASE(2)
        INF_SM_CASE(4)
        INF_SM_CASE(8)
        INF_SM_CASE(16)
#undef INF_SM_CASE
    }
    if constexpr (BWD)
        hipLaunchKernelGGL((softmax_bwd_block<E>), dim3((unsigned)p.rows), dim3(256), 0, s, p);
    else
        hipLaunchKernelGGL((softmax_fwd_block<E, EO>), dim3((unsigned)p.rows), dim3(256), 0, s, p);
    return (int)hipGetLastError();
}

int launch_softmax_fwd(const SoftmaxParams& p, SmType t, int vec_ok, hipStream_t s) {
    switch (t) {
        case SmType::F32: return launch_sm<float, float, false>(p, vec_ok, s);
        case SmType::BF16: return launch_sm<uint16_t, uint16_t, false>(p, vec_ok, s);
        case SmType::I32: return launch_sm<int32_t, float, false>(p, vec_ok, s);
        case SmType::F64:
            hipLaunchKernelGGL(softmax_fwd_f64, dim3((unsigned)p.rows), dim3(256), 0, s, p);
            return (int)hipGetLastError();
    }
    return (int)hipErrorInvalidValue;
}
int launch_softmax_bwd(const SoftmaxParams& p, SmType t, int vec_ok, hipStream_t s) {
    switch (t) {
        case SmType::F32: return launch_sm<float, float, true>(p, vec_ok, s);
        case SmType::BF16: return launch_sm<uint16_t, uint16_t, true>(p, vec_ok, s);
        case SmType::F64:
            hipLaunchKernelGGL(softmax_bwd_f64, dim3((unsigned)p.rows), dim3(256), 0, s, p);
            return (int)hipGetLastError();
        default: return (int)hipErrorInvalidValue;
    }
}

}  // namespace inf
