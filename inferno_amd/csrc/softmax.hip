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
