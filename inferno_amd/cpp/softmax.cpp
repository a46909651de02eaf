// softmax.cpp -- Softmax / SoftmaxBackward (include/inferno/functional/softmax.h).
//
// CPU: the softmax axis is moved last and made dense (a no-op for the usual
//      last-axis case), and the reference's three passes run per row
//      (softmax_kernels.h:77-102): max with a lowest() start,
//      e = (float)exp((double)(x - max)), fp32 running sum, divide; backward
//      dot = sum g*y in axis order, dx = y*(g - dot) (softmaxbackward.h:111-128).
// HIP: a dense last axis runs inf_softmax_fwd / inf_softmax_bwd over rows; any
//      other axis (or layout) runs inf_softmax_fwd_axis / inf_softmax_bwd_axis
//      on the operands' own strides, as the reference's device path walks them
//      (cudasoftmax.cu:16-97): no transposed copies.
// Dtypes follow the reference's dispatch (softmax.cpp:25, dtype_dispatch.h:8-52):
// Float32 -> Float32, Int32 -> Float32, Float64 -> Float64 (double
// arithmetic), plus BFloat16 (fp32 arithmetic); the backward works in
// promote_t of its operands (Float64 if either is).
#include <cfloat>
#include <cmath>
#include <limits>

#include "detail.h"
#include "inferno/functional/softmax.h"
#include "inferno/gradengine/engine.h"

namespace Inferno {

namespace {

constexpr int kMaxSoftmaxRank = 8;  // the axis entry points' rank limit

int norm_axis(int axis, size_t nd) {
    int a = axis < 0 ? axis + (int)nd : axis;
    if (a < 0 || a >= (int)nd) throw Error("Softmax: invalid axis");
    return a;
}

// Dense rows with `axis` last (no grad link).
Tensor rows_of(const Tensor& t, int axis) {
    NoGradGuard ng;
    Tensor x = axis == (int)t.ndim() - 1 ? t : t.transpose(axis, (int)t.ndim() - 1);
    return x.is_contiguous() ? x : x.contiguous();
}

// Whether t's `axis` is its last dim with unit stride and its rows dense
// (the row kernels' layout).
bool dense_rows(const Tensor& t, int axis) { return axis == (int)t.ndim() - 1 && t.is_contiguous(); }

std::vector<int64_t> i64(const std::vector<size_t>& v) { return std::vector<int64_t>(v.begin(), v.end()); }

Tensor restore_axis(const Tensor& rows, int axis, size_t nd) {
    NoGradGuard ng;
    if (axis == (int)nd - 1) return rows;
    return rows.transpose(axis, (int)nd - 1).contiguous();
}

// The reference's three passes in RT arithmetic (softmax_kernels.h:77-102):
// max from lowest() with a strict >, e = (RT)exp((double)(x - max)), RT running
// sum, divide.  Loads return the element converted to RT (an Int32 converts to
// float, as cpu_softmax<int, float> does in every use).
template <typename RT, typename Load, typename Store>
void cpu_softmax_rows(size_t rows, size_t cols, Load ld, Store st) {
    std::vector<RT> e(cols);
    for (size_t r = 0; r < rows; ++r) {
        RT mx = std::numeric_limits<RT>::lowest();
        for (size_t k = 0; k < cols; ++k) {
            const RT x = ld(r * cols + k);
            if (x > mx) mx = x;
        }
        RT sum = RT(0);
        for (size_t k = 0; k < cols; ++k) {
            e[k] = (RT)std::exp((double)(ld(r * cols + k) - mx));
            sum += e[k];
        }
        for (size_t k = 0; k < cols; ++k) st(r * cols + k, e[k] / sum);
    }
}

// dot = sum g*y in axis order, dx = y*(g - dot), in RT = promote_t<y, g>
// (softmaxbackward.h:111-128).
template <typename RT, typename LoadY, typename LoadG, typename Store>
void cpu_softmax_bwd_rows(size_t rows, size_t cols, LoadY ly, LoadG lg, Store st) {
    for (size_t r = 0; r < rows; ++r) {
        RT dot = RT(0);
        for (size_t k = 0; k < cols; ++k) dot += lg(r * cols + k) * ly(r * cols + k);
        for (size_t k = 0; k < cols; ++k) st(r * cols + k, ly(r * cols + k) * (lg(r * cols + k) - dot));
    }
}

// Output dtype of Softmax: promote_t<AT, float> over the dtypes dispatchAny
// takes (softmax.cpp:25, dtype_dispatch.h:8-52), plus BFloat16 (fp32
// arithmetic, bf16 storage).
DType softmax_out_dtype(DType in) {
    switch (in) {
        case DType::Float32:
        case DType::Int32: return DType::Float32;
        case DType::Float64: return DType::Float64;
        case DType::BFloat16: return DType::BFloat16;
        default: throw Error(std::string("Softmax: unsupported dtype ") + dtype_name(in));
    }
}

// promote_t of the backward's two operands (dispatchFloatTwo,
// softmaxbackward.cpp:40-45): Float64 if either is, else the saved output's.
DType softmax_grad_dtype(DType y, DType g) {
    const auto floating = [](DType d) { return d == DType::Float32 || d == DType::Float64 || d == DType::BFloat16; };
    if (!floating(y) || !floating(g))
        throw Error(std::string("SoftmaxBackward: floating operands expected, got ") + dtype_name(y) + " and " +
                    dtype_name(g));
    if (y == DType::Float64 || g == DType::Float64) return DType::Float64;
    return y;
}

inf_dtype sm_dt(DType dt) {
    switch (dt) {
        case DType::Float32: return INF_F32;
        case DType::BFloat16: return INF_BF16;
        case DType::Float64: return INF_F64;
        case DType::Int32: return INF_I32;
        default: throw Error(std::string("Softmax: unsupported dtype ") + dtype_name(dt));
    }
}

}  // namespace

Tensor Softmax(Tensor& A, int axis) {
    const DType odt = softmax_out_dtype(A.dtype());
    const int ax = norm_axis(axis, A.ndim());
    if (!A.device().is_cpu() && !dense_rows(A, ax) && (int)A.ndim() <= kMaxSoftmaxRank) {
        Tensor out(odt, A.shape(), "softmax", A.device(), false);
        if (A.numel()) {
            detail::DeviceGuard g(A.device().index);
            const auto shape = i64(A.shape()), sa = i64(A.strides()), so = i64(out.strides());
            detail::status_check(inf_softmax_fwd_axis(A.data_ptr(), sa.data(), out.data_ptr(), so.data(), (int)A.ndim(),
                                                      shape.data(), ax, sm_dt(A.dtype()), detail::stream_of(A)),
                                 "inf_softmax_fwd_axis");
        }
        out.set_requires_grad(true);
        if (grad_enabled && A.requires_grad()) GetImpl(out)->gradfn() = std::make_shared<SoftmaxBackward>(A, out, ax);
        return out;
    }
    Tensor x = rows_of(A, ax);
    const size_t cols = x.shape().back();
    const size_t rows = cols ? x.numel() / cols : 0;
    Tensor y(odt, x.shape(), "softmax", A.device(), false);
    if (rows && cols) {
        if (A.device().is_cpu()) {
            const char* px = static_cast<const char*>(x.data_ptr());
            char* py = static_cast<char*>(y.data_ptr());
            const size_t ei = dtype_size(x.dtype()), eo = dtype_size(odt);
            const DType idt = x.dtype();
            auto st = [&](size_t i, double v) { detail::store_elem(py + i * eo, odt, v); };
            if (odt == DType::Float64)
                cpu_softmax_rows<double>(rows, cols, [&](size_t i) { return detail::load_elem(px + i * ei, idt); }, st);
            else
                cpu_softmax_rows<float>(rows, cols, [&](size_t i) { return (float)detail::load_elem(px + i * ei, idt); },
                                        st);
        } else {
            detail::DeviceGuard g(A.device().index);
            detail::status_check(inf_softmax_fwd(x.data_ptr(), y.data_ptr(), (int64_t)rows, (int64_t)cols,
                                                 (int64_t)cols, (int64_t)cols, sm_dt(x.dtype()), detail::stream_of(A)),
                                 "inf_softmax_fwd");
        }
    }
    Tensor out = restore_axis(y, ax, A.ndim());
    out.set_requires_grad(true);  // as the reference does (softmax.cpp:40)
    if (grad_enabled && A.requires_grad()) GetImpl(out)->gradfn() = std::make_shared<SoftmaxBackward>(A, out, ax);
    return out;
}

SoftmaxBackward::SoftmaxBackward(const Tensor& A, const Tensor& out, int axis)
    : m_A(A), m_out(make_view(out, out.shape(), out.strides(), out.offset(), "softmax_saved")), m_axis(axis) {
    set_name("SoftmaxBackward");
}

void SoftmaxBackward::backward() {
    NoGradGuard ng;
    Tensor g = Engine::grad_in(this, 0);
    if (!m_out.device().is_cpu() && !(dense_rows(m_out, m_axis) && dense_rows(g, m_axis)) &&
        (int)m_out.ndim() <= kMaxSoftmaxRank) {
        const DType rdt = softmax_grad_dtype(m_out.dtype(), g.dtype());
        if (m_out.dtype() != g.dtype())
            throw Error(std::string("SoftmaxBackward: on HIP the output and its gradient must share a dtype, got ") +
                        dtype_name(m_out.dtype()) + " and " + dtype_name(g.dtype()));
        Tensor dx(rdt, m_out.shape(), "softmax_grad", m_out.device(), false);
        if (dx.numel()) {
            detail::DeviceGuard dg(m_out.device().index);
            const auto shape = i64(m_out.shape()), sy = i64(m_out.strides()), sg = i64(g.strides()),
                       sd = i64(dx.strides());
            detail::status_check(inf_softmax_bwd_axis(m_out.data_ptr(), sy.data(), g.data_ptr(), sg.data(),
                                                      dx.data_ptr(), sd.data(), (int)m_out.ndim(), shape.data(), m_axis,
                                                      sm_dt(m_out.dtype()), detail::stream_of(m_out)),
                                 "inf_softmax_bwd_axis");
        }
        auto e = GetImpl(m_A)->grad_edge();
        if (e) Engine::accumulate(e.get(), 0, dx);
        return;
    }
    Tensor y = rows_of(m_out, m_axis);
    Tensor gr = rows_of(g, m_axis);
    const DType rdt = softmax_grad_dtype(y.dtype(), gr.dtype());
    const size_t cols = y.shape().back();
    const size_t rows = cols ? y.numel() / cols : 0;
    Tensor dx(rdt, y.shape(), "softmax_grad", y.device(), false);
    if (rows && cols) {
        if (y.device().is_cpu()) {
            const char* py = static_cast<const char*>(y.data_ptr());
            const char* pg = static_cast<const char*>(gr.data_ptr());
            char* pd = static_cast<char*>(dx.data_ptr());
            const size_t ey = dtype_size(y.dtype()), eg = dtype_size(gr.dtype()), ed = dtype_size(rdt);
            const DType ydt = y.dtype(), gdt = gr.dtype();
            auto st = [&](size_t i, double v) { detail::store_elem(pd + i * ed, rdt, v); };
            if (rdt == DType::Float64)
                cpu_softmax_bwd_rows<double>(rows, cols, [&](size_t i) { return detail::load_elem(py + i * ey, ydt); },
                                             [&](size_t i) { return detail::load_elem(pg + i * eg, gdt); }, st);
            else
                cpu_softmax_bwd_rows<float>(
                    rows, cols, [&](size_t i) { return (float)detail::load_elem(py + i * ey, ydt); },
                    [&](size_t i) { return (float)detail::load_elem(pg + i * eg, gdt); }, st);
        } else {
            if (y.dtype() != gr.dtype())
                throw Error(std::string("SoftmaxBackward: on HIP the output and its gradient must share a dtype, got ") +
                            dtype_name(y.dtype()) + " and " + dtype_name(gr.dtype()));
            detail::DeviceGuard dg(y.device().index);
            detail::status_check(inf_softmax_bwd(y.data_ptr(), gr.data_ptr(), dx.data_ptr(), (int64_t)rows,
                                                 (int64_t)cols, (int64_t)cols, (int64_t)cols, (int64_t)cols,
                                                 sm_dt(y.dtype()), detail::stream_of(y)),
                                 "inf_softmax_bwd");
        }
    }
    auto e = GetImpl(m_A)->grad_edge();
    if (e) Engine::accumulate(e.get(), 0, restore_axis(dx, m_axis, m_A.ndim()));
}

void SoftmaxBackward::release() {
    m_A = Tensor();
    m_out = Tensor();
}

void SoftmaxBackward::get_inputs(std::vector<Tensor>& out) const { out.push_back(m_A); }

}  // namespace Inferno
