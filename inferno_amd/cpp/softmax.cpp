// softmax.cpp -- Softmax / SoftmaxBackward (include/inferno/functional/softmax.h).
//
// The softmax axis is moved last and made dense (a no-op for the usual
// last-axis case), so both devices work on rows:
//   CPU: the reference's three passes (softmax_kernels.h:77-102): max with a
//        lowest() start, e = (float)exp((double)(x - max)), fp32 running sum,
//        divide; backward dot = sum g*y in axis order, dx = y*(g - dot)
//        (softmaxbackward.h:111-128).
//   HIP: inf_softmax_fwd / inf_softmax_bwd.
#include <cfloat>
#include <cmath>

#include "detail.h"
#include "inferno/functional/softmax.h"
#include "inferno/gradengine/engine.h"

namespace Inferno {

namespace {

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

Tensor restore_axis(const Tensor& rows, int axis, size_t nd) {
    NoGradGuard ng;
    if (axis == (int)nd - 1) return rows;
    return rows.transpose(axis, (int)nd - 1).contiguous();
}

template <typename Load, typename Store>
void cpu_softmax_rows(size_t rows, size_t cols, Load ld, Store st) {
    std::vector<float> e(cols);
    for (size_t r = 0; r < rows; ++r) {
        float mx = -FLT_MAX;
        for (size_t k = 0; k < cols; ++k) {
            const float x = ld(r * cols + k);
            if (x > mx) mx = x;
        }
        float sum = 0.f;
        for (size_t k = 0; k < cols; ++k) {
            e[k] = (float)std::exp((double)(ld(r * cols + k) - mx));
            sum += e[k];
        }
        for (size_t k = 0; k < cols; ++k) st(r * cols + k, e[k] / sum);
    }
}

template <typename LoadY, typename LoadG, typename Store>
void cpu_softmax_bwd_rows(size_t rows, size_t cols, LoadY ly, LoadG lg, Store st) {
    for (size_t r = 0; r < rows; ++r) {
        float dot = 0.f;
        for (size_t k = 0; k < cols; ++k) dot += lg(r * cols + k) * ly(r * cols + k);
        for (size_t k = 0; k < cols; ++k) st(r * cols + k, ly(r * cols + k) * (lg(r * cols + k) - dot));
    }
}

void check_float(const Tensor& t) {
    if (t.dtype() != DType::Float32 && t.dtype() != DType::BFloat16)
        throw Error(std::string("Softmax: Float32 or BFloat16 expected, got ") + dtype_name(t.dtype()));
}

}  // namespace

Tensor Softmax(Tensor& A, int axis) {
    check_float(A);
    const int ax = norm_axis(axis, A.ndim());
    Tensor x = rows_of(A, ax);
    const size_t cols = x.shape().back();
    const size_t rows = cols ? x.numel() / cols : 0;
    Tensor y(A.dtype(), x.shape(), "softmax", A.device(), false);
    if (rows && cols) {
        if (A.device().is_cpu()) {
            if (A.dtype() == DType::Float32) {
                const float* px = static_cast<const float*>(x.data_ptr());
                float* py = static_cast<float*>(y.data_ptr());
                cpu_softmax_rows(rows, cols, [&](size_t i) { return px[i]; }, [&](size_t i, float v) { py[i] = v; });
            } else {
                const bfloat16* px = static_cast<const bfloat16*>(x.data_ptr());
                bfloat16* py = static_cast<bfloat16*>(y.data_ptr());
                cpu_softmax_rows(rows, cols, [&](size_t i) { return (float)px[i]; },
                                 [&](size_t i, float v) { py[i] = bfloat16(v); });
            }
        } else {
            detail::DeviceGuard g(A.device().index);
            detail::status_check(inf_softmax_fwd(x.data_ptr(), y.data_ptr(), (int64_t)rows, (int64_t)cols,
                                                 (int64_t)cols, (int64_t)cols, detail::inf_dt(A.dtype(), "Softmax"),
                                                 detail::stream_of(A)),
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
    Tensor y = rows_of(m_out, m_axis);
    Tensor gr = rows_of(g, m_axis);
    const size_t cols = y.shape().back();
    const size_t rows = cols ? y.numel() / cols : 0;
    Tensor dx(y.dtype(), y.shape(), "softmax_grad", y.device(), false);
    if (rows && cols) {
        if (y.device().is_cpu()) {
            if (y.dtype() == DType::Float32) {
                const float* py = static_cast<const float*>(y.data_ptr());
                const float* pg = static_cast<const float*>(gr.data_ptr());
                float* pd = static_cast<float*>(dx.data_ptr());
                cpu_softmax_bwd_rows(rows, cols, [&](size_t i) { return py[i]; }, [&](size_t i) { return pg[i]; },
                                     [&](size_t i, float v) { pd[i] = v; });
            } else {
                const bfloat16* py = static_cast<const bfloat16*>(y.data_ptr());
                const bfloat16* pg = static_cast<const bfloat16*>(gr.data_ptr());
                bfloat16* pd = static_cast<bfloat16*>(dx.data_ptr());
                cpu_softmax_bwd_rows(rows, cols, [&](size_t i) { return (float)py[i]; },
                                     [&](size_t i) { return (float)pg[i]; },
                                     [&](size_t i, float v) { pd[i] = bfloat16(v); });
            }
        } else {
            detail::DeviceGuard dg(y.device().index);
            detail::status_check(
                inf_softmax_bwd(y.data_ptr(), gr.data_ptr(), dx.data_ptr(), (int64_t)rows, (int64_t)cols, (int64_t)cols,
                                (int64_t)cols, (int64_t)cols, detail::inf_dt(y.dtype(), "SoftmaxBackward"),
                                detail::stream_of(y)),
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
