// tensor.cpp -- TensorImpl and Tensor (include/inferno/core/tensor.h, tensorimpl.h).
#include <algorithm>
#include <numeric>

#include "detail.h"
#include "inferno/gradengine/engine.h"
#include "inferno/gradfn/node.h"

namespace Inferno {

using detail::DeviceGuard;
using detail::hip_check;
using detail::status_check;

// ---------------------------------------------------------------- TensorImpl
TensorImpl::TensorImpl(DType dtype, std::vector<size_t> shape, std::string name, Device device, bool requires_grad)
    : m_dtype(dtype),
      m_shape(std::move(shape)),
      m_strides(Tensor::calculate_strides(m_shape)),
      m_device(device),
      m_name(std::move(name)),
      m_requires_grad(requires_grad) {
    m_storage = make_storage(numel() * dtype_size(dtype), device);
}

TensorImpl::TensorImpl(std::shared_ptr<Storage> storage, DType dtype, std::vector<size_t> shape,
                       std::vector<size_t> strides, size_t offset, std::string name, Device device, bool requires_grad)
    : m_dtype(dtype),
      m_shape(std::move(shape)),
      m_strides(std::move(strides)),
      m_offset(offset),
      m_storage(std::move(storage)),
      m_device(device),
      m_name(std::move(name)),
      m_requires_grad(requires_grad) {}

size_t TensorImpl::numel() const {
    return std::accumulate(m_shape.begin(), m_shape.end(), (size_t)1, std::multiplies<size_t>());
}

bool TensorImpl::is_contiguous() const { return m_strides == Tensor::calculate_strides(m_shape); }

void* TensorImpl::data_ptr() const {
    if (!m_storage || !m_storage->raw_ptr()) return nullptr;
    return static_cast<char*>(m_storage->raw_ptr()) + m_offset * dtype_size(m_dtype);
}

std::shared_ptr<Node> TensorImpl::grad_edge() {
    if (m_gradfn) return m_gradfn;
    if (!m_requires_grad) return nullptr;
    if (!m_accumulate) {
        m_accumulate = std::make_shared<AccumulateGrad>(weak_from_this());
        m_accumulate->set_name("AccumulateGrad(" + m_name + ")");
    }
    return m_accumulate;
}

Tensor make_view(const Tensor& base, std::vector<size_t> shape, std::vector<size_t> strides, size_t offset,
                 const std::string& name) {
    auto b = GetImpl(base);
    Tensor t;
    SetImpl(t, std::make_shared<TensorImpl>(b->storage(), b->dtype(), std::move(shape), std::move(strides), offset,
                                            name, b->device(), false));
    return t;
}

std::shared_ptr<TensorImpl> GetImpl(const Tensor& t) { return t.m_impl; }
void SetImpl(Tensor& t, std::shared_ptr<TensorImpl> impl) { t.m_impl = std::move(impl); }

// -------------------------------------------------------------------- Tensor
static TensorImpl& impl_of(const std::shared_ptr<TensorImpl>& p) {
    if (!p) throw Error("use of an undefined Tensor");
    return *p;
}

Tensor::Tensor(DType dtype, std::vector<size_t> shape, std::string name, Device device, bool requires_grad)
    : m_impl(std::make_shared<TensorImpl>(dtype, std::move(shape), std::move(name), device, requires_grad)) {}

Tensor::Tensor(DType dtype, std::initializer_list<size_t> shape, std::string name, Device device, bool requires_grad)
    : Tensor(dtype, std::vector<size_t>(shape), std::move(name), device, requires_grad) {}

void Tensor::init_from_host(DType dtype, const void* data, size_t count, HostKind kind, std::vector<size_t> shape,
                            std::string name, Device device, bool requires_grad) {
    const size_t n = std::accumulate(shape.begin(), shape.end(), (size_t)1, std::multiplies<size_t>());
    if (n != count) throw Error("Tensor: data has " + std::to_string(count) + " elements, shape needs " + std::to_string(n));
    auto host = std::make_shared<TensorImpl>(dtype, shape, name, Device::cpu(), false);
    char* dst = static_cast<char*>(host->data_ptr());
    const size_t esz = dtype_size(dtype);
    for (size_t i = 0; i < n; ++i) {
        double v = 0;
        switch (kind) {
            case HostKind::F32: v = static_cast<const float*>(data)[i]; break;
            case HostKind::F64: v = static_cast<const double*>(data)[i]; break;
            case HostKind::I32: v = static_cast<const int32_t*>(data)[i]; break;
            case HostKind::I64: v = (double)static_cast<const int64_t*>(data)[i]; break;
            case HostKind::U8: v = static_cast<const uint8_t*>(data)[i]; break;
            case HostKind::I8: v = static_cast<const int8_t*>(data)[i]; break;
            case HostKind::BF16: v = (float)static_cast<const bfloat16*>(data)[i]; break;
        }
        detail::store_elem(dst + i * esz, dtype, v);
    }
    Tensor h;
    h.m_impl = host;
    if (device.is_cpu()) {
        m_impl = host;
    } else {
        m_impl = GetImpl(h.to(device));
    }
    m_impl->set_requires_grad(requires_grad);
}

const Device& Tensor::device() const { return impl_of(m_impl).device(); }
DType Tensor::dtype() const { return impl_of(m_impl).dtype(); }
std::shared_ptr<Storage>& Tensor::data() const { return impl_of(m_impl).storage(); }
std::shared_ptr<Tensor>& Tensor::grad() const { return impl_of(m_impl).grad(); }
Tensor Tensor::Getgrad() const {
    auto& g = grad();
    if (!g) throw Error("Getgrad: tensor '" + name() + "' has no gradient");
    return *g;
}
std::vector<size_t>& Tensor::shape() const { return impl_of(m_impl).shape(); }
std::vector<size_t>& Tensor::strides() const { return impl_of(m_impl).strides(); }
size_t& Tensor::offset() const { return impl_of(m_impl).offset(); }
std::string Tensor::name() const { return impl_of(m_impl).name(); }
size_t Tensor::ndim() const { return shape().size(); }
bool Tensor::requires_grad() const { return impl_of(m_impl).requires_grad(); }
void Tensor::set_requires_grad(bool flag) { impl_of(m_impl).set_requires_grad(flag); }
size_t Tensor::numel() const { return impl_of(m_impl).numel(); }
size_t Tensor::size() const { return numel() * dtype_size(dtype()); }
bool Tensor::is_contiguous() const { return impl_of(m_impl).is_contiguous(); }
void* Tensor::data_ptr() const { return impl_of(m_impl).data_ptr(); }

std::vector<size_t> Tensor::calculate_strides(const std::vector<size_t>& shape) {
    std::vector<size_t> st(shape.size(), 1);
    for (int i = (int)shape.size() - 2; i >= 0; --i) st[i] = st[i + 1] * shape[i + 1];
    return st;
}

Tensor Tensor::full(const std::vector<size_t>& shape, double value, DType dtype, Device device,
                    const std::string& name) {
    Tensor t(dtype, shape, name, device, false);
    const size_t n = t.numel(), esz = dtype_size(dtype);
    if (device.is_cpu()) {
        char* p = static_cast<char*>(t.data_ptr());
        for (size_t i = 0; i < n; ++i) detail::store_elem(p + i * esz, dtype, value);
    } else {
        uint64_t bits = 0;
        detail::store_elem(&bits, dtype, value);
        if (esz > 4) throw Error("Tensor::full: 8-byte dtypes are not supported on HIP");
        DeviceGuard g(device.index);
        status_check(inf_fill(t.data_ptr(), (int64_t)n, (int)esz, (uint32_t)bits, detail::stream_of(t)), "inf_fill");
    }
    return t;
}
Tensor Tensor::ones(const std::vector<size_t>& s, DType dt, Device d, const std::string& n) { return full(s, 1.0, dt, d, n); }
Tensor Tensor::zeros(const std::vector<size_t>& s, DType dt, Device d, const std::string& n) { return full(s, 0.0, dt, d, n); }
Tensor Tensor::ones_like(const Tensor& t) { return ones(t.shape(), t.dtype(), t.device(), "ones_like"); }
Tensor Tensor::zeros_like(const Tensor& t) { return zeros(t.shape(), t.dtype(), t.device(), "zeros_like"); }

Tensor detail::dense_copy(const Tensor& src) {
    Tensor out(src.dtype(), src.shape(), src.name() + "_contig", src.device(), false);
    const size_t esz = dtype_size(src.dtype());
    if (src.numel() == 0) return out;
    if (src.device().is_cpu()) {
        detail::copy_strided_host(static_cast<const char*>(src.data_ptr()), src.strides(),
                                  static_cast<char*>(out.data_ptr()), out.strides(), src.shape(), esz);
    } else {
        if (src.ndim() > 8) throw Error("contiguous: rank > 8 is not supported on HIP");
        auto shape = detail::to_i64(src.shape());
        auto sst = detail::to_i64(src.strides());
        auto dst = detail::to_i64(out.strides());
        DeviceGuard g(src.device().index);
        status_check(inf_copy_strided(src.data_ptr(), sst.data(), out.data_ptr(), dst.data(), (int)src.ndim(),
                                      shape.data(), (int)esz, detail::stream_of(src)),
                     "inf_copy_strided");
    }
    return out;
}

Tensor Tensor::contiguous() const {
    if (is_contiguous()) return *this;
    Tensor out = detail::dense_copy(*this);
    if (grad_enabled && requires_grad()) {
        out.set_requires_grad(true);
        GetImpl(out)->gradfn() = std::make_shared<ContiguousBackward>(*this);
    }
    return out;
}

Tensor Tensor::to(const Device& dst) const {
    const Device& src = device();
    if (src == dst) return *this;
    Tensor c;
    {
        NoGradGuard ng;
        c = is_contiguous() ? *this : detail::dense_copy(*this);
    }
    Tensor out(dtype(), shape(), name(), dst, false);
    const size_t nbytes = size();
    if (nbytes) {
        if (src.is_cpu()) {
            DeviceGuard g(dst.index);
            hipStream_t s = detail::stream_for(dst.index);
            hip_check(hipMemcpyAsync(out.data_ptr(), c.data_ptr(), nbytes, hipMemcpyHostToDevice, s), "hipMemcpyAsync H2D");
            hip_check(hipStreamSynchronize(s), "hipStreamSynchronize");
        } else if (dst.is_cpu()) {
            DeviceGuard g(src.index);
            hipStream_t s = detail::stream_for(src.index);
            hip_check(hipMemcpyAsync(out.data_ptr(), c.data_ptr(), nbytes, hipMemcpyDeviceToHost, s), "hipMemcpyAsync D2H");
            hip_check(hipStreamSynchronize(s), "hipStreamSynchronize");
        } else {
            DeviceGuard g(src.index);
            hipStream_t s = detail::stream_for(src.index);
            hip_check(hipStreamSynchronize(detail::stream_for(dst.index)), "hipStreamSynchronize");
            hip_check(hipMemcpyAsync(out.data_ptr(), c.data_ptr(), nbytes, hipMemcpyDeviceToDevice, s), "hipMemcpyAsync D2D");
            hip_check(hipStreamSynchronize(s), "hipStreamSynchronize");
        }
    }
    out.set_requires_grad(requires_grad());
    return out;
}

static int norm_dim(int d, size_t nd, const char* what) {
    const int n = (int)nd;
    if (d < 0) d += n;
    if (d < 0 || d >= n) throw Error(std::string(what) + ": dimension out of range");
    return d;
}

Tensor Tensor::transpose(int dima, int dimb) const {
    const int a = norm_dim(dima, ndim(), "transpose"), b = norm_dim(dimb, ndim(), "transpose");
    auto sh = shape();
    auto st = strides();
    std::swap(sh[a], sh[b]);
    std::swap(st[a], st[b]);
    Tensor out = make_view(*this, sh, st, offset(), name() + "_T");
    if (requires_grad()) {
        out.set_requires_grad(true);
        if (grad_enabled) GetImpl(out)->gradfn() = std::make_shared<TransposeBackward>(*this, a, b);
    }
    return out;
}

Tensor Tensor::slice(int axis, size_t start, size_t end, size_t step) const {
    const int ax = norm_dim(axis, ndim(), "slice");
    if (step == 0) throw Error("slice: step must be >= 1");
    if (start > end || end >= shape()[ax]) throw Error("slice: range out of bounds");
    auto sh = shape();
    auto st = strides();
    sh[ax] = (end - start) / step + 1;  // inclusive end
    st[ax] *= step;
    Tensor out = make_view(*this, sh, st, offset() + start * strides()[ax], name() + "_slice");
    if (requires_grad()) {
        out.set_requires_grad(true);
        if (grad_enabled) GetImpl(out)->gradfn() = std::make_shared<SliceBackward>(*this, ax, start, step);
    }
    return out;
}

Tensor Tensor::reshape(const std::vector<size_t>& newshape) const {
    const size_t n = std::accumulate(newshape.begin(), newshape.end(), (size_t)1, std::multiplies<size_t>());
    if (n != numel()) throw Error("reshape: element count mismatch");
    if (!is_contiguous()) throw Error("reshape: tensor is not contiguous (call contiguous() first)");
    Tensor out = make_view(*this, newshape, calculate_strides(newshape), offset(), name() + "_reshape");
    if (requires_grad()) {
        out.set_requires_grad(true);
        if (grad_enabled) GetImpl(out)->gradfn() = std::make_shared<ReshapeBackward>(*this);
    }
    return out;
}

Tensor Tensor::unflatten(int dim, const std::vector<size_t>& sizes) const {
    const int d = norm_dim(dim, ndim(), "unflatten");
    const size_t prod = std::accumulate(sizes.begin(), sizes.end(), (size_t)1, std::multiplies<size_t>());
    if (sizes.empty() || prod != shape()[d]) throw Error("unflatten: sizes do not multiply to the dimension");
    std::vector<size_t> sh, st;
    for (int i = 0; i < (int)ndim(); ++i) {
        if (i != d) {
            sh.push_back(shape()[i]);
            st.push_back(strides()[i]);
            continue;
        }
        size_t inner = strides()[i];
        std::vector<size_t> sub(sizes.size());
        for (int j = (int)sizes.size() - 1; j >= 0; --j) {
            sub[j] = inner;
            inner *= sizes[j];
        }
        sh.insert(sh.end(), sizes.begin(), sizes.end());
        st.insert(st.end(), sub.begin(), sub.end());
    }
    Tensor out = make_view(*this, sh, st, offset(), name() + "_unflatten");
    if (requires_grad()) {
        out.set_requires_grad(true);
        if (grad_enabled) GetImpl(out)->gradfn() = std::make_shared<ReshapeBackward>(*this);
    }
    return out;
}

void Tensor::backward() const { Engine::backward(*this); }
void Tensor::backward(const Tensor& gradient) const { Engine::backward(*this, gradient); }

std::vector<double> Tensor::to_host_double() const {
    Tensor h = to(Device::cpu());
    Tensor c;
    {
        NoGradGuard ng;
        c = h.is_contiguous() ? h : detail::dense_copy(h);
    }
    std::vector<double> out(c.numel());
    const char* p = static_cast<const char*>(c.data_ptr());
    const size_t esz = dtype_size(c.dtype());
    for (size_t i = 0; i < out.size(); ++i) out[i] = detail::load_elem(p + i * esz, c.dtype());
    return out;
}

std::vector<float> Tensor::to_host_float() const {
    auto d = to_host_double();
    return std::vector<float>(d.begin(), d.end());
}

double Tensor::item_double_impl() const {
    if (numel() != 1) throw Error("item: tensor has " + std::to_string(numel()) + " elements");
    return to_host_double()[0];
}
int64_t Tensor::item_int64_impl() const { return (int64_t)item_double_impl(); }

Tensor Tensor::operator+(const Tensor& other) const { return add(*this, other); }
Tensor Tensor::operator*(const Tensor& other) const { return multiply(*this, other); }

Tensor scalar_like(const Tensor& like, double value) {
    return Tensor::full({1}, value, like.dtype(), like.device(), "scalar");
}

}  // namespace Inferno
