// mask_ops.cpp -- triu and masked_fill (include/inferno/core/ops.h), the mask
// half of the reference's unfused attention chain (InfernoApp/main.cpp:746-748,
// 781-811).  Same signatures and semantics as src/inferno/core/ops.cpp:1235-1398:
// dense output of the input's shape on the input's device, no backward node
// (the output does not require grad).  CPU tensors run the element loops of
// cpu_triu / cpu_masked_fill (src/inferno/core/cpuops.h:617-705); HIP tensors
// run inf_triu / inf_masked_fill.  Both copy elements bit for bit, so any
// dtype works; the fill value is converted to the input dtype as
// static_cast<AT>(value) does.
#include <cstring>
#include <string>
#include <vector>

#include "detail.h"
#include "inferno/core/ops.h"

namespace Inferno {

namespace {

bool is_int_mask(DType dt) { return dt == DType::Int32 || dt == DType::Int8 || dt == DType::Bool; }

bool nonzero(const char* p, size_t bytes) {
    for (size_t b = 0; b < bytes; ++b)
        if (p[b]) return true;
    return false;
}

}  // namespace

Tensor triu(const Tensor& A, int diagonal) {
    if (A.ndim() < 2) throw Error("triu requires tensor rank >= 2");
    Tensor out(A.dtype(), A.shape(), "triu(" + A.name() + ")", A.device());
    const size_t n = out.numel();
    if (n == 0) return out;
    const size_t esz = dtype_size(A.dtype());
    const size_t rank = A.ndim();
    if (A.device().is_cpu()) {
        // cpu_triu: unravel each output index, read the view through its strides.
        const char* a = static_cast<const char*>(A.data_ptr());
        char* o = static_cast<char*>(out.data_ptr());
        const auto& shape = A.shape();
        const auto& st = A.strides();
        std::vector<size_t> idx(rank, 0);
        for (size_t lin = 0; lin < n; ++lin) {
            size_t tmp = lin;
            for (int d = (int)rank - 1; d >= 0; --d) {
                idx[d] = tmp % shape[d];
                tmp /= shape[d];
            }
            size_t so = 0;
            for (size_t d = 0; d < rank; ++d) so += idx[d] * st[d];
            const size_t row = idx[rank - 2], col = idx[rank - 1];
            if ((int)col - (int)row >= diagonal)
                std::memcpy(o + lin * esz, a + so * esz, esz);
            else
                std::memset(o + lin * esz, 0, esz);
        }
        return out;
    }
    const auto shape = detail::to_i64(A.shape()), st = detail::to_i64(A.strides());
    detail::DeviceGuard dg(A.device().index);
    detail::status_check(inf_triu(A.data_ptr(), st.data(), out.data_ptr(), (int)rank, shape.data(), diagonal,
                                  (int)esz, detail::stream_of(A)),
                         "inf_triu");
    return out;
}

Tensor masked_fill(const Tensor& input, const Tensor& mask, float value) {
    if (!is_int_mask(mask.dtype()))
        throw Error(std::string("masked_fill: the mask must be Int32, Int8 or Bool, got ") + dtype_name(mask.dtype()));
    detail::same_device(input, mask, "masked_fill");
    const size_t rank = input.ndim(), mrank = mask.ndim();
    if (mrank > rank) throw Error("masked_fill: the mask has more dimensions than the input");
    const size_t lead = rank - mrank;
    for (size_t d = 0; d < mrank; ++d)
        if (mask.shape()[d] != 1 && mask.shape()[d] != input.shape()[lead + d])
            throw Error("masked_fill: the mask does not broadcast to the input's shape");
    Tensor out(input.dtype(), input.shape(), "masked_fill_out", input.device());
    const size_t n = out.numel();
    if (n == 0) return out;
    const size_t esz = dtype_size(input.dtype()), mesz = dtype_size(mask.dtype());
    uint64_t fill = 0;  // static_cast<AT>(value), as bits
    detail::store_elem(&fill, input.dtype(), (double)value);
    if (input.device().is_cpu()) {
        // cpu_masked_fill: the mask's shape / strides padded on the left; a
        // size-1 mask dimension always reads index 0.
        std::vector<size_t> pshape(rank, 1), pstride(rank, 0);
        for (size_t d = 0; d < mrank; ++d) {
            pshape[lead + d] = mask.shape()[d];
            pstride[lead + d] = mask.strides()[d];
        }
        const char* in = static_cast<const char*>(input.data_ptr());
        const char* mk = static_cast<const char*>(mask.data_ptr());
        char* o = static_cast<char*>(out.data_ptr());
        const auto& shape = input.shape();
        const auto& st = input.strides();
        std::vector<size_t> idx(rank, 0);
        for (size_t lin = 0; lin < n; ++lin) {
            size_t tmp = lin;
            for (int d = (int)rank - 1; d >= 0; --d) {
                idx[d] = tmp % shape[d];
                tmp /= shape[d];
            }
            size_t io = 0, mo = 0;
            for (size_t d = 0; d < rank; ++d) {
                io += idx[d] * st[d];
                mo += (pshape[d] == 1 ? 0 : idx[d]) * pstride[d];
            }
            if (nonzero(mk + mo * mesz, mesz))
                std::memcpy(o + lin * esz, &fill, esz);
            else
                std::memcpy(o + lin * esz, in + io * esz, esz);
        }
        return out;
    }
    const auto shape = detail::to_i64(input.shape()), st = detail::to_i64(input.strides());
    const auto mshape = detail::to_i64(mask.shape()), mst = detail::to_i64(mask.strides());
    detail::DeviceGuard dg(input.device().index);
    detail::status_check(inf_masked_fill(input.data_ptr(), st.data(), mask.data_ptr(), mshape.data(), mst.data(),
                                         (int)mrank, (int)mesz, out.data_ptr(), (int)rank, shape.data(), fill,
                                         (int)esz, detail::stream_of(input)),
                         "inf_masked_fill");
    return out;
}

}  // namespace Inferno
