// elementwise.hip -- the small memory-bound ops the Tensor layer needs on the
// GPU around the attention path: fill (ones_like seeds of the autograd engine),
// add (gradient accumulation), multiply (scalar scale and the O*dO product
// that injects an upstream gradient), and a strided copy (Tensor::contiguous,
// and writing a gradient into a view of a larger tensor).  None of these is on
// the timed path; they are grid-stride loops over elements.
#include "common.h"
#include "kernels.h"

namespace inf {

template <typename E>
__global__ __launch_bounds__(256) void fill_kernel(E* dst, int64_t n, E value) {
    for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (int64_t)gridDim.x * 256)
        dst[i] = value;
}

// op: 0 = add, 1 = multiply.  a_scalar / b_scalar: that operand is one element.
template <typename Tg, int OP>
__global__ __launch_bounds__(256) void binary_kernel(const typename Tg::T* a, const typename Tg::T* b,
                                                     typename Tg::T* out, int64_t n, int a_scalar,
                                                     int b_scalar) {
    const float as = a_scalar ? Tg::ld(a) : 0.f;
    const float bs = b_scalar ? Tg::ld(b) : 0.f;
    for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (int64_t)gridDim.x * 256) {
        const float x = a_scalar ? as : Tg::ld(a + i);
        const float y = b_scalar ? bs : Tg::ld(b + i);
        Tg::st(out + i, OP == 0 ? x + y : x * y);
    }
}

template <typename E>
__global__ __launch_bounds__(256) void copy_strided_kernel(const E* src, E* dst, StridedCopy c) {
    for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < c.n; i += (int64_t)gridDim.x * 256) {
        int64_t rem = i, so = 0, dof = 0;
        for (int d = c.ndim - 1; d >= 0; --d) {
            const int64_t idx = rem % c.shape[d];
            rem /= c.shape[d];
            so += idx * c.sstride[d];
            dof += idx * c.dstride[d];
        }
        dst[dof] = src[so];
    }
}

// triu (cpu_triu, src/inferno/core/cpuops.h:617-656): output element i (dense)
// takes the view's element when col - row >= diagonal, else all-zero bits.
template <typename E>
__global__ __launch_bounds__(256) void triu_kernel(const E* src, E* dst, StridedCopy c, int diagonal) {
    for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < c.n; i += (int64_t)gridDim.x * 256) {
        int64_t rem = i, so = 0, row = 0, col = 0;
        for (int d = c.ndim - 1; d >= 0; --d) {
            const int64_t idx = rem % c.shape[d];
            rem /= c.shape[d];
            so += idx * c.sstride[d];
            if (d == c.ndim - 1) col = idx;
            if (d == c.ndim - 2) row = idx;
        }
        dst[i] = ((int)col - (int)row >= diagonal) ? src[so] : E(0);
    }
}

// masked_fill (cpu_masked_fill, src/inferno/core/cpuops.h:659-705): output
// element i (dense) = fill where the broadcast mask element is non-zero.
template <typename E, typename M>
__global__ __launch_bounds__(256) void masked_fill_kernel(const E* in, const M* mask, E* out, MaskedFill m,
                                                          E fill) {
    for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < m.n; i += (int64_t)gridDim.x * 256) {
        int64_t rem = i, io = 0, mo = 0;
        for (int d = m.ndim - 1; d >= 0; --d) {
            const int64_t idx = rem % m.shape[d];
            rem /= m.shape[d];
            io += idx * m.istride[d];
            mo += idx * m.mstride[d];
        }
        out[i] = mask[mo] != M(0) ? fill : in[io];
    }
}

static dim3 grid_for(int64_t n) {
    int64_t blocks = (n + 255) / 256;
    if (blocks > 65536) blocks = 65536;
    if (blocks < 1) blocks = 1;
    return dim3((unsigned)blocks);
}

int launch_fill(void* dst, int64_t n, int elem_bytes, uint32_t bits, hipStream_t s) {
    if (elem_bytes == 4)
        hipLaunchKernelGGL(fill_kernel<uint32_t>, grid_for(n), dim3(256), 0, s, (uint32_t*)dst, n, bits);
    else if (elem_bytes == 2)
        hipLaunchKernelGGL(fill_kernel<uint16_t>, grid_for(n), dim3(256), 0, s, (uint16_t*)dst, n,
                           (uint16_t)bits);
    else
        hipLaunchKernelGGL(fill_kernel<uint8_t>, grid_for(n), dim3(256), 0, s, (uint8_t*)dst, n,
                           (uint8_t)bits);
    return (int)hipGetLastError();
}

int launch_binary(int op, const void* a, const void* b, void* out, int64_t n, int a_scalar, int b_scalar,
                  int bf16, hipStream_t s) {
    const dim3 g = grid_for(n);
    if (bf16) {
        if (op == 0)
            hipLaunchKernelGGL((binary_kernel<BF16, 0>), g, dim3(256), 0, s, (const uint16_t*)a,
                               (const uint16_t*)b, (uint16_t*)out, n, a_scalar, b_scalar);
        else
            hipLaunchKernelGGL((binary_kernel<BF16, 1>), g, dim3(256), 0, s, (const uint16_t*)a,
                               (const uint16_t*)b, (uint16_t*)out, n, a_scalar, b_scalar);
    } else {
        if (op == 0)
            hipLaunchKernelGGL((binary_kernel<F32, 0>), g, dim3(256), 0, s, (const float*)a, (const float*)b,
                               (float*)out, n, a_scalar, b_scalar);
        else
            hipLaunchKernelGGL((binary_kernel<F32, 1>), g, dim3(256), 0, s, (const float*)a, (const float*)b,
                               (float*)out, n, a_scalar, b_scalar);
    }
    return (int)hipGetLastError();
}

int launch_copy_strided(const void* src, void* dst, const StridedCopy& c, int elem_bytes, hipStream_t s) {
    const dim3 g = grid_for(c.n);
    if (elem_bytes == 4)
        hipLaunchKernelGGL(copy_strided_kernel<uint32_t>, g, dim3(256), 0, s, (const uint32_t*)src,
                           (uint32_t*)dst, c);
    else if (elem_bytes == 2)
        hipLaunchKernelGGL(copy_strided_kernel<uint16_t>, g, dim3(256), 0, s, (const uint16_t*)src,
                           (uint16_t*)dst, c);
    else if (elem_bytes == 8)
        hipLaunchKernelGGL(copy_strided_kernel<uint64_t>, g, dim3(256), 0, s, (const uint64_t*)src,
                           (uint64_t*)dst, c);
    else
        hipLaunchKernelGGL(copy_strided_kernel<uint8_t>, g, dim3(256), 0, s, (const uint8_t*)src,
                           (uint8_t*)dst, c);
    return (int)hipGetLastError();
}

int launch_triu(const void* src, void* dst, const StridedCopy& c, int diagonal, int elem_bytes, hipStream_t s) {
    const dim3 g = grid_for(c.n);
    if (elem_bytes == 4)
        hipLaunchKernelGGL(triu_kernel<uint32_t>, g, dim3(256), 0, s, (const uint32_t*)src, (uint32_t*)dst, c,
                           diagonal);
    else if (elem_bytes == 2)
        hipLaunchKernelGGL(triu_kernel<uint16_t>, g, dim3(256), 0, s, (const uint16_t*)src, (uint16_t*)dst, c,
                           diagonal);
    else if (elem_bytes == 8)
        hipLaunchKernelGGL(triu_kernel<uint64_t>, g, dim3(256), 0, s, (const uint64_t*)src, (uint64_t*)dst, c,
                           diagonal);
    else
        hipLaunchKernelGGL(triu_kernel<uint8_t>, g, dim3(256), 0, s, (const uint8_t*)src, (uint8_t*)dst, c,
                           diagonal);
    return (int)hipGetLastError();
}

template <typename E>
static void masked_fill_t(const void* in, const void* mask, void* out, const MaskedFill& m, int mask_bytes,
                          E fill, hipStream_t s) {
    const dim3 g = grid_for(m.n);
    if (mask_bytes == 4)
        hipLaunchKernelGGL((masked_fill_kernel<E, uint32_t>), g, dim3(256), 0, s, (const E*)in,
                           (const uint32_t*)mask, (E*)out, m, fill);
    else if (mask_bytes == 8)
        hipLaunchKernelGGL((masked_fill_kernel<E, uint64_t>), g, dim3(256), 0, s, (const E*)in,
                           (const uint64_t*)mask, (E*)out, m, fill);
    else
        hipLaunchKernelGGL((masked_fill_kernel<E, uint8_t>), g, dim3(256), 0, s, (const E*)in,
                           (const uint8_t*)mask, (E*)out, m, fill);
}

int launch_masked_fill(const void* in, const void* mask, void* out, const MaskedFill& m, int elem_bytes,
                       int mask_bytes, uint64_t fill_bits, hipStream_t s) {
    if (elem_bytes == 4)
        masked_fill_t<uint32_t>(in, mask, out, m, mask_bytes, (uint32_t)fill_bits, s);
    else if (elem_bytes == 2)
        masked_fill_t<uint16_t>(in, mask, out, m, mask_bytes, (uint16_t)fill_bits, s);
    else if (elem_bytes == 8)
        masked_fill_t<uint64_t>(in, mask, out, m, mask_bytes, (uint64_t)fill_bits, s);
    else
        masked_fill_t<uint8_t>(in, mask, out, m, mask_bytes, (uint8_t)fill_bits, s);
    return (int)hipGetLastError();
}

}  // namespace inf
