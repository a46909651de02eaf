// nn.hip -- gfx950 kernels for the model ops either side of the attention path
// (the GPT training step around MultiHeadAttention): LayerNorm forward and
// backward, tanh-GELU forward and backward, fused cross-entropy forward and
// backward, embedding gather and scatter-add, AdamW, column sums (bias and
// broadcast gradients) and broadcast element-wise add / multiply.
//
// All of them are HBM-bound.  Rows that fit in registers (LayerNorm rows up to
// 4096 elements) are read once and kept in VGPRs, one wave per row, so a
// forward is exactly one read and one write of the activation.  Reductions
// across rows (dgamma, dbeta, bias gradients) are deterministic two-stage
// sums: per-workgroup partials in a caller-provided workspace, then a column
// reduce.  Only the embedding backward uses atomics (the reference's CUDA
// scatter does too, cudascatteraddembedding.cu).
#include "common.h"
#include "kernels.h"

namespace inf {

namespace {

__device__ __forceinline__ f32x4 f4(float a) { return f32x4{a, a, a, a}; }
__device__ __forceinline__ float hsum4(f32x4 v) { return (v[0] + v[1]) + (v[2] + v[3]); }

// tanh-approximation GELU and its derivative (gelu_kernels.h:9-16,
// gelubackward.h:27-44), evaluated in fp32.
constexpr float kGeluAlpha = 0.7978845608028654f;  // sqrt(2/pi)
constexpr float kGeluBeta = 0.044715f;

__device__ __forceinline__ float gelu_f(float x) {
    const float x3 = x * x * x;
    const float inner = kGeluAlpha * (x + kGeluBeta * x3);
    return 0.5f * x * (1.0f + tanhf(inner));
}
__device__ __forceinline__ float gelu_grad_f(float x) {
    const float x2 = x * x;
    const float x3 = x2 * x;
    const float u = kGeluAlpha * (x + kGeluBeta * x3);
    const float t = tanhf(u);
    const float sech2 = 1.0f - t * t;
    return 0.5f * (1.0f + t) + 0.5f * x * sech2 * kGeluAlpha * (1.0f + 3.0f * kGeluBeta * x2);
}

}  // namespace

// ============================================================================
// LayerNorm forward: y = (x - mean) * invstd * gamma + beta per row, with
// invstd = 1 / sqrt(var + eps) and var the biased variance (two passes over the
// row held in registers), mean / invstd saved for the backward
// (layernorm_kernels.h:48-87).  One wave per row; lane l holds columns
// 4*(64*i + l) .. +3 for i < VPT.
// ============================================================================
// With a residual (p.r), the row is first h = x + r, rounded to the element
// type and stored to p.h, and the LayerNorm reads that rounded h: the same
// values as an add kernel followed by this one.
__device__ __forceinline__ f32x4 round_elem(f32x4 v, const float*) { return v; }
__device__ __forceinline__ f32x4 round_elem(f32x4 v, const uint16_t*) {
#pragma unroll
    for (int k = 0; k < 4; ++k) v[k] = bf16_to_f32(f32_to_bf16(v[k]));
    return v;
}

template <int VPT, typename E>
__global__ __launch_bounds__(256) void ln_fwd_kernel(LnParams p) {
    const int lane = threadIdx.x & 63;
    const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (row >= p.rows) return;
    const int dim = p.dim;
    const E* x = (const E*)p.x + row * p.ldx;
    f32x4 v[VPT];
    float s = 0.f;
#pragma unroll
    for (int i = 0; i < VPT; ++i) {
        const int c = 4 * (64 * i + lane);
        v[i] = (c < dim) ? ld4(x + c) : f4(0.f);
        if (p.r && c < dim) {
            v[i] = round_elem(v[i] + ld4((const E*)p.r + row * p.ldr + c), x);
            st4((E*)p.h + row * p.ldh + c, v[i]);
        }
        s += hsum4(v[i]);
    }
    const float fdim = (float)dim;
    const float mean = wave_sum(s) / fdim;
    float q = 0.f;
#pragma unroll
    for (int i = 0; i < VPT; ++i) {
        const int c = 4 * (64 * i + lane);
        if (c < dim) {
            const f32x4 d = v[i] - f4(mean);
            q += hsum4(d * d);
        }
    }
    const float var = wave_sum(q) / fdim;
    const float invstd = 1.0f / sqrtf(var + p.eps);
    E* y = (E*)p.y + row * p.ldy;
#pragma unroll
    for (int i = 0; i < VPT; ++i) {
        const int c = 4 * (64 * i + lane);
        if (c < dim) {
            const f32x4 g = *reinterpret_cast<const f32x4*>(p.gamma + c);
            const f32x4 b = *reinterpret_cast<const f32x4*>(p.beta + c);
            st4(y + c, (v[i] - f4(mean)) * f4(invstd) * g + b);
        }
    }
    if (lane == 0) {
        if (p.mean) p.mean[row] = mean;
        if (p.invstd) p.invstd[row] = invstd;
    }
}

// Any dim (no vector-width or register limit): one wave per row, three passes
// over global memory.
template <typename E>
__global__ __launch_bounds__(256) void ln_fwd_generic_kernel(LnParams p) {
    const int lane = threadIdx.x & 63;
    const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (row >= p.rows) return;
    const int dim = p.dim;
    const typename E::T* x = (const typename E::T*)p.x + row * p.ldx;
    float s = 0.f;
    if (p.r) {
        // h = x + r first (each lane reads back only the columns it wrote)
        const typename E::T* r = (const typename E::T*)p.r + row * p.ldr;
        typename E::T* h = (typename E::T*)p.h + row * p.ldh;
        for (int c = lane; c < dim; c += 64) {
            E::st(h + c, E::ld(x + c) + E::ld(r + c));
            s += E::ld(h + c);
        }
        x = h;
    } else {
        for (int c = lane; c < dim; c += 64) s += E::ld(x + c);
    }
    const float mean = wave_sum(s) / (float)dim;
    float q = 0.f;
    for (int c = lane; c < dim; c += 64) {
        const float d = E::ld(x + c) - mean;
        q += d * d;
    }
    const float invstd = 1.0f / sqrtf(wave_sum(q) / (float)dim + p.eps);
    typename E::T* y = (typename E::T*)p.y + row * p.ldy;
    for (int c = lane; c < dim; c += 64) E::st(y + c, (E::ld(x + c) - mean) * invstd * p.gamma[c] + p.beta[c]);
    if (lane == 0) {
        if (p.mean) p.mean[row] = mean;
        if (p.invstd) p.invstd[row] = invstd;
    }
}

// ============================================================================
// LayerNorm backward (layernormbackward.h:47-97): per row
//   xhat = (x - mean) * invstd, dxhat = dy * gamma,
//   dx = invstd / dim * (dim * dxhat - sum(dxhat) - xhat * sum(dxhat * xhat)),
// and across rows dgamma = sum(dy * xhat), dbeta = sum(dy).  Stage 1: each
// workgroup (4 waves) walks rows with a grid stride, one wave per row, keeps
// its columns' dgamma / dbeta partials in registers, sums its 4 waves in LDS
// and writes one partial row per workgroup to the workspace.  Stage 2
// (col_reduce_kernel) sums the partial rows.
// ============================================================================
template <int VPT, typename E>
__global__ __launch_bounds__(256) void ln_bwd_kernel(LnBwdParams p) {
    constexpr int MAXC = 64 * 4 * VPT;
    __shared__ __attribute__((aligned(16))) float red[2][4][MAXC];
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int dim = p.dim;
    const float fdim = (float)dim;
    f32x4 gam[VPT], adg[VPT], adb[VPT];
#pragma unroll
    for (int i = 0; i < VPT; ++i) {
        const int c = 4 * (64 * i + lane);
        gam[i] = (c < dim) ? *reinterpret_cast<const f32x4*>(p.gamma + c) : f4(0.f);
        adg[i] = f4(0.f);
        adb[i] = f4(0.f);
    }
    const int64_t nw = (int64_t)gridDim.x * 4;
    for (int64_t row = (int64_t)blockIdx.x * 4 + wave; row < p.rows; row += nw) {
        const E* x = (const E*)p.x + row * p.ldx;
        const E* gy = (const E*)p.dy + row * p.lddy;
        const float mean = p.mean[row];
        const float invstd = p.invstd[row];
        f32x4 xh[VPT], dxh[VPT];
        float s1 = 0.f, s2 = 0.f;
#pragma unroll
        for (int i = 0; i < VPT; ++i) {
            const int c = 4 * (64 * i + lane);
            if (c < dim) {
                const f32x4 g = ld4(gy + c);
                xh[i] = (ld4(x + c) - f4(mean)) * f4(invstd);
                dxh[i] = g * gam[i];
                adb[i] += g;
                adg[i] += g * xh[i];
                s1 += hsum4(dxh[i]);
                s2 += hsum4(dxh[i] * xh[i]);
            } else {
                xh[i] = f4(0.f);
                dxh[i] = f4(0.f);
            }
        }
        s1 = wave_sum(s1);
        s2 = wave_sum(s2);
        const float k = invstd / fdim;
        E* dx = (E*)p.dx + row * p.lddx;
#pragma unroll
        for (int i = 0; i < VPT; ++i) {
            const int c = 4 * (64 * i + lane);
            if (c < dim) st4(dx + c, f4(k) * (f4(fdim) * dxh[i] - f4(s1) - xh[i] * f4(s2)));
        }
    }
#pragma unroll
    for (int i = 0; i < VPT; ++i) {
        const int c = 4 * (64 * i + lane);
        *reinterpret_cast<f32x4*>(&red[0][wave][c]) = adg[i];
        *reinterpret_cast<f32x4*>(&red[1][wave][c]) = adb[i];
    }
    __syncthreads();
    float* pg = p.part + (int64_t)blockIdx.x * dim;
    float* pb = p.part + ((int64_t)gridDim.x + blockIdx.x) * dim;
    for (int c = threadIdx.x; c < dim; c += 256) {
        pg[c] = (red[0][0][c] + red[0][1][c]) + (red[0][2][c] + red[0][3][c]);
        pb[c] = (red[1][0][c] + red[1][1][c]) + (red[1][2][c] + red[1][3][c]);
    }
}

// out[c] (+)= sum_r in[r * cols + c] for r < rows: workgroup w owns columns
// [16*w, 16*w + 16); thread (c = tid % 16, g = tid / 16) sums rows g, g+16, ...
// and the 16 row groups are added in LDS in a fixed order.  Deterministic.
// Column sums of partial rows: 16 columns x 16 row groups per workgroup,
// each thread summing its rows in four independent chains (rows r, r+16,
// r+32, r+48 of each group of 64) so four loads are in flight; fixed order,
// deterministic.  blockIdx.y selects one of two (in, out) pairs so LayerNorm's
// dgamma and dbeta reduce in one launch.
__global__ __launch_bounds__(256) void col_reduce_kernel(const float* __restrict__ in0, float* __restrict__ out0,
                                                         const float* __restrict__ in1, float* __restrict__ out1,
                                                         int64_t rows, int64_t cols, int accumulate) {
    __shared__ float red[16][17];
    const float* in = blockIdx.y ? in1 : in0;
    float* out = blockIdx.y ? out1 : out0;
    const int cl = threadIdx.x & 15;
    const int g = threadIdx.x >> 4;
    const int64_t c = (int64_t)blockIdx.x * 16 + cl;
    float s0 = 0.f, s1 = 0.f, s2 = 0.f, s3 = 0.f;
    if (c < cols) {
        int64_t r = g;
        for (; r + 48 < rows; r += 64) {
            s0 += in[r * cols + c];
            s1 += in[(r + 16) * cols + c];
            s2 += in[(r + 32) * cols + c];
            s3 += in[(r + 48) * cols + c];
        }
        for (; r < rows; r += 16) s0 += in[r * cols + c];
    }
    red[g][cl] = (s0 + s1) + (s2 + s3);
    __syncthreads();
    if (g == 0 && c < cols) {
        float t = 0.f;
#pragma unroll
        for (int i = 0; i < 16; ++i) t += red[i][cl];
        out[c] = accumulate ? out[c] + t : t;
    }
}

// Column sums of a dense [rows, cols] matrix in two stages: per-chunk partials
// (chunk = kColChunk rows, so a [8192, 768] gradient runs 768 workgroups), then
// col_reduce over the chunks.
template <typename E>
__global__ __launch_bounds__(256) void col_partial_kernel(const void* __restrict__ x, float* __restrict__ part,
                                                          int64_t rows, int64_t cols, int64_t ldx) {
    const int64_t c = (int64_t)blockIdx.x * 256 + threadIdx.x;
    const int64_t r0 = (int64_t)blockIdx.y * kColChunk;
    if (c >= cols) return;
    const typename E::T* p = (const typename E::T*)x;
    const int64_t r1 = min(rows, r0 + kColChunk);
    float s = 0.f;
    if (r1 - r0 == kColChunk) {  // full chunk: all loads issued before the sum
        float v[kColChunk];
#pragma unroll
        for (int r = 0; r < kColChunk; ++r) v[r] = E::ld(p + (r0 + r) * ldx + c);
#pragma unroll
        for (int r = 0; r < kColChunk; ++r) s += v[r];
    } else {
        for (int64_t r = r0; r < r1; ++r) s += E::ld(p + r * ldx + c);
    }
    part[(int64_t)blockIdx.y * cols + c] = s;
}

// ============================================================================
// GELU forward / backward, element-wise (gelu.cpp, gelubackward.cpp).
// ============================================================================
template <typename E>
__global__ __launch_bounds__(256) void gelu_fwd_kernel(const void* __restrict__ x, void* __restrict__ y, int64_t n) {
    const int64_t i = ((int64_t)blockIdx.x * 256 + threadIdx.x) * 4;
    const typename E::T* xp = (const typename E::T*)x;
    typename E::T* yp = (typename E::T*)y;
    if (i + 3 < n) {
        const f32x4 v = ld4(xp + i);
        st4(yp + i, f32x4{gelu_f(v[0]), gelu_f(v[1]), gelu_f(v[2]), gelu_f(v[3])});
    } else {
        for (int64_t j = i; j < n; ++j) E::st(yp + j, gelu_f(E::ld(xp + j)));
    }
}

template <typename E>
__global__ __launch_bounds__(256) void gelu_bwd_kernel(const void* __restrict__ x, const void* __restrict__ dy,
                                                       void* __restrict__ dx, int64_t n) {
    const int64_t i = ((int64_t)blockIdx.x * 256 + threadIdx.x) * 4;
    const typename E::T* xp = (const typename E::T*)x;
    const typename E::T* gp = (const typename E::T*)dy;
    typename E::T* op = (typename E::T*)dx;
    if (i + 3 < n) {
        const f32x4 v = ld4(xp + i);
        const f32x4 g = ld4(gp + i);
        st4(op + i, f32x4{g[0] * gelu_grad_f(v[0]), g[1] * gelu_grad_f(v[1]), g[2] * gelu_grad_f(v[2]),
                          g[3] * gelu_grad_f(v[3])});
    } else {
        for (int64_t j = i; j < n; ++j) E::st(op + j, E::ld(gp + j) * gelu_grad_f(E::ld(xp + j)));
    }
}

// ============================================================================
// Cross-entropy, mean over rows (cpuops.h:707-749, crossentropylossbackward.h:
// 45-86).  Forward: one wave per row, online max / sum of exp over the row in
// 4-element chunks, row loss = lse - x[target] with lse = max + log(sum); the
// row's lse is kept for the backward.  A target outside [0, vocab) gives a NaN
// row loss (the reference exits).  A second kernel sums the row losses in a
// fixed order.  Backward: dlogits = (exp(x - lse) - [v == target]) * up / rows.
// ============================================================================
template <typename E>
__global__ __launch_bounds__(256) void ce_fwd_kernel(CeParams p) {
    const int lane = threadIdx.x & 63;
    const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (row >= p.rows) return;
    const int64_t V = p.vocab;
    const typename E::T* x = (const typename E::T*)p.logits + row * p.ld;
    float m = -INFINITY, s = 0.f;
    if ((V & 3) == 0) {
        for (int64_t c = 4 * lane; c < V; c += 256) {
            const f32x4 v = ld4(x + c);
            const float mv = fmaxf(fmaxf(v[0], v[1]), fmaxf(v[2], v[3]));
            if (mv > m) {
                s *= expf(m - mv);
                m = mv;
            }
            s += (expf(v[0] - m) + expf(v[1] - m)) + (expf(v[2] - m) + expf(v[3] - m));
        }
    } else {
        for (int64_t c = lane; c < V; c += 64) {
            const float v = E::ld(x + c);
            if (v > m) {
                s *= expf(m - v);
                m = v;
            }
            s += expf(v - m);
        }
    }
    // combine (m, s) over the wave
#pragma unroll
    for (int k = 32; k >= 1; k >>= 1) {
        const float mo = shfl_xor(m, k);
        const float so = shfl_xor(s, k);
        const float mn = fmaxf(m, mo);
        s = (mn == -INFINITY) ? 0.f : s * expf(m - mn) + so * expf(mo - mn);
        m = mn;
    }
    if (lane == 0) {
        const float lse = m + logf(s);
        const int t = p.targets[row];
        const float loss = (t >= 0 && t < V) ? lse - E::ld(x + t) : NAN;
        p.row_loss[row] = loss;
        if (p.lse) p.lse[row] = lse;
    }
}

// loss[0] = sum(row_loss) / rows, one workgroup, fixed summation order.
__global__ __launch_bounds__(256) void ce_mean_kernel(const float* __restrict__ row_loss, float* __restrict__ out,
                                                      int64_t rows) {
    __shared__ float red[256];
    float s = 0.f;
    for (int64_t r = threadIdx.x; r < rows; r += 256) s += row_loss[r];
    red[threadIdx.x] = s;
    __syncthreads();
    for (int w = 128; w >= 1; w >>= 1) {
        if ((int)threadIdx.x < w) red[threadIdx.x] += red[threadIdx.x + w];
        __syncthreads();
    }
    if (threadIdx.x == 0) out[0] = red[0] / (float)rows;
}

template <typename E>
__global__ __launch_bounds__(256) void ce_bwd_kernel(CeParams p) {
    const int lane = threadIdx.x & 63;
    const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (row >= p.rows) return;
    const int64_t V = p.vocab;
    const typename E::T* x = (const typename E::T*)p.logits + row * p.ld;
    typename E::T* g = (typename E::T*)p.grad + row * p.ldg;
    const float scale = p.upstream[0] / (float)p.rows;
    const float lse = p.lse[row];
    const int t = p.targets[row];
    if ((V & 3) == 0) {
        for (int64_t c = 4 * lane; c < V; c += 256) {
            const f32x4 v = ld4(x + c);
            f32x4 r;
#pragma unroll
            for (int j = 0; j < 4; ++j) r[j] = expf(v[j] - lse) * scale - ((c + j == t) ? scale : 0.f);
            st4(g + c, r);
        }
    } else {
        for (int64_t c = lane; c < V; c += 64)
            E::st(g + c, expf(E::ld(x + c) - lse) * scale - ((c == t) ? scale : 0.f));
    }
}

// ============================================================================
// Embedding (embedding_kernels.h:19-31): out[t, :] = table[ids[t], :]; an id
// outside [0, vocab) gives a NaN row.  Backward (EmbeddingBackward,
// embeddingbackward.cpp:35-45): dtable[ids[t], :] += dout[t, :] with fp32
// atomic adds into a zeroed table gradient.
// ============================================================================
template <typename E>
__global__ __launch_bounds__(256) void embed_fwd_kernel(EmbParams p) {
    const int64_t C4 = p.dim / 4;
    const int64_t f = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (f >= p.n_tokens * C4) return;
    const int64_t t = f / C4;
    const int64_t c = 4 * (f % C4);
    const int id = p.ids[t];
    typename E::T* o = (typename E::T*)p.out + t * p.dim + c;
    if (id < 0 || id >= p.vocab) {
        st4(o, f4(NAN));
        return;
    }
    st4(o, ld4((const typename E::T*)p.table + (int64_t)id * p.dim + c));
}

__global__ __launch_bounds__(256) void embed_bwd_kernel(EmbParams p) {
    const int64_t C4 = p.dim / 4;
    const int64_t f = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (f >= p.n_tokens * C4) return;
    const int64_t t = f / C4;
    const int64_t c = 4 * (f % C4);
    const int id = p.ids[t];
    if (id < 0 || id >= p.vocab) return;
    const f32x4 g = *reinterpret_cast<const f32x4*>((const float*)p.dout + t * p.dim + c);
    float* d = (float*)p.out + (int64_t)id * p.dim + c;
    unsafeAtomicAdd(d + 0, g[0]);
    unsafeAtomicAdd(d + 1, g[1]);
    unsafeAtomicAdd(d + 2, g[2]);
    unsafeAtomicAdd(d + 3, g[3]);
}

// Deterministic variant (the library's deterministic mode): workgroup w owns
// vocab rows [w R, w R + R) in an LDS accumulator and walks the tokens in
// order, adding the gradient row of each token whose id falls in its range, so
// every row of dtable is its tokens' sum in token order.  Thread i owns
// columns i, i + 256, ... of every row, so no two threads touch one word.  The
// ids are scanned 256 at a time (one per thread); each wave's matches go to LDS
// as a ballot mask, and the workgroup then takes the matched tokens in order.
__global__ __launch_bounds__(256) void embed_bwd_det_kernel(EmbParams p, int rows_per_wg, int zero_first) {
    extern __shared__ float acc[];  // rows_per_wg * dim
    __shared__ uint64_t s_mask[2][4];
    const int tid = threadIdx.x;
    const int wave = tid >> 6;
    const int64_t v0 = (int64_t)blockIdx.x * rows_per_wg;
    const int rows = (int)min((int64_t)rows_per_wg, p.vocab - v0);
    const int dim = (int)p.dim;
    float* dt = (float*)p.out + v0 * dim;
    for (int r = 0; r < rows; ++r)
        for (int c = tid; c < dim; c += 256) acc[r * dim + c] = zero_first ? 0.f : dt[(int64_t)r * dim + c];
    int buf = 0;
    for (int64_t t0 = 0; t0 < p.n_tokens; t0 += 256, buf ^= 1) {
        const int64_t t = t0 + tid;
        const int id = t < p.n_tokens ? p.ids[t] : -1;
        const int64_t r = (int64_t)id - v0;
        const bool mine = id >= 0 && id < p.vocab && r >= 0 && r < rows;
        const uint64_t m = __ballot(mine);
        if ((tid & 63) == 0) s_mask[buf][wave] = m;
        __syncthreads();  // the masks of this chunk are visible; the other buffer is free again
#pragma unroll
        for (int w = 0; w < 4; ++w) {
            uint64_t mw = s_mask[buf][w];
            while (mw) {
                const int bit = __builtin_ctzll(mw);
                mw &= mw - 1;
                const int64_t tt = t0 + 64 * w + bit;
                const int rr = (int)((int64_t)p.ids[tt] - v0);
                const float* g = (const float*)p.dout + tt * p.dim;
                for (int c = tid; c < dim; c += 256) acc[rr * dim + c] += g[c];
            }
        }
    }
    for (int r = 0; r < rows; ++r)
        for (int c = tid; c < dim; c += 256) dt[(int64_t)r * dim + c] = acc[r * dim + c];
}

// ============================================================================
// AdamW (adamw.h:67-111, one parameter tensor per launch):
//   m = b1 m + (1-b1) g;  v = b2 v + (1-b2) g^2;
//   upd = (m / bc1) / (sqrt(v / bc2) + eps) + wd * p;  p -= lr * upd.
// ============================================================================
// One AdamW element update (cpu_adamw_step_impl, adamw.h:67-111), shared by
// the single- and multi-tensor kernels.  No FMA contraction: every product and
// sum rounds separately, as in the reference's CPU loop, and the two kernels
// cannot round differently.
__device__ __forceinline__ void adamw_elem(float g, float& m, float& v, float& p, float lr, float b1, float b2,
                                           float eps, float wd, float bc1, float bc2) {
#pragma clang fp contract(off)
    m = b1 * m + (1.0f - b1) * g;
    v = b2 * v + (1.0f - b2) * g * g;
    const float mhat = m / bc1;
    const float vhat = v / bc2;
    float upd = mhat / (sqrtf(vhat) + eps);
    if (wd != 0.0f) upd += wd * p;
    p -= lr * upd;
}

template <typename E>
__global__ __launch_bounds__(256) void adamw_kernel(AdamWParams a) {
    const int64_t i = ((int64_t)blockIdx.x * 256 + threadIdx.x) * 4;
    typename E::T* P = (typename E::T*)a.p;
    const typename E::T* G = (const typename E::T*)a.g;
    float* M = a.m;
    float* Vv = a.v;
    auto one = [&](int64_t j) {
        const float g = E::ld(G + j);
        float mi = M[j], vi = Vv[j], pi = E::ld(P + j);
        adamw_elem(g, mi, vi, pi, a.lr, a.beta1, a.beta2, a.eps, a.weight_decay, a.bc1, a.bc2);
        E::st(P + j, pi);
        M[j] = mi;
        Vv[j] = vi;
    };
    if (i + 3 < a.n) {
#pragma unroll
        for (int j = 0; j < 4; ++j) one(i + j);
    } else {
        for (int64_t j = i; j < a.n; ++j) one(j);
    }
}

// Multi-tensor AdamW: 4 elements per thread with 16-byte (fp32) / 8-byte (bf16)
// accesses; every tensor starts 16-byte aligned (checked on the host), so only
// a tensor's last partial group of 4 goes element by element.
template <typename E>
__global__ __launch_bounds__(256) void adamw_multi_kernel(AdamWMultiParams a) {
    const int w = blockIdx.x;
    int t = 0;
    while (t + 1 < a.n_tensors && a.block0[t + 1] <= w) ++t;  // wave-uniform, <= 48 steps
    const int64_t n = a.n[t];
    const int64_t i = ((int64_t)(w - a.block0[t]) * 256 + threadIdx.x) * 4;
    typename E::T* P = (typename E::T*)a.p[t];
    const typename E::T* G = (const typename E::T*)a.g[t];
    float* M = a.m[t];
    float* Vv = a.v[t];
    if (i + 3 < n) {
        const f32x4 g = ld4(G + i);
        f32x4 p = ld4(P + i);
        f32x4 m = *reinterpret_cast<const f32x4*>(M + i);
        f32x4 v = *reinterpret_cast<const f32x4*>(Vv + i);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            float mj = m[j], vj = v[j], pj = p[j];
            adamw_elem(g[j], mj, vj, pj, a.lr, a.beta1, a.beta2, a.eps, a.weight_decay, a.bc1, a.bc2);
            m[j] = mj;
            v[j] = vj;
            p[j] = pj;
        }
        st4(P + i, p);
        *reinterpret_cast<f32x4*>(M + i) = m;
        *reinterpret_cast<f32x4*>(Vv + i) = v;
    } else {
        for (int64_t j = i; j < n; ++j) {
            float mj = M[j], vj = Vv[j], pj = E::ld(P + j);
            adamw_elem(E::ld(G + j), mj, vj, pj, a.lr, a.beta1, a.beta2, a.eps, a.weight_decay, a.bc1, a.bc2);
            E::st(P + j, pj);
            M[j] = mj;
            Vv[j] = vj;
        }
    }
}

// ============================================================================
// Broadcast binary: out[i] = a[i] (op) b[i % nb] (b repeats over leading dims:
// bias over rows, a positional table over the batch).  cuda_add / cuda_multiply
// (cudaadd.cu, cudamultiply.cu) for the trailing-broadcast case.
// ============================================================================
template <typename E, int OP>
__global__ __launch_bounds__(256) void bcast_kernel(const void* __restrict__ a, const void* __restrict__ b,
                                                    void* __restrict__ out, int64_t n, int64_t nb, int vec) {
    const typename E::T* A = (const typename E::T*)a;
    const typename E::T* Bp = (const typename E::T*)b;
    typename E::T* O = (typename E::T*)out;
    const int64_t i = ((int64_t)blockIdx.x * 256 + threadIdx.x) * 4;
    if (vec && i + 3 < n) {
        const f32x4 x = ld4(A + i);
        const f32x4 y = ld4(Bp + (i % nb));
        st4(O + i, OP == 0 ? x + y : x * y);
    } else {
        for (int64_t j = i; j < min(n, i + 4); ++j) {
            const float x = E::ld(A + j), y = E::ld(Bp + (j % nb));
            E::st(O + j, OP == 0 ? x + y : x * y);
        }
    }
}

// ============================================================================
// Row argmax (the greedy next-token pick): one workgroup per row; threads scan
// 4-column groups t, t + 256, ... (16-byte loads when the row allows, several
// in flight) keeping (value, first index); then wave and workgroup reductions
// in which the larger value wins and equal values keep the smaller index.
// ============================================================================
__device__ __forceinline__ void argmax_merge(float& best, int& idx, float ob, int oi) {
    const bool take = oi >= 0 && (idx < 0 || ob > best || (ob == best && oi < idx));
    best = take ? ob : best;
    idx = take ? oi : idx;
}

template <typename E>
__global__ __launch_bounds__(256) void argmax_rows_kernel(const void* __restrict__ x, int64_t cols, int64_t ld,
                                                          int vec, int32_t* __restrict__ out) {
    __shared__ float sb[4];
    __shared__ int si[4];
    const int tid = threadIdx.x;
    const typename E::T* p = (const typename E::T*)x + (int64_t)blockIdx.x * ld;
    float best = -INFINITY;
    int idx = -1;
    if (vec) {
        constexpr int U = 4;  // 4-column groups per thread per step
        for (int64_t c0 = 4 * (int64_t)tid; c0 < cols; c0 += 4 * 256 * U) {
            f32x4 v[U];
#pragma unroll
            for (int u = 0; u < U; ++u) {
                const int64_t c = c0 + 4 * 256 * u;
                v[u] = c < cols ? ld4(p + c) : f32x4{-INFINITY, -INFINITY, -INFINITY, -INFINITY};
            }
#pragma unroll
            for (int u = 0; u < U; ++u)
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const int64_t c = c0 + 4 * 256 * u + j;
                    if (c < cols && (idx < 0 || v[u][j] > best)) {
                        best = v[u][j];
                        idx = (int)c;
                    }
                }
        }
    } else {
        for (int64_t c = tid; c < cols; c += 256) {
            const float v = E::ld(p + c);
            if (idx < 0 || v > best) {
                best = v;
                idx = (int)c;
            }
        }
    }
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) argmax_merge(best, idx, shfl_xor(best, m), __shfl_xor(idx, m, 64));
    if ((tid & 63) == 0) {
        sb[tid >> 6] = best;
        si[tid >> 6] = idx;
    }
    __syncthreads();
    if (tid == 0) {
        for (int w = 1; w < 4; ++w) argmax_merge(best, idx, sb[w], si[w]);
        out[blockIdx.x] = idx;
    }
}

// ============================================================================
// launchers
// ============================================================================
namespace {
inline unsigned blocks_for(int64_t n, int64_t per) { return (unsigned)((n + per - 1) / per); }
}  // namespace

template <typename E>
static int ln_fwd_t(const LnParams& p, hipStream_t s) {
    const dim3 grid(blocks_for(p.rows, 4));
    const int vpt = (p.dim + 255) / 256;
    if (p.vec && vpt <= 16) {
        using T = typename E::T;
        switch (vpt) {
            case 1: hipLaunchKernelGGL((ln_fwd_kernel<1, T>), grid, dim3(256), 0, s, p); break;
            case 2: hipLaunchKernelGGL((ln_fwd_kernel<2, T>), grid, dim3(256), 0, s, p); break;
            case 3: hipLaunchKernelGGL((ln_fwd_kernel<3, T>), grid, dim3(256), 0, s, p); break;
            case 4: hipLaunchKernelGGL((ln_fwd_kernel<4, T>), grid, dim3(256), 0, s, p); break;
            case 5: case 6: case 7: case 8: hipLaunchKernelGGL((ln_fwd_kernel<8, T>), grid, dim3(256), 0, s, p); break;
            default: hipLaunchKernelGGL((ln_fwd_kernel<16, T>), grid, dim3(256), 0, s, p); break;
        }
    } else {
        hipLaunchKernelGGL((ln_fwd_generic_kernel<E>), grid, dim3(256), 0, s, p);
    }
    return (int)hipGetLastError();
}

int launch_ln_fwd(const LnParams& p, int bf16, hipStream_t s) { return bf16 ? ln_fwd_t<BF16>(p, s) : ln_fwd_t<F32>(p, s); }

int ln_bwd_blocks(int64_t rows) {
    const int64_t b = (rows + 3) / 4;
    return (int)(b < kLnBwdMaxBlocks ? b : kLnBwdMaxBlocks);
}

template <typename T>
static int ln_bwd_t(const LnBwdParams& p, hipStream_t s) {
    const int nb = ln_bwd_blocks(p.rows);
    const int vpt = (p.dim + 255) / 256;
    const dim3 grid((unsigned)nb);
    switch (vpt) {
        case 1: hipLaunchKernelGGL((ln_bwd_kernel<1, T>), grid, dim3(256), 0, s, p); break;
        case 2: hipLaunchKernelGGL((ln_bwd_kernel<2, T>), grid, dim3(256), 0, s, p); break;
        case 3: hipLaunchKernelGGL((ln_bwd_kernel<3, T>), grid, dim3(256), 0, s, p); break;
        case 4: hipLaunchKernelGGL((ln_bwd_kernel<4, T>), grid, dim3(256), 0, s, p); break;
        case 5: case 6: case 7: case 8: hipLaunchKernelGGL((ln_bwd_kernel<8, T>), grid, dim3(256), 0, s, p); break;
        default: return (int)hipErrorInvalidValue;  // dim <= kLnBwdMaxDim (checked by the caller)
    }
    const dim3 rgrid(blocks_for(p.dim, 16), 2);  // y: dgamma, dbeta
    hipLaunchKernelGGL(col_reduce_kernel, rgrid, dim3(256), 0, s, p.part, p.dgamma, p.part + (int64_t)nb * p.dim,
                       p.dbeta, (int64_t)nb, (int64_t)p.dim, p.accumulate);
    return (int)hipGetLastError();
}

int launch_ln_bwd(const LnBwdParams& p, int bf16, hipStream_t s) {
    return bf16 ? ln_bwd_t<uint16_t>(p, s) : ln_bwd_t<float>(p, s);
}

int launch_col_sum(const void* x, float* out, float* part, int64_t rows, int64_t cols, int64_t ldx, int accumulate,
                   int bf16, hipStream_t s) {
    const int64_t chunks = col_sum_chunks(rows);
    const dim3 g1(blocks_for(cols, 256), (unsigned)chunks);
    if (bf16)
        hipLaunchKernelGGL(col_partial_kernel<BF16>, g1, dim3(256), 0, s, x, part, rows, cols, ldx);
    else
        hipLaunchKernelGGL(col_partial_kernel<F32>, g1, dim3(256), 0, s, x, part, rows, cols, ldx);
    hipLaunchKernelGGL(col_reduce_kernel, dim3(blocks_for(cols, 16)), dim3(256), 0, s, part, out, part, out, chunks,
                       cols, accumulate);
    return (int)hipGetLastError();
}

int col_sum_chunks(int64_t rows) { return (int)((rows + kColChunk - 1) / kColChunk); }

int launch_gelu_fwd(const void* x, void* y, int64_t n, int bf16, hipStream_t s) {
    const dim3 grid(blocks_for(n, 1024));
    if (bf16)
        hipLaunchKernelGGL(gelu_fwd_kernel<BF16>, grid, dim3(256), 0, s, x, y, n);
    else
        hipLaunchKernelGGL(gelu_fwd_kernel<F32>, grid, dim3(256), 0, s, x, y, n);
    return (int)hipGetLastError();
}

int launch_gelu_bwd(const void* x, const void* dy, void* dx, int64_t n, int bf16, hipStream_t s) {
    const dim3 grid(blocks_for(n, 1024));
    if (bf16)
        hipLaunchKernelGGL(gelu_bwd_kernel<BF16>, grid, dim3(256), 0, s, x, dy, dx, n);
    else
        hipLaunchKernelGGL(gelu_bwd_kernel<F32>, grid, dim3(256), 0, s, x, dy, dx, n);
    return (int)hipGetLastError();
}

int launch_ce_fwd(const CeParams& p, float* loss, int bf16, hipStream_t s) {
    const dim3 grid(blocks_for(p.rows, 4));
    if (bf16)
        hipLaunchKernelGGL(ce_fwd_kernel<BF16>, grid, dim3(256), 0, s, p);
    else
        hipLaunchKernelGGL(ce_fwd_kernel<F32>, grid, dim3(256), 0, s, p);
    hipLaunchKernelGGL(ce_mean_kernel, dim3(1), dim3(256), 0, s, p.row_loss, loss, p.rows);
    return (int)hipGetLastError();
}

int launch_ce_bwd(const CeParams& p, int bf16, hipStream_t s) {
    const dim3 grid(blocks_for(p.rows, 4));
    if (bf16)
        hipLaunchKernelGGL(ce_bwd_kernel<BF16>, grid, dim3(256), 0, s, p);
    else
        hipLaunchKernelGGL(ce_bwd_kernel<F32>, grid, dim3(256), 0, s, p);
    return (int)hipGetLastError();
}

int launch_embed_fwd(const EmbParams& p, int bf16, hipStream_t s) {
    const dim3 grid(blocks_for(p.n_tokens * (p.dim / 4), 256));
    if (bf16)
        hipLaunchKernelGGL(embed_fwd_kernel<BF16>, grid, dim3(256), 0, s, p);
    else
        hipLaunchKernelGGL(embed_fwd_kernel<F32>, grid, dim3(256), 0, s, p);
    return (int)hipGetLastError();
}

int launch_embed_bwd(const EmbParams& p, hipStream_t s) {
    const dim3 grid(blocks_for(p.n_tokens * (p.dim / 4), 256));
    hipLaunchKernelGGL(embed_bwd_kernel, grid, dim3(256), 0, s, p);
    return (int)hipGetLastError();
}

int launch_embed_bwd_det(const EmbParams& p, int zero_first, hipStream_t s) {
    // rows per workgroup: up to 64 KB of LDS accumulator, at most 32 rows
    const int rows = (int)std::max<int64_t>(1, std::min<int64_t>(32, 16384 / p.dim));
    const size_t lds = (size_t)rows * p.dim * sizeof(float);
    if (lds > 65536) return (int)hipErrorInvalidValue;
    hipLaunchKernelGGL(embed_bwd_det_kernel, dim3(blocks_for(p.vocab, rows)), dim3(256), lds, s, p, rows,
                       zero_first ? 1 : 0);
    return (int)hipGetLastError();
}

int launch_adamw(const AdamWParams& a, int bf16, hipStream_t s) {
    const dim3 grid(blocks_for(a.n, 1024));
    if (bf16)
        hipLaunchKernelGGL(adamw_kernel<BF16>, grid, dim3(256), 0, s, a);
    else
        hipLaunchKernelGGL(adamw_kernel<F32>, grid, dim3(256), 0, s, a);
    return (int)hipGetLastError();
}

int launch_adamw_multi(const AdamWMultiParams& a, int bf16, hipStream_t s) {
    const dim3 grid((unsigned)a.block0[a.n_tensors]);
    if (bf16)
        hipLaunchKernelGGL(adamw_multi_kernel<BF16>, grid, dim3(256), 0, s, a);
    else
        hipLaunchKernelGGL(adamw_multi_kernel<F32>, grid, dim3(256), 0, s, a);
    return (int)hipGetLastError();
}

int launch_argmax_rows(const void* x, int64_t rows, int64_t cols, int64_t ld, int32_t* out, int bf16,
                       hipStream_t s) {
    const size_t align = bf16 ? 8 : 16;
    const int vec = cols % 4 == 0 && ld % 4 == 0 && reinterpret_cast<uintptr_t>(x) % align == 0;
    const dim3 grid((unsigned)rows);
    if (bf16)
        hipLaunchKernelGGL(argmax_rows_kernel<BF16>, grid, dim3(256), 0, s, x, cols, ld, vec, out);
    else
        hipLaunchKernelGGL(argmax_rows_kernel<F32>, grid, dim3(256), 0, s, x, cols, ld, vec, out);
    return (int)hipGetLastError();
}

int launch_bcast(int op, const void* a, const void* b, void* out, int64_t n, int64_t nb, int vec, int bf16,
                 hipStream_t s) {
    const dim3 grid(blocks_for(n, 1024));
    if (bf16) {
        if (op == 0)
            hipLaunchKernelGGL((bcast_kernel<BF16, 0>), grid, dim3(256), 0, s, a, b, out, n, nb, vec);
        else
            hipLaunchKernelGGL((bcast_kernel<BF16, 1>), grid, dim3(256), 0, s, a, b, out, n, nb, vec);
    } else {
        if (op == 0)
            hipLaunchKernelGGL((bcast_kernel<F32, 0>), grid, dim3(256), 0, s, a, b, out, n, nb, vec);
        else
            hipLaunchKernelGGL((bcast_kernel<F32, 1>), grid, dim3(256), 0, s, a, b, out, n, nb, vec);
    }
    return (int)hipGetLastError();
}

}  // namespace inf
