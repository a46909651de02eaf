// decode.hip -- single-query attention against a KV cache (memory-bound).
//
// Work split: workgroup (bh, split) streams `chunk` consecutive cached keys of
// one (b, h).  D/4 lanes share a key row (one 16-byte load each) and form a
// key group; the workgroup's 256/(D/4) groups take interleaved keys, so the
// groups of one wave read consecutive rows (one wave instruction = 1 KB of
// contiguous K or V); the row dot product is reduced inside the group with DPP
// row operations.  Each group runs its own online softmax over U = 4 keys
// per step with the K and V loads of the step issued together, so nothing
// waits on a workgroup barrier inside the stream.  The groups are merged in the
// wave and then across the four waves in LDS; with one split the workgroup
// writes O itself, otherwise it writes its (max, sum, unnormalised o) and
// decode_combine merges the splits of a row.  (Merging in the last-arriving
// split instead needs device-scope release/acquire fences per workgroup, which
// measured 20x slower on MI355X.)
// Scores are in the log2 domain (q is pre-scaled by scale * log2 e).  No key
// is masked: the query sits at the end of the cache, so the causal rule
// j <= i + (Tk - 1) admits all of them (InfernoApp/main.cpp:747-748, Tq = 1).
#include <mutex>

#include "common.h"
#include "kernels.h"

namespace inf {

constexpr int kDecodeU = 4;  // keys per group per step

// Scratch of inf_attn_decode_static: the split partials (B*H*nsplit*(D+2)
// floats) in a file-scope device array instead of a caller's workspace.  Every
// device the library runs on holds its own copy at its own address until the
// process ends.  In host code the array's name is only a stand-in: the
// kernels get the device address hipGetSymbolAddress returns with that device
// current, looked up once per device and kept.  Calls that overlap on one
// device share the array and race.
static __device__ __align__(256) float scratch[kDecodeScratchBytes / sizeof(float)];

namespace {
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
float* g_scratch[kMaxDevices] = {};
}  // namespace

int decode_scratch(float** out) {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return (int)e;
    if (dev < 0 || dev >= kMaxDevices) return (int)hipErrorInvalidDevice;
    std::lock_guard<std::mutex> lk(g_scratch_mu);
    if (!g_scratch[dev]) {
        void* ptr = nullptr;
        e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
        if (e != hipSuccess) return (int)e;
        g_scratch[dev] = static_cast<float*>(ptr);
    }
    *out = g_scratch[dev];
    return 0;
}

template <typename E>
__device__ __forceinline__ void store_out(E* dst, float v) {
    if constexpr (sizeof(E) == 4)
        *dst = v;
    else
        *dst = f32_to_bf16(v);
}

template <int D, typename E>
__global__ __launch_bounds__(256) void decode_split_kernel(DecodeParams p) {
    constexpr int TPK = D / 4;     // lanes per key row
    constexpr int NG = 256 / TPK;  // key groups per workgroup
    constexpr int U = kDecodeU;
    __shared__ float m_s[4];
    __shared__ float l_s[4];
    __shared__ __attribute__((aligned(16))) float o_s[4][D + 4];

    const int tid = threadIdx.x;
    const int grp = tid / TPK;
    const int c4 = tid % TPK;
    const int split = blockIdx.x % p.nsplit;
    const int bh = blockIdx.x / p.nsplit;
    const int b = bh / p.H, h = bh % p.H;
    const int j0 = split * p.chunk;
    const int j1 = min(p.Tk, j0 + p.chunk);

    const E* K = (const E*)p.k + b * p.sk.b + h * p.sk.h + 4 * c4;
    const E* V = (const E*)p.v + b * p.sv.b + h * p.sv.h + 4 * c4;
    const f32x4 q4 = ld4((const E*)p.q + b * p.sq.b + h * p.sq.h + 4 * c4) * p.c;

    float m = -INFINITY, l = 0.f;
    f32x4 acc = f32x4{0.f, 0.f, 0.f, 0.f};
    const int steps = (p.chunk + NG * U - 1) / (NG * U);
    for (int it = 0; it < steps; ++it) {
        f32x4 kr[U], vr[U];
        int jj[U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            jj[u] = j0 + (it * U + u) * NG + grp;
            if (jj[u] < j1) {
                kr[u] = ld4_nt(K + (int64_t)jj[u] * p.sk.t);
                vr[u] = ld4_nt(V + (int64_t)jj[u] * p.sv.t);
            } else {
                kr[u] = vr[u] = f32x4{0.f, 0.f, 0.f, 0.f};
            }
        }
        float s[U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const float d = group_sum<TPK>(q4[0] * kr[u][0] + q4[1] * kr[u][1] + q4[2] * kr[u][2] +
                                           q4[3] * kr[u][3]);
            s[u] = (jj[u] < j1) ? d : -INFINITY;
        }
        float mx = m;
#pragma unroll
        for (int u = 0; u < U; ++u) mx = fmaxf(mx, s[u]);
        const float mref = (mx == -INFINITY) ? 0.f : mx;  // no valid key yet: keep everything at 0
        const float alpha = fast_exp2(m - mref);
        acc *= alpha;
        l *= alpha;
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const float pu = fast_exp2(s[u] - mref);
            l += pu;
            acc += pu * vr[u];
        }
        m = mx;
    }

    // Merge the key groups: first the groups of each wave (lanes l, l^16, l^32,
    // l^48 hold the same head-dim slice), then the four waves through LDS.
    float mw = m;
#pragma unroll
    for (int msk = TPK; msk < 64; msk <<= 1) mw = fmaxf(mw, shfl_xor(mw, msk));
    const float wref = (mw == -INFINITY) ? 0.f : mw;
    const float sc = fast_exp2(m - wref);  // a group without keys has m = -inf -> 0
    acc *= sc;
    l *= sc;
#pragma unroll
    for (int msk = TPK; msk < 64; msk <<= 1) {
        acc[0] += shfl_xor(acc[0], msk);
        acc[1] += shfl_xor(acc[1], msk);
        acc[2] += shfl_xor(acc[2], msk);
        acc[3] += shfl_xor(acc[3], msk);
        l += shfl_xor(l, msk);
    }
    const int wave = tid >> 6, lane = tid & 63;
    if (lane < TPK) {
        if (lane == 0) {
            m_s[wave] = mw;
            l_s[wave] = l;
        }
        *reinterpret_cast<f32x4*>(&o_s[wave][4 * lane]) = acc;
    }
    __syncthreads();
    if (tid < D) {
        float M = fmaxf(fmaxf(m_s[0], m_s[1]), fmaxf(m_s[2], m_s[3]));
        float L = 0.f, o = 0.f;
#pragma unroll
        for (int w = 0; w < 4; ++w) {
            const float wt = fast_exp2(m_s[w] - M);
            L += l_s[w] * wt;
            o += o_s[w][tid] * wt;
        }
        if (p.nsplit == 1) {
            store_out<E>((E*)p.o + b * p.so.b + h * p.so.h + tid, o / L);
        } else {
            float* out = p.part + ((int64_t)bh * p.nsplit + split) * (D + 2);
            out[tid] = o;
            if (tid == 0) {
                out[D] = M;
                out[D + 1] = L;
            }
        }
    }
}

// Merge the splits of one row: each wave reads every split's (max, sum) at
// once (lane s holds split s; at most 64 splits) and wave 0 publishes the split
// weights in LDS; then lane d sums o[d] over the splits with all loads
// independent of each other.
template <int D, typename E>
__global__ __launch_bounds__(D > 64 ? D : 64) void decode_combine_kernel(DecodeParams p) {
    __shared__ float wsh[64];
    const int bh = blockIdx.x;
    const int b = bh / p.H, h = bh % p.H;
    const int t = threadIdx.x;
    const int lane = t & 63;
    const int ns = p.nsplit;
    const float* part = p.part + (int64_t)bh * ns * (D + 2);
    float ms = -INFINITY, ls = 0.f;
    if (lane < ns) {
        ms = part[lane * (D + 2) + D];
        ls = part[lane * (D + 2) + D + 1];
    }
    const float M = wave_max(ms);
    const float w = (lane < ns) ? fast_exp2(ms - M) : 0.f;
    const float L = wave_sum(ls * w);
    if (t < 64) wsh[lane] = w;
    __syncthreads();
    if (t < D) {
        float o = 0.f;
#pragma unroll 8
        for (int sp = 0; sp < ns; ++sp) o += part[sp * (D + 2) + t] * wsh[sp];
        store_out<E>((E*)p.o + b * p.so.b + h * p.so.h + t, o / L);
    }
}

template <int D, typename E>
static int launch_dec_t(const DecodeParams& p, hipStream_t s) {
    hipLaunchKernelGGL((decode_split_kernel<D, E>), dim3((unsigned)(p.B * p.H * p.nsplit)), dim3(256), 0, s, p);
    if (p.nsplit > 1)
        hipLaunchKernelGGL((decode_combine_kernel<D, E>), dim3((unsigned)(p.B * p.H)), dim3(D > 64 ? D : 64), 0, s,
                           p);
    return (int)hipGetLastError();
}

int launch_attn_decode(const DecodeParams& p, int bf16, hipStream_t s) {
    switch (p.D) {
        case 32: return bf16 ? launch_dec_t<32, uint16_t>(p, s) : launch_dec_t<32, float>(p, s);
        case 64: return bf16 ? launch_dec_t<64, uint16_t>(p, s) : launch_dec_t<64, float>(p, s);
        case 128: return bf16 ? launch_dec_t<128, uint16_t>(p, s) : launch_dec_t<128, float>(p, s);
        default: return (int)hipErrorInvalidValue;
    }
}

// Splits per row: the smallest power of two giving >= 4096 workgroups (16 per
// CU), capped at 64 (the combine holds one split per lane) and so that every
// split holds at least one step of every group.  Many
// short splits stream best: reading config 5's 402.8 MB with 16 splits per
// row measured 6.33 TB/s against 5.87 TB/s with 4, and 5.5 TB/s with one
// 1024-thread workgroup per row.
void decode_plan(int B, int H, int Tk, int D, int* nsplit, int* chunk) {
    const int ng = 256 / (D / 4);
    const int step = ng * kDecodeU;
    const int64_t bh = (int64_t)B * H;
    int max_split = (Tk + step - 1) / step;
    if (max_split < 1) max_split = 1;
    int ns = 1;
    while (bh * ns < 4096 && ns * 2 <= max_split && ns < 64) ns *= 2;
    int ch = (Tk + ns - 1) / ns;
    ch = (ch + step - 1) / step * step;
    *nsplit = (Tk + ch - 1) / ch;
    *chunk = ch;
}

}  // namespace inf
