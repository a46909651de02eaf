// decode.hip -- single-query attention against a KV cache (memory-bound).
//
// Split-KV: workgroup (bh, split) reads kDecodeChunk = 256 consecutive cached
// keys of one (b, h).  D/4 threads share a key row (one 16-byte load each, so a
// wave instruction covers 64*16 B of contiguous rows); every thread issues all
// of its K loads before consuming any, and all of its V loads before the
// chunk's max / sum reductions.  Scores live in LDS; the chunk's
// max m, sum l = sum_j exp2(s_j - m) and unnormalised o = sum_j p_j v_j are
// written to the workspace, and decode_combine merges the splits of a row
// with the usual log-sum-exp rescale.  No key is masked: the query sits at
// the end of the cache, so the causal rule j <= i + (Tk - 1) admits all of
// them (InfernoApp/main.cpp:747-748 with Tq = 1).
#include "common.h"
#include "kernels.h"

namespace inf {

template <int D, typename E>
__global__ __launch_bounds__(256) void decode_split_kernel(DecodeParams p) {
    constexpr int TPK = D / 4;             // threads per key row
    constexpr int KPP = 256 / TPK;         // keys per pass
    constexpr int CH = kDecodeChunk;
    constexpr int NP = CH / KPP;           // passes per chunk
    __shared__ float sc[CH];
    __shared__ float red[4];
    __shared__ __attribute__((aligned(16))) float ored[KPP][D + 4];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int kg = tid / TPK;
    const int c4 = tid % TPK;
    const int split = blockIdx.x % p.nsplit;
    const int bh = blockIdx.x / p.nsplit;
    const int b = bh / p.H, h = bh % p.H;
    const int j0 = split * CH;
    const int j1 = min(p.Tk, j0 + CH);

    const E* K = (const E*)p.k + b * p.sk.b + h * p.sk.h;
    const E* V = (const E*)p.v + b * p.sv.b + h * p.sv.h;
    const f32x4 q4 = ld4((const E*)p.q + b * p.sq.b + h * p.sq.h + 4 * c4);

    // All K loads first; the V loads go out right after the scores, so they are
    // in flight during the max / sum reductions.  Peak live data: NP x 16 B.
    f32x4 r4[NP];
#pragma unroll
    for (int i = 0; i < NP; ++i) {
        const int j = j0 + i * KPP + kg;
        r4[i] = (j < j1) ? ld4(K + (int64_t)j * p.sk.t + 4 * c4) : f32x4{0.f, 0.f, 0.f, 0.f};
    }

    // scores (log2 domain)
#pragma unroll
    for (int i = 0; i < NP; ++i) {
        float s = q4[0] * r4[i][0] + q4[1] * r4[i][1] + q4[2] * r4[i][2] + q4[3] * r4[i][3];
#pragma unroll
        for (int m = TPK / 2; m >= 1; m >>= 1) s += shfl_xor(s, m);
        const int j = j0 + i * KPP + kg;
        if (c4 == 0) sc[i * KPP + kg] = (j < j1) ? s * p.c : -INFINITY;
    }
#pragma unroll
    for (int i = 0; i < NP; ++i) {
        const int j = j0 + i * KPP + kg;
        r4[i] = (j < j1) ? ld4(V + (int64_t)j * p.sv.t + 4 * c4) : f32x4{0.f, 0.f, 0.f, 0.f};
    }
    __syncthreads();

    // chunk max
    float mx = wave_max(sc[tid]);
    if (lane == 0) red[wave] = mx;
    __syncthreads();
    mx = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    __syncthreads();
    // chunk sum
    const float e_t = fast_exp2(sc[tid] - mx);
    float sm = wave_sum(e_t);
    if (lane == 0) red[wave] = sm;

    // o partial over this thread's keys
    f32x4 acc = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int i = 0; i < NP; ++i) {
        const float pj = fast_exp2(sc[i * KPP + kg] - mx);
        acc += pj * r4[i];
    }
    *reinterpret_cast<f32x4*>(&ored[kg][4 * c4]) = acc;
    __syncthreads();

    float* out = p.part + ((int64_t)bh * p.nsplit + split) * (D + 2);
    if (tid < D) {
        float o = 0.f;
#pragma unroll 8
        for (int r = 0; r < KPP; ++r) o += ored[r][tid];
        out[tid] = o;
    }
    if (tid == 0) {
        out[D] = mx;
        out[D + 1] = red[0] + red[1] + red[2] + red[3];
    }
}

template <int D, typename E>
__global__ __launch_bounds__(128) void decode_combine_kernel(DecodeParams p) {
    const int bh = blockIdx.x;
    const int b = bh / p.H, h = bh % p.H;
    const int d = threadIdx.x;
    const float* part = p.part + (int64_t)bh * p.nsplit * (D + 2);
    float M = -INFINITY;
    for (int s = 0; s < p.nsplit; ++s) M = fmaxf(M, part[s * (D + 2) + D]);
    float L = 0.f, o = 0.f;
    for (int s = 0; s < p.nsplit; ++s) {
        const float wgt = fast_exp2(part[s * (D + 2) + D] - M);
        L += part[s * (D + 2) + D + 1] * wgt;
        if (d < D) o += part[s * (D + 2) + d] * wgt;
    }
    if (d < D) {
        E* dst = (E*)p.o + b * p.so.b + h * p.so.h + d;
        if (sizeof(E) == 4)
            *(float*)dst = o / L;
        else
            *(uint16_t*)dst = f32_to_bf16(o / L);
    }
}

template <int D, typename E>
static int launch_dec_t(const DecodeParams& p, hipStream_t s) {
    hipLaunchKernelGGL((decode_split_kernel<D, E>), dim3((unsigned)(p.B * p.H * p.nsplit)),
                       dim3(256), 0, s, p);
    hipLaunchKernelGGL((decode_combine_kernel<D, E>), dim3((unsigned)(p.B * p.H)), dim3(128), 0,
                       s, p);
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

}  // namespace inf
