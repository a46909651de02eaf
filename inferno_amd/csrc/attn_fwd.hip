// attn_fwd.hip -- fused causal attention forward for gfx950.
//
// One workgroup = 4 waves = 128 query rows of one (b, h); each wave owns 32
// rows for the whole kernel.  K and V tiles of BN keys are streamed through
// LDS (double-buffered, one barrier per tile, the next tile's global loads in
// flight in registers while the current one is consumed).  Per wave and tile:
//
//   S^T (keys x queries) = K Q^T      v_mfma_f32_32x32x2_f32, A = K from LDS,
//                                     B = Q^T resident in VGPRs
//   online softmax on S^T             query = lane%32, so the row max needs one
//                                     xor-32 exchange; the row sum stays
//                                     per-lane until the end
//   O^T (d x queries) += V^T P^T      A = V^T from LDS, B = P^T straight from
//                                     the S^T accumulators (reduction index
//                                     permuted to match their layout)
//
// V is stored transposed in LDS (Vt[d][key]) so that the four keys a lane
// feeds to four consecutive MFMAs are adjacent: one ds_read_b128 per four
// MFMAs in both products, issued well ahead of use, instead of a dependent
// ds_read_b32 per MFMA.  V tiles are fetched with a row-fastest lane mapping
// (16 keys x 4 column chunks per wave) so the transposing LDS stores hit 64
// distinct banks.
//
// Keeping queries on the lane axis in both products is what lets P stay in
// registers.  The scale is folded into exp2: p = exp2(s*c - m*c) with
// c = scale*log2(e).  Masked scores (key > query + Tk - Tq, or key >= Tk)
// become -inf, so their probabilities are exactly 0, as the reference's
// -1e9f fill followed by exp((double)(-1e9 - max)) is.  The row
// log-sum-exp (natural log) is stored for the backward pass.
//
// Scheduling: workgroup w takes query tile (n_qtiles - 1 - w / (B*H)) of head
// w % (B*H), so the longest causal rows start first; when B*H is a multiple
// of 8, all tiles of a head land on the same XCD (dispatch is round-robin
// over the 8 XCDs), so a head's K/V is fetched into one L2.
#include "common.h"
#include "kernels.h"

namespace inf {

template <int D>
struct FwdTile {
    static constexpr int BN = (D >= 128) ? 32 : 64;  // keys per LDS tile
    static constexpr int KS = D + 4;                 // K row stride in LDS (floats)
    static constexpr int VTS = BN + 4;               // V^T row stride in LDS (floats)
};

template <int D, typename E>
__global__ __launch_bounds__(256, 2) void attn_fwd_kernel(FwdParams p) {
    constexpr int BM = kFwdBM;
    constexpr int BN = FwdTile<D>::BN;
    constexpr int KS = FwdTile<D>::KS;
    constexpr int VTS = FwdTile<D>::VTS;
    constexpr int HD = D / 2;        // reduction elements per lane half
    constexpr int NKB = BN / 32;     // 32-key blocks per tile
    constexpr int NDB = D / 32;      // 32-wide head-dim blocks
    constexpr int C4 = D / 4;        // 4-element chunks per row
    constexpr int LPT = BN * C4 / 256;  // 4-element loads per thread per tensor per tile

    __shared__ __attribute__((aligned(16))) float Ks[2][BN][KS];
    __shared__ __attribute__((aligned(16))) float Vt[2][D][VTS];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int l32 = lane & 31;
    const int g = lane >> 5;

    const int BH = p.B * p.H;
    const int w = blockIdx.x;
    const int qtile = p.n_qtiles - 1 - w / BH;
    const int bh = w % BH;
    const int b = bh / p.H;
    const int h = bh % p.H;

    const E* Q = (const E*)p.q + b * p.sq.b + h * p.sq.h;
    const E* K = (const E*)p.k + b * p.sk.b + h * p.sk.h;
    const E* V = (const E*)p.v + b * p.sv.b + h * p.sv.h;
    E* O = (E*)p.o + b * p.so.b + h * p.so.h;

    const int q0w = qtile * BM + wave * 32;  // first query row of this wave
    const int qrow = q0w + l32;              // this lane's query row

    // Q^T operand: lane (l32, g) holds Q[qrow][g*HD + i], i = 0..HD-1.
    float qf[HD];
    if (qrow < p.Tq) {
        const E* src = Q + (int64_t)qrow * p.sq.t + g * HD;
#pragma unroll
        for (int i = 0; i < HD; i += 4) {
            f32x4 t = ld4(src + i);
            qf[i] = t[0];
            qf[i + 1] = t[1];
            qf[i + 2] = t[2];
            qf[i + 3] = t[3];
        }
    } else {
#pragma unroll
        for (int i = 0; i < HD; ++i) qf[i] = 0.f;
    }

    // Keys this workgroup needs, and this wave's visible limit (exclusive).
    int kv_end = p.Tk;
    if (p.causal) kv_end = min(p.Tk, qtile * BM + BM + p.off);
    const int n_tiles = (kv_end + BN - 1) / BN;
    const int wave_kend = p.causal ? min(kv_end, q0w + 32 + p.off) : kv_end;

    // K: chunk f -> (row f / C4, column chunk f % C4), row-major 16-byte loads.
    // V: chunk f -> (row f % 16 + 16 * (f / (16 * C4)), column chunk (f / 16) % C4).
    f32x4 kr[LPT], vr[LPT];
    auto gload = [&](int t) {
#pragma unroll
        for (int i = 0; i < LPT; ++i) {
            const int f = tid + 256 * i;
            const int krow = t * BN + f / C4;
            const int vrow = t * BN + (f & 15) + 16 * (f / (16 * C4));
            kr[i] = f32x4{0.f, 0.f, 0.f, 0.f};
            vr[i] = f32x4{0.f, 0.f, 0.f, 0.f};
            if (krow < p.Tk) kr[i] = ld4(K + (int64_t)krow * p.sk.t + 4 * (f % C4));
            if (vrow < p.Tk) vr[i] = ld4(V + (int64_t)vrow * p.sv.t + 4 * ((f >> 4) % C4));
        }
    };
    auto sstore = [&](int buf) {
#pragma unroll
        for (int i = 0; i < LPT; ++i) {
            const int f = tid + 256 * i;
            *reinterpret_cast<f32x4*>(&Ks[buf][f / C4][4 * (f % C4)]) = kr[i];
            const int vrow = (f & 15) + 16 * (f / (16 * C4));
            const int vc = 4 * ((f >> 4) % C4);
            Vt[buf][vc + 0][vrow] = vr[i][0];
            Vt[buf][vc + 1][vrow] = vr[i][1];
            Vt[buf][vc + 2][vrow] = vr[i][2];
            Vt[buf][vc + 3][vrow] = vr[i][3];
        }
    };

    f32x16 o[NDB];
#pragma unroll
    for (int i = 0; i < NDB; ++i) o[i] = f32x16{};
    float m_run = -INFINITY;  // running max of raw scores for row qrow
    float l_run = 0.f;        // this lane's partial sum of p (its half of the keys)
    const float c = p.c;

    gload(0);
    sstore(0);
    __syncthreads();

    for (int t = 0; t < n_tiles; ++t) {
        const int buf = t & 1;
        const int k0 = t * BN;
        if (t + 1 < n_tiles) gload(t + 1);

        if (k0 < wave_kend) {
            // ---- S^T = K Q^T --------------------------------------------------
            f32x16 s[NKB];
#pragma unroll
            for (int kb = 0; kb < NKB; ++kb) s[kb] = f32x16{};
#pragma unroll
            for (int i = 0; i < HD; i += 4) {
#pragma unroll
                for (int kb = 0; kb < NKB; ++kb) {
                    const f32x4 a =
                        *reinterpret_cast<const f32x4*>(&Ks[buf][kb * 32 + l32][g * HD + i]);
                    s[kb] = mfma32x32x2(a[0], qf[i + 0], s[kb]);
                    s[kb] = mfma32x32x2(a[1], qf[i + 1], s[kb]);
                    s[kb] = mfma32x32x2(a[2], qf[i + 2], s[kb]);
                    s[kb] = mfma32x32x2(a[3], qf[i + 3], s[kb]);
                }
            }

            // ---- mask, online softmax ------------------------------------------
            const bool need_mask =
                (k0 + BN > p.Tk) || (p.causal && (k0 + BN - 1 > q0w + p.off));
            if (need_mask) {
                const int lim = p.causal ? min(p.Tk - 1, qrow + p.off) : p.Tk - 1;
#pragma unroll
                for (int kb = 0; kb < NKB; ++kb)
#pragma unroll
                    for (int r = 0; r < 16; ++r) {
                        const int key = k0 + kb * 32 + 8 * (r >> 2) + 4 * g + (r & 3);
                        if (key > lim) s[kb][r] = -INFINITY;
                    }
            }
            float mloc = -INFINITY;
#pragma unroll
            for (int kb = 0; kb < NKB; ++kb)
#pragma unroll
                for (int r = 0; r < 16; ++r) mloc = fmaxf(mloc, s[kb][r]);
            mloc = fmaxf(mloc, shfl_xor(mloc, 32));
            const float m_new = fmaxf(m_run, mloc);
            const float alpha = fast_exp2((m_run - m_new) * c);  // m_run = -inf -> 0
            const float mc = m_new * c;
            float lsum = 0.f;
#pragma unroll
            for (int kb = 0; kb < NKB; ++kb)
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const float e = fast_exp2(fmaf(s[kb][r], c, -mc));
                    s[kb][r] = e;
                    lsum += e;
                }
            l_run = fmaf(l_run, alpha, lsum);
            m_run = m_new;
#pragma unroll
            for (int db = 0; db < NDB; ++db) o[db] *= alpha;

            // ---- O^T += V^T P^T --------------------------------------------------
            // reg 4j+cc of s[kb] holds key kb*32 + 8j + 4g + cc
#pragma unroll
            for (int kb = 0; kb < NKB; ++kb)
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    f32x4 va[NDB];
#pragma unroll
                    for (int db = 0; db < NDB; ++db)
                        va[db] = *reinterpret_cast<const f32x4*>(
                            &Vt[buf][db * 32 + l32][kb * 32 + 8 * j + 4 * g]);
#pragma unroll
                    for (int cc = 0; cc < 4; ++cc)
#pragma unroll
                        for (int db = 0; db < NDB; ++db)
                            o[db] = mfma32x32x2(va[db][cc], s[kb][4 * j + cc], o[db]);
                }
        }

        if (t + 1 < n_tiles) sstore(buf ^ 1);
        __syncthreads();
    }

    // ---- epilogue ---------------------------------------------------------------
    const float l_tot = l_run + shfl_xor(l_run, 32);
    const float inv = 1.f / l_tot;
    if (qrow < p.Tq) {
        E* dst = O + (int64_t)qrow * p.so.t;
#pragma unroll
        for (int db = 0; db < NDB; ++db)
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                f32x4 val;
                val[0] = o[db][4 * j + 0] * inv;
                val[1] = o[db][4 * j + 1] * inv;
                val[2] = o[db][4 * j + 2] * inv;
                val[3] = o[db][4 * j + 3] * inv;
                st4(dst + db * 32 + 8 * j + 4 * g, val);
            }
        if (g == 0 && p.lse) p.lse[(int64_t)bh * p.Tq + qrow] = m_run * p.scale + logf(l_tot);
    }
}

template <int D, typename E>
static int launch_fwd_t(const FwdParams& p, hipStream_t s) {
    const dim3 grid((unsigned)(p.n_qtiles * p.B * p.H));
    hipLaunchKernelGGL((attn_fwd_kernel<D, E>), grid, dim3(256), 0, s, p);
    return (int)hipGetLastError();
}

int launch_attn_fwd(const FwdParams& p, int bf16, hipStream_t s) {
    if (bf16) return launch_attn_fwd_bf16(p, s);
    switch (p.D) {
        case 32: return launch_fwd_t<32, float>(p, s);
        case 64: return launch_fwd_t<64, float>(p, s);
        case 128: return launch_fwd_t<128, float>(p, s);
        default: return (int)hipErrorInvalidValue;
    }
}

}  // namespace inf
