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
// Scheduling: dispatch group g = w / (B*H) of head w % (B*H).  Without a
// split plan, group g is query tile n_qtiles - 1 - g, so the longest causal
// rows start first; when B*H is a multiple of 8, all tiles of a head land on
// the same XCD (dispatch is round-robin over the 8 XCDs), so a head's K/V is
// fetched into one L2.  With a split plan (fwd_plan, causal shapes whose
// heaviest query tiles would otherwise set the makespan), the heaviest query
// tiles' key ranges are cut into chunks run by separate groups, the groups are
// ordered heaviest first, and each chunk leaves (unnormalised O, row max, row
// sum) in a workspace slot that attn_fwd_merge_kernel combines with the same
// log-sum-exp weighting as the decode combine.
#include <algorithm>
#include <array>
#include <functional>
#include <map>
#include <mutex>
#include <vector>

#include "common.h"
#include "kernels.h"

namespace inf {

template <int D>
struct FwdTile {
    static constexpr int BN = (D >= 128) ? 32 : 64;  // keys per LDS tile
    static constexpr int KS = D + 4;                 // K row stride in LDS (floats)
    static constexpr int VTS = BN + 4;               // V^T row stride in LDS (floats)
    // Software-pipelined loop (two score blocks live): fits two waves per
    // SIMD up to D = 64; D = 128 keeps one score block.
    static constexpr bool PIPE = D <= 64;
    // V chunk f of a tile: row and first column (elements) within the tile.
    static constexpr int vrow(int f) { return (f & 15) + 16 * (f / (16 * (D / 4))); }
    static constexpr int vcol(int f) { return 4 * ((f >> 4) % (D / 4)); }
    // Chunk tid + 256 i sits at (row, column) of chunk tid plus that of chunk
    // 256 i, for K and V, for every thread and load of a tile.
    static constexpr bool chunks_split() {
        constexpr int C4 = D / 4, LPT = BN * C4 / 256;
        for (int i = 0; i < LPT; ++i)
            for (int tid = 0; tid < 256; ++tid) {
                const int f = tid + 256 * i;
                if (f / C4 != tid / C4 + 256 * i / C4 || f % C4 != tid % C4) return false;
                if (vrow(f) != vrow(tid) + vrow(256 * i) || vcol(f) != vcol(tid) + vcol(256 * i)) return false;
            }
        return true;
    }
};

// Headroom of the forward's lazy rescaling, in exp2 units: P <= 2^8.
constexpr float kLazyLog2 = 8.f;

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
    int qtile, t_begin = 0, t_end = 0x7fffffff, slot = -1;
    if (p.n_groups) {
        const FwdGroup grp = p.groups[w / BH];
        qtile = grp.qt;
        t_begin = grp.t0;
        t_end = grp.t1;
        slot = grp.slot;
    } else {
        qtile = p.n_qtiles - 1 - w / BH;
    }
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
    const int n_tiles = min((kv_end + BN - 1) / BN, t_end);
    const int wave_kend = p.causal ? min(kv_end, q0w + 32 + p.off) : kv_end;

    // K: chunk f -> (row f / C4, column chunk f % C4), row-major 16-byte loads.
    // V: chunk f -> (row f % 16 + 16 * (f / (16 * C4)), column chunk (f / 16) % C4).
    // Loads go through a buffer resource per tile: each chunk's offset is a
    // per-thread part (chunk tid) plus a uniform part (chunk 256 i), and rows
    // at or past `lim` (<= Tk) are outside the resource and read as zeros, so
    // a load costs no address arithmetic, compare or branch.
    static_assert(FwdTile<D>::chunks_split(), "chunk offsets must split into thread + load parts");
    static_assert(sizeof(E) == 4, "fp32 storage (bf16 has its own kernel)");
    f32x4 kr[LPT], vr[LPT];
    const uint32_t k_voff = (uint32_t)(((int64_t)(tid / C4) * p.sk.t + 4 * (tid % C4)) * 4);
    const uint32_t v_voff = (uint32_t)(((int64_t)FwdTile<D>::vrow(tid) * p.sv.t + FwdTile<D>::vcol(tid)) * 4);
    auto gload_k = [&](int t, int lim) {
        const auto rs = row_rsrc((const float*)K, p.sk.t, t * BN, min(lim - t * BN, BN), D);
#pragma unroll
        for (int i = 0; i < LPT; ++i)
            kr[i] = buffer_ld4(rs, k_voff, (uint32_t)(((int64_t)(256 * i / C4) * p.sk.t) * 4));
    };
    auto gload_v = [&](int t, int lim) {
        const auto rs = row_rsrc((const float*)V, p.sv.t, t * BN, min(lim - t * BN, BN), D);
#pragma unroll
        for (int i = 0; i < LPT; ++i)
            vr[i] = buffer_ld4(rs, v_voff,
                               (uint32_t)(((int64_t)FwdTile<D>::vrow(256 * i) * p.sv.t + FwdTile<D>::vcol(256 * i)) * 4));
    };
    auto gload = [&](int t) {
        gload_k(t, p.Tk);
        gload_v(t, p.Tk);
    };
    auto sstore_k = [&](int buf) {
#pragma unroll
        for (int i = 0; i < LPT; ++i) {
            const int f = tid + 256 * i;
            *reinterpret_cast<f32x4*>(&Ks[buf][f / C4][4 * (f % C4)]) = kr[i];
        }
    };
    auto sstore_v = [&](int buf) {
#pragma unroll
        for (int i = 0; i < LPT; ++i) {
            const int f = tid + 256 * i;
            const int vrow = (f & 15) + 16 * (f / (16 * C4));
            const int vc = 4 * ((f >> 4) % C4);
            Vt[buf][vc + 0][vrow] = vr[i][0];
            Vt[buf][vc + 1][vrow] = vr[i][1];
            Vt[buf][vc + 2][vrow] = vr[i][2];
            Vt[buf][vc + 3][vrow] = vr[i][3];
        }
    };
    auto sstore = [&](int buf) {
        sstore_k(buf);
        sstore_v(buf);
    };

    f32x16 o[NDB];
#pragma unroll
    for (int i = 0; i < NDB; ++i) o[i] = f32x16{};
    float m_run = -INFINITY;  // running max of raw scores for row qrow
    float l_run = 0.f;        // this lane's partial sum of p (its half of the keys)
    const float c = p.c;

    // S^T block of key tile in Ks[buf]: s[kb] reg 4j+cc holds key kb*32 + 8j + 4g + cc.
    auto scores = [&](int buf, f32x16 (&s)[NKB]) {
#pragma unroll
        for (int kb = 0; kb < NKB; ++kb) s[kb] = f32x16{};
#pragma unroll
        for (int i = 0; i < HD; i += 4) {
#pragma unroll
            for (int kb = 0; kb < NKB; ++kb) {
                const f32x4 a = *reinterpret_cast<const f32x4*>(&Ks[buf][kb * 32 + l32][g * HD + i]);
                s[kb] = mfma32x32x2(a[0], qf[i + 0], s[kb]);
                s[kb] = mfma32x32x2(a[1], qf[i + 1], s[kb]);
                s[kb] = mfma32x32x2(a[2], qf[i + 2], s[kb]);
                s[kb] = mfma32x32x2(a[3], qf[i + 3], s[kb]);
            }
        }
    };

    // Mask, online softmax and O^T += V^T P^T for key tile t (V^T in Vt[vbuf]).
    auto softmax_pv = [&](f32x16 (&s)[NKB], int t, int vbuf) {
        const int k0 = t * BN;
        const bool need_mask = (k0 + BN > p.Tk) || (p.causal && (k0 + BN - 1 > q0w + p.off));
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
        // Lazy rescaling: a row's reference max m_run moves only when the row
        // sees a score more than kLazyLog2 / c above it, so P stays
        // <= 2^kLazyLog2; the O / l rescale and its exp2 run only on tiles where
        // some row of the wave moved (VALU issue adds to fp32 MFMA time one for
        // one), and for the other rows it multiplies by exactly 1, so every row
        // depends on its own scores only.  O / l and the LSE do not depend on
        // the reference.  m_run = -inf with a visible key always moves it.
        const bool grow = mloc > m_run + kLazyLog2 / c;
        if (__any(grow)) {
            // A row can see no key of a chunk that does not start at key 0:
            // keep m = -inf, l = 0, O = 0 for it instead of exp2(NaN).
            const float alpha = grow ? fast_exp2((m_run - mloc) * c) : 1.f;  // m_run = -inf -> 0
            l_run *= alpha;
#pragma unroll
            for (int db = 0; db < NDB; ++db) o[db] *= alpha;
            m_run = grow ? mloc : m_run;
        }
        const float mc = m_run == -INFINITY ? 0.f : m_run * c;
        // row sum as four independent partial chains
        float ls[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int kb = 0; kb < NKB; ++kb)
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const float e = fast_exp2(fmaf(s[kb][r], c, -mc));
                s[kb][r] = e;
                ls[r & 3] += e;
            }
        l_run += (ls[0] + ls[1]) + (ls[2] + ls[3]);

        // reg 4j+cc of s[kb] holds key kb*32 + 8j + 4g + cc
#pragma unroll
        for (int kb = 0; kb < NKB; ++kb)
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                f32x4 va[NDB];
#pragma unroll
                for (int db = 0; db < NDB; ++db)
                    va[db] = *reinterpret_cast<const f32x4*>(&Vt[vbuf][db * 32 + l32][kb * 32 + 8 * j + 4 * g]);
#pragma unroll
                for (int cc = 0; cc < 4; ++cc)
#pragma unroll
                    for (int db = 0; db < NDB; ++db)
                        o[db] = mfma32x32x2(va[db][cc], s[kb][4 * j + cc], o[db]);
            }
    };

    if constexpr (FwdTile<D>::PIPE) {
        // Software pipeline: S of tile t+1 is issued before the softmax of tile
        // t, so the matrix pipe has independent work while the softmax runs.
        // K runs one tile ahead of V: at the top of step t, Ks[i&1] and
        // Ks[(i+1)&1] hold K_t (already consumed) and K_{t+1}, Vt[i&1] holds
        // V_t (i = t - t_begin).  Step t writes K_{t+2} over K_t and V_{t+1}
        // over V_{t-1}, both last read before the previous barrier.
        gload(t_begin);  // bounds-checked rows: safe even past the last tile
        sstore_k(0);
        sstore_v(0);
        gload_k(t_begin + 1, t_begin + 1 < n_tiles ? p.Tk : 0);
        sstore_k(1);
        __syncthreads();
        f32x16 sa[NKB], sb[NKB];
        if (t_begin * BN < wave_kend) scores(0, sa);
        __syncthreads();  // Ks[0] is overwritten at the end of the first step

        // The prefetch and the stores run unconditionally (straight-line code
        // keeps the loads overlapped); past the last tile they move zeros
        // into buffers that are not read again.
        auto step = [&](int t, f32x16 (&cur)[NKB], f32x16 (&nxt)[NKB]) {
            const int i = t - t_begin;
            const bool has_next = t + 1 < n_tiles;
            gload_k(t + 2, t + 2 < n_tiles ? p.Tk : 0);
            gload_v(t + 1, has_next ? p.Tk : 0);
            if (has_next && (t + 1) * BN < wave_kend) scores((i + 1) & 1, nxt);
            if (t * BN < wave_kend) softmax_pv(cur, t, i & 1);
            sstore_k(i & 1);
            sstore_v((i + 1) & 1);
            __syncthreads();
        };
        for (int t = t_begin; t < n_tiles; t += 2) {
            step(t, sa, sb);
            if (t + 1 < n_tiles) step(t + 1, sb, sa);
        }
    } else {
        gload(t_begin);  // bounds-checked rows: safe even past the last tile
        sstore(0);
        __syncthreads();
        for (int t = t_begin; t < n_tiles; ++t) {
            const int buf = (t - t_begin) & 1;
            if (t + 1 < n_tiles) gload(t + 1);
            if (t * BN < wave_kend) {
                f32x16 s[NKB];
                scores(buf, s);
                softmax_pv(s, t, buf);
            }
            if (t + 1 < n_tiles) sstore(buf ^ 1);
            __syncthreads();
        }
    }

    // ---- epilogue ---------------------------------------------------------------
    const float l_tot = l_run + shfl_xor(l_run, 32);
    if (slot >= 0) {
        // partial of a split query tile: unnormalised O, row max, row sum
        if (qrow < p.Tq) {
            const int r = wave * 32 + l32;
            float* po = p.part + ((int64_t)slot * BH + bh) * (BM * D) + (int64_t)r * D;
#pragma unroll
            for (int db = 0; db < NDB; ++db)
#pragma unroll
                for (int j = 0; j < 4; ++j)
                    st4(po + db * 32 + 8 * j + 4 * g,
                        f32x4{o[db][4 * j + 0], o[db][4 * j + 1], o[db][4 * j + 2], o[db][4 * j + 3]});
            if (g == 0) {
                float* pml = p.part + (int64_t)p.n_slots * BH * BM * D + (((int64_t)slot * BH + bh) * BM + r) * 2;
                pml[0] = m_run;
                pml[1] = l_tot;
            }
        }
        return;
    }
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

// Combines the partial slots of each split query tile: per row
// M = max_s m_s, w_s = exp2((m_s - M) c), O = sum_s w_s O_s / sum_s w_s l_s,
// LSE = M * scale + ln(sum_s w_s l_s).  One thread per (row, 4 columns).
template <int D, typename E>
__global__ __launch_bounds__(256) void attn_fwd_merge_kernel(FwdParams p) {
    constexpr int BM = kFwdBM;
    constexpr int C4 = D / 4;
    constexpr int TPT = BM * C4;  // threads per (split tile, head)
    const int BH = p.B * p.H;
    const int64_t gid = (int64_t)blockIdx.x * 256 + threadIdx.x;
    const int64_t unit = gid / TPT;  // (split tile, head)
    if (unit >= (int64_t)p.n_split * BH) return;
    const int si = (int)(unit / BH);
    const int bh = (int)(unit % BH);
    const int rem = (int)(gid % TPT);
    const int r = rem / C4;
    const int c4 = rem % C4;
    const int qrow = p.split_qt[si] * BM + r;
    if (qrow >= p.Tq) return;
    const int s0 = p.split_slot0[si], ns = p.split_count[si];
    const float* ml = p.part + (int64_t)p.n_slots * BH * BM * D;
    float M = -INFINITY;
    for (int s = 0; s < ns; ++s) M = fmaxf(M, ml[(((int64_t)(s0 + s) * BH + bh) * BM + r) * 2]);
    float L = 0.f;
    f32x4 acc = f32x4{0.f, 0.f, 0.f, 0.f};
    for (int s = 0; s < ns; ++s) {
        const int64_t base = ((int64_t)(s0 + s) * BH + bh) * BM + r;
        const float m = ml[base * 2];
        if (m == -INFINITY) continue;
        const float wgt = fast_exp2((m - M) * p.c);
        L = fmaf(ml[base * 2 + 1], wgt, L);
        const f32x4 v = *reinterpret_cast<const f32x4*>(p.part + base * D + 4 * c4);
        acc[0] = fmaf(v[0], wgt, acc[0]);
        acc[1] = fmaf(v[1], wgt, acc[1]);
        acc[2] = fmaf(v[2], wgt, acc[2]);
        acc[3] = fmaf(v[3], wgt, acc[3]);
    }
    const float inv = 1.f / L;
    const int b = bh / p.H, h = bh % p.H;
    E* dst = (E*)p.o + b * p.so.b + h * p.so.h + (int64_t)qrow * p.so.t + 4 * c4;
    st4(dst, f32x4{acc[0] * inv, acc[1] * inv, acc[2] * inv, acc[3] * inv});
    if (c4 == 0 && p.lse) p.lse[(int64_t)bh * p.Tq + qrow] = M * p.scale + logf(L);
}

template <int D, typename E>
static void launch_merge_t(const FwdParams& p, hipStream_t s) {
    const int64_t threads = (int64_t)p.n_split * p.B * p.H * kFwdBM * (D / 4);
    hipLaunchKernelGGL((attn_fwd_merge_kernel<D, E>), dim3((unsigned)((threads + 255) / 256)), dim3(256), 0, s, p);
}

template <int D, typename E>
static int launch_fwd_t(const FwdParams& p, hipStream_t s) {
    const int BH = p.B * p.H;
    const dim3 grid((unsigned)((p.n_groups ? p.n_groups : p.n_qtiles) * BH));
    hipLaunchKernelGGL((attn_fwd_kernel<D, E>), grid, dim3(256), 0, s, p);
    if (p.n_split) launch_merge_t<D, E>(p, s);
    return (int)hipGetLastError();
}

// ---- split plan ----------------------------------------------------------------
// Makespan of a dispatch order on the device: workgroup w goes to XCD w % 8,
// and inside an XCD each workgroup starts on the slot that frees first (slots =
// resident workgroups).  Costs are in key tiles plus a fixed per-workgroup
// overhead (Q load, first K/V tile not hidden behind compute, epilogue).
static double fwd_makespan(const int* cost, int n_groups, int BH, int slots_per_xcd, double overhead) {
    double worst = 0.0;
    std::vector<double> heap((size_t)slots_per_xcd);
    for (int x = 0; x < 8; ++x) {
        std::fill(heap.begin(), heap.end(), 0.0);  // min-heap of slot free times
        int64_t w = 0;
        for (int gi = 0; gi < n_groups; ++gi)
            for (int i = 0; i < BH; ++i, ++w) {
                if (w % 8 != x) continue;
                std::pop_heap(heap.begin(), heap.end(), std::greater<double>());
                heap.back() += cost[gi] + overhead;
                std::push_heap(heap.begin(), heap.end(), std::greater<double>());
            }
        worst = std::max(worst, *std::max_element(heap.begin(), heap.end()));
    }
    return worst;
}

// Resident forward workgroups per XCD on the current device (8 XCDs), and
// the device's CU count.
struct FwdSlots {
    int per_xcd, cus;
};
// An error left pending by an earlier HIP call on this thread is returned
// (named in the detail text) instead of being cleared by the queries here.
static int fwd_slots(int D, int bf16, FwdSlots* out) {
    static std::mutex mu;
    static std::map<std::array<int, 3>, FwdSlots> cache;
    const hipError_t pending = hipGetLastError();
    int dev = -1;
    if (hipGetDevice(&dev) != hipSuccess) {
        (void)hipGetLastError();  // no device (a CPU-only host sizing workspaces): MI355X defaults
        dev = -1;
    } else if (pending != hipSuccess) {
        return report_pending_error(pending, "attention forward planner");
    }
    std::lock_guard<std::mutex> lk(mu);
    const std::array<int, 3> key{dev, D, bf16};
    auto it = cache.find(key);
    if (it != cache.end()) {
        *out = it->second;
        return 0;
    }
    // MI355X: 256 CUs; fp32: two D <= 64 workgroups per CU, one at D = 128.
    int cus = 256, per_cu = bf16 ? (D >= 128 ? 2 : 4) : (D >= 128 ? 1 : 2);
    if (dev >= 0) {
        int n = 0, occ = 0;
        if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess && n > 0) cus = n;
        hipError_t e = hipErrorInvalidValue;
        if (bf16) e = (hipError_t)fwd_bf16_occupancy(D, &occ);
        else if (D == 32) e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&occ, attn_fwd_kernel<32, float>, 256, 0);
        else if (D == 64) e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&occ, attn_fwd_kernel<64, float>, 256, 0);
        else if (D == 128) e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&occ, attn_fwd_kernel<128, float>, 256, 0);
        if (e == hipSuccess && occ > 0) per_cu = occ;
        (void)hipGetLastError();  // a failed query of ours: the defaults stand
    }
    const FwdSlots slots{std::max(1, cus * per_cu / 8), cus};
    cache[key] = slots;
    *out = slots;
    return 0;
}

// Causal forward split plan.  Without a split the query tiles run heaviest
// first, one workgroup per (tile, head).  When the whole grid fits in the
// resident slots at once, the heaviest tile alone sets the kernel time (1.9x
// to 3.2x measured at B1 H2 T8192 D128 and B1 H4 T2048 D128), so its key range
// is cut.  With more workgroups than slots the tail balances itself (a
// workgroup left alone on a CU runs faster), and at B8 H12 T1024 D64 a split
// made the forward 4% slower, merge pass included: such grids never split.
// Each candidate chunk length CH cuts every tile with more than CH key tiles
// into ceil(n / CH) near-equal chunks; the candidate with the smallest
// simulated makespan (plus the merge pass) wins if it beats the unsplit order
// by more than 2%.
//
// bf16 (constants fitted to measurements at T = 1024..8192, D = 32..128): a
// bf16 key tile costs about a fifth of an fp32 one, so the workgroup's fixed
// cost and the merge weigh more in its units; up to four workgroups share a CU,
// whose resident workgroups together run about 1.1 tiles in the time one runs
// alone, so the makespan is also bounded below by the total work over the
// CUs; and tiles under 32 key tiles (2048 keys) never split (B1 H12 T1024 D64
// measured 19.9 us unsplit, 24.1 us split).
static constexpr double kFwdOverhead[2] = {0.35, 2.0};   // per-workgroup fixed cost, in key tiles (fp32, bf16)
static constexpr double kFwdMergeCost[2] = {0.5, 12.0};  // merge kernel, in key tiles
static constexpr double kFwdCuRate[2] = {0.0, 1.1};      // tiles per CU per tile time (0: no bound)
static constexpr int kFwdMinSplitTiles[2] = {0, 32};

static void fwd_plan_compute(int B, int H, int Tq, int Tk, int D, int bf16, FwdSlots slots, FwdPlan* out) {
    const int BM = kFwdBM, BN = bf16 ? kFwdBf16BN : D >= 128 ? FwdTile<128>::BN : FwdTile<64>::BN;
    const int ix = bf16 ? 1 : 0;
    const double overhead = kFwdOverhead[ix], merge_cost = kFwdMergeCost[ix], cap = kFwdCuRate[ix] * slots.cus;
    const int slots_per_xcd = slots.per_xcd;
    const int nq = (Tq + BM - 1) / BM;
    const int BH = B * H;
    const int off = Tk - Tq;
    if ((int64_t)nq * BH > 8LL * slots_per_xcd) return;
    std::vector<int> nt((size_t)nq);
    int max_nt = 0;
    for (int q = 0; q < nq; ++q) {
        const int kend = std::min(Tk, (q + 1) * BM + off);
        nt[(size_t)q] = std::max(0, (kend + BN - 1) / BN);
        max_nt = std::max(max_nt, nt[(size_t)q]);
    }
    if (max_nt < kFwdMinSplitTiles[ix]) return;
    auto span = [&](const std::vector<int>& c) {
        double m = fwd_makespan(c.data(), (int)c.size(), BH, slots_per_xcd, overhead);
        if (cap > 0) {
            double work = 0.0;
            for (int x : c) work += x + overhead;
            m = std::max(m, work * BH / cap);
        }
        return m;
    };
    std::vector<int> cost;
    for (int q = nq - 1; q >= 0; --q) cost.push_back(nt[(size_t)q]);
    const double base = span(cost);
    double best = base * 0.98;
    int best_ch = 0;
    struct G { int n, qt, t0, t1; };
    auto build = [&](int ch, std::vector<G>& g, int& n_split) {
        g.clear();
        n_split = 0;
        for (int q = 0; q < nq; ++q) {
            const int n = nt[(size_t)q];
            if (n > ch) {
                const int k = (n + ch - 1) / ch;
                ++n_split;
                for (int j = 0; j < k; ++j) {
                    const int a = (int)((int64_t)n * j / k), b = (int)((int64_t)n * (j + 1) / k);
                    g.push_back({b - a, q, a, b});
                }
            } else {
                g.push_back({n, q, 0, n});
            }
        }
        std::stable_sort(g.begin(), g.end(), [](const G& x, const G& y) {
            return x.n != y.n ? x.n > y.n : x.qt > y.qt;
        });
    };
    std::vector<G> g;
    for (int ch = max_nt - 1; ch >= std::max(2, max_nt / 8); --ch) {
        int n_split = 0;
        build(ch, g, n_split);
        if ((int)g.size() > kMaxFwdGroups || n_split > kMaxFwdGroups / 2) continue;
        cost.resize(g.size());
        for (size_t i = 0; i < g.size(); ++i) cost[i] = g[i].n;
        const double ms = span(cost) + merge_cost;
        if (ms < best) {
            best = ms;
            best_ch = ch;
        }
    }
    if (!best_ch) return;
    int n_split = 0;
    build(best_ch, g, n_split);
    // slots: consecutive per split tile, in query-tile order
    std::vector<int> slot0((size_t)nq, -1), count((size_t)nq, 0);
    for (const G& x : g)
        if (x.t1 - x.t0 < nt[(size_t)x.qt]) ++count[(size_t)x.qt];
    int ns = 0;
    for (int q = 0; q < nq; ++q)
        if (count[(size_t)q]) {
            slot0[(size_t)q] = ns;
            out->split_qt[out->n_split] = q;
            out->split_slot0[out->n_split] = ns;
            out->split_count[out->n_split] = count[(size_t)q];
            ++out->n_split;
            ns += count[(size_t)q];
        }
    std::vector<int> next((size_t)nq, 0);
    for (const G& x : g) {
        FwdGroup& o = out->groups[out->n_groups++];
        o.qt = x.qt;
        o.t0 = x.t0;
        o.t1 = x.t1;
        o.slot = count[(size_t)x.qt] ? slot0[(size_t)x.qt] + next[(size_t)x.qt]++ : -1;
    }
    out->n_slots = ns;
}

int fwd_plan(int B, int H, int Tq, int Tk, int D, int causal, int bf16, FwdPlan* out) {
    *out = FwdPlan{};
    bf16 = bf16 ? 1 : 0;
    if (!causal || (D != 32 && D != 64 && D != 128)) return 0;
    FwdSlots slots{};
    if (const int e = fwd_slots(D, bf16, &slots)) return e;
    static std::mutex mu;
    static std::map<std::array<int, 7>, FwdPlan> cache;
    const std::array<int, 7> key{B * H, Tq, Tk, D, bf16, slots.per_xcd, slots.cus};
    {
        std::lock_guard<std::mutex> lk(mu);
        auto it = cache.find(key);
        if (it != cache.end()) {
            *out = it->second;
            return 0;
        }
    }
    fwd_plan_compute(B, H, Tq, Tk, D, bf16, slots, out);
    // The bf16 D = 128 forward raises the P.V MFMAs' wave priority (a wave that
    // reaches them issues them ahead of the other wave's softmax VALU work on
    // its SIMD); on grids that fit one round of workgroup slots that measured
    // 5-7% slower (B2 H8 T4096, B1 H16 T4096, B4 H8 T2048, B1 H8 T8192: 512
    // workgroups on 512 slots) and on larger ones 1-10% faster (config 4, B4
    // H16 T2048, B8 H16 T1024, B8 H12 T1024).
    out->pv_prio = (int64_t)((Tq + kFwdBM - 1) / kFwdBM) * B * H > 8LL * slots.per_xcd;
    std::lock_guard<std::mutex> lk(mu);
    if (cache.size() > 256) cache.clear();
    cache[key] = *out;
    return 0;
}

size_t fwd_workspace_bytes(const FwdPlan& plan, int B, int H, int D) {
    return (size_t)plan.n_slots * B * H * kFwdBM * (size_t)(D + 2) * sizeof(float);
}

int launch_attn_fwd(const FwdParams& p, int bf16, hipStream_t s) {
    if (bf16) {
        const int e = launch_attn_fwd_bf16(p, s);
        if (e || !p.n_split) return e;
        switch (p.D) {  // the merge reads fp32 partials and writes bf16 O
            case 32: launch_merge_t<32, uint16_t>(p, s); break;
            case 64: launch_merge_t<64, uint16_t>(p, s); break;
            case 128: launch_merge_t<128, uint16_t>(p, s); break;
            default: return (int)hipErrorInvalidValue;
        }
        return (int)hipGetLastError();
    }
    switch (p.D) {
        case 32: return launch_fwd_t<32, float>(p, s);
        case 64: return launch_fwd_t<64, float>(p, s);
        case 128: return launch_fwd_t<128, float>(p, s);
        default: return (int)hipErrorInvalidValue;
    }
}

}  // namespace inf
