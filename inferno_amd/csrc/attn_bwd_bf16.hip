// attn_bwd_bf16.hip -- fused causal attention backward, bf16 inputs, fp32
// accumulation, on gfx950 bf16 MFMAs.
//
// Same ownership as the fp32 kernel (attn_bwd.hip): each wave owns a run of
// keys, with 8 waves x 32 keys = 256 keys per workgroup at D = 64 (4 x 32 at
// D = 32; D = 128 has its own kernel below, 8 waves x 16 keys): K and V
// operands and the dK^T / dV^T accumulators in VGPRs for the whole kernel
// (atomic-free dK, dV),
// query tiles of 32 rows, dQ through LDS and fp32 atomics into the
// accumulator.  At bf16 speed the dQ atomics are a device-wide throughput
// limit (at config 2 the kernel measured 23% faster with them left out);
// 256-key blocks add each dQ element once per 256 keys instead of per 128.  A bf16 MFMA reduces 16 (32x32x16)
// or 32 (16x16x32) elements with each lane supplying 8 consecutive ones, so
// every operand must be contiguous along its reduction index:
//   S = Q K^T, dP = dO V^T      reduce over d: Q, dO row-major in LDS; K, V rows
//                               in VGPRs
//   dV^T += dO^T P, dK^T += Q^T dS
//                               reduce over queries: dO and Q are also staged
//                               transposed (queries contiguous per head-dim row);
//                               P and dS come straight from the S / dP
//                               accumulators, registers 8m..8m+7 = queries
//                               16m + 4g + {0..3} and 16m + 8 + 4g + {0..3}
//   dQ += dS K                  reduce over keys: dS (bf16) through LDS with
//                               keys contiguous, K staged transposed once per
//                               workgroup; v_mfma_f32_16x16x32_bf16 tiles.  At
//                               D = 64 each wave's 16x16 dQ block reads the same
//                               K^T rows for every tile: half of them are held
//                               in VGPRs (all of them would spill)
// Transposed staging writes dwords that pack two rows' elements, so the LDS
// stores stay 32-bit.  Softmax statistics, P and dS are computed in fp32.
#include <type_traits>

#include "bwd_split.h"
#include "common.h"
#include "kernels.h"

namespace inf {

typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));

__device__ __forceinline__ f32x4 mfma16x16x32bf16(bf16x8 a, bf16x8 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

// Short rows' delta (bwd_split.h) for the key-block-0 workgroup, before its
// main loop, query-major from LDS.  K and V of the block's first BK keys and a
// batch of PR short query rows of Q and dO are staged in LDS (over the main
// loop's arrays, which are not live yet), then wave w takes the row tile of RT
// rows at batch + RT w: lane (lr, gq) holds row q = tile + lr, with its Q and
// dO values (the B operand, the main loop's k order) in registers, and walks
// the tile's visible keys in key tiles of RT keys, K and V rows (the A
// operand) read from LDS.  S^T and dP^T come from the main loop's MFMA shape
// with A and B swapped: the same products in the same k order.  Each lane adds
// e and e * dP over its keys in key order in fp64, the row's lane groups are
// added in a fixed pattern, and the row's first lane stores delta = sum(e dP)
// / sum(e) as hi + lo to the workspace and, for the D <= 64 kernel, -hi to sdl
// (its staging reads it from there).  No barrier between the staging and the
// end of a batch.
//   M32 = true:  v_mfma_f32_32x32x16_bf16, RT = 32, lane (l32, g) supplies
//                columns 16 kk + 8 g .. + 7, register r is key 8 (r/4) + 4 g + r%4
//   M32 = false: v_mfma_f32_16x16x32_bf16, RT = 16, lane (l16, g4) supplies
//                columns 32 kk + 8 g4 .. + 7, register r is key 4 g4 + r
template <int D, int NW, int BK, int PR, int PSTR, bool M32>
__device__ __forceinline__ void bwd_short_prologue(const BwdParams& p, int bh, const __bf16* Q, const __bf16* K,
                                                   const __bf16* V, const __bf16* dO, int q_begin, int qs_end,
                                                   __bf16 (*ks)[PSTR], __bf16 (*vs)[PSTR], __bf16 (*qs)[PSTR],
                                                   __bf16 (*ds)[PSTR], float* sdl) {
    constexpr int NT = 64 * NW;
    constexpr int RT = M32 ? 32 : 16;
    constexpr int NCH = M32 ? D / 16 : D / 32;  // MFMAs per product
    constexpr int CW = M32 ? 16 : 32;           // columns per MFMA
    constexpr int NR = M32 ? 16 : 4;            // output registers
    constexpr int C8 = D / 8;                   // 16-byte chunks per row
    static_assert(PR == NW * RT, "one row tile per wave per batch");
    typedef typename std::conditional<M32, f32x16, f32x4>::type Acc;
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int lr = M32 ? (lane & 31) : (lane & 15);
    const int gq = M32 ? (lane >> 5) : (lane >> 4);
    const float c = p.c;
    // K and V of the keys these rows can see (at most the block), staged once
    const int kmax = p.causal ? min(p.Tk, min(qs_end, p.Tq) - 1 + p.off + 1) : p.Tk;  // <= BK
    {
        const auto rk = row_rsrc(K, p.sk.t, 0, kmax, D);
        const auto rv = row_rsrc(V, p.sv.t, 0, kmax, D);
        for (int f = tid; f < BK * C8; f += NT) {
            const int r = f / C8, c8 = f % C8;
            *reinterpret_cast<bf16x8*>(&ks[r][8 * c8]) = buffer_ld8bf(rk, (uint32_t)(((int64_t)r * p.sk.t + 8 * c8) * 2), 0);
            *reinterpret_cast<bf16x8*>(&vs[r][8 * c8]) = buffer_ld8bf(rv, (uint32_t)(((int64_t)r * p.sv.t + 8 * c8) * 2), 0);
        }
    }
    for (int b0 = q_begin; b0 < qs_end; b0 += PR) {
        {
            const int nrow = min(p.Tq - b0, PR);
            const auto rq = row_rsrc(Q, p.sq.t, b0, nrow, D);
            const auto rdo = row_rsrc(dO, p.sdo.t, b0, nrow, D);
            for (int f = tid; f < PR * C8; f += NT) {
                const int r = f / C8, c8 = f % C8;
                *reinterpret_cast<bf16x8*>(&qs[r][8 * c8]) = buffer_ld8bf(rq, (uint32_t)(((int64_t)r * p.sq.t + 8 * c8) * 2), 0);
                *reinterpret_cast<bf16x8*>(&ds[r][8 * c8]) = buffer_ld8bf(rdo, (uint32_t)(((int64_t)r * p.sdo.t + 8 * c8) * 2), 0);
            }
        }
        __syncthreads();
        const int t0 = b0 + RT * wave;
        if (t0 < qs_end) {
            const int row = t0 + lr;
            bf16x8 qf[NCH], df[NCH];
#pragma unroll
            for (int kk = 0; kk < NCH; ++kk) {
                qf[kk] = *reinterpret_cast<const bf16x8*>(&qs[RT * wave + lr][CW * kk + 8 * gq]);
                df[kk] = *reinterpret_cast<const bf16x8*>(&ds[RT * wave + lr][CW * kk + 8 * gq]);
            }
            const float L = row < p.Tq ? p.lse[(int64_t)bh * p.Tq + row] * kLog2e : 0.f;
            const int kend = p.causal ? min(p.Tk, min(t0 + RT - 1, p.Tq - 1) + p.off + 1) : p.Tk;
            double le = 0.0, we = 0.0;
            for (int u = 0; u * RT < kend; ++u) {
                Acc s, dp;
#pragma unroll
                for (int kk = 0; kk < NCH; ++kk) {
                    const bf16x8 ka = *reinterpret_cast<const bf16x8*>(&ks[u * RT + lr][CW * kk + 8 * gq]);
                    const bf16x8 va = *reinterpret_cast<const bf16x8*>(&vs[u * RT + lr][CW * kk + 8 * gq]);
                    if constexpr (M32) {
                        s = mfma32x32x16bf16(ka, qf[kk], kk == 0 ? Acc{} : s);
                        dp = mfma32x32x16bf16(va, df[kk], kk == 0 ? Acc{} : dp);
                    } else {
                        s = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ka, qf[kk], kk == 0 ? Acc{} : s, 0, 0, 0);
                        dp = __builtin_amdgcn_mfma_f32_16x16x32_bf16(va, df[kk], kk == 0 ? Acc{} : dp, 0, 0, 0);
                    }
                }
#pragma unroll
                for (int r = 0; r < NR; ++r) {
                    const int key = u * RT + (M32 ? 8 * (r >> 2) + 4 * gq + (r & 3) : 4 * gq + r);
                    const bool vis = key < p.Tk && row < p.Tq && (!p.causal || key <= row + p.off);
                    const float e = bwd_short_weight(p, row, vis, fast_exp2(fmaf(s[r], c, -L)));
                    le += (double)e;
                    we += (double)e * (double)dp[r];
                }
            }
            if constexpr (!M32) {
                le += __shfl_xor(le, 16);
                we += __shfl_xor(we, 16);
            }
            le += __shfl_xor(le, 32);
            we += __shfl_xor(we, 32);
            if (gq == 0 && bwd_short_row(p, row)) {
                const double dl = we / le;
                const float hi = (float)dl;
                p.delta[(int64_t)bh * p.Tq + row] = hi;
                p.delta_lo[(int64_t)bh * p.Tq + row] = (float)(dl - (double)hi);
                if (sdl) sdl[row] = -hi;
            }
        }
        __syncthreads();  // the batch's rows are read before the next batch overwrites them
    }
}

// DWS: every query row is short (Tk within one key block), so the staging
// takes delta from the workspace for every row instead of forming it from O
// and dO.
// SHORT: the launch has short rows (p.n_short > 0; DWS implies it).
template <int D, bool DWS, bool SHORT>
__global__ __launch_bounds__(64 * bwd_bf16_waves(D), (bwd_bf16_waves(D) == 8 || D >= 128) ? 1 : 2) void bwd_main_bf16_kernel(BwdParams p) {
    constexpr int NW = bwd_bf16_waves(D);  // waves per workgroup, 32 keys each
    constexpr int NT = 64 * NW;            // threads
    constexpr int BQ = kBwdBQ;             // 32 query rows per step
    constexpr int BK = 32 * NW;            // keys per workgroup
    constexpr int NKK = D / 16;          // S / dP MFMAs along d
    constexpr int NDB = D / 32;          // 32-wide d blocks of dK^T / dV^T
    constexpr int C8 = D / 8;            // 8-element chunks per row
    constexpr int QS = D + 8;            // row-major Q / dO stride (bf16)
    // Transposed Q / dO: each row stores the queries in the order the dV / dK
    // MFMAs take them (a lane's 8 queries 16m + 4g + {0..3} and 16m + 8 + 4g +
    // {0..3} contiguous at 16m + 8g), so an operand is one 16-byte read
    // instead of two 8-byte ones (1.5-2% faster at D = 32 and 64).
    constexpr int TS = BQ + 8;           // row stride (bf16): 20 dwords keep the 16-byte reads conflict-free
    // dS and K^T row strides of an odd multiple of 32 bytes: the dQ product's
    // 16-byte reads (lane (l16, g4) at row l16, byte 16 g4 of a 64-byte slice)
    // are then conflict-free on gfx950's LDS (BK + 8 measured 1.67x slower
    // per read; config 2 backward -0.8%, D = 32 -1%).
    constexpr int SS = BK + 16;          // dS stride (bf16)
    constexpr int KTS = BK + 16;         // K^T stride (bf16)
    constexpr int QTASK = (BQ / 2) * C8;                 // (row pair, chunk) tasks per tensor
    constexpr int QLPT = (2 * QTASK + NT - 1) / NT;      // Q and dO together, per thread
    constexpr int KTASK = (BK / 2) * C8;
    constexpr int KLPT = (KTASK + NT - 1) / NT;
    constexpr int NDQ = 2 * (D / 16);    // 16x16 dQ blocks of a query tile, NDQ / NW per wave
    static_assert(NDQ % NW == 0, "whole dQ blocks per wave");
    static_assert(D <= 64, "D = 128 runs bwd_main_bf16_w16_kernel");
    // LSE staged in base 2 (scaled by log2(e) once per row instead of once per
    // score: backward -2% at config 2); D = 32 measured 7% slower staged that
    // way and scales where it reads.
    constexpr float kLseStage = D == 64 ? kLog2e : 1.f;
    constexpr float kLseRead = D == 64 ? 1.f : kLog2e;

    // LDS: the main loop's arrays (staged query tile and dS double-buffered:
    // one barrier per tile) and, over the same bytes, the short-row prologue's
    // (K and V of the key block, a batch of short Q / dO rows)
    constexpr int PSTR = D + 8;  // prologue row stride (bf16)
    constexpr int PR = 32 * NW;  // prologue rows per batch
    struct MainLds {
        __bf16 Qs2[2][BQ][QS];
        __bf16 dOs2[2][BQ][QS];
        __bf16 QTs2[2][D][TS];
        __bf16 dOTs2[2][D][TS];
        __bf16 dSs2[2][BQ][SS];
        __bf16 KTs[D][KTS];
        float lse_s2[2][BQ];
        float dl_s2[2][BQ];
    };
    struct ProLds {
        __bf16 k[BK][PSTR], v[BK][PSTR], q[PR][PSTR], d[PR][PSTR];
    };
    __shared__ __attribute__((aligned(16))) union {
        MainLds m;
        ProLds pr;
    } lds;
    auto& Qs2 = lds.m.Qs2;
    auto& dOs2 = lds.m.dOs2;
    auto& QTs2 = lds.m.QTs2;
    auto& dOTs2 = lds.m.dOTs2;
    auto& dSs2 = lds.m.dSs2;
    auto& KTs = lds.m.KTs;
    auto& lse_s2 = lds.m.lse_s2;
    auto& dl_s2 = lds.m.dl_s2;
    // minus the short rows' delta, rows [0, n_short) (n_short <= BK unless DWS)
    __shared__ float sdl_s[BK];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int l32 = lane & 31;
    const int g = lane >> 5;
    const int l16 = lane & 15;
    const int g4 = lane >> 4;

    const BwdWork wk = bwd_work<BK>(p);
    if (wk.bh >= p.B * p.H) return;  // padding workgroup of a split plan's grid
    const int kblk = wk.kblk;
    const int bh = wk.bh;
    const int b = bh / p.H;
    const int h = bh % p.H;

    const __bf16* Q = (const __bf16*)p.q + b * p.sq.b + h * p.sq.h;
    const __bf16* K = (const __bf16*)p.k + b * p.sk.b + h * p.sk.h;
    const __bf16* V = (const __bf16*)p.v + b * p.sv.b + h * p.sv.h;
    const __bf16* dO = (const __bf16*)p.dout + b * p.sdo.b + h * p.sdo.h;
    float* dQa = p.dq_acc + b * p.sacc.b + h * p.sacc.h;
    const float* LSE = p.lse + (int64_t)bh * p.Tq;

    const int k0 = kblk * BK;
    const int k0w = k0 + wave * 32;
    const int key = k0w + l32;

    // K / V operands: MFMA kk takes row `key`, columns 16kk + 8g .. +7.
    bf16x8 kf[NKK], vf[NKK];
#pragma unroll
    for (int kk = 0; kk < NKK; ++kk) {
        if (key < p.Tk) {
            kf[kk] = *reinterpret_cast<const bf16x8*>(K + (int64_t)key * p.sk.t + 16 * kk + 8 * g);
            vf[kk] = *reinterpret_cast<const bf16x8*>(V + (int64_t)key * p.sv.t + 16 * kk + 8 * g);
        } else {
            kf[kk] = vf[kk] = bf16x8{};
        }
    }

    f32x16 dv_acc[NDB], dk_acc[NDB];
#pragma unroll
    for (int i = 0; i < NDB; ++i) {
        dv_acc[i] = f32x16{};
        dk_acc[i] = f32x16{};
    }

    const int q_begin = wk.q_begin;
    const int q_end = wk.q_end;
    const float c = p.c;

    // Q / dO staging, prefetched one query tile ahead in registers: tile q0's
    // rows are loaded while tile q0 - BQ computes.  The staged tile and dS are
    // double-buffered, so each tile needs one barrier: a tile stages the next
    // one into the buffer the previous tile read (every wave passed the
    // previous barrier after its reads), writes its dS, and meets the others
    // at the barrier before the dQ product reads dS.  (With single buffers and
    // two barriers per tile the kernel measured 6% slower at config 2.)
    bf16x8 ra[QLPT], rb[QLPT];
    float r_lse = 0.f;
    float r_dl[QLPT];  // DWS: the delta tasks' rows' delta from the workspace
    // Loads through buffer resources over rows [q0, lim) (<= Tq): rows past
    // them read as zeros, with no address arithmetic or branch per load; raw
    // values only, so no arithmetic waits on the loads here.  Chunk f is a
    // (row pair, chunk) task of Q (f < QTASK) or dO (f < 2 QTASK), or, on the
    // threads the two leave free, a (row, chunk) task of the row dot
    // delta = rowsum(dO * O) (ra = O, rb = dO): delta is formed here instead
    // of in a pass over O and dO before the kernel.  The kind is uniform over
    // each wave for every head dim (QTASK is a multiple of 64), which keeps
    // the selected resources in SGPRs.
    static_assert(QTASK % 64 == 0, "Q / dO split must be wave-uniform");
    static_assert(4 * QTASK == NT, "Q, dO and delta tasks fill the workgroup once");
    const __bf16* Ob = (const __bf16*)p.o + b * p.so.b + h * p.so.h;
    const float* DLs = p.delta + (int64_t)bh * p.Tq;
    int staged_q0 = 0;  // first row of the tile in the staging registers
    auto gload_q = [&](int q0, int lim) {
        staged_q0 = q0;
        const int rows = min(lim - q0, BQ);
        const auto rq = row_rsrc(Q, p.sq.t, q0, rows, D);
        const auto rdo = row_rsrc(dO, p.sdo.t, q0, rows, D);
#pragma unroll
        for (int i = 0; i < QLPT; ++i) {
            const int f = tid + NT * i;
            ra[i] = rb[i] = bf16x8{};
            const int which = __builtin_amdgcn_readfirstlane(f / QTASK);  // 0: Q, 1: dO, 2-3: delta
            if (which >= 2) {
                const int rem = f - 2 * QTASK;
                const int row = rem / C8, c8 = rem % C8;
                if constexpr (DWS) {
                    r_dl[i] = buffer_ld1(row_rsrc(DLs, 1, q0, rows, 1), (uint32_t)row * 4, 0);
                } else {
                    const auto ro = row_rsrc(Ob, p.so.t, q0, rows, D);
                    ra[i] = buffer_ld8bf(ro, (uint32_t)(((int64_t)row * p.so.t + 8 * c8) * 2), 0);
                    rb[i] = buffer_ld8bf(rdo, (uint32_t)(((int64_t)row * p.sdo.t + 8 * c8) * 2), 0);
                }
                continue;
            }
            const int rem = f % QTASK;
            const int qp = rem % (BQ / 2), c8 = rem / (BQ / 2);
            const int64_t st = which ? p.sdo.t : p.sq.t;
            const auto rs = which ? rdo : rq;
            const uint32_t voff = (uint32_t)(((int64_t)(2 * qp) * st + 8 * c8) * 2);
            ra[i] = buffer_ld8bf(rs, voff, 0);
            rb[i] = buffer_ld8bf(rs, voff, (uint32_t)(st * 2));
        }
        // lanes past the tile's rows (all but the first BQ threads) read zeros
        r_lse = buffer_ld1(row_rsrc(LSE, 1, q0, rows, 1), (uint32_t)tid * 4, 0);
    };
    auto sstore_q = [&](int sb) {
        __bf16(*Qs)[QS] = Qs2[sb];
        __bf16(*dOs)[QS] = dOs2[sb];
        __bf16(*QTs)[TS] = QTs2[sb];
        __bf16(*dOTs)[TS] = dOTs2[sb];
        float* lse_s = lse_s2[sb];
        float* dl_s = dl_s2[sb];
#pragma unroll
        for (int i = 0; i < QLPT; ++i) {
            const int f = tid + NT * i;
            const int which = f / QTASK;
            if (which >= 2) {
                // delta of row `row`: this lane's 8 products, then the sum over
                // the C8 adjacent lanes of the row (DPP), in a fixed order
                const int rem = f - 2 * QTASK;
                if constexpr (DWS) {
                    if (rem % C8 == 0) dl_s[rem / C8] = -r_dl[i];
                } else {
                    float d = 0.f;
#pragma unroll
                    for (int e = 0; e < 8; ++e) d = fmaf((float)ra[i][e], (float)rb[i][e], d);
                    d = group_sum<C8>(d);
                    if (rem % C8 == 0) {
                        // staged negated: the dP accumulator starts at -delta; a
                        // short row's (formed by the prologue) comes from sdl_s
                        const int qi = staged_q0 + rem / C8;
                        dl_s[rem / C8] = SHORT && kblk == 0 && bwd_short_row(p, qi) ? sdl_s[qi] : -d;
                    }
                }
                continue;
            }
            const int rem = f % QTASK;
            const int qp = rem % (BQ / 2), c8 = rem / (BQ / 2);
            __bf16(*rows)[QS] = which ? dOs : Qs;
            __bf16(*cols)[TS] = which ? dOTs : QTs;
            *reinterpret_cast<bf16x8*>(&rows[2 * qp][8 * c8]) = ra[i];
            *reinterpret_cast<bf16x8*>(&rows[2 * qp + 1][8 * c8]) = rb[i];
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                bf16x2 pr;
                pr[0] = ra[i][e];
                pr[1] = rb[i][e];
                // query q = 16m + 8h + 4g + c at 16m + 8g + 4h + c
                const int q = 2 * qp;
                const int pos = (q & 16) | ((q & 4) << 1) | ((q & 8) >> 1) | (q & 3);
                *reinterpret_cast<bf16x2*>(&cols[8 * c8 + e][pos]) = pr;
            }
        }
        if (tid < BQ) lse_s[tid] = r_lse * kLseStage;
    };

    // Short rows (bwd_split.h): their delta before the main loop.
    const int qs_end = SHORT && kblk == 0 ? min(q_end, p.n_short) : q_begin;  // short rows: [q_begin, qs_end)
    if (SHORT && q_begin < qs_end)
        bwd_short_prologue<D, NW, BK, PR, PSTR, true>(p, bh, Q, K, V, dO, q_begin, qs_end, lds.pr.k, lds.pr.v,
                                                      lds.pr.q, lds.pr.d, DWS ? nullptr : sdl_s);

    // K^T of the key block (keys contiguous per d row), for dQ.
#pragma unroll
    for (int i = 0; i < KLPT; ++i) {
        const int f = tid + NT * i;
        if (f >= KTASK) continue;
        const int kp = f % (BK / 2), c8 = f / (BK / 2);
        const int r0 = k0 + 2 * kp;
        const bf16x8 a = r0 < p.Tk ? *reinterpret_cast<const bf16x8*>(K + (int64_t)r0 * p.sk.t + 8 * c8) : bf16x8{};
        const bf16x8 c = r0 + 1 < p.Tk ? *reinterpret_cast<const bf16x8*>(K + (int64_t)(r0 + 1) * p.sk.t + 8 * c8)
                                       : bf16x8{};
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            bf16x2 pr;
            pr[0] = a[e];
            pr[1] = c[e];
            *reinterpret_cast<bf16x2*>(&KTs[8 * c8 + e][2 * kp]) = pr;
        }
    }

    gload_q(q_begin, p.Tq);
    sstore_q(0);
    __syncthreads();

    // The first KR K^T operands of this wave's dQ block, the same for every
    // query tile, held in VGPRs (KR = 4 of 8 at D = 64 fits the 256-VGPR
    // budget of 2 waves per SIMD; 3.5% faster at config 2; K^T is staged and
    // visible after the barrier above).
    constexpr int KR = (NDQ / NW) == 1 && D == 64 ? 4 : 0;
    bf16x8 ktr[KR > 0 ? KR : 1];
#pragma unroll
    for (int kk = 0; kk < KR; ++kk) {
        const int dc = (wave * (NDQ / NW)) >> 1;
        ktr[kk] = *reinterpret_cast<const bf16x8*>(&KTs[16 * dc + l16][32 * kk + 8 * g4]);
    }

    // The prefetch and its store are straight-line (a row limit of 0 past the
    // last tile): conditional blocks would make the compiler wait for every
    // outstanding memory operation, the previous tile's dQ atomics included,
    // at the top of each tile.
    int cb = 0;
    for (int q0 = q_begin; q0 < q_end; q0 += BQ, cb ^= 1) {
        gload_q(q0 + BQ, q0 + BQ < q_end ? p.Tq : 0);
        __bf16(*Qs)[QS] = Qs2[cb];
        __bf16(*dOs)[QS] = dOs2[cb];
        __bf16(*QTs)[TS] = QTs2[cb];
        __bf16(*dOTs)[TS] = dOTs2[cb];
        __bf16(*dSs)[SS] = dSs2[cb];
        const float* lse_s = lse_s2[cb];
        const float* dl_s = dl_s2[cb];

        const bool active = !p.causal || (q0 + BQ - 1 + p.off >= k0w);
        bf16x8 pb[2], dsb[2];
        if (active && k0w < p.Tk) {
            f32x16 s, dp;
            bf16x8 qa[NKK], da[NKK];
#pragma unroll
            for (int kk = 0; kk < NKK; ++kk) {
                qa[kk] = *reinterpret_cast<const bf16x8*>(&Qs[l32][16 * kk + 8 * g]);
                da[kk] = *reinterpret_cast<const bf16x8*>(&dOs[l32][16 * kk + 8 * g]);
            }
            // dP starts at -delta of its row (register r: query row
            // 8 (r / 4) + 4 g + r % 4), so dS = P * dP needs no subtraction
            f32x16 dp0;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const f32x4 nd = *reinterpret_cast<const f32x4*>(&dl_s[8 * j + 4 * g]);
#pragma unroll
                for (int cc = 0; cc < 4; ++cc) dp0[4 * j + cc] = nd[cc];
            }
            // all operand reads are issued before the first MFMA (the
            // scheduler would otherwise pair each read with its MFMA and wait
            // out one LDS latency per product)
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int kk = 0; kk < NKK; ++kk) {
                s = mfma32x32x16bf16(qa[kk], kf[kk], kk == 0 ? f32x16{} : s);  // zero accumulator as an operand
                dp = mfma32x32x16bf16(da[kk], vf[kk], kk == 0 ? dp0 : dp);
            }
            // transposed Q / dO operands of the dV / dK products, read while P and dS are formed
            bf16x8 ado[2][NDB], aq[2][NDB];
#pragma unroll
            for (int m = 0; m < 2; ++m) {
#pragma unroll
                for (int db = 0; db < NDB; ++db) {
                    ado[m][db] = *reinterpret_cast<const bf16x8*>(&dOTs[db * 32 + l32][16 * m + 8 * g]);
                    aq[m][db] = *reinterpret_cast<const bf16x8*>(&QTs[db * 32 + l32][16 * m + 8 * g]);
                }
            }
            __builtin_amdgcn_sched_barrier(0);
            // P and dS; register r holds query row 8*(r/4) + 4*g + r%4 of the
            // tile.  Only tiles that cross the causal diagonal or the end of
            // the queries / keys evaluate the visibility test.
            auto p_ds = [&](auto masked) {
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const f32x4 L = *reinterpret_cast<const f32x4*>(&lse_s[8 * j + 4 * g]) * kLseRead;
#pragma unroll
                    for (int cc = 0; cc < 4; ++cc) {
                        const int r = 4 * j + cc;
                        float pr = fast_exp2(fmaf(s[r], c, -L[cc]));
                        if constexpr (decltype(masked)::value) {
                            const int qi = q0 + 8 * j + 4 * g + cc;
                            const bool vis = (qi < p.Tq) && (key < p.Tk) && (!p.causal || key <= qi + p.off);
                            pr = vis ? pr : 0.f;
                        }
                        pb[r >> 3][r & 7] = (__bf16)pr;
                        dsb[r >> 3][r & 7] = (__bf16)(pr * dp[r]);
                    }
                }
            };
            const bool need_mask = q0 + BQ > p.Tq || k0w + 32 > p.Tk || (p.causal && k0w + 31 > q0 + p.off);
            if (need_mask)
                p_ds(std::true_type{});
            else
                p_ds(std::false_type{});
            if (bwd_one_key_tile(p, q0, k0w)) {  // a row with one visible key: dS = P (dP - dP) = 0
#pragma unroll
                for (int r = 0; r < 16; ++r)
                    if (bwd_one_key_row(p, q0 + 8 * (r >> 2) + 4 * g + (r & 3))) dsb[r >> 3][r & 7] = (__bf16)0.f;
            }
            // dV^T += dO^T P ; dK^T += Q^T dS  (reduce over the 32 queries, 16 per MFMA)
#pragma unroll
            for (int m = 0; m < 2; ++m)
#pragma unroll
                for (int db = 0; db < NDB; ++db) {
                    dv_acc[db] = mfma32x32x16bf16(ado[m][db], pb[m], dv_acc[db]);
                    dk_acc[db] = mfma32x32x16bf16(aq[m][db], dsb[m], dk_acc[db]);
                }
        } else {
            pb[0] = pb[1] = dsb[0] = dsb[1] = bf16x8{};
        }
        // dS block of this wave -> LDS (rows = queries, columns = the 128 keys)
        if (!p.dq_direct) {
#pragma unroll
            for (int r = 0; r < 16; ++r) dSs[8 * (r >> 2) + 4 * g + (r & 3)][wave * 32 + l32] = dsb[r >> 3][r & 7];
        }
        // the other buffer was last read by the previous tile, before the
        // previous barrier: stage the next tile there (zeros after the last)
        sstore_q(cb ^ 1);
        __syncthreads();

        // ---- dQ tile (32 x D) += dS (32 x BK) K (BK x D), 16x16 blocks ---------
        // Each wave takes NDQ / NW adjacent blocks.  fp32 atomics through a
        // buffer resource over the tile's rows: rows past Tq fall outside it
        // and the hardware drops those adds.
        if (p.dq_direct) continue;
        const auto rdq = row_rsrc(dQa, p.sacc.t, q0, min(p.Tq - q0, BQ), D);
#pragma unroll
        for (int bi = 0; bi < NDQ / NW; ++bi) {
            const int blk = wave * (NDQ / NW) + bi;  // adjacent blocks share K^T rows
            const int qh = blk & 1;
            const int dc = blk >> 1;
            f32x4 acc;
            bf16x8 a[BK / 32], bb[BK / 32];
#pragma unroll
            for (int kk = 0; kk < BK / 32; ++kk) {
                a[kk] = *reinterpret_cast<const bf16x8*>(&dSs[16 * qh + l16][32 * kk + 8 * g4]);
                bb[kk] = kk < KR ? ktr[kk < KR ? kk : 0] : *reinterpret_cast<const bf16x8*>(&KTs[16 * dc + l16][32 * kk + 8 * g4]);
            }
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int kk = 0; kk < BK / 32; ++kk)
                acc = mfma16x16x32bf16(a[kk], bb[kk], kk == 0 ? f32x4{0.f, 0.f, 0.f, 0.f} : acc);
            const uint32_t voff = (uint32_t)(((int64_t)(16 * qh + 4 * g4) * p.sacc.t + 16 * dc + l16) * 4);
#pragma unroll
            for (int r = 0; r < 4; ++r)
                buffer_atomic_add(rdq, acc[r] * p.scale, voff, (uint32_t)((int64_t)r * p.sacc.t * 4));
        }
    }

    if (!bwd_fixup<NT>(p, wk, dk_acc, dv_acc)) return;
    if (key < p.Tk) {
        uint16_t* dKp = (uint16_t*)p.dk + b * p.sdk.b + h * p.sdk.h + (int64_t)key * p.sdk.t;
        uint16_t* dVp = (uint16_t*)p.dv + b * p.sdv.b + h * p.sdv.h + (int64_t)key * p.sdv.t;
#pragma unroll
        for (int db = 0; db < NDB; ++db)
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                f32x4 a, v;
#pragma unroll
                for (int cc = 0; cc < 4; ++cc) {
                    a[cc] = dk_acc[db][4 * j + cc] * p.scale;
                    v[cc] = dv_acc[db][4 * j + cc];
                }
                st4(dKp + db * 32 + 8 * j + 4 * g, a);
                st4(dVp + db * 32 + 8 * j + 4 * g, v);
            }
    }
}

// D = 128: 8 waves x 16 keys (128 keys per workgroup) on v_mfma_f32_16x16x32_bf16,
// two waves per SIMD (244 VGPRs; 216 in the DQD instantiation).  (32 keys per wave on 32x32 MFMAs needs
// ~470 registers per wave at D = 128: one wave per SIMD; against that layout
// this one measured 11-28% faster at T <= 2048 and 2% at config 4, whose
// 64 key blocks per head make the dQ atomics the limit: 39% faster there
// with the atomics left out.)  Per wave: K / V operands of its 16
// keys and the dK^T / dV^T accumulators (8 blocks of 16 d x 16 keys each) in
// VGPRs.  A 16x16x32 MFMA reduces 32 elements, each lane (row or column l16,
// group g4) supplying 8 consecutive ones:
//   S = Q K^T, dP = dO V^T   (per 16-query half): A = Q rows from LDS, B = K
//                            rows of the wave's keys (registers); output lane
//                            = key l16, registers r = queries 4 g4 + r
//   dV^T += dO^T P, dK^T += Q^T dS: B = P / dS straight from the S / dP
//                            outputs (a lane's 8 queries 4 g4 + {0..3} and
//                            16 + 4 g4 + {0..3}); A = dO^T / Q^T read from the
//                            same Q / dO rows by transpose reads
//                            (ds_read_b64_tr_b16), two per operand
//   dQ += dS K               dS through LDS (keys contiguous), K^T staged once;
//                            each wave one 16-query half x two 16-wide d blocks
//
// DQD: the launch has the query-major dQ pass (p.dq_direct), so no dQ product
// here; then Q / dO tiles go straight into LDS (direct-to-LDS buffer loads,
// one tile ahead, each step waiting for them before its barrier), where the
// atomics of the dQ product would otherwise sit in the same in-order memory
// counter as those loads.
template <int D, bool SHORT, bool DQD>
__global__ __launch_bounds__(512, 1) void bwd_main_bf16_w16_kernel(BwdParams p) {
    static_assert(D == 128, "16-key waves are the D = 128 kernel");
    constexpr int NW = 8;
    constexpr int NT = 64 * NW;
    constexpr int BQ = kBwdBQ;           // 32
    constexpr int KW = 16;               // keys per wave
    constexpr int BK = KW * NW;          // 128 keys per workgroup
    constexpr int NKC = D / 32;          // 32-wide d chunks: reduction steps of S / dP
    constexpr int NDB = D / 16;          // 16-row d blocks of dK^T / dV^T
    constexpr int C8 = D / 8;
    // Row strides of 288 bytes (an odd multiple of 32): the 16-byte operand
    // reads, lane (l16, g4) at row l16 and byte 16 g4 of a 64-byte slice, are
    // then conflict-free on gfx950's LDS (272 bytes, D + 8, measured 1.67x
    // slower); the 8-byte transpose reads are conflict-free with either.
    constexpr int QS = D + 16;           // row-major Q / dO stride (bf16)
    constexpr int SS = BK + 16;          // dS stride
    constexpr int KTS = BK + 16;         // K^T stride
    constexpr int QTASK = (BQ / 2) * C8; // 256: Q tasks on threads 0..255, dO on 256..511
    constexpr int KTASK = (BK / 2) * C8;
    constexpr int KLPT = (KTASK + NT - 1) / NT;
    static_assert(2 * QTASK == NT, "one Q / dO staging task per thread");

    // LDS: the main loop's arrays and, over the same bytes, the short-row
    // prologue's (K and V of the key block, a batch of short Q / dO rows)
    constexpr int PSTR = D + 8;  // prologue row stride (bf16)
    constexpr int PR = 16 * NW;  // prologue rows per batch
    struct MainLds {
        __bf16 Qs2[2][BQ][QS];
        __bf16 dOs2[2][BQ][QS];
        __bf16 dSs2[2][BQ][SS];
        __bf16 KTs[D][KTS];
        float lse_s2[2][BQ];
        float dl_s2[2][BQ];
    };
    struct ProLds {
        __bf16 k[BK][PSTR], v[BK][PSTR], q[PR][PSTR], d[PR][PSTR];
    };
    __shared__ __attribute__((aligned(16))) union {
        MainLds m;
        ProLds pr;
    } lds;
    auto& Qs2 = lds.m.Qs2;
    auto& dOs2 = lds.m.dOs2;
    auto& dSs2 = lds.m.dSs2;
    auto& KTs = lds.m.KTs;
    auto& lse_s2 = lds.m.lse_s2;
    auto& dl_s2 = lds.m.dl_s2;

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int l16 = lane & 15;
    const int g4 = lane >> 4;

    const BwdWork wk = bwd_work<BK>(p);
    if (wk.bh >= p.B * p.H) return;  // padding workgroup of a split plan's grid
    const int kblk = wk.kblk;
    const int bh = wk.bh;
    const int b = bh / p.H;
    const int h = bh % p.H;

    const __bf16* Q = (const __bf16*)p.q + b * p.sq.b + h * p.sq.h;
    const __bf16* K = (const __bf16*)p.k + b * p.sk.b + h * p.sk.h;
    const __bf16* V = (const __bf16*)p.v + b * p.sv.b + h * p.sv.h;
    const __bf16* dO = (const __bf16*)p.dout + b * p.sdo.b + h * p.sdo.h;
    float* dQa = p.dq_acc + b * p.sacc.b + h * p.sacc.h;
    const float* LSE = p.lse + (int64_t)bh * p.Tq;
    const float* DL = p.delta + (int64_t)bh * p.Tq;

    const int k0 = kblk * BK;
    const int k0w = k0 + wave * KW;
    const int key = k0w + l16;

    // K / V operands: chunk kk takes row `key`, columns 32 kk + 8 g4 .. +7.
    bf16x8 kf[NKC], vf[NKC];
#pragma unroll
    for (int kk = 0; kk < NKC; ++kk) {
        if (key < p.Tk) {
            kf[kk] = *reinterpret_cast<const bf16x8*>(K + (int64_t)key * p.sk.t + 32 * kk + 8 * g4);
            vf[kk] = *reinterpret_cast<const bf16x8*>(V + (int64_t)key * p.sv.t + 32 * kk + 8 * g4);
        } else {
            kf[kk] = vf[kk] = bf16x8{};
        }
    }

    f32x4 dv_acc[NDB], dk_acc[NDB];
#pragma unroll
    for (int i = 0; i < NDB; ++i) {
        dv_acc[i] = f32x4{0.f, 0.f, 0.f, 0.f};
        dk_acc[i] = f32x4{0.f, 0.f, 0.f, 0.f};
    }

    const int q_begin = wk.q_begin;
    const int q_end = wk.q_end;
    const float c = p.c;

    // Q / dO staging, row-major only (double-buffered with dS, one barrier
    // per tile): thread (rq, cq) stores 16-byte
    // chunk cq of rows rq and rq + 16, so a wave's 16 lanes of one row write
    // 256 consecutive bytes (conflict-free).  The dV^T / dK^T operands read
    // the same rows transposed (ds_read_b64_tr_b16).
    bf16x8 ra[2], rb[2];
    float r_lse[2] = {0.f, 0.f}, r_dl[2] = {0.f, 0.f};
    // 0: Q, 1: dO; wave-uniform, and read as such so the row stride is a
    // scalar (a per-lane value there made the compiler loop over its lanes'
    // values for the buffer loads' scalar offset)
    const int which = __builtin_amdgcn_readfirstlane(tid / QTASK);
    const int rem = tid % QTASK;
    const int cq = rem % C8, rq = rem / C8;
    static_assert(QTASK == (BQ / 2) * C8 && C8 == 16, "16 chunks x 16 row pairs per tensor");
    // register set rs (0 / 1, compile-time at every call) <- tile q0
    auto gload_q = [&](auto rs_c, int q0, int lim) {
        constexpr int rs = decltype(rs_c)::value;
        const int rows = min(lim - q0, BQ);
        const int64_t st = which ? p.sdo.t : p.sq.t;
        const auto rsrc = row_rsrc(which ? dO : Q, st, q0, rows, D);
        const uint32_t voff = (uint32_t)(((int64_t)rq * st + 8 * cq) * 2);
        ra[rs] = buffer_ld8bf(rsrc, voff, 0);
        rb[rs] = buffer_ld8bf(rsrc, voff, (uint32_t)((BQ / 2) * st * 2));
        r_lse[rs] = buffer_ld1(row_rsrc(LSE, 1, q0, rows, 1), (uint32_t)tid * 4, 0);
        r_dl[rs] = buffer_ld1(row_rsrc(DL, 1, q0, rows, 1), (uint32_t)tid * 4, 0);
    };
    auto sstore_q = [&](auto rs_c, int sb) {
        constexpr int rs = decltype(rs_c)::value;
        __bf16(*rows)[QS] = which ? dOs2[sb] : Qs2[sb];
        *reinterpret_cast<bf16x8*>(&rows[rq][8 * cq]) = ra[rs];
        *reinterpret_cast<bf16x8*>(&rows[rq + BQ / 2][8 * cq]) = rb[rs];
        if (tid < BQ) {
            lse_s2[sb][tid] = r_lse[rs] * kLog2e;  // LSE in base 2
            dl_s2[sb][tid] = r_dl[rs];
        }
    };
    using R0 = std::integral_constant<int, 0>;
    using R1 = std::integral_constant<int, 1>;
    // DQD: LSE / delta alone through registers (two tiles ahead), and Q / dO
    // by direct-to-LDS loads: a tile of one tensor is 32 rows of QS / 8 16-byte
    // slots (the last two of each row padding) = NJQ one-KiB instructions,
    // waves 0-3 loading Q and 4-7 dO, wave w's share being instructions
    // w % 4, w % 4 + 4, ... (one past the last repeats the last: the same
    // bytes into the same slots, no load behind a branch).
    auto gload_l = [&](auto rs_c, int q0, int lim) {
        constexpr int rs = decltype(rs_c)::value;
        const int rows = min(lim - q0, BQ);
        r_lse[rs] = buffer_ld1(row_rsrc(LSE, 1, q0, rows, 1), (uint32_t)tid * 4, 0);
        r_dl[rs] = buffer_ld1(row_rsrc(DL, 1, q0, rows, 1), (uint32_t)tid * 4, 0);
    };
    auto sstore_l = [&](auto rs_c, int sb) {
        constexpr int rs = decltype(rs_c)::value;
        if (tid < BQ) {
            lse_s2[sb][tid] = r_lse[rs] * kLog2e;  // LSE in base 2
            dl_s2[sb][tid] = r_dl[rs];
        }
    };
    constexpr int SQ = QS / 8;
    constexpr int NJQ = BQ * SQ / 64;
    static_assert(BQ * SQ % 64 == 0, "a tile must fill whole instructions");
    constexpr int NIQ = (NJQ + 3) / 4;
    const int64_t st_q = which ? p.sdo.t : p.sq.t;
    uint32_t q_voff[NIQ];
    int q_lds[NIQ];
#pragma unroll
    for (int i = 0; i < NIQ; ++i) {
        const int j = min(((tid >> 6) & 3) + 4 * i, NJQ - 1);
        const int slot = 64 * j + lane;
        q_voff[i] = (uint32_t)(((int64_t)(slot / SQ) * st_q + 8 * min(slot % SQ, C8 - 1)) * 2);
        q_lds[i] = 1024 * j;
    }
    auto dload_q = [&](int sb, int q0, int lim) {
        const int rows = min(lim - q0, BQ);
        const auto rsrc = row_rsrc(which ? dO : Q, st_q, q0, rows, D);
        char* base = which ? reinterpret_cast<char*>(&dOs2[sb][0][0]) : reinterpret_cast<char*>(&Qs2[sb][0][0]);
#pragma unroll
        for (int i = 0; i < NIQ; ++i) buffer_ld16_lds(rsrc, base + q_lds[i], q_voff[i]);
    };

    // Short rows (bwd_split.h): their delta before the main loop.
    const int qs_end = SHORT && kblk == 0 ? min(q_end, p.n_short) : q_begin;  // short rows: [q_begin, qs_end)
    if (SHORT && q_begin < qs_end)
        bwd_short_prologue<D, NW, BK, PR, PSTR, false>(p, bh, Q, K, V, dO, q_begin, qs_end, lds.pr.k, lds.pr.v,
                                                       lds.pr.q, lds.pr.d, nullptr);

    // K^T of the key block (keys contiguous per d row), for dQ.
#pragma unroll
    for (int i = 0; i < KLPT; ++i) {
        if constexpr (DQD) break;
        const int f = tid + NT * i;
        if (f >= KTASK) continue;
        const int kp = f % (BK / 2), c8 = f / (BK / 2);
        const int r0 = k0 + 2 * kp;
        const bf16x8 a = r0 < p.Tk ? *reinterpret_cast<const bf16x8*>(K + (int64_t)r0 * p.sk.t + 8 * c8) : bf16x8{};
        const bf16x8 c = r0 + 1 < p.Tk ? *reinterpret_cast<const bf16x8*>(K + (int64_t)(r0 + 1) * p.sk.t + 8 * c8)
                                       : bf16x8{};
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            bf16x2 pr;
            pr[0] = a[e];
            pr[1] = c[e];
            *reinterpret_cast<bf16x2*>(&KTs[8 * c8 + e][2 * kp]) = pr;
        }
    }

    // Q / dO tiles are loaded two tiles ahead (two register sets), stored one
    // tile ahead: a load that misses the L2 has a whole tile more to arrive.
    // (DQD: Q / dO straight into LDS one tile ahead, LSE / delta as above.)
    if constexpr (DQD) {
        dload_q(0, q_begin, p.Tq);
        gload_l(R0{}, q_begin, p.Tq);
        sstore_l(R0{}, 0);
        gload_l(R1{}, q_begin + BQ, q_begin + BQ < q_end ? p.Tq : 0);
        __builtin_amdgcn_s_waitcnt(0);  // this wave's loads have landed in LDS
    } else {
        gload_q(R0{}, q_begin, p.Tq);
        sstore_q(R0{}, 0);
        gload_q(R1{}, q_begin + BQ, q_begin + BQ < q_end ? p.Tq : 0);
    }
    __syncthreads();

    // dQ blocks of this wave: query half qhw, d blocks 2 dcw and 2 dcw + 1
    const int qhw = wave & 1;
    const int dcw = wave >> 1;

    // step of tile q0 in LDS buffer cb; register set LS holds tile q0 + BQ,
    // the other set takes tile q0 + 2 BQ
    auto step = [&](int q0, int cb, auto ls_c) {
        constexpr int LS = decltype(ls_c)::value;
        if constexpr (DQD) {
            gload_l(std::integral_constant<int, 1 - LS>{}, q0 + 2 * BQ, q0 + 2 * BQ < q_end ? p.Tq : 0);
            if (q0 + BQ < q_end) dload_q(cb ^ 1, q0 + BQ, p.Tq);
        } else {
            gload_q(std::integral_constant<int, 1 - LS>{}, q0 + 2 * BQ, q0 + 2 * BQ < q_end ? p.Tq : 0);
        }
        __bf16(*Qs)[QS] = Qs2[cb];
        __bf16(*dOs)[QS] = dOs2[cb];
        __bf16(*dSs)[SS] = dSs2[cb];
        const float* lse_s = lse_s2[cb];
        const float* dl_s = dl_s2[cb];

        const bool active = !p.causal || (q0 + BQ - 1 + p.off >= k0w);
        bf16x8 pb, dsb;
        if (active && k0w < p.Tk) {
            f32x4 s[2], dp[2];
            bf16x8 qa[2][NKC], da[2][NKC];
#pragma unroll
            for (int qh = 0; qh < 2; ++qh)
#pragma unroll
                for (int kk = 0; kk < NKC; ++kk) {
                    qa[qh][kk] = *reinterpret_cast<const bf16x8*>(&Qs[16 * qh + l16][32 * kk + 8 * g4]);
                    da[qh][kk] = *reinterpret_cast<const bf16x8*>(&dOs[16 * qh + l16][32 * kk + 8 * g4]);
                }
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int kk = 0; kk < NKC; ++kk)
#pragma unroll
                for (int qh = 0; qh < 2; ++qh) {
                    s[qh] = mfma16x16x32bf16(qa[qh][kk], kf[kk], kk == 0 ? f32x4{0.f, 0.f, 0.f, 0.f} : s[qh]);
                    dp[qh] = mfma16x16x32bf16(da[qh][kk], vf[kk], kk == 0 ? f32x4{0.f, 0.f, 0.f, 0.f} : dp[qh]);
                }
            // P and dS: register r of half qh is query 16 qh + 4 g4 + r
            const f32x4 L0 = *reinterpret_cast<const f32x4*>(&lse_s[4 * g4]);
            const f32x4 L1 = *reinterpret_cast<const f32x4*>(&lse_s[16 + 4 * g4]);
            const f32x4 D0 = *reinterpret_cast<const f32x4*>(&dl_s[4 * g4]);
            const f32x4 D1 = *reinterpret_cast<const f32x4*>(&dl_s[16 + 4 * g4]);
            auto p_ds = [&](auto masked) {
#pragma unroll
                for (int qh = 0; qh < 2; ++qh)
#pragma unroll
                    for (int r = 0; r < 4; ++r) {
                        const float Lq = qh ? L1[r] : L0[r];
                        const float Dq = qh ? D1[r] : D0[r];
                        float pr = fast_exp2(fmaf(s[qh][r], c, -Lq));
                        if constexpr (decltype(masked)::value) {
                            const int qi = q0 + 16 * qh + 4 * g4 + r;
                            const bool vis = (qi < p.Tq) && (key < p.Tk) && (!p.causal || key <= qi + p.off);
                            pr = vis ? pr : 0.f;
                        }
                        pb[4 * qh + r] = (__bf16)pr;
                        dsb[4 * qh + r] = (__bf16)(pr * (dp[qh][r] - Dq));
                    }
            };
            const bool need_mask = q0 + BQ > p.Tq || k0w + KW > p.Tk || (p.causal && k0w + KW - 1 > q0 + p.off);
            if (need_mask)
                p_ds(std::true_type{});
            else
                p_ds(std::false_type{});
            if (bwd_one_key_tile(p, q0, k0w)) {  // a row with one visible key: dS = P (dP - dP) = 0
#pragma unroll
                for (int r = 0; r < 8; ++r)
                    if (bwd_one_key_row(p, q0 + 16 * (r >> 2) + 4 * g4 + (r & 3))) dsb[r] = (__bf16)0.f;
            }
            // dV^T += dO^T P ; dK^T += Q^T dS over the 32 queries (one MFMA per d block).
            // The B operands' element j is query 16 (j / 4) + 4 g4 + j % 4, so lane
            // (l16, g4) takes column 16 db + l16 of rows 4 g4 + {0..3} and 16 + 4 g4
            // + {0..3}: two transpose reads, lane s of the 16 addressing row
            // 4 g4 + s / 4 at columns 16 db + 4 (s % 4).
            bf16x8 ado[NDB], aq[NDB];
            const int tr_row = 4 * g4 + (l16 >> 2), tr_col = 4 * (l16 & 3);
#pragma unroll
            for (int db = 0; db < NDB; ++db) {
                const bf16x4 dlo = ds_read_tr16(&dOs[tr_row][16 * db + tr_col]);
                const bf16x4 dhi = ds_read_tr16(&dOs[tr_row + 16][16 * db + tr_col]);
                const bf16x4 qlo = ds_read_tr16(&Qs[tr_row][16 * db + tr_col]);
                const bf16x4 qhi = ds_read_tr16(&Qs[tr_row + 16][16 * db + tr_col]);
                ado[db] = __builtin_shufflevector(dlo, dhi, 0, 1, 2, 3, 4, 5, 6, 7);
                aq[db] = __builtin_shufflevector(qlo, qhi, 0, 1, 2, 3, 4, 5, 6, 7);
            }
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int db = 0; db < NDB; ++db) {
                dv_acc[db] = mfma16x16x32bf16(ado[db], pb, dv_acc[db]);
                dk_acc[db] = mfma16x16x32bf16(aq[db], dsb, dk_acc[db]);
            }
        } else {
            pb = dsb = bf16x8{};
        }
        if constexpr (DQD) {
            sstore_l(ls_c, cb ^ 1);
            __builtin_amdgcn_s_waitcnt(0);  // this wave's Q / dO loads have landed in LDS
            __syncthreads();
            return;
        } else {
            // dS of this wave -> LDS (rows = queries, columns = the block's keys)
#pragma unroll
            for (int r = 0; r < 8; ++r) dSs[16 * (r >> 2) + 4 * g4 + (r & 3)][wave * KW + l16] = dsb[r];
            sstore_q(ls_c, cb ^ 1);
            __syncthreads();
        }

        // ---- dQ (32 x D) += dS (32 x BK) K (BK x D): this wave's two 16x16 blocks
        const auto rdq = row_rsrc(dQa, p.sacc.t, q0, min(p.Tq - q0, BQ), D);
        f32x4 acc0, acc1;
        bf16x8 a[BK / 32], b0[BK / 32], b1[BK / 32];
#pragma unroll
        for (int kk = 0; kk < BK / 32; ++kk) {
            a[kk] = *reinterpret_cast<const bf16x8*>(&dSs[16 * qhw + l16][32 * kk + 8 * g4]);
            b0[kk] = *reinterpret_cast<const bf16x8*>(&KTs[32 * dcw + l16][32 * kk + 8 * g4]);
            b1[kk] = *reinterpret_cast<const bf16x8*>(&KTs[32 * dcw + 16 + l16][32 * kk + 8 * g4]);
        }
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int kk = 0; kk < BK / 32; ++kk) {
            acc0 = mfma16x16x32bf16(a[kk], b0[kk], kk == 0 ? f32x4{0.f, 0.f, 0.f, 0.f} : acc0);
            acc1 = mfma16x16x32bf16(a[kk], b1[kk], kk == 0 ? f32x4{0.f, 0.f, 0.f, 0.f} : acc1);
        }
        const uint32_t voff = (uint32_t)(((int64_t)(16 * qhw + 4 * g4) * p.sacc.t + 32 * dcw + l16) * 4);
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            buffer_atomic_add(rdq, acc0[r] * p.scale, voff, (uint32_t)((int64_t)r * p.sacc.t * 4));
            buffer_atomic_add(rdq, acc1[r] * p.scale, voff + 64, (uint32_t)((int64_t)r * p.sacc.t * 4));
        }
    };
    for (int q0 = q_begin; q0 < q_end; q0 += 2 * BQ) {
        step(q0, 0, R1{});
        if (q0 + BQ < q_end) step(q0 + BQ, 1, R0{});
    }

    // split plans: the fix-up takes the accumulators as two f32x16 each
    f32x16 dk16[NDB / 4], dv16[NDB / 4];
#pragma unroll
    for (int i = 0; i < NDB / 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                dk16[i][4 * j + r] = dk_acc[4 * i + j][r];
                dv16[i][4 * j + r] = dv_acc[4 * i + j][r];
            }
    if (!bwd_fixup<NT>(p, wk, dk16, dv16)) return;
    if (key < p.Tk) {
        uint16_t* dKp = (uint16_t*)p.dk + b * p.sdk.b + h * p.sdk.h + (int64_t)key * p.sdk.t;
        uint16_t* dVp = (uint16_t*)p.dv + b * p.sdv.b + h * p.sdv.h + (int64_t)key * p.sdv.t;
#pragma unroll
        for (int i = 0; i < NDB / 4; ++i)
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int db = 4 * i + j;
                f32x4 a, v;
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    a[r] = dk16[i][4 * j + r] * p.scale;
                    v[r] = dv16[i][4 * j + r];
                }
                st4(dKp + 16 * db + 4 * g4, a);
                st4(dVp + 16 * db + 4 * g4, v);
            }
    }
}


// ---- query-major dQ pass (bf16, long key ranges) ---------------------------
//
// 4 waves x 32 query rows per workgroup (heaviest query tiles first), key
// tiles of BN keys streamed through LDS as K rows and V rows; Q and dO rows of
// the wave's queries in VGPRs, LSE and delta one value per lane.  Per tile,
// with queries on the lane axis:
//   S^T = K Q^T, dP^T = V dO^T, P^T = exp2(S^T c - L), dS^T = P^T (dP^T - delta)
//   dQ^T += K^T dS^T (dS^T straight from registers, as the forward's P^T, and
//                     K^T read from the K rows by transpose reads, as the
//                     forward's V^T)
// dQ accumulates in fp32 VGPRs and is written once (bf16, times the scale):
// no accumulator, no atomics, no conversion pass, and the same sum order on
// every run.  It recomputes S and dP (two more products per score than the
// atomic path's dQ), so it pays only where the atomics bound the fused
// kernel (bwd_dq_direct): at D = 128 with many key blocks.  (At D = 64 it
// measured 28% slower than the atomics at B1 H16 T8192.)
//
// The K row stride serves both reads of K without bank conflicts: 16-byte
// row reads (lane l32 at row l32, 16 g bytes in) need an odd number of
// 16-byte units, and the transpose reads (4 rows x 32 bytes per 16 lanes)
// need the rows' 32-byte windows disjoint modulo 256 bytes: 304 B at D = 128,
// 144 B at D = 64, 112 B at D = 32.
template <int D>
struct DqBf16Tile {
    static constexpr int BN = D >= 128 ? 32 : 64;
    static constexpr int KS = D == 128 ? D + 24 : D == 64 ? D + 8 : D + 24;  // K row stride (bf16)
    static constexpr int VS = D + 8;                                         // V row stride (bf16)
    static constexpr int SK = KS / 8, SV = VS / 8;                           // 16-byte slots per row
    static constexpr int NJK = (BN * SK + 63) / 64, NJV = (BN * SV + 63) / 64;  // load instructions
    // rows allocated: the last instruction's slots past the tile land in spare rows
    static constexpr int KROWS = (NJK * 1024 + 2 * KS - 1) / (2 * KS);
    static constexpr int VROWS = (NJV * 1024 + 2 * VS - 1) / (2 * VS);
};

template <int D>
__global__ __launch_bounds__(256, 2) void bwd_dq_bf16_kernel(BwdParams p) {
    using T = DqBf16Tile<D>;
    constexpr int BM = kBwdDqBM;
    constexpr int BN = T::BN, KS = T::KS, VS = T::VS, SK = T::SK, SV = T::SV;
    constexpr int NJK = T::NJK, NJV = T::NJV;
    constexpr int NKK = D / 16;
    constexpr int NKB = BN / 32;
    constexpr int NDB = D / 32;
    constexpr int C8 = D / 8;
    constexpr int NI = ((NJK > NJV ? NJK : NJV) + 3) / 4;  // load instructions per wave and kind

    // Two buffers as separate arrays, each step's named at compile time, so
    // the compiler can tell the loads into one from the reads of the other.
    __shared__ __attribute__((aligned(16))) __bf16 Ks0[T::KROWS][KS];
    __shared__ __attribute__((aligned(16))) __bf16 Ks1[T::KROWS][KS];
    __shared__ __attribute__((aligned(16))) __bf16 Vs0[T::VROWS][VS];
    __shared__ __attribute__((aligned(16))) __bf16 Vs1[T::VROWS][VS];

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

    const __bf16* Q = (const __bf16*)p.q + b * p.sq.b + h * p.sq.h;
    const __bf16* K = (const __bf16*)p.k + b * p.sk.b + h * p.sk.h;
    const __bf16* V = (const __bf16*)p.v + b * p.sv.b + h * p.sv.h;
    const __bf16* dO = (const __bf16*)p.dout + b * p.sdo.b + h * p.sdo.h;

    const int q0w = qtile * BM + wave * 32;
    const int qrow = q0w + l32;
    bf16x8 qf[NKK], df[NKK];
#pragma unroll
    for (int kk = 0; kk < NKK; ++kk) {
        if (qrow < p.Tq) {
            qf[kk] = *reinterpret_cast<const bf16x8*>(Q + (int64_t)qrow * p.sq.t + 16 * kk + 8 * g);
            df[kk] = *reinterpret_cast<const bf16x8*>(dO + (int64_t)qrow * p.sdo.t + 16 * kk + 8 * g);
        } else {
            qf[kk] = df[kk] = bf16x8{};
        }
    }
    const float Lq = qrow < p.Tq ? p.lse[(int64_t)bh * p.Tq + qrow] * kLog2e : 0.f;
    const float Dq = qrow < p.Tq ? p.delta[(int64_t)bh * p.Tq + qrow] : 0.f;
    const bool one_key = qrow < p.Tq && bwd_one_key_row(p, qrow);
    const bool one_key_wave = p.causal ? (-p.off >= q0w && -p.off < q0w + 32) : p.Tk == 1;  // wave-uniform

    int kv_end = p.Tk;
    if (p.causal) kv_end = min(p.Tk, qtile * BM + BM + p.off);
    const int nt = (kv_end + BN - 1) / BN;
    const int wave_kend = p.causal ? min(kv_end, q0w + 32 + p.off) : kv_end;

    // Key tile u goes from memory straight into LDS through gfx950's 16-byte
    // direct-to-LDS buffer loads: the 64 lanes of one instruction fill 1 KiB
    // at the instruction's LDS base, lane l at +16 l, so a tile's padded rows
    // are one run of 16-byte slots and instruction j fills slots 64 j ..
    // 64 j + 63, each lane loading the chunk of its slot (a pad slot repeats
    // its row's last chunk; slots past the tile, in the spare rows, read
    // outside the resource: zeros).  Wave w issues instructions w, w + 4, ...,
    // and one past the last repeats the last (the same bytes into the same
    // slots), so no load is behind a branch.  The resources cover the tile's
    // rows, so keys past Tk land as zeros.
    const int64_t kstep = (int64_t)BN * p.sk.t, vstep = (int64_t)BN * p.sv.t;
    const __bf16* kt = K;
    const __bf16* vt = V;
    const int wave_u = __builtin_amdgcn_readfirstlane(wave);
    uint32_t k_voff[NI], v_voff[NI];
    int k_lds[NI], v_lds[NI];
#pragma unroll
    for (int i = 0; i < NI; ++i) {
        const int jk = min(wave_u + 4 * i, NJK - 1), jv = min(wave_u + 4 * i, NJV - 1);
        const int sk = 64 * jk + lane, sv = 64 * jv + lane;
        k_voff[i] = sk < BN * SK ? (uint32_t)(((int64_t)(sk / SK) * p.sk.t + 8 * min(sk % SK, C8 - 1)) * 2)
                                 : 0x80000000u;
        v_voff[i] = sv < BN * SV ? (uint32_t)(((int64_t)(sv / SV) * p.sv.t + 8 * min(sv % SV, C8 - 1)) * 2)
                                 : 0x80000000u;
        k_lds[i] = 1024 * jk;
        v_lds[i] = 1024 * jv;
    }
    auto rows_of = [&](int u) { return u < nt ? min(p.Tk - u * BN, BN) : 0; };
    auto dload = [&](__bf16 (&Kd)[T::KROWS][KS], __bf16 (&Vd)[T::VROWS][VS], int rows) {
        const auto rk = row_rsrc(kt, p.sk.t, 0, rows, D);
        const auto rv = row_rsrc(vt, p.sv.t, 0, rows, D);
#pragma unroll
        for (int i = 0; i < NI; ++i) {
            buffer_ld16_lds(rk, reinterpret_cast<char*>(&Kd[0][0]) + k_lds[i], k_voff[i]);
            buffer_ld16_lds(rv, reinterpret_cast<char*>(&Vd[0][0]) + v_lds[i], v_voff[i]);
        }
        kt += kstep;
        vt += vstep;
    };
    using B0 = std::integral_constant<int, 0>;
    using B1 = std::integral_constant<int, 1>;

    // transposed K reads: this lane's key-row offset and column offset
    const int tr_row = (lane & 15) >> 2;
    const int tr_col = 16 * ((lane >> 4) & 1) + 4 * (lane & 3);

    f32x16 dq[NDB];
#pragma unroll
    for (int i = 0; i < NDB; ++i) dq[i] = f32x16{};
    const float c = p.c;

    dload(Ks0, Vs0, rows_of(0));
    __builtin_amdgcn_s_waitcnt(0);  // this wave's loads have landed in LDS
    __syncthreads();

    // Step u reads buffer u % 2 while tile u + 1 loads into the other one,
    // which every wave finished reading before the previous step's barrier;
    // the step ends by waiting for its loads, then the barrier.
    auto step = [&](int u, auto buf_c) {
        constexpr int BUF = decltype(buf_c)::value;
        __bf16(&Kc)[T::KROWS][KS] = BUF ? Ks1 : Ks0;
        __bf16(&Vc)[T::VROWS][VS] = BUF ? Vs1 : Vs0;
        const int k0 = u * BN;
        dload(BUF ? Ks0 : Ks1, BUF ? Vs0 : Vs1, rows_of(u + 1));
        if (k0 < wave_kend) {
            f32x16 s[NKB], dp[NKB];
            bf16x8 ak[NKK][NKB], av[NKK][NKB];
#pragma unroll
            for (int kk = 0; kk < NKK; ++kk)
#pragma unroll
                for (int kb = 0; kb < NKB; ++kb) {
                    ak[kk][kb] = *reinterpret_cast<const bf16x8*>(&Kc[kb * 32 + l32][16 * kk + 8 * g]);
                    av[kk][kb] = *reinterpret_cast<const bf16x8*>(&Vc[kb * 32 + l32][16 * kk + 8 * g]);
                }
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int kk = 0; kk < NKK; ++kk)
#pragma unroll
                for (int kb = 0; kb < NKB; ++kb) {
                    s[kb] = mfma32x32x16bf16(ak[kk][kb], qf[kk], kk == 0 ? f32x16{} : s[kb]);
                    dp[kb] = mfma32x32x16bf16(av[kk][kb], df[kk], kk == 0 ? f32x16{} : dp[kb]);
                }
            // register r of block kb: key k0 + kb*32 + 8 (r / 4) + 4 g + r % 4, query qrow
            const bool need_mask = (k0 + BN > p.Tk) || (qtile * BM + BM > p.Tq) || (p.causal && (k0 + BN - 1 > q0w + p.off));
            const int lim = p.causal ? min(p.Tk - 1, qrow + p.off) : p.Tk - 1;
            bf16x8 dsb[NKB][2];
            // the visibility test only on tiles that cross the diagonal or the ends
            auto p_ds = [&](auto masked) {
#pragma unroll
                for (int kb = 0; kb < NKB; ++kb)
#pragma unroll
                    for (int r = 0; r < 16; ++r) {
                        float pr = fast_exp2(fmaf(s[kb][r], c, -Lq));
                        if constexpr (decltype(masked)::value) {
                            const int key = k0 + kb * 32 + 8 * (r >> 2) + 4 * g + (r & 3);
                            pr = (key <= lim && qrow < p.Tq) ? pr : 0.f;
                        }
                        dsb[kb][r >> 3][r & 7] = (__bf16)(pr * (dp[kb][r] - Dq));
                    }
            };
            if (need_mask)
                p_ds(std::true_type{});
            else
                p_ds(std::false_type{});
            if (one_key_wave && k0 == 0) {  // a row with one visible key: dS = P (dP - dP) = 0
#pragma unroll
                for (int kb = 0; kb < NKB; ++kb)
                    if (one_key) dsb[kb][0] = dsb[kb][1] = bf16x8{};
            }
            // dQ^T[d][q] += K^T[d][keys] dS^T[keys][q]: MFMA m of key block kb takes
            // dS^T of keys 16 m + 4 g + {0..3} and 16 m + 8 + 4 g + {0..3}; lane
            // (group G = lane / 16, i = lane % 16) addresses key row key + i / 4,
            // columns db*32 + 16 (G % 2) + 4 (i % 4) and receives column
            // db*32 + l32 of keys key + {0..3} (then + 8 + {0..3})
            bf16x8 akt[NDB][NKB][2];
#pragma unroll
            for (int db = 0; db < NDB; ++db)
#pragma unroll
                for (int kb = 0; kb < NKB; ++kb)
#pragma unroll
                    for (int m = 0; m < 2; ++m) {
                        const __bf16* kp = &Kc[kb * 32 + 16 * m + 4 * g + tr_row][db * 32 + tr_col];
                        const bf16x4 lo = ds_read_tr16(kp);
                        const bf16x4 hi = ds_read_tr16(kp + 8 * KS);
                        akt[db][kb][m] = __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
                    }
            __builtin_amdgcn_sched_barrier(0);
            // At D = 128 the dQ MFMAs run at raised wave priority (issued ahead of the
            // other wave's softmax VALU work): config 4 455 -> 439 us, B8 H12 T1024
            // -1%, B2 H8 T4096 +1.6%; D = 32 / 64 measured within 1% and keep the default.
            if constexpr (D >= 128) __builtin_amdgcn_s_setprio(1);
#pragma unroll
            for (int kb = 0; kb < NKB; ++kb)
#pragma unroll
                for (int m = 0; m < 2; ++m)
#pragma unroll
                    for (int db = 0; db < NDB; ++db) dq[db] = mfma32x32x16bf16(akt[db][kb][m], dsb[kb][m], dq[db]);
            if constexpr (D >= 128) __builtin_amdgcn_s_setprio(0);
        }
        __builtin_amdgcn_s_waitcnt(0);
        __syncthreads();
    };
    for (int u = 0; u < nt; u += 2) {
        step(u, B0{});
        if (u + 1 < nt) step(u + 1, B1{});
    }
    if (qrow < p.Tq) {
        uint16_t* dst = (uint16_t*)p.dq + b * p.sdq.b + h * p.sdq.h + (int64_t)qrow * p.sdq.t;
#pragma unroll
        for (int db = 0; db < NDB; ++db)
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                f32x4 val;
#pragma unroll
                for (int cc = 0; cc < 4; ++cc) val[cc] = dq[db][4 * j + cc] * p.scale;
                st4(dst + db * 32 + 8 * j + 4 * g, val);
            }
    }
}

int launch_bwd_dq_bf16(const BwdParams& p, hipStream_t s) {
    const dim3 grid((unsigned)(p.n_qtiles * p.B * p.H));
    switch (p.D) {
        case 32: hipLaunchKernelGGL((bwd_dq_bf16_kernel<32>), grid, dim3(256), 0, s, p); break;
        case 64: hipLaunchKernelGGL((bwd_dq_bf16_kernel<64>), grid, dim3(256), 0, s, p); break;
        case 128: hipLaunchKernelGGL((bwd_dq_bf16_kernel<128>), grid, dim3(256), 0, s, p); break;
        default: return (int)hipErrorInvalidValue;
    }
    return (int)hipGetLastError();
}

int bwd_main_bf16_occupancy(int D, int* blocks_per_cu) {
    switch (D) {
        case 32: return (int)hipOccupancyMaxActiveBlocksPerMultiprocessor(blocks_per_cu, bwd_main_bf16_kernel<32, false, false>, 64 * bwd_bf16_waves(32), 0);
        case 64: return (int)hipOccupancyMaxActiveBlocksPerMultiprocessor(blocks_per_cu, bwd_main_bf16_kernel<64, false, false>, 64 * bwd_bf16_waves(64), 0);
        case 128: return (int)hipOccupancyMaxActiveBlocksPerMultiprocessor(blocks_per_cu, bwd_main_bf16_w16_kernel<128, false, false>, 512, 0);
        default: return (int)hipErrorInvalidValue;
    }
}

int launch_bwd_main_bf16(const BwdParams& p, hipStream_t s) {
    // every row short (Tk within the key block): delta from the workspace for all
    const bool dws = p.n_short >= p.Tq;
    const dim3 grid((unsigned)(p.n_groups ? p.n_groups * bwd_padded_heads(p.B * p.H) : p.n_kblocks * p.B * p.H));
    switch (p.D) {
        case 32:
            if (dws) hipLaunchKernelGGL((bwd_main_bf16_kernel<32, true, true>), grid, dim3(64 * bwd_bf16_waves(32)), 0, s, p);
            else if (p.n_short > 0) hipLaunchKernelGGL((bwd_main_bf16_kernel<32, false, true>), grid, dim3(64 * bwd_bf16_waves(32)), 0, s, p);
            else hipLaunchKernelGGL((bwd_main_bf16_kernel<32, false, false>), grid, dim3(64 * bwd_bf16_waves(32)), 0, s, p);
            break;
        case 64:
            if (dws) hipLaunchKernelGGL((bwd_main_bf16_kernel<64, true, true>), grid, dim3(64 * bwd_bf16_waves(64)), 0, s, p);
            else if (p.n_short > 0) hipLaunchKernelGGL((bwd_main_bf16_kernel<64, false, true>), grid, dim3(64 * bwd_bf16_waves(64)), 0, s, p);
            else hipLaunchKernelGGL((bwd_main_bf16_kernel<64, false, false>), grid, dim3(64 * bwd_bf16_waves(64)), 0, s, p);
            break;
        case 128:
            if (p.dq_direct) {
                if (p.n_short > 0) hipLaunchKernelGGL((bwd_main_bf16_w16_kernel<128, true, true>), grid, dim3(512), 0, s, p);
                else hipLaunchKernelGGL((bwd_main_bf16_w16_kernel<128, false, true>), grid, dim3(512), 0, s, p);
            } else {
                if (p.n_short > 0) hipLaunchKernelGGL((bwd_main_bf16_w16_kernel<128, true, false>), grid, dim3(512), 0, s, p);
                else hipLaunchKernelGGL((bwd_main_bf16_w16_kernel<128, false, false>), grid, dim3(512), 0, s, p);
            }
            break;
        default: return (int)hipErrorInvalidValue;
    }
    return (int)hipGetLastError();
}

}  // namespace inf
