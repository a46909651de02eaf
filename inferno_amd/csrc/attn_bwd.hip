// attn_bwd.hip -- fused causal attention backward for gfx950 (recompute).
//
// Kernel 1 (bwd_pre): delta[i] = sum_d dO[i,d] * O[i,d] per query row (the
// row dot that SoftmaxBackward computes as sum_j dP_ij P_ij), and zeroes the
// fp32 dQ accumulator.  (The bf16 main kernel at D <= 64 forms delta itself,
// and then this pass only zeroes.)
//
// Kernel 2 (bwd_main): one workgroup = 4 waves = 128 keys of one (b, h); each
// wave owns 32 keys and keeps K and V for them in VGPRs plus its dK^T and dV^T
// accumulators for the whole kernel, so dK and dV are written exactly once,
// with no atomics.  The workgroup walks query tiles of 32 rows from the first
// row that can see its keys to the end.  Per tile and wave:
//
//   S  (q x keys)   = Q K^T          A = Q from LDS, B = K^T in VGPRs
//   dP (q x keys)   = dO V^T         A = dO from LDS, B = V^T in VGPRs
//   P  = exp2(S*c - lse*log2e), masked entries exactly 0
//   dS = P * (dP - delta)
//   dV^T += dO^T P                   B = P straight from the S accumulators
//   dK^T += Q^T dS                   B = dS straight from the dP accumulators
//
// All four keep keys on the lane axis.  dQ = dS K needs queries on the lane
// axis instead, so each wave writes its dS block to LDS, and after a barrier
// the four waves compute the tile's dQ (32 x D over all 128 keys) with
// v_mfma_f32_16x16x4_f32 and add it to the fp32 accumulator with one
// global atomic add per element per 128-key block.  Workgroup w takes key
// block w / (B*H), so the blocks with the most query tiles start first.
//
// bf16 inputs use the bf16-MFMA main kernel (attn_bwd_bf16.hip) between the
// same pre kernel and a final bwd_cvt that turns the fp32 dQ accumulator into
// bf16 dq.
#include <type_traits>

#include <algorithm>
#include <array>
#include <cmath>
#include <map>
#include <mutex>
#include <vector>

#include "bwd_split.h"
#include "common.h"
#include "kernels.h"

namespace inf {

// Batch, head and position of row `row` of the [B, H, Tq] rows: 32-bit
// divisions when the row count fits (every practical shape), as 64-bit ones
// cost tens of instructions per thread in these memory-bound passes.
__device__ __forceinline__ void bwd_row_split(const BwdParams& p, int64_t rows, int64_t row, int64_t& b, int64_t& h,
                                              int64_t& i) {
    if (rows <= 0xffffffffLL) {
        const uint32_t r = (uint32_t)row, bh = r / (uint32_t)p.Tq;
        i = r - bh * (uint32_t)p.Tq;
        b = bh / (uint32_t)p.H;
        h = bh - (uint32_t)b * (uint32_t)p.H;
    } else {
        const int64_t bh = row / p.Tq;
        i = row % p.Tq;
        b = bh / p.H;
        h = bh % p.H;
    }
}

// delta = rowsum(dO * O) per query row, and the zeroing of the fp32 dQ
// accumulator and the split plan's arrival counters.  Each thread takes one
// 16-byte chunk of O and dO (4 fp32 or 8 bf16 elements; TPR threads per row)
// and the row's threads sum their products with DPP moves.
template <int D, typename E>
constexpr int bwd_pre_tpr() { return D / (16 / (int)sizeof(E)); }
template <int D, typename E>
constexpr int bwd_pre_rows_per_block() { return 256 / bwd_pre_tpr<D, E>(); }

template <int D, typename E>
__global__ __launch_bounds__(256) void bwd_pre_kernel(BwdParams p) {
    constexpr int VEC = 16 / (int)sizeof(E);   // elements per 16-byte chunk
    constexpr int TPR = bwd_pre_tpr<D, E>();    // threads per row
    constexpr int RPB = bwd_pre_rows_per_block<D, E>();
    const int tid = threadIdx.x;
    const int64_t row = (int64_t)blockIdx.x * RPB + tid / TPR;
    const int c = tid % TPR;
    const int64_t rows = (int64_t)p.B * p.H * p.Tq;
    float s = 0.f;
    if (row < rows) {
        int64_t b, h, i;
        bwd_row_split(p, rows, row, b, h, i);
        if (p.pre_delta) {
            const E* po = (const E*)p.o + b * p.so.b + h * p.so.h + i * p.so.t + VEC * c;
            const E* pd = (const E*)p.dout + b * p.sdo.b + h * p.sdo.h + i * p.sdo.t + VEC * c;
            if constexpr (sizeof(E) == 4) {
                const f32x4 o4 = ld4(po), d4 = ld4(pd);
                s = o4[0] * d4[0] + o4[1] * d4[1] + o4[2] * d4[2] + o4[3] * d4[3];
            } else {
                const u16x8 o8 = *reinterpret_cast<const u16x8*>(po);
                const u16x8 d8 = *reinterpret_cast<const u16x8*>(pd);
#pragma unroll
                for (int k = 0; k < 8; ++k) s = fmaf(bf16_to_f32(o8[k]), bf16_to_f32(d8[k]), s);
            }
        }
        if (!p.dq_direct) {
            f32x4* acc = reinterpret_cast<f32x4*>(p.dq_acc + b * p.sacc.b + h * p.sacc.h + i * p.sacc.t + VEC * c);
#pragma unroll
            for (int k = 0; k < VEC / 4; ++k) acc[k] = f32x4{0.f, 0.f, 0.f, 0.f};
        }
    }
    // (p.pre_delta is uniform: the whole grid takes or skips the exchange)
    if (p.pre_delta) {
        s = group_sum<TPR>(s);
        if (row < rows && c == 0) p.delta[row] = s;
    }
    if (blockIdx.x == 0)
        for (int i = tid; i < p.n_split * p.B * p.H; i += 256) p.counters[i] = 0u;
}

// bwd_pre without delta (the bf16 main kernel at D <= 64 forms it): the fp32
// dQ accumulator is one dense [B, H, Tq, D] block, so it is cleared as a flat
// array (16-byte stores over a grid-stride loop), with the split plan's
// arrival counters.
__global__ __launch_bounds__(256) void bwd_zero_kernel(BwdParams p) {
    const int64_t n4 = (int64_t)p.B * p.H * p.Tq * p.D / 4;
    f32x4* acc = reinterpret_cast<f32x4*>(p.dq_acc);
    for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n4; i += (int64_t)gridDim.x * 256)
        acc[i] = f32x4{0.f, 0.f, 0.f, 0.f};
    if (blockIdx.x == 0)
        for (int i = threadIdx.x; i < p.n_split * p.B * p.H; i += 256) p.counters[i] = 0u;
}

template <int D>
struct BwdTile {
    static constexpr int NW = bwd_waves(0, D);  // waves per workgroup, 32 keys each
    static constexpr int BK = 32 * NW;       // keys per workgroup
    static constexpr int QS = D + 4;         // Q / dO row stride in LDS (floats)
    static constexpr int SS = BK + 4;        // dS row stride
    static constexpr int KTS = BK + 4;       // K^T row stride
};

// SHORT: the launch has short rows (p.n_short > 0); without them the kernel
// carries neither the prologue nor the low part of delta.
template <int D, typename E, bool SHORT>
__global__ __launch_bounds__(64 * bwd_waves(0, D), (bwd_waves(0, D) == 8 || D >= 128) ? 1 : 2) void bwd_main_kernel(
    BwdParams p) {
    constexpr int NW = BwdTile<D>::NW;
    constexpr int NT = 64 * NW;
    constexpr int BQ = kBwdBQ;
    constexpr int BK = BwdTile<D>::BK;
    constexpr int HD = D / 2;
    constexpr int NDB = D / 32;
    constexpr int C4 = D / 4;
    constexpr int QS = BwdTile<D>::QS;
    constexpr int SS = BwdTile<D>::SS;
    constexpr int KTS = BwdTile<D>::KTS;
    constexpr int QLPT = BQ * C4 / NT;    // 4-element loads per thread for a Q / dO tile
    constexpr int KLPT = BK * C4 / NT;    // for the K^T staging
    constexpr int NDQ = 2 * (D / 16);     // 16x16 dQ blocks of a query tile, NDQ / NW per wave
    static_assert(BQ * C4 % NT == 0 && BK * C4 % NT == 0 && NDQ % NW == 0, "whole passes");

    __shared__ __attribute__((aligned(16))) float Qs[BQ][QS];
    __shared__ __attribute__((aligned(16))) float dOs[BQ][QS];
    __shared__ __attribute__((aligned(16))) float dSs[BQ][SS];
    __shared__ __attribute__((aligned(16))) float Kts[D][KTS];
    __shared__ __attribute__((aligned(16))) float lse_s[BQ];
    __shared__ __attribute__((aligned(16))) float dl_s[BQ];
    __shared__ __attribute__((aligned(16))) float dlo_s[BQ];  // low part of the short rows' delta (else 0)

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

    const E* Q = (const E*)p.q + b * p.sq.b + h * p.sq.h;
    const E* K = (const E*)p.k + b * p.sk.b + h * p.sk.h;
    const E* V = (const E*)p.v + b * p.sv.b + h * p.sv.h;
    const E* dO = (const E*)p.dout + b * p.sdo.b + h * p.sdo.h;
    float* dQa = p.dq_acc + b * p.sacc.b + h * p.sacc.h;
    const float* LSE = p.lse + (int64_t)bh * p.Tq;
    const float* DL = p.delta + (int64_t)bh * p.Tq;
    const float* DLO = p.delta_lo + (int64_t)bh * p.Tq;

    const int k0 = kblk * BK;
    const int k0w = k0 + wave * 32;
    const int key = k0w + l32;  // this lane's key

    // K^T and V^T operands: lane (l32, g) holds row `key`, columns g*HD + i.
    float kf[HD], vf[HD];
    if (key < p.Tk) {
        const E* ks = K + (int64_t)key * p.sk.t + g * HD;
        const E* vs = V + (int64_t)key * p.sv.t + g * HD;
#pragma unroll
        for (int i = 0; i < HD; i += 4) {
            const f32x4 a = ld4(ks + i);
            const f32x4 c = ld4(vs + i);
            kf[i] = a[0]; kf[i + 1] = a[1]; kf[i + 2] = a[2]; kf[i + 3] = a[3];
            vf[i] = c[0]; vf[i + 1] = c[1]; vf[i + 2] = c[2]; vf[i + 3] = c[3];
        }
    } else {
#pragma unroll
        for (int i = 0; i < HD; ++i) kf[i] = vf[i] = 0.f;
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

    // Query-tile staging.  With PF (D <= 64, where the registers fit) the next
    // tile's Q, dO, LSE and delta are loaded into registers while the current
    // tile computes and stored to LDS right after the dS barrier, when every
    // wave is done with the staged copies: two barriers per tile.  The
    // prefetch is straight-line (a row limit of 0 past the last tile) and keeps
    // raw values, so no wait for it lands inside the MFMA blocks.
    // The loads go through buffer resources over rows [q0, lim): chunk
    // tid + NT i sits NT i / C4 rows below chunk tid, and rows past the
    // resource read as zeros, so a load needs no address arithmetic or branch.
    constexpr bool PF = D <= 64;
    // The LSE is staged in base 2 (scaled by log2(e) once per row instead of
    // once per score) except at D = 64, which measured 2% slower that way at
    // config 2; at D = 32 the staging keeps the kernel within the registers
    // of three workgroups per CU (B4 H16 T1024: 134 -> 119 us).
    constexpr float kLseStage = D == 64 ? 1.f : kLog2e;
    constexpr float kLseRead = D == 64 ? kLog2e : 1.f;
    static_assert(NT % C4 == 0, "chunk rows must split into thread + load parts");
    static_assert(sizeof(E) == 4, "fp32 storage (bf16 has its own kernel)");
    f32x4 ra[QLPT], rd[QLPT];
    float r_lse = 0.f, r_dl = 0.f, r_dlo = 0.f;
    const uint32_t q_voff = (uint32_t)(((int64_t)(tid / C4) * p.sq.t + 4 * (tid % C4)) * 4);
    const uint32_t do_voff = (uint32_t)(((int64_t)(tid / C4) * p.sdo.t + 4 * (tid % C4)) * 4);
    auto gload_q = [&](int q0, int lim) {
        const int rows = min(lim - q0, BQ);
        const auto rq = row_rsrc((const float*)Q, p.sq.t, q0, rows, D);
        const auto rdo = row_rsrc((const float*)dO, p.sdo.t, q0, rows, D);
#pragma unroll
        for (int i = 0; i < QLPT; ++i) {
            ra[i] = buffer_ld4(rq, q_voff, (uint32_t)((int64_t)(NT * i / C4) * p.sq.t * 4));
            rd[i] = buffer_ld4(rdo, do_voff, (uint32_t)((int64_t)(NT * i / C4) * p.sdo.t * 4));
        }
        // lanes past the tile's rows (all but the first BQ threads) read zeros
        r_lse = buffer_ld1(row_rsrc(LSE, 1, q0, rows, 1), (uint32_t)tid * 4, 0);
        r_dl = buffer_ld1(row_rsrc(DL, 1, q0, rows, 1), (uint32_t)tid * 4, 0);
        // rows past the short ones (and every row outside key block 0) read 0
        if constexpr (SHORT) {
            const int n_sh = kblk == 0 ? max(0, min(p.n_short - q0, rows)) : 0;
            r_dlo = buffer_ld1(row_rsrc(DLO, 1, q0, n_sh, 1), (uint32_t)tid * 4, 0);
        }
    };
    auto sstore_q = [&]() {
#pragma unroll
        for (int i = 0; i < QLPT; ++i) {
            const int f = tid + NT * i;
            *reinterpret_cast<f32x4*>(&Qs[f / C4][4 * (f % C4)]) = ra[i];
            *reinterpret_cast<f32x4*>(&dOs[f / C4][4 * (f % C4)]) = rd[i];
        }
        if (tid < BQ) {
            lse_s[tid] = r_lse * kLseStage;
            dl_s[tid] = r_dl;
            if constexpr (SHORT) dlo_s[tid] = r_dlo;
        }
    };
    // Short rows (bwd_split.h): before the main loop, their delta from this
    // block's own S and dP.  Per short tile each wave forms S^T and dP^T of its
    // 32 keys (the main loop's chains with the operands swapped, so lane
    // (l32, g) holds query q0 + l32 and keys 8 (r / 4) + 4 g + r % 4 of the
    // wave), the weights e = exp2(S c - lse log2 e) (1 for a one-key row's
    // key), and per query sum(e) and sum(e dP) in fp64 (exact products) over
    // its registers and the lane pair (l32, l32 + 32); the workgroup's first
    // BQ threads add the waves' sums in wave order and store delta = sum(e dP)
    // / sum(e) as hi + lo.  Each tile's loads are issued while the previous one
    // computes; the main loop's first barrier orders the last sums' reads
    // before it writes the dS tile they sit in.
    const int qs_end = SHORT && kblk == 0 ? min(q_end, p.n_short) : q_begin;  // short tiles: [q_begin, qs_end)
    if (SHORT && q_begin < qs_end) {
        double* part = reinterpret_cast<double*>(&dSs[0][0]);  // [NW][BQ] pairs (sum e, sum e dP)
        static_assert(2 * NW * BQ * sizeof(double) <= sizeof(dSs), "the sums fit the dS tile");
        gload_q(q_begin, p.Tq);
        for (int q0 = q_begin; q0 < qs_end; q0 += BQ) {
            sstore_q();
            __syncthreads();
            if (q0 + BQ < qs_end) gload_q(q0 + BQ, p.Tq);
            double l = 0.0, w = 0.0;
            if ((!p.causal || (q0 + BQ - 1 + p.off >= k0w)) && k0w < p.Tk) {
                f32x16 st, dpt;
#pragma unroll
                for (int i = 0; i < HD; i += 4) {
                    const f32x4 qa = *reinterpret_cast<const f32x4*>(&Qs[l32][g * HD + i]);
                    const f32x4 da = *reinterpret_cast<const f32x4*>(&dOs[l32][g * HD + i]);
                    st = mfma32x32x2(kf[i + 0], qa[0], i == 0 ? f32x16{} : st);
                    dpt = mfma32x32x2(vf[i + 0], da[0], i == 0 ? f32x16{} : dpt);
                    st = mfma32x32x2(kf[i + 1], qa[1], st);
                    dpt = mfma32x32x2(vf[i + 1], da[1], dpt);
                    st = mfma32x32x2(kf[i + 2], qa[2], st);
                    dpt = mfma32x32x2(vf[i + 2], da[2], dpt);
                    st = mfma32x32x2(kf[i + 3], qa[3], st);
                    dpt = mfma32x32x2(vf[i + 3], da[3], dpt);
                }
                const int qi = q0 + l32;
                const float L = lse_s[l32] * kLseRead;
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const int kj = k0w + 8 * (r >> 2) + 4 * g + (r & 3);
                    const bool vis = (qi < p.Tq) && (kj < p.Tk) && (!p.causal || kj <= qi + p.off);
                    const float e = bwd_short_weight(p, qi, vis, fast_exp2(fmaf(st[r], c, -L)));
                    l += (double)e;
                    w += (double)e * (double)dpt[r];
                }
            }
            l += __shfl_xor(l, 32);
            w += __shfl_xor(w, 32);
            if (g == 0) {
                part[2 * (wave * BQ + l32)] = l;
                part[2 * (wave * BQ + l32) + 1] = w;
            }
            __syncthreads();
            if (tid < BQ) bwd_short_delta_store<NW, BQ>(p, bh, q0 + tid, part + 2 * tid);
        }
    }

    // K^T of the whole key block in LDS, for the dQ product.
#pragma unroll
    for (int i = 0; i < KLPT; ++i) {
        const int f = tid + NT * i;
        const int r = f / C4;
        const int c4 = f % C4;
        f32x4 val = f32x4{0.f, 0.f, 0.f, 0.f};
        if (k0 + r < p.Tk) val = ld4(K + (int64_t)(k0 + r) * p.sk.t + 4 * c4);
        Kts[4 * c4 + 0][r] = val[0];
        Kts[4 * c4 + 1][r] = val[1];
        Kts[4 * c4 + 2][r] = val[2];
        Kts[4 * c4 + 3][r] = val[3];
    }


    // With PF the next tile's loads are in flight while a tile computes.
    // Without short rows (EARLY) they are issued right after the store that
    // frees their registers, ahead of the tile's dQ atomics, so the store's
    // wait for them (the memory counter drains in issue order) does not wait
    // for the atomics as well (config 2 302 -> 297 us); the short-row
    // variant, tighter on registers, measured 3% slower that way and issues
    // them at the top of the tile.
    constexpr bool EARLY = PF && !SHORT;
    // Without PF (D = 128) a tile's loads go out in the previous tile's dQ
    // section (ahead of its atomics, where fewer registers are live) and are
    // stored at the top of the tile (B8 H12 T1024 686 -> 678 us, config 4
    // 5972 -> 5937 us).
    constexpr bool LATE_EARLY = !PF;
    if constexpr (PF) {
        gload_q(q_begin, p.Tq);
        sstore_q();
        __syncthreads();
        if constexpr (EARLY) gload_q(q_begin + BQ, q_begin + BQ < q_end ? p.Tq : 0);
    }
    if constexpr (LATE_EARLY) gload_q(q_begin, p.Tq);

    for (int q0 = q_begin; q0 < q_end; q0 += BQ) {
        if constexpr (PF && !EARLY) {
            gload_q(q0 + BQ, q0 + BQ < q_end ? p.Tq : 0);
        } else if constexpr (LATE_EARLY) {
            sstore_q();
            __syncthreads();
        }

        // Does any query of this tile see any key of this wave?
        const bool active = !p.causal || (q0 + BQ - 1 + p.off >= k0w);
        f32x16 ds;
        if (active && k0w < p.Tk) {
            f32x16 s, dp;
#pragma unroll
            for (int i = 0; i < HD; i += 4) {
                const f32x4 qa = *reinterpret_cast<const f32x4*>(&Qs[l32][g * HD + i]);
                const f32x4 da = *reinterpret_cast<const f32x4*>(&dOs[l32][g * HD + i]);
                s = mfma32x32x2(qa[0], kf[i + 0], i == 0 ? f32x16{} : s);  // zero accumulator as an operand
                dp = mfma32x32x2(da[0], vf[i + 0], i == 0 ? f32x16{} : dp);
                s = mfma32x32x2(qa[1], kf[i + 1], s);
                dp = mfma32x32x2(da[1], vf[i + 1], dp);
                s = mfma32x32x2(qa[2], kf[i + 2], s);
                dp = mfma32x32x2(da[2], vf[i + 2], dp);
                s = mfma32x32x2(qa[3], kf[i + 3], s);
                dp = mfma32x32x2(da[3], vf[i + 3], dp);
            }
            // P and dS; reg r holds query row 8*(r/4) + 4*g + r%4 of the tile.
            // Only tiles that cross the causal diagonal or the end of the
            // queries / keys evaluate the visibility test.
            auto p_ds = [&](auto masked) {
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const f32x4 L = *reinterpret_cast<const f32x4*>(&lse_s[8 * j + 4 * g]) * kLseRead;
                    const f32x4 Dl = *reinterpret_cast<const f32x4*>(&dl_s[8 * j + 4 * g]);
                    const f32x4 Dlo = SHORT ? *reinterpret_cast<const f32x4*>(&dlo_s[8 * j + 4 * g])
                                            : f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
                    for (int cc = 0; cc < 4; ++cc) {
                        const int r = 4 * j + cc;
                        float pr = fast_exp2(fmaf(s[r], c, -L[cc]));
                        if constexpr (decltype(masked)::value) {
                            const int qi = q0 + 8 * j + 4 * g + cc;
                            const bool vis = (qi < p.Tq) && (key < p.Tk) && (!p.causal || key <= qi + p.off);
                            pr = vis ? pr : 0.f;
                        }
                        s[r] = pr;
                        ds[r] = pr * (SHORT ? (dp[r] - Dl[cc]) - Dlo[cc] : dp[r] - Dl[cc]);
                    }
                }
            };
            const bool need_mask = q0 + BQ > p.Tq || k0w + 32 > p.Tk || (p.causal && k0w + 31 > q0 + p.off);
            if (need_mask)
                p_ds(std::true_type{});
            else
                p_ds(std::false_type{});
            // A row with one visible key: dS = P (dP - dP) = 0.  (At D = 32 without
            // short rows the kernel keeps three workgroups per CU only without this
            // fix, 168 VGPRs; its short-row prologue, on small problems, forms
            // delta = dP bit for bit instead.)
            if constexpr (D != 32 || SHORT) {
                if (bwd_one_key_tile(p, q0, k0w)) {
#pragma unroll
                    for (int r = 0; r < 16; ++r)
                        if (bwd_one_key_row(p, q0 + 8 * (r >> 2) + 4 * g + (r & 3))) ds[r] = 0.f;
                }
            }
            // dV^T += dO^T P ; dK^T += Q^T dS
#pragma unroll
            for (int kk = 0; kk < 16; ++kk) {
                const int qr = 8 * (kk >> 2) + 4 * g + (kk & 3);
#pragma unroll
                for (int db = 0; db < NDB; ++db) {
                    const float ado = dOs[qr][db * 32 + l32];
                    const float aq = Qs[qr][db * 32 + l32];
                    dv_acc[db] = mfma32x32x2(ado, s[kk], dv_acc[db]);
                    dk_acc[db] = mfma32x32x2(aq, ds[kk], dk_acc[db]);
                }
            }
        } else {
            ds = f32x16{};
        }
        // dS block of this wave -> LDS (rows = queries, columns = the 128 keys);
        // with the query-major dQ pass (dq_direct) there is no dQ product here
        if (!p.dq_direct) {
#pragma unroll
            for (int r = 0; r < 16; ++r) dSs[8 * (r >> 2) + 4 * g + (r & 3)][wave * 32 + l32] = ds[r];
        }
        __syncthreads();
        if constexpr (PF) sstore_q();  // the next tile (zeros after the last one, never read)
        if constexpr (EARLY) gload_q(q0 + 2 * BQ, q0 + 2 * BQ < q_end ? p.Tq : 0);
        if constexpr (LATE_EARLY) gload_q(q0 + BQ, q0 + BQ < q_end ? p.Tq : 0);
        if (p.dq_direct) {
            __syncthreads();
            continue;
        }

        // ---- dQ tile (32 x D) += dS (32 x BK) K (BK x D) ---------------------
        // Each wave takes NDQ / NW adjacent 16x16 blocks; lane group g4
        // reduces keys g4 * BK/4 .. + BK/4 - 1.  fp32 atomics through a buffer
        // resource over the tile's rows: rows past Tq fall outside it and the
        // hardware drops those adds.
        const auto rdq = row_rsrc(dQa, p.sacc.t, q0, min(p.Tq - q0, BQ), D);
#pragma unroll
        for (int bi = 0; bi < NDQ / NW; ++bi) {
            const int blk = wave * (NDQ / NW) + bi;  // adjacent blocks share K^T rows
            const int qh = blk & 1;
            const int dc = blk >> 1;
            f32x4 acc;
#pragma unroll
            for (int kk = 0; kk < BK / 4; kk += 4) {
                const f32x4 a = *reinterpret_cast<const f32x4*>(&dSs[16 * qh + l16][g4 * (BK / 4) + kk]);
                const f32x4 bb = *reinterpret_cast<const f32x4*>(&Kts[16 * dc + l16][g4 * (BK / 4) + kk]);
                acc = mfma16x16x4(a[0], bb[0], kk == 0 ? f32x4{0.f, 0.f, 0.f, 0.f} : acc);
                acc = mfma16x16x4(a[1], bb[1], acc);
                acc = mfma16x16x4(a[2], bb[2], acc);
                acc = mfma16x16x4(a[3], bb[3], acc);
            }
            const uint32_t voff = (uint32_t)(((int64_t)(16 * qh + 4 * g4) * p.sacc.t + 16 * dc + l16) * 4);
#pragma unroll
            for (int r = 0; r < 4; ++r)
                buffer_atomic_add(rdq, acc[r] * p.scale, voff, (uint32_t)((int64_t)r * p.sacc.t * 4));
        }
        __syncthreads();
    }

    // ---- dK = scale * dK^T^T, dV = dV^T^T ------------------------------------------
    if (!bwd_fixup<NT>(p, wk, dk_acc, dv_acc)) return;
    if (key < p.Tk) {
        E* dKp = (E*)p.dk + b * p.sdk.b + h * p.sdk.h + (int64_t)key * p.sdk.t;
        E* dVp = (E*)p.dv + b * p.sdv.b + h * p.sdv.h + (int64_t)key * p.sdv.t;
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

// dQ accumulator (fp32) -> bf16 dq, when dq has the accumulator's dense
// [B, H, Tq, D] layout and 16-byte aligned rows: a flat pass, 8 elements
// (two 16-byte loads, one 16-byte store) per thread.
__global__ __launch_bounds__(256) void bwd_cvt_flat_kernel(BwdParams p) {
    const int64_t n8 = (int64_t)p.B * p.H * p.Tq * p.D / 8;
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= n8) return;
    const f32x4* a = reinterpret_cast<const f32x4*>(p.dq_acc) + 2 * i;
    const f32x4 x = a[0], y = a[1];
    u16x8 h;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        h[k] = f32_to_bf16(x[k]);
        h[4 + k] = f32_to_bf16(y[k]);
    }
    reinterpret_cast<u16x8*>(p.dq)[i] = h;
}

// dQ accumulator (fp32) -> bf16 dq on dq's own strides.
template <int D>
__global__ __launch_bounds__(256) void bwd_cvt_kernel(BwdParams p) {
    constexpr int TPR = D / 4;
    constexpr int RPB = 256 / TPR;
    const int tid = threadIdx.x;
    const int64_t row = (int64_t)blockIdx.x * RPB + tid / TPR;
    const int c4 = tid % TPR;
    const int64_t rows = (int64_t)p.B * p.H * p.Tq;
    if (row >= rows) return;
    int64_t b, h, i;
    bwd_row_split(p, rows, row, b, h, i);
    const f32x4 a = *reinterpret_cast<const f32x4*>(p.dq_acc + b * p.sacc.b + h * p.sacc.h +
                                                     i * p.sacc.t + 4 * c4);
    st4((uint16_t*)p.dq + b * p.sdq.b + h * p.sdq.h + i * p.sdq.t + 4 * c4, a);
}

// Query-major dQ pass, fp32 (the deterministic mode: the main kernel then
// skips its dQ product).  One workgroup = 4 waves x 32 query rows of one
// (b, h), laid out as the forward: each lane keeps its query row of Q and dO
// as the B operand (Q^T, dO^T) in VGPRs, with that row's log-sum-exp and
// delta; tiles of 32 keys stream through LDS as K and V rows and K^T
// (double-buffered, one barrier per tile).  Per wave and tile:
//   S^T = K Q^T, dP^T = V dO^T        v_mfma_f32_32x32x2_f32, A from LDS
//   P^T = exp2(S^T c - lse log2 e), dS^T = P^T (dP^T - delta)
//   dQ^T += K^T dS^T                  B = dS^T straight from the accumulators
//                                     (as the forward feeds P^T to P V)
// dQ stays in VGPRs and is stored once, times the scale: every element is the
// sum of its key tiles in key order, with no accumulator, zeroing or atomics,
// so the result is the same on every run.  It recomputes S and dP (two more
// products per score than the atomic dQ of the main kernel).
template <int D>
__global__ __launch_bounds__(256, D >= 128 ? 1 : 2) void bwd_dq_kernel(BwdParams p) {
    constexpr int BM = kBwdDqBM;
    constexpr int BN = 32;               // keys per tile
    constexpr int HD = D / 2;            // reduction elements per lane half
    constexpr int NDB = D / 32;          // 32-wide d blocks of dQ^T
    constexpr int C4 = D / 4;            // 4-element chunks per row
    constexpr int KS = D + 4;            // K / V row stride in LDS (floats)
    constexpr int TS = BN + 4;           // K^T row stride in LDS (floats)
    constexpr int LPT = BN * C4 / 256;   // 4-element loads per thread per tensor per tile
    static_assert(BM == 128 && BN * C4 % 256 == 0, "4 waves x 32 rows, whole staging passes");
    static_assert(256 % C4 == 0, "chunk rows must split into thread + load parts");

    __shared__ __attribute__((aligned(16))) float Ks[2][BN][KS];
    __shared__ __attribute__((aligned(16))) float Vs[2][BN][KS];
    __shared__ __attribute__((aligned(16))) float Kt[2][D][TS];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int l32 = lane & 31;
    const int g = lane >> 5;

    const int BH = p.B * p.H;
    const int w = blockIdx.x;
    const int qtile = p.n_qtiles - 1 - w / BH;  // the longest causal rows first
    const int bh = w % BH;
    const int b = bh / p.H;
    const int h = bh % p.H;

    const float* Q = (const float*)p.q + b * p.sq.b + h * p.sq.h;
    const float* K = (const float*)p.k + b * p.sk.b + h * p.sk.h;
    const float* V = (const float*)p.v + b * p.sv.b + h * p.sv.h;
    const float* dO = (const float*)p.dout + b * p.sdo.b + h * p.sdo.h;

    const int q0w = qtile * BM + wave * 32;
    const int qrow = q0w + l32;
    // B operands: lane (l32, g) holds row qrow, columns g*HD + i.
    float qf[HD], df[HD];
    if (qrow < p.Tq) {
        const float* qs = Q + (int64_t)qrow * p.sq.t + g * HD;
        const float* ds = dO + (int64_t)qrow * p.sdo.t + g * HD;
#pragma unroll
        for (int i = 0; i < HD; i += 4) {
            const f32x4 a = ld4(qs + i);
            const f32x4 c = ld4(ds + i);
            qf[i] = a[0]; qf[i + 1] = a[1]; qf[i + 2] = a[2]; qf[i + 3] = a[3];
            df[i] = c[0]; df[i + 1] = c[1]; df[i + 2] = c[2]; df[i + 3] = c[3];
        }
    } else {
#pragma unroll
        for (int i = 0; i < HD; ++i) qf[i] = df[i] = 0.f;
    }
    const float Lq = qrow < p.Tq ? p.lse[(int64_t)bh * p.Tq + qrow] * kLog2e : 0.f;
    const float Dq = qrow < p.Tq ? p.delta[(int64_t)bh * p.Tq + qrow] : 0.f;
    const float Dqlo = bwd_short_row(p, qrow) ? p.delta_lo[(int64_t)bh * p.Tq + qrow] : 0.f;
    const bool one_key = qrow < p.Tq && bwd_one_key_row(p, qrow);
    const bool one_key_wave = p.causal ? (-p.off >= q0w && -p.off < q0w + 32) : p.Tk == 1;  // wave-uniform

    int kv_end = p.Tk;
    if (p.causal) kv_end = min(p.Tk, qtile * BM + BM + p.off);
    const int nt = (kv_end + BN - 1) / BN;
    const int wave_kend = p.causal ? min(kv_end, q0w + 32 + p.off) : kv_end;

    // Chunk f of a tile -> (row f / C4, column chunk f % C4); chunk tid + 256 i
    // is 256 i / C4 rows below chunk tid.  Rows at or past the resource's end
    // (<= Tk) read as zeros.
    f32x4 kr[LPT], vr[LPT];
    const uint32_t k_voff = (uint32_t)(((int64_t)(tid / C4) * p.sk.t + 4 * (tid % C4)) * 4);
    const uint32_t v_voff = (uint32_t)(((int64_t)(tid / C4) * p.sv.t + 4 * (tid % C4)) * 4);
    auto gload = [&](int u) {
        const int rows = u < nt ? min(p.Tk - u * BN, BN) : 0;
        const auto rk = row_rsrc(K, p.sk.t, u * BN, rows, D);
        const auto rv = row_rsrc(V, p.sv.t, u * BN, rows, D);
#pragma unroll
        for (int i = 0; i < LPT; ++i) {
            kr[i] = buffer_ld4(rk, k_voff, (uint32_t)((int64_t)(256 * i / C4) * p.sk.t * 4));
            vr[i] = buffer_ld4(rv, v_voff, (uint32_t)((int64_t)(256 * i / C4) * p.sv.t * 4));
        }
    };
    auto sstore = [&](int buf) {
#pragma unroll
        for (int i = 0; i < LPT; ++i) {
            const int f = tid + 256 * i;
            const int r = f / C4, c4 = f % C4;
            *reinterpret_cast<f32x4*>(&Ks[buf][r][4 * c4]) = kr[i];
            *reinterpret_cast<f32x4*>(&Vs[buf][r][4 * c4]) = vr[i];
#pragma unroll
            for (int e = 0; e < 4; ++e) Kt[buf][4 * c4 + e][r] = kr[i][e];
        }
    };

    f32x16 dq[NDB];
#pragma unroll
    for (int i = 0; i < NDB; ++i) dq[i] = f32x16{};
    const float c = p.c;

    gload(0);
    sstore(0);
    __syncthreads();
    for (int u = 0; u < nt; ++u) {
        const int buf = u & 1;
        const int k0 = u * BN;
        gload(u + 1);  // zero rows past the last tile: straight-line
        if (k0 < wave_kend) {
            f32x16 s = f32x16{}, dp = f32x16{};
#pragma unroll
            for (int i = 0; i < HD; i += 4) {
                const f32x4 a = *reinterpret_cast<const f32x4*>(&Ks[buf][l32][g * HD + i]);
                const f32x4 v = *reinterpret_cast<const f32x4*>(&Vs[buf][l32][g * HD + i]);
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    s = mfma32x32x2(a[j], qf[i + j], s);
                    dp = mfma32x32x2(v[j], df[i + j], dp);
                }
            }
            // reg r: key k0 + 8 (r / 4) + 4 g + r % 4 of query qrow
            const bool need_mask = (k0 + BN > p.Tk) || (qtile * BM + BM > p.Tq) || (p.causal && (k0 + BN - 1 > q0w + p.off));
            const int lim = p.causal ? min(p.Tk - 1, qrow + p.off) : p.Tk - 1;
            // the visibility test only on tiles that cross the diagonal or the ends
            auto p_ds = [&](auto masked) {
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    float pr = fast_exp2(fmaf(s[r], c, -Lq));
                    if constexpr (decltype(masked)::value) {
                        const int key = k0 + 8 * (r >> 2) + 4 * g + (r & 3);
                        pr = (key <= lim && qrow < p.Tq) ? pr : 0.f;
                    }
                    s[r] = pr * ((dp[r] - Dq) - Dqlo);  // dS^T
                }
            };
            if (need_mask)
                p_ds(std::true_type{});
            else
                p_ds(std::false_type{});
            if (one_key_wave && k0 == 0 && one_key) s = f32x16{};  // one visible key: dS = P (dP - dP) = 0
            // dQ^T[d][q] += K^T[d][keys] dS^T[keys][q]: MFMA (j, cc) reduces keys 8j + cc, 8j + 4 + cc
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                f32x4 kt[NDB];
#pragma unroll
                for (int db = 0; db < NDB; ++db)
                    kt[db] = *reinterpret_cast<const f32x4*>(&Kt[buf][db * 32 + l32][8 * j + 4 * g]);
#pragma unroll
                for (int cc = 0; cc < 4; ++cc)
#pragma unroll
                    for (int db = 0; db < NDB; ++db) dq[db] = mfma32x32x2(kt[db][cc], s[4 * j + cc], dq[db]);
            }
        }
        sstore(buf ^ 1);
        __syncthreads();
    }
    if (qrow < p.Tq) {
        float* dst = (float*)p.dq + b * p.sdq.b + h * p.sdq.h + (int64_t)qrow * p.sdq.t;
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

// ---- split plan (host) ------------------------------------------------------------
//
// Under a causal mask key block j has ~(Tq - 128 j) / 32 query tiles, so at
// config-2 sizes the first key blocks carry up to 8x the work of the last.
// Measured on MI355X: a workgroup alone on a CU runs ~1.85x faster than each
// of two sharing it (two resident workgroups give ~8% more throughput than
// one), so the heaviest workgroups, which always share their CU with lighter
// ones, set the kernel's length.  bwd_plan simulates the dispatch (workgroup w
// to XCD w % 8, each XCD's workgroups placed in order on its least-loaded CU
// with a free slot) for splits of the heaviest key blocks' tile ranges into
// chunks, and keeps the best if it beats the unsplit order by 3%.

static constexpr double kBwdPairGain = 0.08;  // throughput gained per extra resident workgroup
// Per-workgroup fixed cost (K/V loads, K^T staging) and the partial store /
// reduction of a split chunk, in query tiles of that dtype's kernel.  A bf16
// tile costs a fraction of an fp32 one while the fixed costs take about the
// same time; the bf16 figures are set from measurement (splits lost 5-8% at
// B4 H12 and config 2 with smaller ones), so bf16 splits only grids far below
// the device's size.
static constexpr double kBwdOverhead[2] = {0.3, 5.0};
static constexpr double kBwdFixup[2] = {0.4, 8.0};
// The short-row prologue of key block 0 (the S and dP chains of each short
// query tile, run once more to form delta) per short tile, in the same units.
static constexpr double kBwdShortTile[2] = {0.55, 0.5};

static double share_rate(size_t k) { return k <= 1 ? 1.0 : (1.0 + kBwdPairGain * (double)(k - 1)) / (double)k; }

// Makespan, in query tiles of a workgroup alone on a CU, of workgroups of the
// given costs in dispatch order.
static double cu_makespan(const std::vector<double>& cost, int cus_per_xcd, int slots) {
    double worst = 0.0;
    std::vector<std::vector<double>> res((size_t)cus_per_xcd);
    for (int x = 0; x < 8; ++x) {
        for (auto& r : res) r.clear();
        size_t next = (size_t)x;
        auto fill = [&]() {
            while (next < cost.size()) {
                int best = -1;
                for (int c = 0; c < cus_per_xcd; ++c)
                    if ((int)res[(size_t)c].size() < slots &&
                        (best < 0 || res[(size_t)c].size() < res[(size_t)best].size()))
                        best = c;
                if (best < 0) break;
                res[(size_t)best].push_back(cost[next]);
                next += 8;
            }
        };
        fill();
        double t = 0.0;
        for (;;) {
            double dt = INFINITY;
            for (const auto& r : res)
                for (double v : r) dt = std::min(dt, v / share_rate(r.size()));
            if (!(dt < INFINITY)) break;
            t += dt;
            for (auto& r : res) {
                const double rate = share_rate(r.size());
                for (double& v : r) v -= dt * rate;
                r.erase(std::remove_if(r.begin(), r.end(), [](double v) { return v <= 1e-9; }), r.end());
            }
            fill();
        }
        worst = std::max(worst, t);
    }
    return worst;
}

// Resident backward workgroups per CU, and CUs per XCD, on the current device.
// An error left pending by an earlier HIP call on this thread is returned
// (named in the detail text) instead of being cleared by the queries here.
static int bwd_slots(int D, int bf16, int* per_cu, int* cus_per_xcd) {
    static std::mutex mu;
    static std::map<std::array<int, 3>, std::pair<int, int>> cache;
    const hipError_t pending = hipGetLastError();
    int dev = -1;
    if (hipGetDevice(&dev) != hipSuccess) {
        (void)hipGetLastError();  // no device (a CPU-only host sizing workspaces): MI355X defaults
        dev = -1;
    } else if (pending != hipSuccess) {
        return report_pending_error(pending, "attention backward planner");
    }
    std::lock_guard<std::mutex> lk(mu);
    const std::array<int, 3> key{dev, D, bf16};
    auto it = cache.find(key);
    if (it == cache.end()) {
        int cus = 256, occ = (D >= 128 || bwd_waves(bf16, D) == 8) ? 1 : 2;  // MI355X defaults
        if (dev >= 0) {
            int n = 0, o = 0;
            if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess && n > 0) cus = n;
            hipError_t e = hipErrorInvalidValue;
            if (!bf16 && D == 32)
                e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&o, bwd_main_kernel<32, float, false>, 64 * bwd_waves(0, 32), 0);
            if (!bf16 && D == 64)
                e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&o, bwd_main_kernel<64, float, false>, 64 * bwd_waves(0, 64), 0);
            if (!bf16 && D == 128)
                e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&o, bwd_main_kernel<128, float, false>, 64 * bwd_waves(0, 128), 0);
            if (bf16) e = (hipError_t)bwd_main_bf16_occupancy(D, &o);
            if (e == hipSuccess && o > 0) occ = o;
            (void)hipGetLastError();  // a failed query of ours: the defaults stand
        }
        it = cache.emplace(key, std::make_pair(occ, std::max(1, cus / 8))).first;
    }
    *per_cu = it->second.first;
    *cus_per_xcd = it->second.second;
    return 0;
}

static void bwd_plan_compute(int B, int H, int Tq, int Tk, int D, int bf16, int per_cu, int cus_per_xcd,
                             BwdPlan* out) {
    const int BH = B * H;
    const int bk = bwd_keys_per_wg(bf16, D);
    const int nkb = (Tk + bk - 1) / bk;
    const int off = Tk - Tq;
    if ((int64_t)nkb * BH > 8LL * 8 * cus_per_xcd * per_cu) return;  // the tail is a small share
    std::vector<int> t0((size_t)nkb), nt((size_t)nkb);
    int max_nt = 0;
    for (int j = 0; j < nkb; ++j) {
        t0[(size_t)j] = std::max(0, j * bk - off) / kBwdBQ;
        nt[(size_t)j] = (Tq + kBwdBQ - 1) / kBwdBQ - t0[(size_t)j];
        max_nt = std::max(max_nt, nt[(size_t)j]);
    }
    // query tiles [0, s_tiles) of key block 0 hold its short rows and run the prologue
    const int s_tiles = (bwd_short_rows(B, H, Tq, Tk, 1, bk) + kBwdBQ - 1) / kBwdBQ;
    struct G { double cost; int kb, a, b, chunk, n; };
    // A key block of more than ch tiles is split into ceil(n / ch) chunks of
    // near-equal cost, block 0's short tiles counted with the prologue's share
    // pro.  The chunk size is chosen with pro = 0: counting the prologue there
    // moved the choice to plans measured slower (config 2 fp32: ch 27-31, which
    // leave key block 1 whole, +6-10%), while cutting block 0 at the weighted
    // midpoint recovered half of the prologue's cost at the chosen size.
    auto build = [&](int ch, double pro, std::vector<G>& g) {
        g.clear();
        for (int j = 0; j < nkb; ++j) {
            const int n = nt[(size_t)j], s = j == 0 ? s_tiles : 0;
            const int k = n > ch ? (n + ch - 1) / ch : 1;
            auto work = [&](int t) { return (double)t + pro * std::min(t, s); };  // tiles [0, t)
            int a = 0;
            for (int c = 0; c < k; ++c) {
                int e = n;
                if (c + 1 < k) {  // the cut nearest cost share c + 1, leaving a tile for each later chunk
                    const double target = work(n) * (c + 1) / k;
                    e = a + 1;
                    while (e < n - (k - c - 1) && work(e) < target) ++e;
                    if (e > a + 1 && target - work(e - 1) < work(e) - target) --e;
                }
                const double cost = work(e) - work(a) + kBwdOverhead[bf16] + (k > 1 ? kBwdFixup[bf16] : 0.0);
                g.push_back({cost, j, t0[(size_t)j] + a, t0[(size_t)j] + e, c, k});
                a = e;
            }
        }
        std::stable_sort(g.begin(), g.end(), [](const G& x, const G& y) { return x.cost > y.cost; });
    };
    // dispatch order of a plan's grid: group-major, BHp heads per group (padding
    // heads cost nothing); the unsplit grid has B*H heads per key block
    auto makespan = [&](const std::vector<G>& g, int heads) {
        std::vector<double> cost;
        cost.reserve(g.size() * (size_t)heads);
        for (const G& x : g)
            for (int i = 0; i < heads; ++i) cost.push_back(i < BH ? x.cost : 0.0);
        return cu_makespan(cost, cus_per_xcd, per_cu);
    };
    std::vector<G> g;
    build(max_nt, 0.0, g);
    const double base = makespan(g, BH);
    double best = base * 0.97;
    int best_ch = 0;
    for (int ch = max_nt - 1; ch >= std::max(2, max_nt / 8); --ch) {
        build(ch, 0.0, g);
        int n_split = 0;
        for (const G& x : g) n_split += x.chunk == 0 && x.n > 1;
        if ((int)g.size() > kMaxBwdGroups || n_split == 0) continue;
        const double ms = makespan(g, bwd_padded_heads(BH));
        if (ms < best) {
            best = ms;
            best_ch = ch;
        }
    }
    if (!best_ch) return;
    build(best_ch, kBwdShortTile[bf16], g);
    std::vector<int> chunks((size_t)nkb, 1), split_of((size_t)nkb, -1), slot0((size_t)nkb, 0);
    for (const G& x : g) chunks[(size_t)x.kb] = x.n;
    int n_split = 0, n_slots = 0;
    for (int j = 0; j < nkb; ++j) {
        if (chunks[(size_t)j] > 1) {
            split_of[(size_t)j] = n_split++;
            slot0[(size_t)j] = n_slots;
            n_slots += chunks[(size_t)j];
        }
    }
    for (const G& x : g) {
        BwdGroup& o = out->groups[out->n_groups++];
        o.kb = x.kb;
        o.t0 = x.a;
        o.t1 = x.b;
        o.split = split_of[(size_t)x.kb];
        o.chunk = x.chunk;
        o.n_chunks = x.n;
        o.slot0 = slot0[(size_t)x.kb];
    }
    out->n_split = n_split;
    out->n_slots = n_slots;
}

int bwd_plan(int B, int H, int Tq, int Tk, int D, int causal, int bf16, BwdPlan* out) {
    *out = BwdPlan{};
    out->bk = bwd_keys_per_wg(bf16, D);
    if (!causal) return 0;
    int per_cu = 0, cus_per_xcd = 0;
    if (const int e = bwd_slots(D, bf16, &per_cu, &cus_per_xcd)) return e;
    static std::mutex mu;
    static std::map<std::array<int, 7>, BwdPlan> cache;
    const std::array<int, 7> key{B * H, Tq, Tk, D, bf16, per_cu, cus_per_xcd};
    {
        std::lock_guard<std::mutex> lk(mu);
        auto it = cache.find(key);
        if (it != cache.end()) {
            *out = it->second;
            return 0;
        }
    }
    bwd_plan_compute(B, H, Tq, Tk, D, bf16 ? 1 : 0, per_cu, cus_per_xcd, out);
    std::lock_guard<std::mutex> lk(mu);
    if (cache.size() > 256) cache.clear();
    cache[key] = *out;
    return 0;
}

size_t bwd_split_workspace_bytes(const BwdPlan& plan, int B, int H, int D) {
    if (!plan.n_split) return 0;
    const size_t bh = (size_t)B * H;
    const size_t part = (size_t)plan.n_slots * bh * 2 * (size_t)D * plan.bk * sizeof(float);
    return part + (size_t)plan.n_split * bh * sizeof(unsigned);
}

template <int D, typename E>
static int launch_bwd_t(const BwdParams& p_in, hipStream_t s) {
    BwdParams p = p_in;
    // The bf16 main kernel at D <= 64 forms delta itself while staging each
    // query tile; bwd_pre then only zeroes, unless the query-major dQ pass
    // (which reads delta) follows.
    p.pre_delta = (sizeof(E) == 2 && D <= 64) ? p.dq_direct : 1;
    constexpr int RPB = 256 / (D / 4);
    const int64_t rows = (int64_t)p.B * p.H * p.Tq;
    const dim3 pre_grid((unsigned)((rows + RPB - 1) / RPB));  // bwd_cvt: 4 elements per thread
    constexpr int PRE_RPB = bwd_pre_rows_per_block<D, E>();
    const dim3 delta_grid((unsigned)((rows + PRE_RPB - 1) / PRE_RPB));
    if (!p.pre_delta && !p.dq_direct) {
        // zeroing only: a few grid-stride workgroups per CU
        const int64_t n4 = rows * D / 4;
        const unsigned zb = (unsigned)std::min<int64_t>((n4 + 255) / 256, 2048);
        hipLaunchKernelGGL(bwd_zero_kernel, dim3(zb), dim3(256), 0, s, p);
    } else {
        hipLaunchKernelGGL((bwd_pre_kernel<D, E>), delta_grid, dim3(256), 0, s, p);
    }
    if constexpr (sizeof(E) == 2) {
        const int e = launch_bwd_main_bf16(p, s);
        if (e) return e;
        if (p.dq_direct) {
            const int e2 = launch_bwd_dq_bf16(p, s);
            if (e2) return e2;
        } else {
            const bool dense = p.sdq.t == D && p.sdq.h == (int64_t)p.Tq * D && p.sdq.b == (int64_t)p.H * p.Tq * D &&
                               reinterpret_cast<uintptr_t>(p.dq) % 16 == 0;
            if (dense)
                hipLaunchKernelGGL(bwd_cvt_flat_kernel, dim3((unsigned)((rows * D / 8 + 255) / 256)), dim3(256), 0, s, p);
            else
                hipLaunchKernelGGL((bwd_cvt_kernel<D>), pre_grid, dim3(256), 0, s, p);
        }
    } else {
        const dim3 grid((unsigned)(p.n_groups ? p.n_groups * bwd_padded_heads(p.B * p.H) : p.n_kblocks * p.B * p.H));
        if (p.n_short > 0)
            hipLaunchKernelGGL((bwd_main_kernel<D, E, true>), grid, dim3(64 * bwd_waves(0, D)), 0, s, p);
        else
            hipLaunchKernelGGL((bwd_main_kernel<D, E, false>), grid, dim3(64 * bwd_waves(0, D)), 0, s, p);
        if (p.dq_direct)
            hipLaunchKernelGGL((bwd_dq_kernel<D>), dim3((unsigned)(p.n_qtiles * p.B * p.H)), dim3(256), 0, s, p);
    }
    return (int)hipGetLastError();
}

int launch_attn_bwd(const BwdParams& p, int bf16, hipStream_t s) {
    switch (p.D) {
        case 32: return bf16 ? launch_bwd_t<32, uint16_t>(p, s) : launch_bwd_t<32, float>(p, s);
        case 64: return bf16 ? launch_bwd_t<64, uint16_t>(p, s) : launch_bwd_t<64, float>(p, s);
        case 128: return bf16 ? launch_bwd_t<128, uint16_t>(p, s) : launch_bwd_t<128, float>(p, s);
        default: return (int)hipErrorInvalidValue;
    }
}

}  // namespace inf
