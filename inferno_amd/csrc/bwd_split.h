// bwd_split.h -- work assignment of a backward workgroup and the fix-up that
// completes a split key block (shared by the fp32 and bf16 main kernels).
//
// Without a plan, workgroup w takes key block w / (B*H) and every query tile
// that can see it.  With a plan, w takes group w / BHp and head w % BHp, with
// BHp = B*H rounded up to a multiple of 8 (workgroups of the padding heads
// exit at once): a key block and a range of its query tiles.  When a key
// block's tiles are split over several groups, each group ends with partial
// dK^T / dV^T accumulators; every group stores its partial, and the group that
// finishes last (an arrival counter per (key block, b, h)) sums all partials in
// chunk order and stores dK and dV.  No workgroup waits for another, so the
// split cannot stall the grid.
//
// The partials are handed over through device-coherent accesses: the writer
// stores them with device-scope (sc1) buffer stores, which write through the
// XCD's L2, and waits for their completion before counting; the last arriver
// reads them with device-scope (sc1) loads, which bypass both cache levels.
// This holds wherever the chunks run.  (A device-scope fence would instead
// write back and invalidate the whole L2 of the XCD, evicting every other
// resident workgroup's tiles: measured 18% slower at config 2 fp32, 2.1x at
// bf16.)  The grid is still laid out group-major over B*H padded to a multiple
// of 8, which keeps a head's chunks on one XCD under the round-robin dispatch
// and so its K / V tiles in one L2.
#pragma once

#include "common.h"
#include "kernels.h"

namespace inf {

struct BwdWork {
    int kblk, bh;
    int q_begin, q_end;  // query rows [q_begin, q_end), q_begin a multiple of kBwdBQ
    int split, chunk, n_chunks, slot0;
};

// Heads per group in the launch grid of a split plan.
__host__ __device__ inline int bwd_padded_heads(int BH) { return (BH + 7) / 8 * 8; }

// Work of this workgroup (BK keys per key block); bh >= B*H marks a padding
// workgroup (none to do).
template <int BK>
__device__ __forceinline__ BwdWork bwd_work(const BwdParams& p) {
    const int BH = p.B * p.H;
    const int w = blockIdx.x;
    BwdWork r;
    r.bh = w % BH;
    if (p.n_groups) {
        const int BHp = bwd_padded_heads(BH);
        r.bh = w % BHp;
        const BwdGroup g = p.groups[w / BHp];
        r.kblk = g.kb;
        r.q_begin = g.t0 * kBwdBQ;
        r.q_end = min(p.Tq, g.t1 * kBwdBQ);
        r.split = g.split;
        r.chunk = g.chunk;
        r.n_chunks = g.n_chunks;
        r.slot0 = g.slot0;
    } else {
        r.kblk = w / BH;
        int qb = p.causal ? max(0, r.kblk * BK - p.off) : 0;
        r.q_begin = (qb / kBwdBQ) * kBwdBQ;
        r.q_end = p.Tq;
        r.split = -1;
        r.chunk = 0;
        r.n_chunks = 1;
        r.slot0 = 0;
    }
    return r;
}

// ---- rows whose visible keys all lie in key block 0 ----------------------------
//
// SoftmaxBackward forms dS_ij = P_ij (dP_ij - sum_k P_ik dP_ik) from its own
// P and dP (softmaxbackward.h:109-128 in the reference): with one visible key
// P = 1 and dS = 0 exactly, and with few keys or a near one-hot softmax dS is
// a small difference.  The fused kernels take delta = rowsum(dO * O) instead,
// which is the same sum in exact arithmetic but rounds differently (and, for
// bf16, reads O rounded to bf16), so on such rows dQ and dK would carry that
// rounding at the scale of |dO . O|.  Query rows [0, n_short) see only keys of
// key block 0 (causal: i + off < keys per workgroup; non-causal: Tk within one
// block), so a block-0 workgroup holds all of their scores.  Before its main
// loop it forms their delta itself: S and dP with the MFMA shape of its main
// loop, e = exp2(S c - lse log2 e) as the main loop forms P, and delta =
// sum_j e_j dP_j / sum_j e_j, the softmax of the row normalised over its own
// keys as the reference's e / sum is.  (The main loop's P sums to 1 only
// within the log-sum-exp's rounding, ~1e-6 at sharp scores; a near one-hot
// row's dP_max - delta is of the size 1 - P_max, so delta from the
// unnormalised P would carry that rounding magnified by 1 / (1 - P_max).)
// The sums are taken in fp64 and delta is stored as hi + lo, two fp32 values:
// one fp32 delta would round dP - delta at 2^-24 |dP| (1e-4 relative at P_max
// = 1 - 1e-3), while dP - hi is exact (the two are within a factor of two) and
// the fp32 kernels' - lo keeps the result to the rounding of dS itself.  A row
// whose only visible key is key 0 weighs it 1, so its delta equals its dP bit
// for bit and dS = P (dP - delta) = 0 exactly, as in the reference.  The
// delta goes to the workspace, where the main loop (and the query-major dQ
// pass) read it; the prologue runs before the accumulators and the main
// loop's prefetch are live, so it leaves the main loop's registers alone.

// Whether query row i is one whose delta the block-0 workgroup forms, and
// whether its only visible key is key 0.
__device__ __forceinline__ bool bwd_short_row(const BwdParams& p, int i) { return i < p.n_short; }
__device__ __forceinline__ bool bwd_one_key_row(const BwdParams& p, int i) {
    return p.causal ? i + p.off == 0 : p.Tk == 1;
}

// Whether the 32-row query tile at q0 holds a row whose only visible key is
// key 0 while the wave's keys start at k0w (wave-uniform): the kernels then
// set that row's dS to 0 after forming the tile's dS.
__device__ __forceinline__ bool bwd_one_key_tile(const BwdParams& p, int q0, int k0w) {
    if (k0w != 0) return false;
    if (!p.causal) return p.Tk == 1;
    const int r = -p.off;  // the row with i + off == 0
    return r >= q0 && r < q0 + kBwdBQ && r < p.Tq;
}

// The weight of key j in short row i's delta: e = exp2(S c - lse log2 e) when
// visible (vis), 1 for the one key of a one-key row, else 0.
__device__ __forceinline__ float bwd_short_weight(const BwdParams& p, int i, bool vis, float e) {
    return vis ? (bwd_one_key_row(p, i) ? 1.f : e) : 0.f;
}

// Short row i's delta from NW per-wave pairs (sum e, sum e dP) in fp64,
// spaced 2 * STRIDE doubles apart (wave order): delta = sum(e dP) / sum(e)
// stored as hi (the fp32 nearest) + lo (the rest, rounded).  Rows outside the
// short ones store nothing.
template <int NW, int STRIDE>
__device__ __forceinline__ void bwd_short_delta_store(const BwdParams& p, int bh, int i, const double* sums) {
    if (!bwd_short_row(p, i)) return;
    double l = 0.0, w = 0.0;
#pragma unroll
    for (int v = 0; v < NW; ++v) {
        l += sums[2 * STRIDE * v];
        w += sums[2 * STRIDE * v + 1];
    }
    const double dl = w / l;
    const float hi = (float)dl;
    p.delta[(int64_t)bh * p.Tq + i] = hi;
    p.delta_lo[(int64_t)bh * p.Tq + i] = (float)(dl - (double)hi);
}

// For a split key block: store this workgroup's dK^T and dV^T accumulators
// (N f32x16 per lane each, NT threads) as its partial, count the arrival, and,
// in the last workgroup to arrive, replace the accumulators by the
// chunk-ordered sum of all partials.  Returns whether this workgroup goes on
// to store dK and dV.  Must be reached by every thread of the workgroup.
template <int NT, int N>
__device__ __forceinline__ bool bwd_fixup(const BwdParams& p, const BwdWork& wk, f32x16 (&dk)[N], f32x16 (&dv)[N]) {
    if (wk.split < 0) return true;
    constexpr int NACC = 2 * N;
    constexpr int kDeviceScope = 0x10;  // buffer cache policy: sc1
    auto acc = [&](int a) -> f32x16& { return a < N ? dk[a] : dv[a - N]; };
    __shared__ int s_last;
    const int tid = threadIdx.x;
    const int BH = p.B * p.H;
    const size_t per_wg = (size_t)NT * NACC * 16;  // floats of one partial
    auto slot_rsrc = [&](int c) {
        return buffer_rsrc(p.part + ((size_t)(wk.slot0 + c) * BH + wk.bh) * per_wg, (uint32_t)(per_wg * 4));
    };
    // lane-major: f32x4 j of accumulator a of thread tid at byte (((4a + j) * NT + tid) * 16
    const uint32_t voff = (uint32_t)tid * 16;
    const auto mine = slot_rsrc(wk.chunk);
#pragma unroll
    for (int a = 0; a < NACC; ++a)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const f32x4 v = f32x4{acc(a)[4 * j], acc(a)[4 * j + 1], acc(a)[4 * j + 2], acc(a)[4 * j + 3]};
            __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, v), mine, (int)voff,
                                                   (4 * a + j) * NT * 16, kDeviceScope);
        }
    __builtin_amdgcn_s_waitcnt(0);  // the partial's stores are complete
    __syncthreads();
    if (tid == 0) s_last = atomicAdd(&p.counters[wk.split * BH + wk.bh], 1u) == (unsigned)(wk.n_chunks - 1);
    __syncthreads();
    if (!s_last) return false;
#pragma unroll
    for (int a = 0; a < NACC; ++a) acc(a) = f32x16{};
    for (int c = 0; c < wk.n_chunks; ++c) {
        const auto src = slot_rsrc(c);
#pragma unroll
        for (int a = 0; a < NACC; ++a)
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const f32x4 v = __builtin_bit_cast(
                    f32x4, __builtin_amdgcn_raw_buffer_load_b128(src, (int)voff, (4 * a + j) * NT * 16, kDeviceScope));
                acc(a)[4 * j] += v[0];
                acc(a)[4 * j + 1] += v[1];
                acc(a)[4 * j + 2] += v[2];
                acc(a)[4 * j + 3] += v[3];
            }
    }
    return true;
}

}  // namespace inf
