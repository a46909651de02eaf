// attn_fwd_bf16.hip -- fused causal attention forward, bf16 inputs, fp32
// accumulation, on v_mfma_f32_32x32x16_bf16 (gfx950).
//
// Same structure as the fp32 kernel (attn_fwd.hip): 4 waves x 32 query rows,
// K/V tiles of 64 keys double-buffered through LDS (loaded straight into LDS
// by direct-to-LDS buffer loads, one tile ahead), S^T = K Q^T and
// O^T += V^T P^T with queries on the lane axis, online softmax in fp32, and
// the same split plan (fwd_plan: a chunk of a long query tile's key range
// leaves fp32 partials that attn_fwd_merge_kernel combines into bf16 O).
// What bf16 changes is the operand shape: one MFMA reduces 16 elements, each
// lane supplying 8 consecutive ones.
//   S^T:  A = K[key][8 d's]  -- a 16-byte row read from the row-major K tile
//         B = Q[q][8 d's]    -- resident in VGPRs (D/4 registers)
//   O^T:  B = P^T[8 keys][q] -- straight from the S^T accumulators: MFMA m of
//         a 32-key block takes registers 8m..8m+7, i.e. keys
//         16m + 4g + {0..3} and 16m + 8 + 4g + {0..3} (converted to bf16)
//         A = V^T[d][the same 8 keys] -- V is staged row-major like K and
//         read transposed by gfx950's ds_read_b64_tr_b16: in each group of 16
//         lanes, output lane i, element k is element i % 4 of the 8 bytes
//         that lane 4k + i / 4 addresses.  With those 16 lanes addressing 4 key
//         rows x 4 chunks of 4 head-dim columns (row r0 + s / 4, columns
//         d0 + 4 (s % 4) for lane s), lane i receives column d0 + i of the 4
//         rows: two such reads (keys 16m + 4g + {0..3}, then + 8) are the
//         operand, the same two 8-byte reads per MFMA as a transposed copy
//         would need, without transposing stores while staging.
// Softmax statistics and the row sum stay fp32; P enters the MFMA rounded to
// bf16.
#include "common.h"
#include "kernels.h"

namespace inf {


template <int D>
struct FwdBf16Tile {
    static constexpr int BN = kFwdBf16BN;  // keys per tile
    static constexpr int KS = D + 8;    // K row stride in LDS (bf16 elements)
    // V row stride (bf16): a transposed read's 4 rows x 32 bytes must fall in
    // disjoint banks, i.e. a stride of 36 (D = 64), 72 or 24 (D = 128 / 32)
    // dwords modulo 64.
    static constexpr int VS = D == 64 ? D + 8 : D + 16;
};

// SPLIT: the launch carries a split plan (groups, partial slots); the
// instantiation without it keeps none of that code in its loop.
// PRIO: the P.V MFMAs run at raised wave priority (D = 128 without a split
// plan, on grids larger than one round of workgroup slots: fwd_plan).
template <int D, bool SPLIT, bool PRIO>
__global__ __launch_bounds__(256, 2) void attn_fwd_bf16_kernel(FwdParams p) {
    constexpr int BM = kFwdBM;
    constexpr int BN = FwdBf16Tile<D>::BN;
    constexpr int KS = FwdBf16Tile<D>::KS;
    constexpr int VS = FwdBf16Tile<D>::VS;
    constexpr int NKK = D / 16;          // MFMAs along the head dim for S^T
    constexpr int NKB = BN / 32;         // 32-key blocks per tile
    constexpr int NDB = D / 32;          // 32-wide head-dim blocks of O^T
    constexpr int C8 = D / 8;            // 8-element chunks per row

    // The two K / V buffers are distinct arrays, each step's named at compile
    // time, so the compiler can tell the direct-to-LDS loads of one from the
    // reads of the other (with one array indexed by the buffer number it waits
    // for those loads before every tile's first LDS read).
    __shared__ __attribute__((aligned(16))) __bf16 Ks0[BN][KS];
    __shared__ __attribute__((aligned(16))) __bf16 Ks1[BN][KS];
    __shared__ __attribute__((aligned(16))) __bf16 Vs0[BN][VS];
    __shared__ __attribute__((aligned(16))) __bf16 Vs1[BN][VS];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int l32 = lane & 31;
    const int g = lane >> 5;

    // Work: query tile and key-tile range [t_begin, t_end) of this workgroup
    // (the whole visible range, heaviest tiles first, without a split plan; a
    // group of the plan with one); a split chunk writes a partial to `slot`.
    const int BH = p.B * p.H;
    const int w = blockIdx.x;
    int qtile, t_begin = 0, t_end = 0x7fffffff, slot = -1;
    if constexpr (SPLIT) {
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

    const __bf16* Q = (const __bf16*)p.q + b * p.sq.b + h * p.sq.h;
    const __bf16* K = (const __bf16*)p.k + b * p.sk.b + h * p.sk.h;
    const __bf16* V = (const __bf16*)p.v + b * p.sv.b + h * p.sv.h;
    uint16_t* O = (uint16_t*)p.o + b * p.so.b + h * p.so.h;

    const int q0w = qtile * BM + wave * 32;
    const int qrow = q0w + l32;

    // Q operand: MFMA kk takes Q[qrow][16kk + 8g .. 16kk + 8g + 7].
    bf16x8 qf[NKK];
#pragma unroll
    for (int kk = 0; kk < NKK; ++kk) {
        if (qrow < p.Tq)
            qf[kk] = *reinterpret_cast<const bf16x8*>(Q + (int64_t)qrow * p.sq.t + 16 * kk + 8 * g);
        else
            qf[kk] = bf16x8{};
    }

    int kv_end = p.Tk;
    if (p.causal) kv_end = min(p.Tk, qtile * BM + BM + p.off);
    const int n_tiles = min((kv_end + BN - 1) / BN, t_end);
    const int wave_kend = p.causal ? min(kv_end, q0w + 32 + p.off) : kv_end;

    // Tile u of the range (keys kb0 + u*BN ...) goes from memory straight into
    // LDS through gfx950's 16-byte direct-to-LDS buffer loads: the 64 lanes of
    // one instruction fill 1 KiB at the instruction's LDS base, lane l at
    // +16 l.  A tile's padded rows are one run of 16-byte slots (SK per K row,
    // SV per V row, the last one or two of each row padding), so instruction j
    // fills slots 64 j .. 64 j + 63, each lane loading the chunk of its slot (a
    // pad slot loads its row's last chunk again; it is never read), and wave w
    // issues instructions w, w + 4, ...  The buffer resources cover the tile's
    // `rows` rows, so rows past them land as zeros, and the tile bases advance
    // by one tile per load (pointer increments, no per-step 64-bit products).
    constexpr int SK = KS / 8, SV = VS / 8;               // 16-byte slots per LDS row
    constexpr int NJK = BN * SK / 64, NJV = BN * SV / 64;  // load instructions per tile
    static_assert(BN * SK % 64 == 0 && BN * SV % 64 == 0, "a tile must fill whole instructions");
    constexpr int NI = ((NJK > NJV ? NJK : NJV) + 3) / 4;  // per wave
    const int kb0 = t_begin * BN;
    const int nt = n_tiles - t_begin;  // tiles in this workgroup's range
    const int klim = p.Tk - kb0;       // keys of the range that exist
    const int64_t kstep = (int64_t)BN * p.sk.t, vstep = (int64_t)BN * p.sv.t;
    const __bf16* kt = K + (int64_t)kb0 * p.sk.t;
    const __bf16* vt = V + (int64_t)kb0 * p.sv.t;
    const int wave_u = __builtin_amdgcn_readfirstlane(wave);
    // Every wave issues NI instructions of each kind: one past a tile's last
    // instruction repeats that one (the same bytes into the same slots), so no
    // load sits behind a branch.
    uint32_t k_voff[NI], v_voff[NI];  // this lane's byte offsets from the tile base
    int k_lds[NI], v_lds[NI];         // the instructions' LDS offsets (wave-uniform)
#pragma unroll
    for (int i = 0; i < NI; ++i) {
        const int jk = min(wave_u + 4 * i, NJK - 1), jv = min(wave_u + 4 * i, NJV - 1);
        const int sk = 64 * jk + lane, sv = 64 * jv + lane;
        k_voff[i] = (uint32_t)(((int64_t)(sk / SK) * p.sk.t + 8 * min(sk % SK, C8 - 1)) * 2);
        v_voff[i] = (uint32_t)(((int64_t)(sv / SV) * p.sv.t + 8 * min(sv % SV, C8 - 1)) * 2);
        k_lds[i] = 1024 * jk;
        v_lds[i] = 1024 * jv;
    }
    auto rows_of = [&](int t) { return t < nt ? min(klim - t * BN, BN) : 0; };
    auto dload = [&](__bf16 (&Kd)[BN][KS], __bf16 (&Vd)[BN][VS], int rows) {
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

    // transposed V reads: this lane's key-row offset and column offset
    const int tr_row = (lane & 15) >> 2;
    const int tr_col = 16 * ((lane >> 4) & 1) + 4 * (lane & 3);

    f32x16 o[NDB];
#pragma unroll
    for (int i = 0; i < NDB; ++i) o[i] = f32x16{};
    float m_run = -INFINITY;
    float l_run = 0.f;
    const float c = p.c;

    dload(Ks0, Vs0, rows_of(0));
    __builtin_amdgcn_s_waitcnt(0);  // this wave's loads have landed in LDS
    __syncthreads();

    // Step u reads buffer BUF (u % 2) while tile u + 1 loads into the other
    // one, which every wave finished reading before the previous step's
    // barrier; the step ends by waiting for its loads, then the barrier.
    auto step = [&](int u, auto buf_c) {
        constexpr int BUF = decltype(buf_c)::value;
        __bf16(&Kc)[BN][KS] = BUF ? Ks1 : Ks0;
        __bf16(&Vc)[BN][VS] = BUF ? Vs1 : Vs0;
        const int k0 = kb0 + u * BN;
        dload(BUF ? Ks0 : Ks1, BUF ? Vs0 : Vs1, rows_of(u + 1));

        if (k0 < wave_kend) {
            f32x16 s[NKB];
#pragma unroll
            for (int kk = 0; kk < NKK; ++kk)
#pragma unroll
                for (int kb = 0; kb < NKB; ++kb) {
                    const bf16x8 a = *reinterpret_cast<const bf16x8*>(&Kc[kb * 32 + l32][16 * kk + 8 * g]);
                    s[kb] = mfma32x32x16bf16(a, qf[kk], kk == 0 ? f32x16{} : s[kb]);
                }

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
            // row max as four independent chains (a single chain of dependent
            // three-input maxima waits out the VALU latency at every step)
            float mp[4] = {-INFINITY, -INFINITY, -INFINITY, -INFINITY};
#pragma unroll
            for (int kb = 0; kb < NKB; ++kb)
#pragma unroll
                for (int r = 0; r < 16; ++r) mp[r & 3] = fmaxf(mp[r & 3], s[kb][r]);
            float mloc = fmaxf(fmaxf(mp[0], mp[1]), fmaxf(mp[2], mp[3]));
            mloc = max_xor32(mloc);
            // Lazy rescaling, per row: the reference max moves only when the
            // row sees a score 2^8 (in exp2 units) above it; the wave skips the
            // O / l rescale when no row moved (a row that did not move would
            // multiply by exactly 1).  P <= 2^8 enters the MFMA as bf16.
            const bool grow = mloc > m_run + 8.f / c;
            if (__any(grow)) {
                const float alpha = grow ? fast_exp2((m_run - mloc) * c) : 1.f;  // m_run = -inf -> 0
                l_run *= alpha;
#pragma unroll
                for (int db = 0; db < NDB; ++db) o[db] *= alpha;
                m_run = grow ? mloc : m_run;
            }
            // A row of a split chunk may have no visible key in the chunk: it
            // keeps m_run = -inf, p = 0, and the merge skips its partial.
            const float mc = SPLIT && m_run == -INFINITY ? 0.f : m_run * c;
            float ls[4];  // row sum as four independent chains
            bf16x8 pb[NKB][2];
#pragma unroll
            for (int kb = 0; kb < NKB; ++kb)
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const float e = fast_exp2(fmaf(s[kb][r], c, -mc));
                    ls[r & 3] = kb == 0 && r < 4 ? e : ls[r & 3] + e;
                    pb[kb][r >> 3][r & 7] = (__bf16)e;
                }
            l_run += (ls[0] + ls[1]) + (ls[2] + ls[3]);

            // At D = 128 without a split plan (two workgroups per CU, each SIMD
            // holding waves of both) the P.V MFMAs run at raised wave priority, so
            // a wave that reaches them issues them ahead of the other wave's
            // softmax VALU work: config 4 forward 310 -> 295 us, B8 H12 T1024
            // 44.9 -> 43.9; it measured 2% slower at D = 64, 6% slower on
            // split-plan grids and 5-7% slower on grids that fit one round of
            // workgroup slots, which keep the default priority.
            constexpr bool kPvPrio = PRIO && D >= 128 && !SPLIT;
            if constexpr (kPvPrio) __builtin_amdgcn_s_setprio(1);
#pragma unroll
            for (int kb = 0; kb < NKB; ++kb)
#pragma unroll
                for (int mm = 0; mm < 2; ++mm) {
                    const int key = kb * 32 + 16 * mm + 4 * g;
#pragma unroll
                    for (int db = 0; db < NDB; ++db) {
                        // lane (group G = lane / 16, i = lane % 16) addresses key row
                        // key + i / 4, columns db*32 + 16 (G % 2) + 4 (i % 4); it receives
                        // column db*32 + l32 of keys key + {0..3} (then + 8 + {0..3})
                        const bf16x4 lo = ds_read_tr16(&Vc[key + tr_row][db * 32 + tr_col]);
                        const bf16x4 hi = ds_read_tr16(&Vc[key + 8 + tr_row][db * 32 + tr_col]);
                        const bf16x8 a = __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
                        o[db] = mfma32x32x16bf16(a, pb[kb][mm], o[db]);
                    }
                }
            if constexpr (kPvPrio) __builtin_amdgcn_s_setprio(0);
        }

        __builtin_amdgcn_s_waitcnt(0);
        __syncthreads();
    };
    for (int u = 0; u < nt; u += 2) {
        step(u, B0{});
        if (u + 1 < nt) step(u + 1, B1{});
    }

    const float l_tot = l_run + shfl_xor(l_run, 32);
    if (SPLIT && slot >= 0) {
        // partial of a split query tile (fp32): unnormalised O, row max, row sum
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
        uint16_t* dst = O + (int64_t)qrow * p.so.t;
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

template <int D>
static void launch_t(const FwdParams& p, dim3 grid, hipStream_t s) {
    if (p.n_groups)
        hipLaunchKernelGGL((attn_fwd_bf16_kernel<D, true, false>), grid, dim3(256), 0, s, p);
    else if (D >= 128 && p.pv_prio)
        hipLaunchKernelGGL((attn_fwd_bf16_kernel<D, false, (D >= 128)>), grid, dim3(256), 0, s, p);
    else
        hipLaunchKernelGGL((attn_fwd_bf16_kernel<D, false, false>), grid, dim3(256), 0, s, p);
}

int launch_attn_fwd_bf16(const FwdParams& p, hipStream_t s) {
    const dim3 grid((unsigned)((p.n_groups ? p.n_groups : p.n_qtiles) * p.B * p.H));
    switch (p.D) {
        case 32: launch_t<32>(p, grid, s); break;
        case 64: launch_t<64>(p, grid, s); break;
        case 128: launch_t<128>(p, grid, s); break;
        default: return (int)hipErrorInvalidValue;
    }
    return (int)hipGetLastError();
}

int fwd_bf16_occupancy(int D, int* blocks_per_cu) {
    switch (D) {
        case 32: return (int)hipOccupancyMaxActiveBlocksPerMultiprocessor(blocks_per_cu, attn_fwd_bf16_kernel<32, true, false>, 256, 0);
        case 64: return (int)hipOccupancyMaxActiveBlocksPerMultiprocessor(blocks_per_cu, attn_fwd_bf16_kernel<64, true, false>, 256, 0);
        case 128: return (int)hipOccupancyMaxActiveBlocksPerMultiprocessor(blocks_per_cu, attn_fwd_bf16_kernel<128, true, false>, 256, 0);
        default: return (int)hipErrorInvalidValue;
    }
}

}  // namespace inf
