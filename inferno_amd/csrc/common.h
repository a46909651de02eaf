// common.h -- shared device helpers for the gfx950 (CDNA4) attention kernels.
//
// Wave64 throughout.  MFMA operand/result layouts used by every kernel here
// (lane l = 0..63, l32 = l % 32, g = l / 32; checked on the GPU by
// tests/test_gpu_parity.py through the attention results themselves):
//   v_mfma_f32_32x32x2_f32   A: lane gives A[l32][g]   B: lane gives B[g][l32]
//                            D: reg r holds D[8*(r/4) + 4*g + r%4][l32]
//   v_mfma_f32_16x16x4_f32   A: lane gives A[l%16][l/16]  B: B[l/16][l%16]
//                            D: reg r holds D[4*(l/16) + r][l%16]
//   v_mfma_f32_32x32x16_bf16 A: lane gives A[l32][8*g .. 8*g+7]  B: B[8*g .. 8*g+7][l32]
//                            D: as 32x32x2
// The reduction index of an MFMA may be permuted freely as long as A and B
// agree, which is how the kernels feed a result tile straight back in as the
// next product's operand without a shuffle.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace inf {

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef uint16_t u16x4 __attribute__((ext_vector_type(4)));
typedef uint16_t u16x8 __attribute__((ext_vector_type(8)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;

__device__ __forceinline__ f32x16 mfma32x32x2(float a, float b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ f32x4 mfma16x16x4(float a, float b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ f32x16 mfma32x32x16bf16(bf16x8 a, bf16x8 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}

// Hardware exp2 (v_exp_f32): exp2(-inf) = 0, ~1 ulp.
__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// Cross-lane exchange within the wave (ds_bpermute; no LDS allocation).
__device__ __forceinline__ float shfl_xor(float v, int mask) {
    int lane = __lane_id();
    int src = lane ^ mask;
    return __int_as_float(__builtin_amdgcn_ds_bpermute(src << 2, __float_as_int(v)));
}

// max(v[l], v[l ^ 32]) in every lane l, on the VALU: v_permlane32_swap of
// two copies of v exchanges the upper half of the first with the lower half of
// the second, so in every lane the two results are v[l] and v[l ^ 32] (in
// either order).
__device__ __forceinline__ float max_xor32(float v) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}

// Sum over aligned groups of W lanes (W = 2..32), result in every lane of the
// group.  Within a 16-lane DPP row it is VALU-only: quad_perm [1,0,3,2] and
// [2,3,0,1] build quad sums, row_half_mirror (lane i <- 7-i) pairs the quads of
// each half-row and row_mirror (lane i <- 15-i) pairs the halves; only W = 32
// needs one cross-row ds_bpermute.
template <int CTRL>
__device__ __forceinline__ float dpp_mov(float x) {
    return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(x), CTRL, 0xF, 0xF, true));
}

template <int W>
__device__ __forceinline__ float group_sum(float v) {
    static_assert(W == 2 || W == 4 || W == 8 || W == 16 || W == 32, "group width");
    if constexpr (W >= 2) v += dpp_mov<0xB1>(v);   // quad_perm [1,0,3,2]
    if constexpr (W >= 4) v += dpp_mov<0x4E>(v);   // quad_perm [2,3,0,1]
    if constexpr (W >= 8) v += dpp_mov<0x141>(v);  // row_half_mirror
    if constexpr (W >= 16) v += dpp_mov<0x140>(v); // row_mirror
    if constexpr (W >= 32) v += shfl_xor(v, 16);
    return v;
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) v = fmaxf(v, shfl_xor(v, m));
    return v;
}
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) v += shfl_xor(v, m);
    return v;
}

// bf16 <-> fp32.  fp32 -> bf16 rounds to nearest even and keeps NaN a (quiet)
// NaN; gfx950 converts in hardware (v_cvt_pk_bf16_f32, two values per
// instruction), branch-free, where a bit-level rounding with a NaN test
// compiles to a divergent branch per element.
__device__ __forceinline__ float bf16_to_f32(uint16_t h) {
    return __uint_as_float(((uint32_t)h) << 16);
}
__device__ __forceinline__ uint16_t f32_to_bf16(float f) {
    return __builtin_bit_cast(uint16_t, static_cast<__bf16>(f));
}

// Element type tags: fp32 storage or bf16 storage (fp32 arithmetic either way).
struct F32 {
    using T = float;
    static __device__ __forceinline__ float ld(const float* p) { return *p; }
    static __device__ __forceinline__ void st(float* p, float v) { *p = v; }
};
struct BF16 {
    using T = uint16_t;
    static __device__ __forceinline__ float ld(const uint16_t* p) { return bf16_to_f32(*p); }
    static __device__ __forceinline__ void st(uint16_t* p, float v) { *p = f32_to_bf16(v); }
};

// Load 4 consecutive elements as fp32 (16-byte load for fp32, 8-byte for bf16).
__device__ __forceinline__ f32x4 ld4(const float* p) { return *reinterpret_cast<const f32x4*>(p); }

// Raw buffer resource over `bytes` bytes from `base` (gfx9 dword 3: raw
// addressing, no swizzle).  A load whose offset falls at or past `bytes`
// returns zeros without a memory access.  Callers pass wave-uniform values;
// reading them through readfirstlane keeps the descriptor in SGPRs even where
// the compiler cannot prove the uniformity itself (a descriptor in VGPRs
// turns every use into a loop over lanes).
__device__ __forceinline__ __amdgpu_buffer_rsrc_t buffer_rsrc(const void* base, uint32_t bytes) {
    const uint64_t a = reinterpret_cast<uint64_t>(base);
    const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)a);
    const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(a >> 32));
    const uint32_t n = __builtin_amdgcn_readfirstlane(bytes);
    return __builtin_amdgcn_make_buffer_rsrc(reinterpret_cast<void*>(((uint64_t)hi << 32) | lo), (short)0, (int)n,
                                             0x00020000);
}
// 16-byte load at byte offset voff (per lane) + soff (uniform).
__device__ __forceinline__ f32x4 buffer_ld4(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
    return __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(r, (int)voff, (int)soff, 0));
}
__device__ __forceinline__ float buffer_ld1(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
    return __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(r, (int)voff, (int)soff, 0));
}
// fp32 atomic add at byte offset voff + soff (dropped outside the resource).
// Cache policy 0: on gfx950 an agent-scope atomicAdd compiles to the same
// instruction without policy bits, so adds from workgroups on different XCDs
// to one address are device-coherent, as HIP's atomicAdd is.
__device__ __forceinline__ void buffer_atomic_add(__amdgpu_buffer_rsrc_t r, float v, uint32_t voff, uint32_t soff) {
    __builtin_amdgcn_raw_ptr_buffer_atomic_fadd_f32(v, r, (int)voff, (int)soff, 0);
}
// Resource over rows [row0, row0 + rows) of a row-major bf16 matrix (row
// stride `st` elements, `cols` used columns); loads return raw bf16 bits.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t row_rsrc(const __bf16* base, int64_t st, int row0, int rows, int cols) {
    const uint32_t bytes = rows > 0 ? (uint32_t)(((int64_t)(rows - 1) * st + cols) * 2) : 0u;
    return buffer_rsrc(base + (int64_t)row0 * st, bytes);
}
__device__ __forceinline__ bf16x8 buffer_ld8bf(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
    return __builtin_bit_cast(bf16x8, __builtin_amdgcn_raw_buffer_load_b128(r, (int)voff, (int)soff, 0));
}
// gfx950's 16-byte direct-to-LDS buffer load: 16 bytes at byte offset voff
// (per lane) of the resource land in LDS at `lds` (wave-uniform) + 16 * lane,
// without passing through VGPRs; the wave's memory counter covers them.
__device__ __forceinline__ void buffer_ld16_lds(__amdgpu_buffer_rsrc_t r, void* lds, uint32_t voff) {
    __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (__attribute__((address_space(3))) void*)lds, 16, voff, 0, 0, 0);
}
// gfx950's ds_read_b64_tr_b16 at an LDS address (8-byte aligned): in each
// group of 16 lanes, output lane i, element k is element i % 4 of the 8 bytes
// that lane 4 k + i / 4 addresses.  With the 16 lanes addressing 4 rows x 4
// chunks of 4 columns of a row-major bf16 tile (row r0 + s / 4, columns
// c0 + 4 (s % 4) for lane s), lane i receives column c0 + i of those 4 rows.
__device__ __forceinline__ bf16x4 ds_read_tr16(const __bf16* p) {
    return __builtin_bit_cast(bf16x4, __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                                          (__attribute__((address_space(3))) s16x4*)(p)));
}
// Resource over rows [row0, row0 + rows) of a row-major fp32 matrix with
// row stride `st` elements and `cols` used columns (rows <= 0: empty).
// Offsets must stay below 2^31 bytes: the caller bounds rows * st * 4.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t row_rsrc(const float* base, int64_t st, int row0, int rows, int cols) {
    const uint32_t bytes = rows > 0 ? (uint32_t)(((int64_t)(rows - 1) * st + cols) * 4) : 0u;
    return buffer_rsrc(base + (int64_t)row0 * st, bytes);
}
__device__ __forceinline__ f32x4 ld4(const uint16_t* p) {
    u16x4 h = *reinterpret_cast<const u16x4*>(p);
    f32x4 r;
    r[0] = bf16_to_f32(h[0]);
    r[1] = bf16_to_f32(h[1]);
    r[2] = bf16_to_f32(h[2]);
    r[3] = bf16_to_f32(h[3]);
    return r;
}
// Streaming (non-temporal) 4-element loads for data read exactly once.
__device__ __forceinline__ f32x4 ld4_nt(const float* p) {
    return __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(p));
}
__device__ __forceinline__ f32x4 ld4_nt(const uint16_t* p) {
    const u16x4 h = __builtin_nontemporal_load(reinterpret_cast<const u16x4*>(p));
    f32x4 r;
    r[0] = bf16_to_f32(h[0]);
    r[1] = bf16_to_f32(h[1]);
    r[2] = bf16_to_f32(h[2]);
    r[3] = bf16_to_f32(h[3]);
    return r;
}
__device__ __forceinline__ void st4(float* p, f32x4 v) { *reinterpret_cast<f32x4*>(p) = v; }
__device__ __forceinline__ void st4(uint16_t* p, f32x4 v) {
    u16x4 h;
    h[0] = f32_to_bf16(v[0]);
    h[1] = f32_to_bf16(v[1]);
    h[2] = f32_to_bf16(v[2]);
    h[3] = f32_to_bf16(v[3]);
    *reinterpret_cast<u16x4*>(p) = h;
}

}  // namespace inf
