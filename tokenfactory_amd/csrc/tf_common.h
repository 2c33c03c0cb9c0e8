// Shared device helpers for the gfx950 full-attention kernels.
//
// Everything here is CDNA4-specific: 64-lane wavefronts, the bf16 MFMA
// instructions v_mfma_f32_16x16x32_bf16 / v_mfma_f32_16x16x16_bf16 /
// v_mfma_f32_32x32x16_bf16, and the OCP e4m3 conversions of gfx950.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace tfa {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

enum : int { DT_BF16 = 0, DT_FP8_E4M3 = 1, DT_FP32 = 2 };

constexpr int kWave = 64;
constexpr float kLog2e = 1.4426950408889634f;

// ---------------------------------------------------------------- loads
// Orders a wave's LDS accesses across its lanes: every lane's earlier LDS
// writes are visible to every lane's later reads (and earlier reads complete
// before later overwrites).  A wave-scope release / acquire around a wave
// barrier, for data passed between the lanes of one wave through LDS.
__device__ __forceinline__ void wave_lds_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

__device__ __forceinline__ u32x4 ld_g16(const void* p) {
  return *reinterpret_cast<const u32x4*>(p);
}
// Streaming (nontemporal) 16-byte load for data read exactly once.
__device__ __forceinline__ u32x4 ld_nt16(const void* p) {
  return __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
}
__device__ __forceinline__ u32x2 ld_g8(const void* p) {
  return *reinterpret_cast<const u32x2*>(p);
}
__device__ __forceinline__ u32x4 ld_s16(const void* p) {
  return *reinterpret_cast<const u32x4*>(p);
}
__device__ __forceinline__ void st_s16(void* p, u32x4 v) {
  *reinterpret_cast<u32x4*>(p) = v;
}
__device__ __forceinline__ void st_s8(void* p, u32x2 v) {
  *reinterpret_cast<u32x2*>(p) = v;
}

// ---------------------------------------------------------------- MFMA
// D = A * B + C.  Operand/result lane layouts (l = lane id):
//  16x16x32: A[i=l%16][k=8*(l/16)+j], B[k=8*(l/16)+j][n=l%16], C[4*(l/16)+r][l%16]
//  16x16x16: A[i=l%16][k=4*(l/16)+j], B[k=4*(l/16)+j][n=l%16], C[4*(l/16)+r][l%16]
//  32x32x16: A[i=l%32][k=8*(l/32)+j], B[k=8*(l/32)+j][n=l%32],
//            C[8*(r/4)+4*(l/32)+r%4][l%32]
__device__ __forceinline__ f32x4 mfma_16x16x32(u32x4 a, u32x4 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a),
                                                 __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
}
__device__ __forceinline__ f32x4 mfma_16x16x16(u32x2 a, u32x2 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(__builtin_bit_cast(bf16x4, a),
                                                   __builtin_bit_cast(bf16x4, b), c, 0, 0, 0);
}
__device__ __forceinline__ f32x16 mfma_32x32x16(u32x4 a, u32x4 b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a),
                                                 __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
}

// ---------------------------------------------------------------- packing
// Two fp32 -> packed bf16 pair (round to nearest even; v_cvt_pk_bf16_f32).
__device__ __forceinline__ uint32_t pack_bf16(float lo, float hi) {
  bf16x2 v = {(__bf16)lo, (__bf16)hi};
  return __builtin_bit_cast(uint32_t, v);
}
// Low (sel_hi=false) or high halves of two dwords -> (b.half | a.half << 16).
__device__ __forceinline__ uint32_t pair_lo(uint32_t a, uint32_t b) {
  return __builtin_amdgcn_perm(a, b, 0x05040100u);
}
__device__ __forceinline__ uint32_t pair_hi(uint32_t a, uint32_t b) {
  return __builtin_amdgcn_perm(a, b, 0x07060302u);
}
__device__ __forceinline__ uint32_t pair_sel(uint32_t a, uint32_t b, int hi) {
  return hi ? pair_hi(a, b) : pair_lo(a, b);
}

// Two OCP e4m3 bytes (low or high 16-bit word of src) -> packed bf16 pair.
// Exact: every e4m3 value, subnormals included, is representable in bf16.
template <bool HI>
__device__ __forceinline__ uint32_t e4m3x2_to_bf16x2(uint32_t src) {
  return __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(src, 1.0f, HI));
}
// 8 e4m3 bytes (two dwords) -> 8 bf16 (four dwords), element order kept.
__device__ __forceinline__ u32x4 e4m3x8_to_bf16x8(uint32_t d0, uint32_t d1) {
  u32x4 r;
  r[0] = e4m3x2_to_bf16x2<false>(d0);
  r[1] = e4m3x2_to_bf16x2<true>(d0);
  r[2] = e4m3x2_to_bf16x2<false>(d1);
  r[3] = e4m3x2_to_bf16x2<true>(d1);
  return r;
}

// ---------------------------------------------------------------- output gate
// The attention output gate of full_attention.py:157-159 on a pair of
// outputs: bf16(o * bf16(silu(g))), the reference's two bf16 tensor ops, each
// rounding to bf16.  silu(x) = x / (1 + exp(-x)) is evaluated in fp32 with the
// hardware exp2 and reciprocal (about 1 ulp each), so after the bf16 rounding
// it agrees with an exactly rounded evaluation except, rarely, by one bf16 ulp;
// +-inf, NaN and huge magnitudes give the same results (inf, NaN, NaN, x, -0).
// o: the two attention outputs already rounded to bf16; gp: two bf16 gates.
__device__ __forceinline__ float bf16_lo(uint32_t p) { return __uint_as_float(p << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t p) { return __uint_as_float(p & 0xffff0000u); }
__device__ __forceinline__ float silu_to_bf16(float g) {
  const float e = __builtin_amdgcn_exp2f(-g * kLog2e);
  return bf16_lo(pack_bf16(g * __builtin_amdgcn_rcpf(1.f + e), 0.f));
}
__device__ __forceinline__ uint32_t gate_pair(uint32_t o, uint32_t gp) {
  return pack_bf16(bf16_lo(o) * silu_to_bf16(bf16_lo(gp)),
                   bf16_hi(o) * silu_to_bf16(bf16_hi(gp)));
}

// |x| of eight bf16 values as bit patterns: for non-negative values the
// integer order is the float order and every NaN pattern sorts above +inf.
__device__ __forceinline__ uint32_t abs_max8(u32x4 v) {
  uint32_t m = 0;
#pragma unroll
  for (int j = 0; j < 4; ++j) m = max(m, max(v[j] & 0x7fffu, (v[j] >> 16) & 0x7fffu));
  return m;
}

// Raises *amax to the largest m of the wave's lanes (bf16 bit patterns of |o|
// from abs_max8): one wave-wide reduction and at most one no-return atomic per
// wave, the per-tensor amax of the dynamic FP8 quantisation that follows the
// attention output (fp8_triton.py:128).  Every lane of the wave calls it;
// amax NULL: nothing to do.
__device__ __forceinline__ void amax_commit(uint32_t* amax, uint32_t m) {
  if (!amax) return;
#pragma unroll
  for (int d = 32; d >= 1; d >>= 1) m = max(m, (uint32_t)__shfl_xor((int)m, d, kWave));
  if ((threadIdx.x & (kWave - 1)) == 0 && m != 0)
    __hip_atomic_fetch_max(amax, m, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Wave index within the workgroup as a scalar (wave-uniform) value, so loops
// and branches keyed on it compile to scalar control flow.
__device__ __forceinline__ int wave_id() {
  return __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
}

// ---------------------------------------------------------------- math
// Sum over the 8 lanes of a row; every lane gets the same bits (each step adds
// the same two operands in every lane of a pair).
__device__ __forceinline__ float row_sum8(float v) {
  v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(
                                     0, __builtin_bit_cast(int, v), 0xB1, 0xF, 0xF, false));
  v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(
                                     0, __builtin_bit_cast(int, v), 0x4E, 0xF, 0xF, false));
  v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(
                                     0, __builtin_bit_cast(int, v), 0x141, 0xF, 0xF, false));
  return v;
}

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

__device__ __forceinline__ float wave_max_xor(float v, int mask) {
  return fmaxf(v, __shfl_xor(v, mask, kWave));
}

__device__ __forceinline__ int64_t clamp_i64(int64_t v, int64_t lo, int64_t hi) {
  return v < lo ? lo : (v > hi ? hi : v);
}

// The pool row a req_to_token entry `v` reads.  The reference's batched
// branches clamp (`.clamp(min=0)`, full_attention.py:217-219), so a negative
// entry reads slot 0; its bsz == 1 branch indexes the pool directly (:188-190),
// where a negative entry v >= -S reads slot S + v as torch indexing does
// (`wrap`).  Anything else outside the pool is clamped into it, so no entry
// can address memory outside the pool (the reference raises there).
__device__ __forceinline__ int64_t pool_row(int64_t v, int64_t pool_slots, bool wrap) {
  if (wrap && v < 0) v += pool_slots;
  return clamp_i64(v, 0, pool_slots - 1);
}

}  // namespace tfa
