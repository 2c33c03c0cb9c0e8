// Causal prefill / extend attention over a bf16 KV pool (bf16 MFMA).
//
// Replaces the reference's extend / mixed branch (qwen3_8/full_attention.py:244-283)
// and the ext_len > 1 case of its bsz == 1 branch (:179-213) for a bf16 pool.
// The reference pads queries to [B, max_ext, Hq, D], gathers and GQA-expands
// the whole padded context and runs a dense masked SDPA; here each request is
// processed at its own length and nothing is padded or expanded.
//
// Work item (from tf_attn_plan_extend): (request b, kv head hk, row0).  The
// rows of a (b, hk) pair are the ext_b * G flattened (token t, q head h) pairs
// of the kv head's q-head group, row = t * G + h; an item covers 256 of them,
// 64 per wave as two 32-row MFMA blocks, so all G heads of a GQA group share
// every K/V tile and every K or V fragment read from LDS feeds two MFMAs.
// Row (t, h) attends to context positions 0 .. P + t, P = L - ext.
//
// Per 32-key tile each wave computes, with v_mfma_f32_32x32x16_bf16 and for
// both of its row blocks,
//   S^T[key, row] = K Q^T        (Q^T register-resident, K from LDS),
//   the online softmax per row (a row's 32 scores live in lanes n and n + 32),
//   O^T[dim, row] += V^T P^T     (V^T read from row-major V in LDS with
//                                 ds_read_b64_tr_b16, P^T packed from S^T),
// so each lane owns one row per block: its max, sum and 128 output dims.
// Two row blocks per wave halve the LDS bytes per MFMA FLOP: at the MFMA peak
// rate the 4 waves of a CU read 64 B/clk of K and V fragments.
//
// Staging: K and V rows go from global memory straight into LDS
// (global_load_lds_dwordx4, 1 KB = two keys per instruction, 4 + 4 per wave
// per tile) two tiles ahead, into 3 K stages and 4 V stages (V is read one
// tile later than K), one pair per QK^T MFMA; one barrier per tile.  Slot ids
// reach LDS the same way, 1024 keys at a time (the low dword of each
// req_to_token entry).  Each tile's softmax runs beside the neighbouring
// tiles' MFMAs (see "one step" below).
// The running max is raised lazily: the accumulators are rescaled only when a
// row's max grows by more than 2^8 (exact in exact arithmetic; p <= 2^8).
#include <math.h>

#include "tf_common.h"
#include "tf_internal.h"

namespace tfa {
namespace {

typedef __attribute__((address_space(3))) void lds_void;
typedef short i16x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) i16x4 lds_i16x4;

constexpr int kD = 256;
constexpr int kWaves = 4;
constexpr int kThreads = kWaves * kWave;
constexpr int kRowsPerWave = 64;                     // two 32-row MFMA blocks
static_assert(kWaves * kRowsPerWave == kExtendItemRows, "item rows");
constexpr int kBN = 32;                              // keys per tile
constexpr int kRowBytes = 2 * kD;                    // 512
// K: key pairs (2i, 2i + 1) at i * kKPair, 32 bytes of padding after each
// pair; key n's 16-byte chunk c sits at chunk c ^ (n & 1) of its row.  The
// MFMA-operand reads (16 consecutive keys, one chunk) then hit 16 distinct
// 16-byte bank groups.
constexpr int kKPair = 2 * kRowBytes + 32;           // 1056
constexpr int kKStage = (kBN / 2) * kKPair;          // 16896
// V: row-major, 512 B per key; key n's chunk c sits at chunk c ^ vswz(n),
// vswz(n) = 10 (n & 1) + 4 ((n >> 1) & 1), which makes every transposing read
// (4 keys x 64 B per 32 lanes) conflict-free.
constexpr int kVStage = kBN * kRowBytes;             // 16384
constexpr int kAhead = 2;                            // tiles staged ahead of QK^T
constexpr int kStages = kAhead + 1;                  // K stages
constexpr int kVStages = kAhead + 2;                 // V stages (read one tile later)
constexpr int kSlotChunk = 1024;
constexpr int kSlotMask = 2 * kSlotChunk - 1;
constexpr int kTilesPerSlotChunk = kSlotChunk / kBN;
constexpr float kRescaleLog2 = 8.f;
constexpr int kQkAhead = 4;                          // K fragments in flight
constexpr int kPvAhead = 4;                          // V fragments in flight

struct __attribute__((aligned(16))) Smem {
  uint8_t k[kStages * kKStage];
  uint8_t v[kVStages * kVStage];
  int32_t slots[2 * kSlotChunk];   // 8 KB: key k's slot id at slots[k % 2048]
};

__device__ __forceinline__ int vswz(int n) { return 10 * (n & 1) + 4 * ((n >> 1) & 1); }

// ---------------------------------------------------------------- staging
// global_load_lds_dword{,x4} as inline assembly: lane l's 4 / 16 bytes land at
// LDS address M0 + 4 l / 16 l.  The compiler's wait-count pass does not see
// these loads (its own waits only get more conservative), so every reader of
// the staged data synchronises explicitly: s_waitcnt vmcnt, then a barrier.
__device__ __forceinline__ uint32_t lds_addr(const void* p) {
  return (uint32_t)(uintptr_t)(const lds_void*)p;
}
__device__ __forceinline__ void dma4(const void* gptr, uint32_t lds) {
  asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dword %0, off"
               :: "v"(gptr), "s"(lds) : "m0");
}
__device__ __forceinline__ void dma16(const void* gptr, uint32_t lds) {
  asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, off"
               :: "v"(gptr), "s"(lds) : "m0");
}

// End of step j: tile j + 1 (issued at step j + 1 - kAhead) must have landed;
// the 8 loads per tile of the newer kAhead - 1 tiles may still be in flight.
__device__ __forceinline__ void vm_wait_staged() {
  static_assert(kAhead == 2 || kAhead == 3, "vmcnt immediates");
  if (kAhead == 2)
    asm volatile("s_waitcnt vmcnt(8)" ::: "memory");
  else
    asm volatile("s_waitcnt vmcnt(16)" ::: "memory");
}

// Slot ids of keys [chunk * 1024, +1024) clamped to [0, kend): wave w moves
// 256 of them (4 dword instructions) into slot-buffer half chunk & 1.
__device__ __forceinline__ void slot_issue(const int64_t* rtt, int chunk, int kend, int w,
                                           int lane, int32_t* slots) {
  const int key0 = chunk * kSlotChunk + 256 * w;
  const uint32_t dst = lds_addr(slots + (chunk & 1) * kSlotChunk + 256 * w);
#pragma unroll
  for (int i = 0; i < 4; ++i) dma4(rtt + min(key0 + 64 * i + lane, kend - 1), dst + 256 * i);
}

// Wave w stages keys 8w .. 8w + 7 of a tile: instruction p moves keys
// 8w + 2p + {0, 1}; lane l fills 16-byte position l % 32 of key 8w + 2p + l / 32.
// The slot id is clamped into the pool where it is used, so that a stray
// req_to_token entry can never address memory outside the pool.
__device__ __forceinline__ int32_t stage_slot(const int32_t* slots, int tile, int w, int g,
                                              int p) {
  return slots[(tile * kBN + 8 * w + 2 * p + g) & kSlotMask];
}

// Per-lane global bases: lane l loads 16-byte chunk (l % 32) ^ (key & 1) of a
// K row and chunk (l % 32) ^ vswz(key) of a V row; key & 1 = l / 32 and
// vswz(key) = 10 (l / 32) + 4 (p & 1) for instruction p.
struct StageBases {
  const uint8_t* k;
  const uint8_t* v[2];   // by p & 1
};

__device__ __forceinline__ StageBases stage_bases(const uint8_t* kb, const uint8_t* vb, int lane) {
  const int pos = lane & 31, g = lane >> 5;
  StageBases sb;
  sb.k = kb + 16 * (pos ^ g);
  sb.v[0] = vb + 16 * (pos ^ (10 * g));
  sb.v[1] = vb + 16 * (pos ^ (10 * g + 4));
  return sb;
}

// Row `slot` (clamped into the pool) of K and V: one 32 x 32 -> 64-bit
// multiply-add per address (slot ids and the slot stride fit 32 bits).
__device__ __forceinline__ void kv_issue(const StageBases& sb, uint32_t slot_bytes, int32_t slot,
                                         int32_t smax, int w, int p, uint8_t* kst, uint8_t* vst) {
  const uint64_t off = (uint64_t)(uint32_t)min(max(slot, 0), smax) * slot_bytes;
  dma16(sb.k + off, lds_addr(kst + (4 * w + p) * kKPair));
  dma16(sb.v[p & 1] + off, lds_addr(vst + (8 * w + 2 * p) * kRowBytes));
}

// ---------------------------------------------------------------- MFMAs
// Register files: O^T (2 blocks x 8 tiles x 16 fp32) fills all 256 AGPRs, so
// S^T must come out of its MFMAs in VGPRs.  This file is compiled with
// -mllvm --amdgpu-mfma-vgpr-form=1, which gives the builtin MFMAs (S^T = K Q^T)
// VGPR results; the PV MFMAs are written as inline assembly with their
// accumulator bound to AGPRs ("+a").  The hazard recognizer cannot see inside
// that assembly, so it carries its own wait states: two ahead of each MFMA for
// sources a VALU just wrote, and 20 (more than the 19 an XDL result needs)
// after the last MFMA of a phase, inside the same statement, so that no copy
// or read the compiler places after the phase can see an unfinished tile.
// acc_settle() issues the same 20 where the accumulators are rewritten.
template <bool kLast>
__device__ __forceinline__ void mfma_acc(f32x16& d, const u32x4& a, const u32x4& b) {
  if (kLast)
    asm volatile("s_nop 1\n\tv_mfma_f32_32x32x16_bf16 %0, %1, %2, %0\n\t"
                 "s_nop 7\n\ts_nop 7\n\ts_nop 3"
                 : "+a"(d) : "v"(a), "v"(b));
  else
    asm volatile("s_nop 1\n\tv_mfma_f32_32x32x16_bf16 %0, %1, %2, %0" : "+a"(d) : "v"(a), "v"(b));
}
__device__ __forceinline__ void acc_settle() { asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 3"); }

// Multiplies an accumulator tile held in AGPRs by a per-lane factor one
// register at a time, so the tile never has to live in VGPRs.  The caller runs
// it only when no MFMA has written the tile within the last 19 wait states,
// and issues acc_settle() before an MFMA next reads it.
__device__ __forceinline__ void scale_acc(f32x16& x, float f) {
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    float e = x[i];
    float tmp;
    asm volatile(
        "v_accvgpr_read_b32 %1, %0\n\t"
        "v_mul_f32 %1, %1, %2\n\t"
        "v_accvgpr_write_b32 %0, %1"
        : "+a"(e), "=&v"(tmp)
        : "v"(f));
    x[i] = e;
  }
}
// ---------------------------------------------------------------- PV operand
// A operand of step q4 for output dims 32 mt + n: register j of lane (g, n)
// is V[key 16 q4 + 8 (j / 4) + 4 g + j % 4][32 mt + n], the key order in which
// P^T leaves the S^T accumulator.  ds_read_b64_tr_b16 hands lane i of each
// 16-lane group element i % 4 of the 8 bytes addressed by lane 4 k + (i % 16) / 4
// as its element k, so lane L addresses V[key 4 g + (L % 16) / 4 (+8)]
// [dims 32 mt + 16 ((L / 16) % 2) + 4 (L % 4) .. +3]; vaddr[mt % 4] holds that
// offset (swizzle included) for q4 = 0.
__device__ __forceinline__ u32x4 v_frag(const uint8_t* vst, const int (&vaddr)[4], int f) {
  const int q4 = f >> 3, mt = f & 7;
  const uint8_t* p = vst + vaddr[mt & 3] + 256 * (mt >> 2) + 16 * q4 * kRowBytes;
  const u32x2 lo = __builtin_bit_cast(
      u32x2, __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)(p)));
  const u32x2 hi = __builtin_bit_cast(
      u32x2, __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)(p + 8 * kRowBytes)));
  return u32x4{lo[0], lo[1], hi[0], hi[1]};
}

// ---------------------------------------------------------------- softmax
// Softmax state of the lane's two rows: reference max m (raw score units),
// moff = m * sl2, running sum l of p = 2^(s sl2 - moff).
struct Rows {
  float m[2], moff[2], l[2];
};

__device__ __forceinline__ void mask_tile(f32x16& s, int k0, int g, int limit) {
#pragma unroll
  for (int r = 0; r < 16; ++r)
    if (k0 + 8 * (r >> 2) + 4 * g + (r & 3) > limit) s[r] = -INFINITY;
}

// Max of lanes n and n + 32 (the two halves of a row's scores).
__device__ __forceinline__ float half_swap_max(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false,
                                                  false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}

// ---------------------------------------------------------------- one step
// Step j runs three tiles at once, each phase one MFMA stream with the other
// work placed one item per MFMA (sched_barrier regions):
//   phase A: S^T(j) = K(j) Q^T (32 MFMAs) | staging of tile j + 2 (slot ids at
//            MFMA 0, K and V rows 4-7) | second-half exps of tile j - 1
//            (MFMAs 12-27);
//   phase B: O^T += V(j - 1)^T P^T(j - 1) (32 MFMAs) | row max of tile j
//            (MFMAs 0-7, lane-half swap 8, reference update 9) | first-half
//            exps of tile j (10-25).
// Row block rb's P^T operand for 16-key step q4 is pt[rb][q4], p[rb][8 q4 ..
// 8 q4 + 7] packed to bf16; phase B overwrites pt[rb][0] (consumed by its
// first 16 MFMAs) with tile j's values from MFMA 17 on.
template <bool kQk, bool kExp>
__device__ __forceinline__ void phase_a(const uint8_t* kst, int kaddr, const u32x4 (&qf)[2][16],
                                        f32x16 (&s)[2], const int32_t* slots, int tile2, int w,
                                        int lane, int32_t smax, const StageBases& sb,
                                        uint32_t slot_bytes, uint8_t* k_dst, uint8_t* v_dst,
                                        const float (&sh)[2][8], Rows& rows, float sl2,
                                        u32x4 (&pt)[2][2]) {
  auto kread = [&](int kk) { return ld_s16(kst + kaddr + 32 * kk); };
  u32x4 fr[kQkAhead + 1];
  if (kQk) {
#pragma unroll
    for (int i = 0; i < kQkAhead; ++i) fr[i] = kread(i);
  }
  int32_t ss[4];
  float p[2][8];
#pragma unroll
  for (int i = 0; i < 32; ++i) {
    const int kk = i >> 1, rb = i & 1;
    // One region per MFMA: the MFMA issues first, this region's other work
    // follows it and overlaps its 32 cycles.
    __builtin_amdgcn_sched_barrier(0);
    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
    __builtin_amdgcn_sched_group_barrier(0x7f7, 64, 0);
    if (kQk) {
      if (rb == 0 && kk + kQkAhead < 16) fr[(kk + kQkAhead) % (kQkAhead + 1)] = kread(kk + kQkAhead);
      s[rb] = mfma_32x32x16(fr[kk % (kQkAhead + 1)], qf[rb][kk], kk == 0 ? f32x16{} : s[rb]);
      if (i == 0) {
#pragma unroll
        for (int q = 0; q < 4; ++q) ss[q] = stage_slot(slots, tile2, w, lane >> 5, q);
      } else if (i >= 4 && i < 8) {
        kv_issue(sb, slot_bytes, ss[i - 4], smax, w, i - 4, k_dst, v_dst);
      }
    }
    if (!kExp) continue;
    if (i >= 12 && i < 28) {
      // Exp e covers score r = e / 2 of block e % 2; each pair is packed as
      // soon as it is complete.
      const int e = i - 12, eb = e & 1, r = e >> 1;
      p[eb][r] = fast_exp2(fmaf(sh[eb][r], sl2, -rows.moff[eb]));
      if (r & 1) {
        pt[eb][1][r >> 1] = pack_bf16(p[eb][r - 1], p[eb][r]);
        rows.l[eb] += p[eb][r - 1] + p[eb][r];
        // Pin the result here: otherwise it is sunk past the rescale branch
        // into phase B's block, where it would run ahead of the PV MFMAs.
        asm volatile("" : "+v"(pt[eb][1][r >> 1]));
      }
      if (e == 15) asm volatile("" : "+v"(rows.l[0]), "+v"(rows.l[1]));
    }
  }
  __builtin_amdgcn_sched_barrier(0);
}

// Phase B; returns, per row block, whether its reference max was raised (the
// caller then rescales that block's accumulators by alpha).
template <bool kPv, bool kSoftmax>
__device__ __forceinline__ void phase_b(const uint8_t* vst, const int (&vaddr)[4],
                                        f32x16 (&acc)[2][8], const f32x16 (&s)[2], Rows& rows,
                                        float sl2, u32x4 (&pt)[2][2], float (&sh)[2][8],
                                        bool (&grew)[2], float (&alpha)[2]) {
  u32x4 fr[kPvAhead + 1];
  if (kPv) {
#pragma unroll
    for (int f = 0; f < kPvAhead; ++f) fr[f] = v_frag(vst, vaddr, f);
  }
  float mx[2];
  float p[2][8];
  uint32_t p_pair[2][4];
#pragma unroll
  for (int i = 0; i < 32; ++i) {
    const int f = i >> 1, rb = i & 1;
    __builtin_amdgcn_sched_barrier(0);   // MFMA first, as in phase_a
    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
    __builtin_amdgcn_sched_group_barrier(0x7f7, 64, 0);
    if (kPv) {
      if (rb == 0 && f + kPvAhead < 16)
        fr[(f + kPvAhead) % (kPvAhead + 1)] = v_frag(vst, vaddr, f + kPvAhead);
      if (i < 31)
        mfma_acc<false>(acc[rb][f & 7], fr[f % (kPvAhead + 1)], pt[rb][f >> 3]);
      else
        mfma_acc<true>(acc[rb][f & 7], fr[f % (kPvAhead + 1)], pt[rb][f >> 3]);
    }
    if (kSoftmax) {
      if (i < 8) {
        const int mb = i >> 2, q = i & 3;
        if (q == 0) mx[mb] = s[mb][0];
#pragma unroll
        for (int r = 4 * q; r < 4 * q + 4; ++r)
          if (r > 0) mx[mb] = fmaxf(mx[mb], s[mb][r]);
      } else if (i == 8) {
#pragma unroll
        for (int mb = 0; mb < 2; ++mb) mx[mb] = half_swap_max(mx[mb]);
      } else if (i == 9) {
        // Lazy reference max, per row: raised only when the row outgrew it by
        // more than 2^kRescaleLog2 (exact in exact arithmetic; p <= 2^8).  The
        // wave-wide vote only decides whether the rescale runs at all.
#pragma unroll
        for (int mb = 0; mb < 2; ++mb) {
          const bool grow = (mx[mb] - rows.m[mb]) * sl2 > kRescaleLog2;
          const float mnew = grow ? mx[mb] : rows.m[mb];
          alpha[mb] = grow ? fast_exp2((rows.m[mb] - mnew) * sl2) : 1.f;
          rows.l[mb] *= alpha[mb];
          rows.m[mb] = mnew;
          rows.moff[mb] = mnew * sl2;
          grew[mb] = __ballot(grow) != 0;
        }
      } else if (i >= 10 && i < 26) {
        const int e = i - 10, eb = e & 1, r = e >> 1;
        p[eb][r] = fast_exp2(fmaf(s[eb][r], sl2, -rows.moff[eb]));
        if (r & 1) {
          p_pair[eb][r >> 1] = pack_bf16(p[eb][r - 1], p[eb][r]);
          rows.l[eb] += p[eb][r - 1] + p[eb][r];
        }
      } else if (i == 26) {
#pragma unroll
        for (int b2 = 0; b2 < 2; ++b2) {
#pragma unroll
          for (int r = 0; r < 8; ++r) sh[b2][r] = s[b2][8 + r];
        }
      }
      // pt[.][0] was last read by MFMA 15; pairs 0-1 are complete at MFMA 17,
      // pairs 2-3 at MFMA 25.
      if (i == 17 || i == 26) {
        const int k0 = i == 17 ? 0 : 2;
#pragma unroll
        for (int b2 = 0; b2 < 2; ++b2)
#pragma unroll
          for (int k = k0; k < k0 + 2; ++k) pt[b2][0][k] = p_pair[b2][k];
      }
    }
  }
  __builtin_amdgcn_sched_barrier(0);
}

__global__ void __launch_bounds__(kThreads) extend_bf16_kernel(ExtendArgs a) {
  __shared__ Smem sm;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int w = wave_id();
  const int g = lane >> 5;
  const int n = lane & 31;

  const int32_t* wk = a.work + 8 * (int64_t)blockIdx.x;
  const int b = wk[0];
  const int hk = wk[1];
  const int row0 = wk[2];
  const int q_start = wk[3];
  const int ext = wk[4];
  const int G = a.group;

  if (ext <= 0) return;   // padding entry of a device-built work list
  int64_t len = a.seq_override > 0 ? (int64_t)a.seq_override : a.seq_lens[b];
  if (len > a.rtt_cols) len = a.rtt_cols;
  const int L = (int)len;
  const int P = L - ext;
  const int rows_total = ext * G;
  if (L <= 0 || row0 >= rows_total) return;

  const int64_t rrow = clamp_i64(a.rpi[b], 0, a.rtt_rows - 1);
  const int64_t* rtt = a.rtt + rrow * a.rtt_stride;

  // This lane's row in each block; padding lanes (row_ok false) compute a
  // valid duplicate row and never write it.
  int limit[2];
#pragma unroll
  for (int rb = 0; rb < 2; ++rb) {
    const int rho = min(row0 + kRowsPerWave * w + 32 * rb + n, rows_total - 1);
    limit[rb] = P + rho / G;   // last visible key
  }

  // Keys [0, kend) are needed by the item; keys below w_full are visible to
  // every row of this wave. Every wave runs all n_tiles tiles (keys past a
  // row's limit are masked; key 0 is visible to every row, so each row's max
  // is finite after tile 0).
  const int blk_last_row = min(row0 + kExtendItemRows, rows_total) - 1;
  const int kend = min(L, P + blk_last_row / G + 1);
  if (kend <= 0) return;
  const int n_tiles = (kend + kBN - 1) / kBN;
  const int last = n_tiles - 1;
  const int w_first = row0 + kRowsPerWave * w;
  const int w_full = w_first < rows_total ? P + w_first / G + 1 : 0;

  const float sl2 = a.scale_log2;
  const uint32_t slot_bytes = (uint32_t)a.hkv * kRowBytes;
  const StageBases sb = stage_bases(a.k_pool + (int64_t)hk * kRowBytes,
                                    a.v_pool + (int64_t)hk * kRowBytes, lane);
  const int32_t smax = (int32_t)min(a.pool_slots - 1, (int64_t)INT32_MAX);

  // LDS read offsets of this lane (see kv_issue / v_frag).
  const int kaddr = (n >> 1) * kKPair + (n & 1) * kRowBytes + 16 * (g ^ (n & 1));
  int vaddr[4];
  {
    const int s16 = lane & 15;
    const int r = s16 >> 2;                    // key within the 4-key group
    const int sw = vswz(r);
    const int c = 2 * ((lane >> 4) & 1) + ((s16 & 3) >> 1);
    const int base = (4 * g + r) * kRowBytes + 16 * (c ^ (sw & 3)) + 8 * (s16 & 1);
#pragma unroll
    for (int m2 = 0; m2 < 4; ++m2) vaddr[m2] = base + 64 * (m2 ^ (sw >> 2));
  }

  // Q^T fragments: lane (g, n) holds q[row n of block rb][16 kk + 8 g .. +8].
  u32x4 qf[2][16];
#pragma unroll
  for (int rb = 0; rb < 2; ++rb) {
    const int rho = min(row0 + kRowsPerWave * w + 32 * rb + n, rows_total - 1);
    const int t = rho / G, h = rho - t * G;
    const __bf16* qp = a.q + (int64_t)(q_start + t) * a.q_stride + (int64_t)(hk * G + h) * kD;
#pragma unroll
    for (int kk = 0; kk < 16; ++kk) qf[rb][kk] = ld_g16(qp + 16 * kk + 8 * g);
  }
  // Consume Q here so that the compiler waits for these loads before the
  // loop; inside it, vmcnt belongs to the staging loads.
#pragma unroll
  for (int rb = 0; rb < 2; ++rb)
#pragma unroll
    for (int kk = 0; kk < 16; ++kk) asm volatile("" ::"v"(qf[rb][kk]));

  Rows rows;
#pragma unroll
  for (int rb = 0; rb < 2; ++rb) {
    rows.m[rb] = -INFINITY;
    rows.moff[rb] = 0.f;
    rows.l[rb] = 0.f;
  }
  f32x16 acc[2][8];
#pragma unroll
  for (int rb = 0; rb < 2; ++rb)
#pragma unroll
    for (int i = 0; i < 8; ++i) acc[rb][i] = f32x16{};

  // ---- prologue: slot ids of the first 1024 keys, then tiles 0 and 1 into
  // stages 0 and 1. Tiles past the last one are stand-ins for the last tile
  // (its slots are staged, so every load stays inside the pool) and are never
  // read.
  slot_issue(rtt, 0, kend, w, lane, sm.slots);
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __syncthreads();
#pragma unroll
  for (int tl = 0; tl < kAhead; ++tl) {
    const int tile = min(tl, last);
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      kv_issue(sb, slot_bytes, stage_slot(sm.slots, tile, w, g, q), smax, w, q,
               sm.k + tl * kKStage, sm.v + tl * kVStage);
    }
  }
  vm_wait_staged();
  __syncthreads();

  // K tile t lives in K stage t % 3, V tile t in V stage t % 4. Step j stages
  // tile j + 2 while QK^T reads K(j) and PV reads V(j - 1); the stages it
  // overwrites held tiles j - 1 (K) and j - 2 (V), finished before the
  // previous barrier.
  f32x16 s[2];
  float sh[2][8];
  u32x4 pt[2][2];
  bool grew[2];
  float alpha[2];
  // Rescales O^T for the reference max raised in the previous step's phase B;
  // runs between phase A and phase B, where O^T holds exactly the tiles
  // before the one whose max raised it.
  auto rescale = [&]() {
    if (grew[0] || grew[1]) {
#pragma unroll
      for (int rb = 0; rb < 2; ++rb) {
        if (grew[rb]) {
#pragma unroll
          for (int i = 0; i < 8; ++i) scale_acc(acc[rb][i], alpha[rb]);
        }
      }
      acc_settle();
    }
  };
  auto step_end = [&]() {
    // Tile j + 1 was issued one step earlier: only this step's 8 tile loads
    // may still be in flight.
    vm_wait_staged();
    __syncthreads();
  };

  // Step 0: S^T(0) and the max / first-half exps of tile 0 (no PV yet).
  phase_a<true, false>(sm.k, kaddr, qf, s, sm.slots, min(kAhead, last), w, lane, smax, sb,
                       slot_bytes, sm.k + kAhead * kKStage, sm.v + kAhead * kVStage, sh, rows,
                       sl2, pt);
  if (kBN > w_full) {
#pragma unroll
    for (int rb = 0; rb < 2; ++rb) mask_tile(s[rb], 0, g, limit[rb]);
  }
  phase_b<false, true>(sm.v, vaddr, acc, s, rows, sl2, pt, sh, grew, alpha);
  step_end();

  for (int j = 1; j < n_tiles; ++j) {
    // Slot ids of the next 1024 keys: issued at tile 4 of chunk c into the
    // half that served chunk c - 1 (last read when tile 32 c - 1 was staged,
    // at step 32 c - 3), first read when tile 32 (c + 1) is staged.
    if (j % kTilesPerSlotChunk == 4 && (j / kTilesPerSlotChunk + 1) * kSlotChunk < kend)
      slot_issue(rtt, j / kTilesPerSlotChunk + 1, kend, w, lane, sm.slots);
    const int kst = j % kStages, kst2 = (j + kAhead) % kStages;
    const int vst = (j - 1) % kVStages, vst2 = (j + kAhead) % kVStages;

    phase_a<true, true>(sm.k + kst * kKStage, kaddr, qf, s, sm.slots, min(j + kAhead, last), w, lane,
                        smax, sb, slot_bytes, sm.k + kst2 * kKStage, sm.v + vst2 * kVStage, sh, rows, sl2,
                  pt);
    const int k0 = j * kBN;
    if (k0 + kBN > w_full) {
#pragma unroll
      for (int rb = 0; rb < 2; ++rb) mask_tile(s[rb], k0, g, limit[rb]);
    }
    rescale();
    phase_b<true, true>(sm.v + vst * kVStage, vaddr, acc, s, rows, sl2, pt, sh, grew, alpha);
    step_end();
  }

  // Tail: second-half exps and PV of the last tile.
  phase_a<false, true>(sm.k, kaddr, qf, s, sm.slots, 0, w, lane, smax, sb, slot_bytes, sm.k, sm.v,
                 sh, rows, sl2, pt);
  rescale();
  phase_b<true, false>(sm.v + (last % kVStages) * kVStage, vaddr, acc, s, rows, sl2, pt, sh,
                       grew, alpha);
  // The last steps staged stand-in tiles nobody reads; they must land before
  // the workgroup's LDS can be handed to another workgroup.
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  acc_settle();

#pragma unroll
  for (int rb = 0; rb < 2; ++rb) {
    const float lt = rows.l[rb] + __shfl_xor(rows.l[rb], 32, kWave);
    const int rho = row0 + kRowsPerWave * w + 32 * rb + n;
    if (rho >= rows_total) continue;
    const int t = rho / G, h = rho - t * G;
    const float inv = 1.f / lt;
    __bf16* o = a.out + (int64_t)(q_start + t) * a.out_stride + (int64_t)(hk * G + h) * kD;
    const __bf16* gt = a.gate ? a.gate + (int64_t)(q_start + t) * a.gate_stride +
                                    (int64_t)(hk * G + h) * a.gate_hstride
                              : nullptr;
#pragma unroll
    for (int mt = 0; mt < 8; ++mt) {
#pragma unroll
      for (int rq = 0; rq < 4; ++rq) {
        const int off = 32 * mt + 8 * rq + 4 * g;
        u32x2 v = {pack_bf16(acc[rb][mt][4 * rq + 0] * inv, acc[rb][mt][4 * rq + 1] * inv),
                   pack_bf16(acc[rb][mt][4 * rq + 2] * inv, acc[rb][mt][4 * rq + 3] * inv)};
        if (gt) {
          const u32x2 gv = ld_g8(gt + off);
          v = u32x2{gate_pair(v[0], gv[0]), gate_pair(v[1], gv[1])};
        }
        *reinterpret_cast<u32x2*>(o + off) = v;
      }
    }
  }
}

}  // namespace

void launch_extend_bf16(const ExtendArgs& a, int32_t n_work, hipStream_t stream) {
  hipLaunchKernelGGL(extend_bf16_kernel, dim3((unsigned)n_work), dim3(kThreads), 0, stream, a);
}

}  // namespace tfa
