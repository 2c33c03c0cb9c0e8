// Causal prefill / extend attention over an fp8-e4m3 KV pool (bf16 MFMA), and
// the tf_attn_extend entry point (bf16 pools run extend_bf16.hip's kernel).
//
// Replaces the reference's extend / mixed branch (qwen3_8/full_attention.py:244-283)
// and the ext_len > 1 case of its bsz == 1 branch (:179-213).  The reference
// pads queries to [B, max_ext, Hq, D], gathers and GQA-expands the whole padded
// context and runs a dense masked SDPA; here each request is processed at its
// own length and nothing is padded or expanded.
//
// Work item (from tf_attn_plan_extend): (request b, kv head hk, row0).  The
// rows of a (b, hk) pair are the ext_b * G flattened (token t, q head h) pairs
// of the kv head's q-head group, row = t * G + h; an item covers 256 of them
// and runs as two workgroups of 128 rows (32 per wave), so all G heads of a
// GQA group share every K/V tile.
// Row (t, h) attends to context positions 0 .. P + t, P = L - ext.
//
// Each wave computes, per 64-key tile j, with v_mfma_f32_32x32x16_bf16:
//   S^T[key, row] = K Q^T        (Q^T register-resident, K from LDS)
//   online softmax of S^T        (a row's 64 scores live in lanes n and n + 32)
//   O^T[dim, row] += V^T P^T     (V^T from LDS, P^T packed straight from S^T)
// so each lane owns one row: its max, sum and 128 of its output dims.  The
// e4m3 rows are widened to bf16 (exactly) on their way into LDS.
//
// Software pipeline (one barrier per tile, no wave-dependent branches around
// the accumulator so it stays in AGPRs):
//   * the QK^T MFMAs of tile j + 1 are issued next to the softmax of tile j,
//     and the exps of tile j next to its PV MFMAs, so VALU work hides under
//     matrix-core time;
//   * tile j + 2 is gathered from HBM into registers while tile j is computed
//     (slot ids come from an LDS slot buffer refilled 1024 keys at a time, so
//     no load waits on a dependent slot lookup in global memory);
//   * K lands in LDS row-major with a 16-byte pad per key row, V is transposed
//     in registers and lands as V^T rows of 64 keys, chunk-swizzled; both are
//     double-buffered (K(j+2) overwrites K(j) during PV(j); V(j+2) is written
//     at the start of the next tile, after every wave has finished PV(j)).
//   * The running max is raised lazily: the accumulator is rescaled only when
//     some row's max grows by more than 2^8, otherwise the old max stays the
//     reference point (exact in exact arithmetic; p <= 2^8 fits bf16's range).
#include <math.h>

#include <type_traits>

#include "tf_common.h"
#include "tf_internal.h"

namespace tfa {
namespace {

constexpr int kD = 256;
constexpr int kWaves = 4;
constexpr int kThreads = kWaves * kWave;
constexpr int kRowsPerWave = 32;
static_assert(2 * kWaves * kRowsPerWave == kExtendItemRows, "two workgroups per item");
constexpr int kBN = 64;                         // keys per tile
constexpr int kKStride = 2 * kD + 16;           // bytes per K row in LDS (padded)
constexpr int kKStage = kBN * kKStride;         // 33792
constexpr int kVtStride = 2 * kBN;              // bytes per V^T row (64 keys)
constexpr int kVtStage = kD * kVtStride;        // 32768
constexpr int kSlotChunk = 1024;                // keys per slot-buffer refill
constexpr int kSlotMask = 2 * kSlotChunk - 1;
constexpr int kTilesPerSlotChunk = kSlotChunk / kBN;
constexpr float kRescaleLog2 = 8.f;             // lazy-rescale threshold (log2 units)


struct __attribute__((aligned(16))) ExtendSmem {
  uint8_t k[2 * kKStage];          // 66 KB
  uint8_t vt[2 * kVtStage];        // 64 KB
  int32_t slots[2 * kSlotChunk];   // 8 KB: key k's slot id at slots[k % 2048]
};

// One tile's gathered rows for this thread: the 8 keys run0 + {0..3, 8..11}
// (run0 = 16 (grp / 2) + 4 (grp % 2), grp = tid / 32), 16 bytes each (chunk
// tid % 32 of the head row: dims 8c .. 8c + 7; fp8 rows keep 8 bytes in .xy).
// Those 8 keys are exactly V^T positions 8 grp .. 8 grp + 7 (see exp_pv_tile).
template <bool FP8>
struct TileRegs {
  u32x4 k[8];
  u32x4 v[8];
};

__device__ __forceinline__ int run_key(int j) { return 8 * (j >> 2) + (j & 3); }

template <bool FP8>
__device__ __forceinline__ void gather_tile(const int32_t* slots, const uint8_t* kb,
                                            const uint8_t* vb, uint32_t lane_off,
                                            int64_t slot_bytes, int key0, int run0,
                                            TileRegs<FP8>& r) {
  const u32x4 s0 = *reinterpret_cast<const u32x4*>(slots + ((key0 + run0) & kSlotMask));
  const u32x4 s1 = *reinterpret_cast<const u32x4*>(slots + ((key0 + run0 + 8) & kSlotMask));
  int64_t off[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) off[j] = (int64_t)(j < 4 ? s0[j] : s1[j - 4]) * slot_bytes + lane_off;
  // K rows first: store_k consumes them a whole tile earlier than store_vt
  // consumes the V rows.
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    if (FP8) {
      const u32x2 x = ld_g8(kb + off[j]);
      r.k[j] = u32x4{x[0], x[1], 0u, 0u};
    } else {
      r.k[j] = ld_g16(kb + off[j]);
    }
  }
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    if (FP8) {
      const u32x2 y = ld_g8(vb + off[j]);
      r.v[j] = u32x4{y[0], y[1], 0u, 0u};
    } else {
      r.v[j] = ld_g16(vb + off[j]);
    }
  }
}

template <bool FP8>
__device__ __forceinline__ void gather_k(const int32_t* slots, const uint8_t* kb, uint32_t lane_off,
                                         int64_t slot_bytes, int key0, int run0,
                                         TileRegs<FP8>& r) {
  const u32x4 s0 = *reinterpret_cast<const u32x4*>(slots + ((key0 + run0) & kSlotMask));
  const u32x4 s1 = *reinterpret_cast<const u32x4*>(slots + ((key0 + run0 + 8) & kSlotMask));
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const int64_t off = (int64_t)(j < 4 ? s0[j] : s1[j - 4]) * slot_bytes + lane_off;
    if (FP8) {
      const u32x2 x = ld_g8(kb + off);
      r.k[j] = u32x4{x[0], x[1], 0u, 0u};
    } else {
      r.k[j] = ld_g16(kb + off);
    }
  }
}

template <bool FP8>
__device__ __forceinline__ void store_k(uint8_t* kst, int run0, int c, const TileRegs<FP8>& r) {
  uint8_t* p = kst + run0 * kKStride + 16 * c;
#pragma unroll
  for (int j = 0; j < 8; ++j)
    st_s16(p + run_key(j) * kKStride, FP8 ? e4m3x8_to_bf16x8(r.k[j][0], r.k[j][1]) : r.k[j]);
}

// V^T row `dim` holds the tile's 64 keys in 8 chunks of 8 positions; chunk pc
// is stored at chunk pc ^ swz(dim), swz(dim) = (dim ^ (dim >> 3)) & 7, which
// keeps both these writes and the PV reads free of bank conflicts.
template <bool FP8>
__device__ __forceinline__ void store_vt(uint8_t* vst, int grp, int c, const TileRegs<FP8>& r) {
  u32x4 in[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) in[j] = FP8 ? e4m3x8_to_bf16x8(r.v[j][0], r.v[j][1]) : r.v[j];
  const int y = (grp ^ c) & 7;
  uint8_t* p = vst + 8 * c * kVtStride;
#pragma unroll
  for (int d = 0; d < 8; ++d) {
    u32x4 o;
#pragma unroll
    for (int w = 0; w < 4; ++w) o[w] = pair_sel(in[2 * w + 1][d >> 1], in[2 * w][d >> 1], d & 1);
    st_s16(p + d * kVtStride + 16 * (y ^ d), o);
  }
}

// Slot ids of keys [chunk * 1024, chunk * 1024 + 1024) clamped to the needed
// range [0, kend): loaded into registers (4 per thread) a few tiles before
// they are written to slot-buffer half (chunk & 1), so the req_to_token read
// latency hides under compute.
struct SlotPrefetch {
  int64_t v[kSlotChunk / kThreads];
};

__device__ __forceinline__ void slot_load(const int64_t* rtt, int chunk, int kend, int tid,
                                          SlotPrefetch& p) {
  const int k0 = chunk * kSlotChunk;
#pragma unroll
  for (int i = 0; i < kSlotChunk / kThreads; ++i) p.v[i] = rtt[min(k0 + tid + i * kThreads, kend - 1)];
}

__device__ __forceinline__ void slot_store(const SlotPrefetch& p, int chunk, int tid,
                                           int64_t pool_slots, bool wrap, int32_t* slots) {
  int32_t* buf = slots + (chunk & 1) * kSlotChunk;
#pragma unroll
  for (int i = 0; i < kSlotChunk / kThreads; ++i)
    buf[tid + i * kThreads] = (int32_t)pool_row(p.v[i], pool_slots, wrap);
}

// S^T (64 keys x 32 rows) = K_tile Q^T: s[hh][r] is key 32 hh + 8 (r / 4) + 4 g + r % 4.
// K fragments are read kQkAhead steps ahead of the MFMAs that consume them.
constexpr int kQkAhead = 3;
__device__ __forceinline__ void qk_tile(const uint8_t* kst, int kread, const u32x4 (&qf)[16],
                                        f32x16 (&s)[2]) {
  u32x4 fr[kQkAhead + 1][2];
#pragma unroll
  for (int p = 0; p < kQkAhead; ++p)
#pragma unroll
    for (int hh = 0; hh < 2; ++hh) fr[p][hh] = ld_s16(kst + kread + hh * 32 * kKStride + 32 * p);
  s[0] = f32x16{};
  s[1] = f32x16{};
#pragma unroll
  for (int kk = 0; kk < 16; ++kk) {
    if (kk + kQkAhead < 16) {
#pragma unroll
      for (int hh = 0; hh < 2; ++hh)
        fr[(kk + kQkAhead) % (kQkAhead + 1)][hh] =
            ld_s16(kst + kread + hh * 32 * kKStride + 32 * (kk + kQkAhead));
    }
#pragma unroll
    for (int hh = 0; hh < 2; ++hh) s[hh] = mfma_32x32x16(fr[kk % (kQkAhead + 1)][hh], qf[kk], s[hh]);
  }
  // Keep the reads kQkAhead steps ahead: the scheduler would otherwise sink
  // them next to their MFMAs and expose the LDS latency.
  __builtin_amdgcn_sched_group_barrier(0x100, 2 * kQkAhead, 0);
#pragma unroll
  for (int i = 0; i < 32 - 2 * kQkAhead; ++i) {
    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
    __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
  }
  __builtin_amdgcn_sched_group_barrier(0x008, 2 * kQkAhead, 0);
}

// Sets the scores of keys past this lane's last visible key to -inf.
__device__ __forceinline__ void mask_tile(f32x16 (&s)[2], int k0, int g, int limit) {
#pragma unroll
  for (int hh = 0; hh < 2; ++hh)
#pragma unroll
    for (int r = 0; r < 16; ++r)
      if (k0 + 32 * hh + 8 * (r >> 2) + 4 * g + (r & 3) > limit) s[hh][r] = -INFINITY;
}

// Phase A of a pipelined step: S^T of tile j + 1 (as qk_tile) with the tile
// staging spread one item per MFMA, so that LDS writes, global-load issue and
// the V transpose overlap matrix-core work instead of stalling in a burst:
//   MFMA 0:      slot ids of K tile kt and V tile vt from the LDS slot buffer
//   MFMAs 0-7:   K rows in registers -> K stage k_dst (one key per MFMA)
//   MFMAs 8-15:  V rows in registers -> transposed V^T stage v_dst (8 dims each)
//   MFMAs 16-23: global loads of tile kt's K rows into the registers just freed
//   MFMAs 24-31: global loads of tile vt's V rows
template <bool FP8>
__device__ __forceinline__ void qk_tile_staged(
    const uint8_t* kst, int kread, const u32x4 (&qf)[16], f32x16 (&s)[2], TileRegs<FP8>& r,
    uint8_t* k_dst, uint8_t* v_dst, int run0, int grp, int c, const int32_t* slots,
    const uint8_t* kb, const uint8_t* vb, uint32_t lane_off, int64_t slot_bytes, int kt, int vt) {
  u32x4 fr[kQkAhead + 1][2];
#pragma unroll
  for (int p = 0; p < kQkAhead; ++p)
#pragma unroll
    for (int hh = 0; hh < 2; ++hh) fr[p][hh] = ld_s16(kst + kread + hh * 32 * kKStride + 32 * p);
  s[0] = f32x16{};
  s[1] = f32x16{};
  u32x4 sk[2], sv[2];
  u32x4 vin[8];
  uint8_t* const kp = k_dst + run0 * kKStride + 16 * c;
  const int y = (grp ^ c) & 7;
  uint8_t* const vp = v_dst + 8 * c * kVtStride;
#pragma unroll
  for (int i = 0; i < 32; ++i) {
    const int kk = i >> 1, hh = i & 1;
    __builtin_amdgcn_sched_barrier(0);
    if (hh == 0 && kk + kQkAhead < 16) {
#pragma unroll
      for (int h2 = 0; h2 < 2; ++h2)
        fr[(kk + kQkAhead) % (kQkAhead + 1)][h2] =
            ld_s16(kst + kread + h2 * 32 * kKStride + 32 * (kk + kQkAhead));
    }
    s[hh] = mfma_32x32x16(fr[kk % (kQkAhead + 1)][hh], qf[kk], s[hh]);
    if (i == 0) {
      const int kk0 = kt * kBN + run0, vk0 = vt * kBN + run0;
      sk[0] = *reinterpret_cast<const u32x4*>(slots + (kk0 & kSlotMask));
      sk[1] = *reinterpret_cast<const u32x4*>(slots + ((kk0 + 8) & kSlotMask));
      sv[0] = *reinterpret_cast<const u32x4*>(slots + (vk0 & kSlotMask));
      sv[1] = *reinterpret_cast<const u32x4*>(slots + ((vk0 + 8) & kSlotMask));
    }
    if (i < 8) {
      st_s16(kp + run_key(i) * kKStride,
             FP8 ? e4m3x8_to_bf16x8(r.k[i][0], r.k[i][1]) : r.k[i]);
    } else if (i < 16) {
      const int d = i - 8;
      if (d == 0) {
#pragma unroll
        for (int j = 0; j < 8; ++j) vin[j] = FP8 ? e4m3x8_to_bf16x8(r.v[j][0], r.v[j][1]) : r.v[j];
      }
      u32x4 o;
#pragma unroll
      for (int w = 0; w < 4; ++w) o[w] = pair_sel(vin[2 * w + 1][d >> 1], vin[2 * w][d >> 1], d & 1);
      st_s16(vp + d * kVtStride + 16 * (y ^ d), o);
    } else if (i < 24) {
      const int j = i - 16;
      const int64_t off = (int64_t)(j < 4 ? sk[0][j] : sk[1][j - 4]) * slot_bytes + lane_off;
      if (FP8) {
        const u32x2 x = ld_g8(kb + off);
        r.k[j] = u32x4{x[0], x[1], 0u, 0u};
      } else {
        r.k[j] = ld_g16(kb + off);
      }
    } else {
      const int j = i - 24;
      const int64_t off = (int64_t)(j < 4 ? sv[0][j] : sv[1][j - 4]) * slot_bytes + lane_off;
      if (FP8) {
        const u32x2 x = ld_g8(vb + off);
        r.v[j] = u32x4{x[0], x[1], 0u, 0u};
      } else {
        r.v[j] = ld_g16(vb + off);
      }
    }
  }
  __builtin_amdgcn_sched_barrier(0);
}

// Online softmax of one tile's scores (raw, unscaled) for this lane's row, in
// two halves so that the rare accumulator rescale can sit between them and the
// exps stay in the same scheduling region as the PV MFMAs that consume them.
//
// softmax_max: the row max over the tile; the reference max m is raised only
// when some row of the wave outgrew it by more than 2^kRescaleLog2 (returns
// true, wave-uniform, with alpha = the factor for the accumulator and l).
__device__ __forceinline__ bool softmax_max(const f32x16 (&s)[2], float& m, float& l, float sl2,
                                            float& alpha) {
  float mx = s[0][0];
#pragma unroll
  for (int r = 1; r < 16; ++r) mx = fmaxf(mx, s[0][r]);
#pragma unroll
  for (int r = 0; r < 16; ++r) mx = fmaxf(mx, s[1][r]);
  mx = wave_max_xor(mx, 32);
  const bool grow = (mx - m) * sl2 > kRescaleLog2;
  const bool any = __ballot(grow) != 0;
  const float mnew = any ? fmaxf(m, mx) : m;
  alpha = any ? fast_exp2((m - mnew) * sl2) : 1.f;
  l *= alpha;
  m = mnew;
  return any;
}

// Exp half of the softmax fused with O^T += V^T P^T.
//
// p = 2^(s sl2 - m sl2) for the tile's 32 scores of this lane, l += sum p, and
// P^T packed as the B operands of four 16-key steps: step q4 takes scores
// 8 q4 .. 8 q4 + 7 (keys 16 q4 + 8 (j / 4) + 4 g + j % 4), and its A operand for
// output dims 32 mt + n is V^T row 32 mt + n, positions 16 q4 + 8 g .. +8.
// The exps of step q4 + 1 are issued one per MFMA of step q4, and the V^T
// reads kPvAhead MFMAs ahead; scheduling barriers keep that order.
constexpr int kPvAhead = 6;
__device__ __forceinline__ void exp_pv_tile(const uint8_t* vst, const int (&vb)[4][2],
                                            const f32x16 (&s)[2], float m, float& l,
                                            float sl2, f32x16 (&acc)[8]) {
  const float moff = m == -INFINITY ? 0.f : m * sl2;
  float p[32];
  u32x4 pt[4];
  auto ex = [&](int i) { p[i] = fast_exp2(fmaf(s[i >> 4][i & 15], sl2, -moff)); };
  auto pack = [&](int q4) {
#pragma unroll
    for (int k = 0; k < 4; ++k) pt[q4][k] = pack_bf16(p[8 * q4 + 2 * k], p[8 * q4 + 2 * k + 1]);
  };
  auto vread = [&](int i) {
    return ld_s16(vst + vb[i / 8][i & 1] + 32 * kVtStride * (i % 8));
  };
  u32x4 fr[kPvAhead + 1];
#pragma unroll
  for (int i = 0; i < kPvAhead; ++i) fr[i] = vread(i);
#pragma unroll
  for (int i = 0; i < 8; ++i) ex(i);
  pack(0);
#pragma unroll
  for (int i = 0; i < 32; ++i) {
    __builtin_amdgcn_sched_barrier(0);
    acc[i % 8] = mfma_32x32x16(fr[i % (kPvAhead + 1)], pt[i / 8], acc[i % 8]);
    if (i + kPvAhead < 32) fr[(i + kPvAhead) % (kPvAhead + 1)] = vread(i + kPvAhead);
    if (i < 24) {
      ex(8 + i);
      if (i % 8 == 7) pack(i / 8 + 1);
    }
  }
  __builtin_amdgcn_sched_barrier(0);
  float ps[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int i = 0; i < 32; ++i) ps[i & 3] += p[i];
  l += (ps[0] + ps[1]) + (ps[2] + ps[3]);
}

// Multiplies an accumulator tile held in AGPRs by a per-lane factor one
// register at a time, so the tile never has to live in VGPRs.
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

template <bool FP8>
__global__ void __launch_bounds__(kThreads)
extend_kernel(ExtendArgs a) {
  __shared__ ExtendSmem sm;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int w = wave_id();
  const int g = lane >> 5;
  const int n = lane & 31;

  // Two workgroups per 256-row work item, 128 rows each.
  const int32_t* wk = a.work + 8 * (int64_t)(blockIdx.x >> 1);
  const int b = wk[0];
  const int hk = wk[1];
  const int row0 = wk[2] + kWaves * kRowsPerWave * (int)(blockIdx.x & 1);
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

  // This lane's row; padding lanes (row_ok false) compute a valid duplicate row
  // and never write it.
  const int rho = row0 + kRowsPerWave * w + n;
  const bool row_ok = rho < rows_total;
  const int t = row_ok ? rho / G : ext - 1;
  const int h = row_ok ? rho - t * G : 0;
  const int limit = P + t;  // last visible key

  // Keys [0, kend) are needed by the block; keys below w_full are visible to
  // every row of this wave.
  const int blk_last_row = min(row0 + kWaves * kRowsPerWave, rows_total) - 1;
  const int kend = min(L, P + blk_last_row / G + 1);
  if (kend <= 0) return;
  const int n_tiles = (kend + kBN - 1) / kBN;
  // Every wave runs all n_tiles tiles (keys past a row's limit are masked, and
  // key 0 is visible to every row, so each row's max is finite after tile 0).
  const int w_first = row0 + kRowsPerWave * w;
  const int w_full = w_first < rows_total ? P + w_first / G + 1 : 0;

  const float kscale = FP8 ? a.k_scale[0] : 1.f;
  const float vscale = FP8 ? a.v_scale[0] : 1.f;
  const float sl2 = a.scale_log2 * kscale;

  // Gather mapping.
  const int grp = tid >> 5;
  const int c = tid & 31;
  const int run0 = 16 * (grp >> 1) + 4 * (grp & 1);
  constexpr int kRowBytes = FP8 ? kD : 2 * kD;
  const int64_t slot_bytes = (int64_t)a.hkv * kRowBytes;
  const uint8_t* kb = a.k_pool + (int64_t)hk * kRowBytes;
  const uint8_t* vb = a.v_pool + (int64_t)hk * kRowBytes;
  const uint32_t lane_off = (FP8 ? 8 : 16) * c;

  // LDS read offsets of this lane.
  const int kread = n * kKStride + 16 * g;
  int vbo[4][2];
  {
    const int z = (n ^ (n >> 3)) & 7;
#pragma unroll
    for (int q4 = 0; q4 < 4; ++q4)
#pragma unroll
      for (int p = 0; p < 2; ++p) vbo[q4][p] = n * kVtStride + 16 * (((2 * q4 + g) ^ z ^ (4 * p)) & 7);
  }

  // Q^T fragments: lane (g, n) holds q[row n][16 kk + 8 g .. +8].
  u32x4 qf[16];
  {
    const __bf16* qp = a.q + (int64_t)(q_start + t) * a.q_stride + (int64_t)(hk * G + h) * kD;
#pragma unroll
    for (int kk = 0; kk < 16; ++kk) qf[kk] = ld_g16(qp + 16 * kk + 8 * g);
  }

  float m = -INFINITY;
  float l = 0.f;
  f32x16 acc[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) acc[i] = f32x16{};

  uint8_t* const kst0 = sm.k;
  uint8_t* const kst1 = sm.k + kKStage;
  uint8_t* const vst0 = sm.vt;
  uint8_t* const vst1 = sm.vt + kVtStage;

  // ---- prologue: K(0), K(1), V(0) in LDS; K(2) and V(1) in registers; S(0)
  // computed. Tiles past the last one are stand-ins for the last tile (its
  // slots are staged, so every load stays inside the pool) and are never read.
  SlotPrefetch spf;
  slot_load(rtt, 0, kend, tid, spf);
  slot_store(spf, 0, tid, a.pool_slots, a.seq_override > 0, sm.slots);
  __syncthreads();
  const int last = n_tiles - 1;
  TileRegs<FP8> regs;
  gather_tile<FP8>(sm.slots, kb, vb, lane_off, slot_bytes, 0, run0, regs);
  store_k<FP8>(kst0, run0, c, regs);
  store_vt<FP8>(vst0, grp, c, regs);
  gather_tile<FP8>(sm.slots, kb, vb, lane_off, slot_bytes, min(1, last) * kBN, run0, regs);
  store_k<FP8>(kst1, run0, c, regs);
  gather_k<FP8>(sm.slots, kb, lane_off, slot_bytes, min(2, last) * kBN, run0, regs);
  __syncthreads();

  f32x16 sa[2];
  qk_tile(kst0, kread, qf, sa);

  // Step j: phase A computes S^T of tile j + 1 while K(j + 2) and V(j + 1)
  // move from registers to LDS and the loads of K(j + 3) and V(j + 2) are
  // issued; phase B is the softmax and PV of tile j. One barrier per step.
  for (int j = 0; j < n_tiles; ++j) {
    const int odd = j & 1;
    uint8_t* const k_this = odd ? kst1 : kst0;   // K(j) stage, gets K(j + 2)
    uint8_t* const k_next = odd ? kst0 : kst1;   // K(j + 1)
    uint8_t* const v_this = odd ? vst1 : vst0;   // V(j)
    uint8_t* const v_next = odd ? vst0 : vst1;   // gets V(j + 1)

    // Slot ids of the next 1024 keys: loaded at tile 4 of a chunk, written at
    // tile 8, first read by the loads issued at tile 13.
    if ((j / kTilesPerSlotChunk + 1) * kSlotChunk < kend) {
      if (j % kTilesPerSlotChunk == 4) slot_load(rtt, j / kTilesPerSlotChunk + 1, kend, tid, spf);
      if (j % kTilesPerSlotChunk == 8)
        slot_store(spf, j / kTilesPerSlotChunk + 1, tid, a.pool_slots, a.seq_override > 0, sm.slots);
    }
    const int k0 = j * kBN;
    if (k0 + kBN > w_full) mask_tile(sa, k0, g, limit);
    f32x16 sn[2];
    qk_tile_staged<FP8>(k_next, kread, qf, sn, regs, k_this, v_next, run0, grp, c, sm.slots,
                        kb, vb, lane_off, slot_bytes, min(j + 3, last), min(j + 2, last));
    float alpha;
    if (softmax_max(sa, m, l, sl2, alpha)) {
#pragma unroll
      for (int i = 0; i < 8; ++i) scale_acc(acc[i], alpha);
    }
    exp_pv_tile(v_this, vbo, sa, m, l, sl2, acc);
    sa[0] = sn[0];
    sa[1] = sn[1];
    __syncthreads();
  }

  if (!row_ok) return;
  l += __shfl_xor(l, 32, kWave);
  const float inv = vscale / l;
  __bf16* o = a.out + (int64_t)(q_start + t) * a.out_stride + (int64_t)(hk * G + h) * kD;
  const __bf16* gt = a.gate ? a.gate + (int64_t)(q_start + t) * a.gate_stride +
                                  (int64_t)(hk * G + h) * a.gate_hstride
                            : nullptr;
#pragma unroll
  for (int mt = 0; mt < 8; ++mt) {
#pragma unroll
    for (int rq = 0; rq < 4; ++rq) {
      const int off = 32 * mt + 8 * rq + 4 * g;
      u32x2 v = {pack_bf16(acc[mt][4 * rq + 0] * inv, acc[mt][4 * rq + 1] * inv),
                 pack_bf16(acc[mt][4 * rq + 2] * inv, acc[mt][4 * rq + 3] * inv)};
      if (gt) {
        const u32x2 gv = ld_g8(gt + off);
        v = u32x2{gate_pair(v[0], gv[0]), gate_pair(v[1], gv[1])};
      }
      *reinterpret_cast<u32x2*>(o + off) = v;
    }
  }
}

}  // namespace
}  // namespace tfa

extern "C" int32_t tf_attn_extend(const void* q, int64_t q_row_stride, const void* k_pool,
                                  const void* v_pool, int64_t pool_slots, int32_t kv_dtype,
                                  const float* k_scale, const float* v_scale,
                                  const int64_t* req_to_token, int64_t rtt_rows,
                                  int64_t rtt_row_stride, int64_t rtt_cols,
                                  const int64_t* req_pool_indices, const int64_t* seq_lens,
                                  int32_t seq_len_override, const int32_t* work,
                                  int32_t n_work, int32_t num_q_heads, int32_t num_kv_heads,
                                  int32_t head_dim, float scale, void* out,
                                  int64_t out_row_stride, const void* gate,
                                  int64_t gate_row_stride, int64_t gate_head_stride,
                                  tf_stream_t stream) {
  using namespace tfa;
  clear_error();
  if (n_work < 0) return fail(TF_ERR_INVALID, "extend: n_work=%d", n_work);
  if (num_kv_heads <= 0 || num_q_heads <= 0 || num_q_heads % num_kv_heads)
    return fail(TF_ERR_INVALID, "extend: num_q_heads=%d not a multiple of num_kv_heads=%d",
                num_q_heads, num_kv_heads);
  if (head_dim != kD)
    return fail(TF_ERR_UNSUPPORTED, "extend: head_dim=%d (only %d is built)", head_dim, kD);
  if (kv_dtype != TF_DTYPE_BF16 && kv_dtype != TF_DTYPE_FP8_E4M3)
    return fail(TF_ERR_UNSUPPORTED, "extend: kv_dtype=%d", kv_dtype);
  if (n_work == 0) return TF_OK;
  if (!q || !k_pool || !v_pool || !req_to_token || !req_pool_indices || !out || !work)
    return fail(TF_ERR_INVALID, "extend: null pointer argument");
  if (!seq_lens && seq_len_override <= 0)
    return fail(TF_ERR_INVALID, "extend: seq_lens is null and no override");
  if (kv_dtype == TF_DTYPE_FP8_E4M3 && (!k_scale || !v_scale))
    return fail(TF_ERR_INVALID, "extend: fp8 pool needs k_scale and v_scale");
  if (pool_slots < 1 || pool_slots > INT32_MAX || rtt_rows < 1 || rtt_cols < 1 ||
      rtt_row_stride < rtt_cols)
    return fail(TF_ERR_INVALID, "extend: bad pool/req_to_token extents");
  if (!aligned16(q) || !aligned16(out) || !aligned16(k_pool) || !aligned16(v_pool) ||
      (q_row_stride * 2) % 16 || (out_row_stride * 2) % 16 || !aligned16(work))
    return fail(TF_ERR_INVALID, "extend: q/out/pools/work must be 16-byte aligned");
  if (gate && (!aligned16(gate) || gate_row_stride % 8 || gate_head_stride % 8 ||
               gate_head_stride < head_dim))
    return fail(TF_ERR_INVALID, "extend: gate must be 16-byte aligned with strides of 8 elements");
  if ((int64_t)num_kv_heads * head_dim * 2 > INT32_MAX)
    return fail(TF_ERR_INVALID, "extend: num_kv_heads=%d too large", num_kv_heads);
  if (q_row_stride < (int64_t)num_q_heads * head_dim ||
      out_row_stride < (int64_t)num_q_heads * head_dim)
    return fail(TF_ERR_INVALID, "extend: row stride smaller than num_q_heads*head_dim");

  ExtendArgs a;
  a.q = static_cast<const __bf16*>(q);
  a.q_stride = q_row_stride;
  a.k_pool = static_cast<const uint8_t*>(k_pool);
  a.v_pool = static_cast<const uint8_t*>(v_pool);
  a.pool_slots = pool_slots;
  a.k_scale = k_scale;
  a.v_scale = v_scale;
  a.rtt = req_to_token;
  a.rtt_rows = rtt_rows;
  a.rtt_stride = rtt_row_stride;
  a.rtt_cols = rtt_cols;
  a.rpi = req_pool_indices;
  a.seq_lens = seq_lens;
  a.seq_override = seq_len_override;
  a.work = work;
  a.hkv = num_kv_heads;
  a.group = num_q_heads / num_kv_heads;
  a.scale_log2 = scale * kLog2e;
  a.out = static_cast<__bf16*>(out);
  a.out_stride = out_row_stride;
  a.gate = static_cast<const __bf16*>(gate);
  a.gate_stride = gate_row_stride;
  a.gate_hstride = gate_head_stride;

  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  if (kv_dtype == TF_DTYPE_FP8_E4M3)
    hipLaunchKernelGGL(extend_kernel<true>, dim3(2u * (unsigned)n_work), dim3(kThreads), 0, s, a);
  else
    launch_extend_bf16(a, n_work, s);
  return launch_status("tf_attn_extend launch");
}
