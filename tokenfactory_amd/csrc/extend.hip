// Causal prefill / extend attention over a bf16 or fp8-e4m3 KV pool (bf16
// MFMA), and the tf_attn_extend entry point.
//
// Replaces the reference's extend / mixed branch (qwen3_8/full_attention.py:244-283)
// and the ext_len > 1 case of its bsz == 1 branch (:179-213).
// The reference pads queries to [B, max_ext, Hq, D], gathers and GQA-expands
// the whole padded context and runs a dense masked SDPA; here each request is
// processed at its own length and nothing is padded or expanded.
//
// Work item (from tf_attn_plan_extend): (request b, kv head hk, row0).  The
// rows of a (b, hk) pair are the ext_b * G flattened (token t, q head h) pairs
// of the kv head's q-head group, row = t * G + h; an item covers 256 of them,
// 32 per wave (one 32-row MFMA block) over 8 waves, so all G heads of a GQA
// group share every K/V tile staged in LDS.
// Row (t, h) attends to context positions 0 .. P + t, P = L - ext.
//
// Per 32-key tile each wave computes, with v_mfma_f32_32x32x16_bf16,
//   S^T[key, row] = K Q^T        (Q^T register-resident, K from LDS),
//   the online softmax per row (a row's 32 scores live in lanes n and n + 32),
//   O^T[dim, row] += V^T P^T     (V^T read from row-major V in LDS with
//                                 ds_read_b64_tr_b16, P^T packed from S^T),
// so each lane owns one row: its max, sum and 128 output dims.
//
// Two waves per SIMD, half a step apart.  O^T (128 registers) and Q^T (64)
// of a 32-row block leave room for a second wave on each SIMD.  Waves 0-3
// ("lead") run QK^T(j), softmax(j), PV(j) between barriers j - 1 and j; waves
// 4-7 ("trail", one per SIMD beside a lead wave) run PV(j - 1), QK^T(j),
// softmax(j).  So while one wave of a SIMD works through its softmax the other
// issues MFMAs, and each wave's waits (LDS, barrier, MFMA results) are covered
// by the other wave's work.
//
// Staging: K and V rows go from global memory straight into LDS
// (global_load_lds_dwordx4, 1 KB = two keys per instruction, 2 + 2 per wave
// per tile) two tiles ahead, into 3 K stages and 4 V stages (the trailing
// waves read V one tile later than K), one barrier per tile.  Slot ids reach
// LDS the same way, 1024 keys at a time (the low dword of each req_to_token
// entry).  fp8 pools: the e4m3 rows go into LDS the same way (one K and one V
// instruction per wave per tile) and one step later each lane widens the 16
// bytes it loaded into the bf16 stages (exact), so the MFMA side is the bf16
// kernel's; scores and outputs are scaled by k_scale / v_scale.
// The running max is raised lazily: the accumulators are rescaled only when a
// row's max grows by more than 2^8 (exact in exact arithmetic; p <= 2^8).
#include <math.h>

#include <type_traits>

#include "tf_common.h"
#include "tf_internal.h"

namespace tfa {
namespace {

typedef __attribute__((address_space(3))) void lds_void;
typedef short i16x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) i16x4 lds_i16x4;

constexpr int kD = 256;
constexpr int kWaves = 8;
constexpr int kLeadWaves = kWaves / 2;
constexpr int kThreads = kWaves * kWave;
constexpr int kRowsPerWave = 32;                     // one 32-row MFMA block
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
constexpr int kAhead = 2;                            // tiles staged ahead
// bf16 pools: the DMA fills the K / V stages the MFMAs read, 3 K stages and 4
// V stages (the trailing waves read V one tile later than K).  fp8 pools: the
// DMA fills two e4m3 stages and the widened tile goes into the bf16 stages one
// step before it is read, so 2 K and 3 V stages suffice.
template <bool FP8> constexpr int kStagesOf = FP8 ? 2 : kAhead + 1;
template <bool FP8> constexpr int kVStagesOf = FP8 ? 3 : kAhead + 2;
constexpr int kF8Half = kBN * kD;                    // 8 KB: one tile of e4m3 K (or V)
constexpr int kF8Stage = 2 * kF8Half;                // K then V
constexpr int kSlotChunk = 1024;
constexpr int kSlotMask = 2 * kSlotChunk - 1;
constexpr int kTilesPerSlotChunk = kSlotChunk / kBN;
constexpr float kRescaleLog2 = 8.f;
constexpr int kQkAhead = 2;                          // K fragments in flight
constexpr int kPvAhead = 2;                          // V fragments in flight

// A wave's 32 rows x 256 dims of bf16 (Q on the way in, the output on the
// way out), row-major with 16-byte chunk c of row r at chunk c ^ r: the
// row-contiguous global side and the MFMA-fragment side both access it
// without bank conflicts beyond two-way.
constexpr int kTileBytes = kRowsPerWave * kRowBytes;   // 16 KB

template <bool FP8>
struct __attribute__((aligned(16))) Smem {
  union {
    struct {
      uint8_t k[kStagesOf<FP8> * kKStage];
      uint8_t v[kVStagesOf<FP8> * kVStage];
      uint8_t f8[FP8 ? 2 * kF8Stage : 16];   // e4m3 rows as they arrive
    };
    uint8_t rows[kWaves][kTileBytes];   // Q in the prologue, the output at the end
  };
  int32_t slots[2 * kSlotChunk];   // 8 KB: key k's slot id at slots[k % 2048]
};
static_assert(sizeof(Smem<true>) <= 160 * 1024 && sizeof(Smem<false>) <= 160 * 1024, "LDS");

__device__ __forceinline__ int swz_chunk(int r, int c) { return (c ^ r) & 31; }

// x through an empty asm: what is computed from it cannot be hoisted out of
// the block (the epilogue's row arithmetic would otherwise be computed in the
// prologue and kept, or spilled, across the whole tile loop).
__device__ __forceinline__ int opaque(int x) {
  asm volatile("" : "+v"(x));
  return x;
}

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

// The tile issued one step earlier must have landed; the loads per wave of the
// tile issued in this step (4 for bf16 rows, 2 for e4m3 rows) may still be in
// flight.
template <bool FP8>
__device__ __forceinline__ void vm_wait_staged() {
  static_assert(kAhead == 2, "vmcnt immediate");
  if (FP8)
    asm volatile("s_waitcnt vmcnt(2)" ::: "memory");
  else
    asm volatile("s_waitcnt vmcnt(4)" ::: "memory");
}

// Slot ids of keys [chunk * 1024, +1024) clamped to [0, kend): wave w moves
// 128 of them (2 dword instructions) into slot-buffer half chunk & 1.
__device__ __forceinline__ void slot_issue(const int64_t* rtt, int chunk, int kend, int w,
                                           int lane, int32_t* slots) {
  const int key0 = chunk * kSlotChunk + 128 * w;
  const uint32_t dst = lds_addr(slots + (chunk & 1) * kSlotChunk + 128 * w);
#pragma unroll
  for (int i = 0; i < 2; ++i) dma4(rtt + min(key0 + 64 * i + lane, kend - 1), dst + 256 * i);
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

// What one step stages: wave w moves keys 4w .. 4w + 3 of `tile`; instruction
// p moves keys 4w + 2p + {0, 1}, lane l filling 16-byte position l % 32 of key
// 4w + 2p + l / 32.  The slot id is clamped into the pool where it is used, so
// that a stray req_to_token entry can never address memory outside the pool.
struct Stager {
  StageBases sb;
  const int32_t* slots;
  uint8_t* k_dst;
  uint8_t* v_dst;
  uint32_t slot_bytes;
  int32_t smax;
  bool wrap;     // bsz == 1 call: negative slot ids index from the pool's end
  int tile;
  int w;
  int g;

  __device__ __forceinline__ int32_t slot(int p) const {
    return slots[(tile * kBN + 4 * w + 2 * p + g) & kSlotMask];
  }
  // Row `slot` of K and V: one 32 x 32 -> 64-bit multiply-add per address
  // (slot ids and the slot stride fit 32 bits).
  __device__ __forceinline__ void issue(int32_t sl, int p) const {
    if (wrap && sl < 0) sl += smax + 1;
    const uint64_t off = (uint64_t)(uint32_t)min(max(sl, 0), smax) * slot_bytes;
    dma16(sb.k + off, lds_addr(k_dst + (2 * w + p) * kKPair));
    dma16(sb.v[p & 1] + off, lds_addr(v_dst + (4 * w + 2 * p) * kRowBytes));
  }
  // The phases' interface: slot ids read at one MFMA, loads issued at the
  // next two.
  struct Ids {
    int32_t s[2];
  };
  __device__ __forceinline__ Ids fetch() const { return Ids{{slot(0), slot(1)}}; }
  __device__ __forceinline__ void issue_part(const Ids& ids, int p) const { issue(ids.s[p], p); }
};

// fp8 pools: wave w moves the e4m3 rows of keys 4w .. 4w + 3 of `tile`, one
// instruction for K and one for V (1 KB each); lane l fills 16-byte chunk
// l % 16 of key 4w + l / 16, row-major in the e4m3 stage (256 bytes per key).
struct Stager8 {
  const uint8_t* k;     // pool bases + kv head + this lane's chunk
  const uint8_t* v;
  const int32_t* slots;
  uint8_t* dst;         // e4m3 stage + this wave's 4 keys
  uint32_t slot_bytes;
  int32_t smax;
  bool wrap;
  int tile;
  int key;              // 4w + l / 16

  struct Ids {
    int32_t s;
  };
  __device__ __forceinline__ Ids fetch() const {
    return Ids{slots[(tile * kBN + key) & kSlotMask]};
  }
  __device__ __forceinline__ void issue_part(const Ids& ids, int p) const {
    int32_t sl = ids.s;
    if (wrap && sl < 0) sl += smax + 1;
    const uint64_t off = (uint64_t)(uint32_t)min(max(sl, 0), smax) * slot_bytes;
    if (p == 0)
      dma16(k + off, lds_addr(dst));
    else
      dma16(v + off, lds_addr(dst + kF8Half));
  }
};

// Widens the e4m3 K and V bytes this lane staged (key `key`, dims 16c .. 16c +
// 15) into the bf16 stages, in the layouts the MFMA operand reads expect (see
// Stager::issue): exact, every e4m3 value is a bf16 value.  Each lane reads only
// the bytes its own load wrote, so s_waitcnt vmcnt orders it; no barrier.
__device__ __forceinline__ void widen_tile(const uint8_t* f8, uint8_t* kdst, uint8_t* vdst,
                                           int key, int c) {
  const uint8_t* src = f8 + key * kD + 16 * c;
  uint8_t* krow = kdst + (key >> 1) * kKPair + (key & 1) * kRowBytes;
  uint8_t* vrow = vdst + key * kRowBytes;
  const int ks = key & 1, vs = vswz(key);
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const u32x2 kx = *reinterpret_cast<const u32x2*>(src + 8 * h);
    const u32x2 vx = *reinterpret_cast<const u32x2*>(src + kF8Half + 8 * h);
    st_s16(krow + 16 * ((2 * c + h) ^ ks), e4m3x8_to_bf16x8(kx[0], kx[1]));
    st_s16(vrow + 16 * ((2 * c + h) ^ vs), e4m3x8_to_bf16x8(vx[0], vx[1]));
  }
}

// ---------------------------------------------------------------- MFMAs
// Register file: at two waves per SIMD each wave has 256 registers; O^T
// (8 tiles x 16 fp32), Q^T (64) and S^T (16) all live in VGPRs.  This file is
// compiled with -mllvm --amdgpu-mfma-vgpr-form=1, which makes the builtin
// MFMAs read and write their accumulators in VGPRs, so no AGPR copies are
// needed and the compiler sees, and spaces, every MFMA dependency itself.
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

// ---------------------------------------------------------------- phases
// Each MFMA phase is one stream of 16 MFMAs with the other work placed one
// item per MFMA (sched_barrier regions, MFMA first in each region): the
// fragment reads kQkAhead / kPvAhead MFMAs ahead and, when the phase carries
// the step's staging, the slot-id reads at MFMA 0 and the two K / V row pairs
// at MFMAs 2 and 3.
template <bool kStage, class S>
__device__ __forceinline__ void qk_phase(const uint8_t* kst, int kaddr, const u32x4 (&qf)[16],
                                         f32x16& s, const S& st) {
  u32x4 fr[kQkAhead + 1];
  __builtin_amdgcn_s_setprio(1);
#pragma unroll
  for (int i = 0; i < kQkAhead; ++i) fr[i] = ld_s16(kst + kaddr + 32 * i);
  typename S::Ids ids;
#pragma unroll
  for (int kk = 0; kk < 16; ++kk) {
    __builtin_amdgcn_sched_barrier(0);
    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
    __builtin_amdgcn_sched_group_barrier(0x7f7, 64, 0);
    if (kk + kQkAhead < 16)
      fr[(kk + kQkAhead) % (kQkAhead + 1)] = ld_s16(kst + kaddr + 32 * (kk + kQkAhead));
    s = mfma_32x32x16(fr[kk % (kQkAhead + 1)], qf[kk], kk == 0 ? f32x16{} : s);
    if (kStage) {
      if (kk == 0)
        ids = st.fetch();
      else if (kk == 2 || kk == 3)
        st.issue_part(ids, kk - 2);
    }
  }
  __builtin_amdgcn_sched_barrier(0);
}

template <bool kStage, class S>
__device__ __forceinline__ void pv_phase(const uint8_t* vst, const int (&vaddr)[4],
                                         f32x16 (&acc)[8], const u32x4 (&pt)[2],
                                         const S& st) {
  u32x4 fr[kPvAhead + 1];
  __builtin_amdgcn_s_setprio(0);
#pragma unroll
  for (int f = 0; f < kPvAhead; ++f) fr[f] = v_frag(vst, vaddr, f);
  typename S::Ids ids;
#pragma unroll
  for (int f = 0; f < 16; ++f) {
    __builtin_amdgcn_sched_barrier(0);
    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
    __builtin_amdgcn_sched_group_barrier(0x7f7, 64, 0);
    if (f + kPvAhead < 16) fr[(f + kPvAhead) % (kPvAhead + 1)] = v_frag(vst, vaddr, f + kPvAhead);
    acc[f & 7] = mfma_32x32x16(fr[f % (kPvAhead + 1)], pt[f >> 3], acc[f & 7]);
    if (kStage) {
      if (f == 0)
        ids = st.fetch();
      else if (f == 2 || f == 3)
        st.issue_part(ids, f - 2);
    }
  }
  __builtin_amdgcn_sched_barrier(0);
}

// ---------------------------------------------------------------- softmax
// Softmax state of the lane's row: reference max m (raw score units),
// moff = m * sl2, running sum l of p = 2^(s sl2 - moff) (this lane's half).
struct Row {
  float m, moff, l;
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

// Row max of the tile, the lazy reference-max update, and P^T packed to bf16:
// pt[q4] holds p for keys 16 q4 + 8 (j / 4) + 4 g + j % 4, two per dword, the
// B operand of PV step q4.  Returns whether any row of the wave raised its
// reference max (alpha is then the lane's factor for the accumulators).
__device__ __forceinline__ bool softmax_tile(const f32x16& s, Row& row, float sl2,
                                             u32x4 (&pt)[2], float& alpha) {
  float mx = s[0];
#pragma unroll
  for (int r = 1; r < 16; ++r) mx = fmaxf(mx, s[r]);
  mx = half_swap_max(mx);
  // Lazy reference max, per row: raised only when the row outgrew it by more
  // than 2^kRescaleLog2.  The wave-wide vote only decides whether the rescale
  // runs at all.
  const bool grow = (mx - row.m) * sl2 > kRescaleLog2;
  const float mnew = grow ? mx : row.m;
  alpha = grow ? fast_exp2((row.m - mnew) * sl2) : 1.f;
  row.l *= alpha;
  row.m = mnew;
  row.moff = mnew * sl2;
#pragma unroll
  for (int q4 = 0; q4 < 2; ++q4) {
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const float p0 = fast_exp2(fmaf(s[8 * q4 + 2 * k], sl2, -row.moff));
      const float p1 = fast_exp2(fmaf(s[8 * q4 + 2 * k + 1], sl2, -row.moff));
      pt[q4][k] = pack_bf16(p0, p1);
      row.l += p0 + p1;
    }
  }
  return __ballot(grow) != 0;
}

template <bool FP8>
__global__ void __launch_bounds__(kThreads) extend_mfma_kernel(ExtendArgs a) {
  __shared__ Smem<FP8> sm;
  constexpr int kKS = kStagesOf<FP8>, kVS = kVStagesOf<FP8>;

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

  // This lane's row; padding lanes compute a valid duplicate row and never
  // write it.
  const int rho_c = min(row0 + kRowsPerWave * w + n, rows_total - 1);
  const int limit = P + rho_c / G;   // last visible key

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

  // fp8 pools: scores and outputs are computed from the e4m3 values and
  // scaled by k_scale / v_scale (folded into the exponent scale and 1 / l).
  const float sl2 = FP8 ? a.scale_log2 * a.k_scale[0] : a.scale_log2;
  typename std::conditional<FP8, Stager8, Stager>::type st;
  if constexpr (FP8) {
    st.k = a.k_pool + (int64_t)hk * kD + 16 * (lane & 15);
    st.v = a.v_pool + (int64_t)hk * kD + 16 * (lane & 15);
    st.slot_bytes = (uint32_t)a.hkv * kD;
    st.key = 4 * w + (lane >> 4);
  } else {
    st.sb = stage_bases(a.k_pool + (int64_t)hk * kRowBytes,
                        a.v_pool + (int64_t)hk * kRowBytes, lane);
    st.slot_bytes = (uint32_t)a.hkv * kRowBytes;
    st.w = w;
    st.g = g;
  }
  st.slots = sm.slots;
  st.smax = (int32_t)min(a.pool_slots - 1, (int64_t)INT32_MAX);
  st.wrap = a.seq_override > 0;
  auto stage_at = [&](int tile, int j) {   // tile `tile` into the stages of step j
    st.tile = tile;
    if constexpr (FP8) {
      st.dst = sm.f8 + (j & 1) * kF8Stage + 4 * w * kD;
    } else {
      st.k_dst = sm.k + (j % kKS) * kKStage;
      st.v_dst = sm.v + (j % kVS) * kVStage;
    }
  };
  auto stage_for = [&](int j) { stage_at(min(j + kAhead, last), j + kAhead); };
  // fp8: tile t's e4m3 rows (issued one step earlier) widened into the bf16
  // stages; only this lane's own loads need to have landed (after the step's
  // own loads when it staged one, `all` when it staged nothing).
  auto widen = [&](int t, auto all) {
    if constexpr (FP8) {
      if (t <= last) {
        if constexpr (decltype(all)::value)
          asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        else
          vm_wait_staged<true>();
        widen_tile(sm.f8 + (t & 1) * kF8Stage, sm.k + (t % kKS) * kKStage,
                   sm.v + (t % kVS) * kVStage, 4 * w + (lane >> 4), lane & 15);
      }
    }
  };
  using Staged = std::true_type;
  using Unstaged = std::false_type;

  // LDS read offsets of this lane (see Stager::issue / v_frag).
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

  // Q: the wave's 32 rows (padding rows repeat the last real row) are loaded
  // row-contiguously, lane L taking 16-byte chunk L % 32 of row 2 i + L / 32,
  // together with the slot ids of the first 1024 keys.
  uint8_t* const my_rows = sm.rows[w];
  {
    u32x4 qv[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int r = 2 * i + g;
      const int rho = min(row0 + kRowsPerWave * w + r, rows_total - 1);
      const int t = rho / G, h = rho - t * G;
      qv[i] = ld_g16(a.q + (int64_t)(q_start + t) * a.q_stride + (int64_t)(hk * G + h) * kD + 8 * n);
    }
    slot_issue(rtt, 0, kend, w, lane, sm.slots);
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int r = 2 * i + g;
      st_s16(my_rows + r * kRowBytes + 16 * swz_chunk(r, n), qv[i]);
    }
  }
  // Q^T fragments: lane (g, n) holds q[row n][16 kk + 8 g .. +8].
  u32x4 qf[16];
#pragma unroll
  for (int kk = 0; kk < 16; ++kk)
    qf[kk] = ld_s16(my_rows + n * kRowBytes + 16 * swz_chunk(n, 2 * kk + g));
  // Consume Q here so that the compiler waits for these reads before the
  // loop; inside it, vmcnt belongs to the staging loads.
#pragma unroll
  for (int kk = 0; kk < 16; ++kk) asm volatile("" ::"v"(qf[kk]));

  Row row{-INFINITY, 0.f, 0.f};
  f32x16 acc[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) acc[i] = f32x16{};

  // ---- prologue: the slot ids (issued with Q) land, every wave has its Q
  // out of the shared rows, then tiles 0 and 1 go into stages 0 and 1. Tiles
  // past the last one are stand-ins for the last tile (its slots are staged,
  // so every load stays inside the pool) and are never read.
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __syncthreads();
#pragma unroll
  for (int tl = 0; tl < kAhead; ++tl) {
    stage_at(min(tl, last), tl);
    const auto ids = st.fetch();
#pragma unroll
    for (int p = 0; p < 2; ++p) st.issue_part(ids, p);
  }
  widen(0, Unstaged{});
  vm_wait_staged<FP8>();
  __syncthreads();

  // bf16: K tile t lives in K stage t % 3, V tile t in V stage t % 4.
  // Between barriers j - 1 and j every wave stages tile j + 2; lead waves read
  // K(j) and V(j), trailing waves V(j - 1) and K(j).  The stages tile j + 2
  // overwrites held tiles j - 1 (K) and j - 2 (V), whose last reads came
  // before barrier j - 1.
  // fp8: e4m3 tile t lives in e4m3 stage t % 2, its widened rows in K stage
  // t % 2 and V stage t % 3.  Between barriers j - 1 and j every wave stages
  // tile j + 2 (over tile j, widened before barrier j - 1) and widens tile
  // j + 1 (over K(j - 1) and V(j - 2), last read before barrier j - 1).
  f32x16 s;
  u32x4 pt[2];
  float alpha;
  auto slot_chunk = [&](int j) {
    // Slot ids of the next 1024 keys: issued at tile 4 of chunk c into the
    // half that served chunk c - 1 (last read when tile 32 c - 1 was staged,
    // before barrier 32 c - 3), first read when tile 32 (c + 1) is staged.
    if (j % kTilesPerSlotChunk == 4 && (j / kTilesPerSlotChunk + 1) * kSlotChunk < kend)
      slot_issue(rtt, j / kTilesPerSlotChunk + 1, kend, w, lane, sm.slots);
  };
  // Softmax of tile j; `grew` records whether a row's reference max was
  // raised, and rescale() then scales O^T, which must hold exactly the tiles
  // before j (it runs right before PV(j)).
  bool grew = false;
  auto softmax_step = [&](int j) {
    const int k0 = j * kBN;
    if (k0 + kBN > w_full) mask_tile(s, k0, g, limit);
    grew = softmax_tile(s, row, sl2, pt, alpha) && j > 0;
  };
  auto rescale = [&]() {
    if (grew) {
#pragma unroll
      for (int i = 0; i < 8; ++i) acc[i] *= alpha;
    }
  };
  auto step_end = [&](auto staged) {
    // Tile j + 1 was issued one step earlier: only this step's tile loads
    // may still be in flight (none after a step that staged nothing).
    if constexpr (decltype(staged)::value)
      vm_wait_staged<FP8>();
    else
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
  };
  // bf16 pools: steps j < n_stage stage tile j + 2, which exists; the last two
  // steps stage nothing (no stand-in loads for the epilogue to wait for), so
  // their waits cover every outstanding load.  No slot-id chunk is due in
  // them.  fp8 pools stage in every step (stand-in tiles past the last): the
  // separate tail steps cost that variant a register spill.
  constexpr bool kTail = !FP8;
  const int n_stage = kTail ? max(n_tiles - kAhead, 0) : n_tiles;

  if (w < kLeadWaves) {
    auto lead_step = [&](int j, auto staged) {
      constexpr bool kS = decltype(staged)::value;
      if constexpr (kS) {
        slot_chunk(j);
        stage_for(j);
      }
      qk_phase<kS>(sm.k + (j % kKS) * kKStage, kaddr, qf, s, st);
      softmax_step(j);
      widen(j + 1, std::integral_constant<bool, !kS>{});
      rescale();
      pv_phase<false>(sm.v + (j % kVS) * kVStage, vaddr, acc, pt, st);
      step_end(staged);
    };
    int j = 0;
    for (; j < n_stage; ++j) lead_step(j, Staged{});
    if constexpr (kTail)
      for (; j < n_tiles; ++j) lead_step(j, Unstaged{});
  } else {
    auto trail_step = [&](int j, auto staged) {   // j >= 1
      constexpr bool kS = decltype(staged)::value;
      if constexpr (kS) {
        slot_chunk(j);
        stage_for(j);
      }
      rescale();
      pv_phase<kS>(sm.v + ((j - 1) % kVS) * kVStage, vaddr, acc, pt, st);
      qk_phase<false>(sm.k + (j % kKS) * kKStage, kaddr, qf, s, st);
      widen(j + 1, std::integral_constant<bool, !kS>{});
      softmax_step(j);
      step_end(staged);
    };
    if (!kTail || n_stage > 0) {
      stage_for(0);
      qk_phase<true>(sm.k, kaddr, qf, s, st);
      widen(1, Unstaged{});
      softmax_step(0);
      step_end(Staged{});
    } else if constexpr (kTail) {
      qk_phase<false>(sm.k, kaddr, qf, s, st);
      widen(1, Staged{});
      softmax_step(0);
      step_end(Unstaged{});
    }
    int j = 1;
    for (; j < n_stage; ++j) trail_step(j, Staged{});
    if constexpr (kTail)
      for (; j < n_tiles; ++j) trail_step(j, Unstaged{});
    rescale();
    pv_phase<false>(sm.v + (last % kVS) * kVStage, vaddr, acc, pt, st);
  }
  // Every wave must be done with the stages before the stage memory holds
  // the output rows (the prologue's stand-in tile of a one-tile item has
  // landed by the last step's wait).
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __syncthreads();

  // Output: O^T / l into the wave's rows in LDS (lane (g, n) holds dims
  // 32 mt + 8 rq + 4 g .. +3 of row n), then row-contiguous 16-byte stores
  // (with the output gate), lane L writing chunk L % 32 of row 2 i + L / 32.
  const float inv = (FP8 ? a.v_scale[0] : 1.f) / (row.l + __shfl_xor(row.l, 32, kWave));
  const int ln = opaque(lane);   // lane coordinates recomputed here, see opaque()
  const int ne = ln & 31, ge = ln >> 5;
#pragma unroll
  for (int mt = 0; mt < 8; ++mt) {
#pragma unroll
    for (int rq = 0; rq < 4; ++rq) {
      const u32x2 v = {pack_bf16(acc[mt][4 * rq + 0] * inv, acc[mt][4 * rq + 1] * inv),
                       pack_bf16(acc[mt][4 * rq + 2] * inv, acc[mt][4 * rq + 3] * inv)};
      st_s8(my_rows + ne * kRowBytes + 16 * swz_chunk(ne, 4 * mt + rq) + 8 * ge, v);
    }
  }
  const int rho0 = row0 + kRowsPerWave * w + ge;
  uint32_t omax = 0;
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const int r = 2 * i + ge;
    const int rho = rho0 + 2 * i;
    if (rho < rows_total) {
      u32x4 v = ld_s16(my_rows + r * kRowBytes + 16 * swz_chunk(r, ne));
      const int t = rho / G, h = rho - t * G;
      if (a.gate) {
        const u32x4 gv = ld_g16(a.gate + (int64_t)(q_start + t) * a.gate_stride +
                                (int64_t)(hk * G + h) * a.gate_hstride + 8 * ne);
#pragma unroll
        for (int k = 0; k < 4; ++k) v[k] = gate_pair(v[k], gv[k]);
      }
      omax = max(omax, abs_max8(v));
      *reinterpret_cast<u32x4*>(a.out + (int64_t)(q_start + t) * a.out_stride +
                                (int64_t)(hk * G + h) * kD + 8 * ne) = v;
    }
  }
  amax_commit(a.amax, omax);
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
                                  uint32_t* out_amax, tf_stream_t stream) {
  using namespace tfa;
  clear_error();
  if (n_work < 0) return fail(TF_ERR_INVALID, "extend: n_work=%d", n_work);
  if (num_kv_heads <= 0 || num_q_heads <= 0 || num_q_heads % num_kv_heads)
    return fail(TF_ERR_INVALID, "extend: num_q_heads=%d not a multiple of num_kv_heads=%d",
                num_q_heads, num_kv_heads);
  const bool generic = head_dim != kD;
  if (generic && !generic_head_dim(head_dim))
    return fail(TF_ERR_UNSUPPORTED, "extend: head_dim=%d (a multiple of 8 between 8 and %d)",
                head_dim, kD);
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
  a.amax = out_amax;

  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  if (generic) {   // head_dim != 256: one wave per row of every work entry
    GenericAttnArgs g{};
    g.q = a.q;
    g.q_stride = a.q_stride;
    g.k_pool = a.k_pool;
    g.v_pool = a.v_pool;
    g.pool_slots = a.pool_slots;
    g.fp8 = kv_dtype == TF_DTYPE_FP8_E4M3;
    g.k_scale = a.k_scale;
    g.v_scale = a.v_scale;
    g.rtt = a.rtt;
    g.rtt_rows = a.rtt_rows;
    g.rtt_stride = a.rtt_stride;
    g.rtt_cols = a.rtt_cols;
    g.rpi = a.rpi;
    g.seq_lens = a.seq_lens;
    g.seq_override = a.seq_override;
    g.work = work;
    g.n_rows = n_work;
    g.hq = num_q_heads;
    g.hkv = num_kv_heads;
    g.head_dim = head_dim;
    g.scale_log2 = a.scale_log2;
    g.out = a.out;
    g.out_stride = a.out_stride;
    g.gate = a.gate;
    g.gate_stride = a.gate_stride;
    g.gate_hstride = a.gate_hstride;
    g.amax = out_amax;
    return launch_generic_attn(g, s);
  }
  if (kv_dtype == TF_DTYPE_FP8_E4M3)
    hipLaunchKernelGGL(extend_mfma_kernel<true>, dim3((unsigned)n_work), dim3(kThreads), 0, s, a);
  else
    hipLaunchKernelGGL(extend_mfma_kernel<false>, dim3((unsigned)n_work), dim3(kThreads), 0, s, a);
  return launch_status("tf_attn_extend launch");
}

