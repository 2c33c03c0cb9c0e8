// Decode attention over the req_to_token -> KV-pool slot indirection.
//
// Replaces the reference's pure-decode branch (qwen3_8/full_attention.py:215-242):
// gather of req_to_token[r, :L] rows, GQA repeat_interleave, length mask and
// SDPA, here fused into one HBM-streaming pass with no padded or expanded copy.
//
// Work decomposition (persistent, balanced)
//   unit = (request item, kv head, group of <= 16 q heads sharing that kv head);
//   a unit's context is cut into 16-token tiles, and the tiles of all units,
//   laid out unit after unit, form one global range of N tiles. The grid has
//   P = one workgroup per CU (all resident at once); workgroup b owns global
//   tiles [floor(b N / P), floor((b+1) N / P)), so every CU gets the same work
//   whatever the length mix. A workgroup walks its range as segments (one unit
//   each); 4 waves take interleaved tiles of a segment. A unit owned entirely by
//   one workgroup is written as final bf16 output; otherwise each owner stores
//   an fp32 partial (O, max, sum) at index b + u (unique, < P + units) and a
//   second small kernel merges them.
//   The whole GQA head group of a kv head shares every K/V row read from HBM.
// Per segment: the slot ids of up to 2048 tokens at a time (int64 req_to_token
// entries clamped to the pool) are staged in LDS with coalesced loads, and the
// group's Q^T MFMA fragments once.
// Per 16-token tile a wave
//   * loads K and V rows with the same row-contiguous pattern (lane (g, n) reads
//     16-byte chunk n (+16) of the rows of tokens 4g + j) using nontemporal
//     loads; the next tile's K is issued as soon as this tile's K is staged and
//     its V as soon as PV has consumed this tile's V, so a tile's worth of loads
//     is always in flight per wave,
//   * stages K through a per-wave, XOR-swizzled LDS tile into the MFMA
//     A-operand layout (row = lane % 16), conflict-free both ways,
//   * S^T[token, head] = K * Q^T with v_mfma_f32_16x16x32_bf16 (heads padded to 16),
//   * online softmax per head (lane-local scores, two xor-shuffles for the max),
//   * O^T[dim, head] += V^T * P^T with v_mfma_f32_16x16x16_bf16, V^T built in
//     registers with v_perm_b32 (fp8: byte permutes + v_cvt_scalef32_pk_bf16_fp8).
//   Every per-head quantity (max, sum, rescale factor, 64 output dims) is then
//   lane-local: lane (g, n) owns head n, dims {128s + 32g + 8r + e} (bf16) or
//   {64g + 16r + e} (fp8).
// The merge lives in its own launch so the streaming kernel needs no
// device-scope fence (on gfx950 those write back and invalidate the XCD's L2).
#include <math.h>

#include <mutex>

#include "tf_common.h"
#include "tf_internal.h"

namespace tfa {
namespace {

constexpr int kD = 256;         // head_dim (Qwen3.8: 256)
constexpr int kWaves = 4;
constexpr int kTile = 16;       // tokens per wave iteration
constexpr int kAcc = 16;        // f32x4 accumulators per lane (64 output dims)
constexpr int kMaxChunk = 2048; // slot ids staged in LDS at a time
constexpr int kMaxItems = 2048; // requests per call (per-item prefix lives in LDS)

struct DecodeArgs {
  const __bf16* q;
  int64_t q_stride;
  const uint8_t* k_pool;
  const uint8_t* v_pool;
  int64_t pool_slots;
  const float* k_scale;
  const float* v_scale;
  const int64_t* rtt;
  int64_t rtt_rows, rtt_stride, rtt_cols;
  const int64_t* rpi;
  const int64_t* seq_lens;
  int32_t seq_override;
  const int32_t* items;
  const int32_t* q_rows;
  int32_t n_items;
  int32_t hkv, group, n_hg;
  float scale_log2;
  __bf16* out;
  int64_t out_stride;
  const __bf16* gate;   // optional output gate (NULL: none)
  int64_t gate_stride, gate_hstride;
  uint32_t* amax;       // optional: raised to max |out| (bf16 bits), amax_commit
  float* ws_ml;
  float* ws_o;
  int32_t n_blocks;   // P: workgroups of the streaming kernel
};

struct WaveState {
  float m, l;
  f32x4 acc[kAcc];
};

// LDS slot for one wave's state, element-major so lanes hit consecutive banks.
struct StateSlot {
  f32x4 acc[kAcc][kWave];
  float m[kWave];
  float l[kWave];
};

// Per-wave K staging tile: 16 token rows x 32 (bf16) or 16 (fp8) 16-byte
// chunks; chunk c of row r sits at r * chunks + (c ^ r) so that both the
// coalesced writes and the MFMA-layout reads are free of bank conflicts.
constexpr int kKStageChunks = 16 * 32;

struct DecodeSmem {
  union {
    struct {
      int32_t slots[kMaxChunk];                 // slot id of each staged token
      u32x4 kstage[kWaves][kKStageChunks];      // per-wave K tile
    } loop;
    StateSlot merge[2];                         // wave-state exchange
  } u;
  u32x4 qfrag[8][kWave];                        // Q^T B-operand fragments, lane-major
  int32_t ipre[kMaxItems + 1];                  // exclusive prefix of per-item tiles
  int32_t wsum[kWaves];
};

// Per-lane register slices of one 16-token tile: K (staged to LDS for the
// S^T = K Q^T MFMA) and V (transposed in registers for the PV MFMA).
template <bool FP8>
struct KBuf {
  u32x4 k[FP8 ? 4 : 8];   // [j * (FP8 ? 1 : 2) + s]: row of token 4g + j, chunk n + 16s
};
template <bool FP8>
struct VBuf {
  u32x4 v[4][FP8 ? 1 : 2];
};

__device__ __forceinline__ void merge_into(WaveState& st, float m2, float l2, const f32x4* acc2) {
  const float M = fmaxf(st.m, m2);
  const float a1 = (st.m == -INFINITY) ? 0.f : fast_exp2(st.m - M);
  const float a2 = (m2 == -INFINITY) ? 0.f : fast_exp2(m2 - M);
  st.l = st.l * a1 + l2 * a2;
#pragma unroll
  for (int i = 0; i < kAcc; ++i) st.acc[i] = st.acc[i] * a1 + acc2[i] * a2;
  st.m = M;
}

__device__ __forceinline__ void reset_state(WaveState& st) {
  st.m = -INFINITY;
  st.l = 0.f;
#pragma unroll
  for (int i = 0; i < kAcc; ++i) st.acc[i] = f32x4{0.f, 0.f, 0.f, 0.f};
}

__device__ __forceinline__ void put_state(StateSlot* s, int lane, const WaveState& st) {
#pragma unroll
  for (int i = 0; i < kAcc; ++i) s->acc[i][lane] = st.acc[i];
  s->m[lane] = st.m;
  s->l[lane] = st.l;
}

__device__ __forceinline__ void take_state(const StateSlot* s, int lane, WaveState& st) {
  f32x4 acc2[kAcc];
#pragma unroll
  for (int i = 0; i < kAcc; ++i) acc2[i] = s->acc[i][lane];
  merge_into(st, s->m[lane], s->l[lane], acc2);
}

// Tree merge of the 4 wave states; wave 0 ends up holding the block state.
__device__ __forceinline__ void block_merge(StateSlot* slots, int w, int lane, WaveState& st) {
  __syncthreads();
  if (w >= 2) put_state(&slots[w - 2], lane, st);
  __syncthreads();
  if (w < 2) take_state(&slots[w], lane, st);
  __syncthreads();
  if (w == 1) put_state(&slots[0], lane, st);
  __syncthreads();
  if (w == 0) take_state(&slots[0], lane, st);
}

// Returns the largest |value| written (bf16 bits) for amax_commit.
template <bool FP8>
__device__ __forceinline__ uint32_t write_output(const DecodeArgs& a, int qrow, int hq, int g,
                                                 const WaveState& st, float vscale) {
  const float inv = vscale / st.l;
  uint32_t m = 0;
  __bf16* o = a.out + (int64_t)qrow * a.out_stride + (int64_t)hq * kD;
  const __bf16* gt =
      a.gate ? a.gate + (int64_t)qrow * a.gate_stride + (int64_t)hq * a.gate_hstride : nullptr;
  // 8 outputs (dims off .. off + 7) per store; gated when the caller passed one.
  auto store8 = [&](int off, u32x4 v) {
    if (gt) {
      const u32x4 gv = ld_g16(gt + off);
#pragma unroll
      for (int k = 0; k < 4; ++k) v[k] = gate_pair(v[k], gv[k]);
    }
    m = max(m, abs_max8(v));
    *reinterpret_cast<u32x4*>(o + off) = v;
  };
  if (FP8) {
#pragma unroll
    for (int r = 0; r < 4; ++r) {
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        u32x4 v;
#pragma unroll
        for (int k = 0; k < 4; ++k)
          v[k] = pack_bf16(st.acc[8 * h + 2 * k][r] * inv, st.acc[8 * h + 2 * k + 1][r] * inv);
        store8(64 * g + 16 * r + 8 * h, v);
      }
    }
  } else {
#pragma unroll
    for (int s = 0; s < 2; ++s) {
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        u32x4 v;
#pragma unroll
        for (int k = 0; k < 4; ++k)
          v[k] = pack_bf16(st.acc[8 * s + 2 * k][r] * inv, st.acc[8 * s + 2 * k + 1][r] * inv);
        store8(128 * s + 32 * g + 8 * r, v);
      }
    }
  }
  return m;
}

// Issue the loads of tile `it` (chunk tokens it*16 .. it*16+15, clamped to the
// chunk's last token so every address is a valid row). K/V rows are streamed
// once, so the loads are nontemporal.
template <bool FP8>
__device__ __forceinline__ void issue_k(KBuf<FP8>& kb, const int32_t* slots, int it, int n_loc,
                                        int g, int n, const uint8_t* kbase,
                                        int64_t slot_bytes) {
  // Same row-contiguous pattern as V: lane (g, n) reads 16-byte chunk n (+16s)
  // of the rows of tokens 4g + j; the MFMA layout is produced through LDS.
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int64_t ks = slots[min(it * kTile + 4 * g + j, n_loc - 1)];
    const uint8_t* kp = kbase + ks * slot_bytes;
#pragma unroll
    for (int s = 0; s < (FP8 ? 1 : 2); ++s) kb.k[j * (FP8 ? 1 : 2) + s] = ld_nt16(kp + 16 * n + 256 * s);
  }
}

// Writes the tile's K chunks to this wave's LDS staging tile (swizzled).
template <bool FP8>
__device__ __forceinline__ void stage_k(const KBuf<FP8>& kb, u32x4* ks, int g, int n) {
  constexpr int kChunks = FP8 ? 16 : 32;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int r = 4 * g + j;
#pragma unroll
    for (int s = 0; s < (FP8 ? 1 : 2); ++s) {
      const int c = n + 16 * s;
      ks[r * kChunks + (c ^ r)] = kb.k[j * (FP8 ? 1 : 2) + s];
    }
  }
}

template <bool FP8>
__device__ __forceinline__ void issue_v(VBuf<FP8>& vb, const int32_t* slots, int it, int n_loc,
                                        int g, int n, const uint8_t* vbase,
                                        int64_t slot_bytes) {
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int64_t vs = slots[min(it * kTile + 4 * g + j, n_loc - 1)];
    const uint8_t* vp = vbase + vs * slot_bytes;
#pragma unroll
    for (int s = 0; s < (FP8 ? 1 : 2); ++s) vb.v[j][s] = ld_nt16(vp + 16 * n + 256 * s);
  }
}

// S^T = K Q^T for the tile, then the online-softmax update of head n; returns
// the tile's probabilities packed as the PV B operand (P^T, 4 tokens per lane).
template <bool FP8>
__device__ __forceinline__ u32x2 qk_softmax(const u32x4* ks, const u32x4 (&qf)[8], int it,
                                            int n_loc, int g, int n, float sl2, WaveState& st) {
  // K fragment of k-step kk for lane (g, n): row n, dims 32kk + 8g .. (bf16:
  // chunk 4kk + g) or, for fp8, dims 64u + 16g .. (chunk 4u + g, two k-steps).
  f32x4 sacc = {0.f, 0.f, 0.f, 0.f};
  if (FP8) {
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const u32x4 kf = ks[n * 16 + ((4 * u + g) ^ n)];
      sacc = mfma_16x16x32(e4m3x8_to_bf16x8(kf[0], kf[1]), qf[2 * u], sacc);
      sacc = mfma_16x16x32(e4m3x8_to_bf16x8(kf[2], kf[3]), qf[2 * u + 1], sacc);
    }
  } else {
#pragma unroll
    for (int kk = 0; kk < 8; ++kk)
      sacc = mfma_16x16x32(ks[n * 32 + ((4 * kk + g) ^ n)], qf[kk], sacc);
  }
  float sc[4];
  float mx = -INFINITY;
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const int t = it * kTile + 4 * g + r;
    sc[r] = (t < n_loc) ? sacc[r] * sl2 : -INFINITY;
    mx = fmaxf(mx, sc[r]);
  }
  mx = wave_max_xor(mx, 16);
  mx = wave_max_xor(mx, 32);
  const float mnew = fmaxf(st.m, mx);
  const float alpha = fast_exp2(st.m - mnew);
  float p[4];
  float psum = 0.f;
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    p[r] = fast_exp2(sc[r] - mnew);
    psum += p[r];
  }
  st.l = st.l * alpha + psum;
  st.m = mnew;
  if (__ballot(alpha != 1.f)) {
#pragma unroll
    for (int i = 0; i < kAcc; ++i) st.acc[i] *= alpha;
  }
  return u32x2{pack_bf16(p[0], p[1]), pack_bf16(p[2], p[3])};
}

// O^T += V^T P^T for the tile.
template <bool FP8>
__device__ __forceinline__ void pv(const VBuf<FP8>& vb, u32x2 pt, WaveState& st) {
  if (FP8) {
#pragma unroll
    for (int e = 0; e < 16; e += 2) {
      const int dw = e >> 2;
      const uint32_t b0 = e & 3;
      const uint32_t sel = b0 | ((4 + b0) << 8) | ((b0 + 1) << 16) | ((5 + b0) << 24);
      const uint32_t x = __builtin_amdgcn_perm(vb.v[1][0][dw], vb.v[0][0][dw], sel);
      const uint32_t y = __builtin_amdgcn_perm(vb.v[3][0][dw], vb.v[2][0][dw], sel);
      const u32x2 va = {e4m3x2_to_bf16x2<false>(x), e4m3x2_to_bf16x2<false>(y)};
      const u32x2 vbb = {e4m3x2_to_bf16x2<true>(x), e4m3x2_to_bf16x2<true>(y)};
      st.acc[e] = mfma_16x16x16(va, pt, st.acc[e]);
      st.acc[e + 1] = mfma_16x16x16(vbb, pt, st.acc[e + 1]);
    }
  } else {
#pragma unroll
    for (int s = 0; s < 2; ++s) {
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const int dw = e >> 1;
        const int hi = e & 1;
        const u32x2 va = {pair_sel(vb.v[1][s][dw], vb.v[0][s][dw], hi),
                          pair_sel(vb.v[3][s][dw], vb.v[2][s][dw], hi)};
        st.acc[8 * s + e] = mfma_16x16x16(va, pt, st.acc[8 * s + e]);
      }
    }
  }
}


// Context length of item i (the request's seq_len, or the bsz == 1 override),
// clamped to the req_to_token row.  A negative batch index marks a padding
// entry of a device-built item list: no work and no output.
__device__ __forceinline__ bool item_is_padding(const DecodeArgs& a, int i) {
  return a.items && a.items[i] < 0;
}

__device__ __forceinline__ int item_len(const DecodeArgs& a, int i) {
  if (item_is_padding(a, i)) return 0;
  const int b = a.items ? a.items[i] : i;
  int64_t len = a.seq_override > 0 ? (int64_t)a.seq_override : a.seq_lens[b];
  if (len > a.rtt_cols) len = a.rtt_cols;
  return len > 0 ? (int)len : 0;
}

__device__ __forceinline__ int item_tiles(const DecodeArgs& a, int i) {
  return (item_len(a, i) + kTile - 1) / kTile;
}

// ipre[i] = sum of tiles of items < i, ipre[n_items] = total (block-wide scan).
__device__ void item_prefix(const DecodeArgs& a, int32_t* ipre, int32_t* wsum) {
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int w = wave_id();
  constexpr int kPer = kMaxItems / (kWaves * kWave);
  int t[kPer];
  int sum = 0;
#pragma unroll
  for (int k = 0; k < kPer; ++k) {
    const int i = tid * kPer + k;
    t[k] = i < a.n_items ? item_tiles(a, i) : 0;
    sum += t[k];
  }
  int incl = sum;
#pragma unroll
  for (int off = 1; off < kWave; off <<= 1) {
    const int v = __shfl_up(incl, off, kWave);
    if (lane >= off) incl += v;
  }
  if (lane == kWave - 1) wsum[w] = incl;
  __syncthreads();
  int excl = incl - sum;
  for (int k = 0; k < w; ++k) excl += wsum[k];
#pragma unroll
  for (int k = 0; k < kPer; ++k) {
    const int i = tid * kPer + k;
    if (i <= a.n_items) ipre[i] = excl;
    excl += t[k];
  }
  if (tid == kWaves * kWave - 1 && a.n_items == kMaxItems) ipre[kMaxItems] = excl;
  __syncthreads();
}

// Workgroup that owns global tile x when N tiles are split over P workgroups.
__device__ __forceinline__ int owner_of(int64_t x, int64_t N, int P) {
  return (int)(((x + 1) * P - 1) / N);
}

template <bool FP8>
__global__ void __launch_bounds__(kWaves * kWave, 2)
decode_kernel(DecodeArgs a) {
  constexpr int kRowBytes = FP8 ? kD : 2 * kD;
  __shared__ DecodeSmem sm;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int w = wave_id();
  const int g = lane >> 4;
  const int n = lane & 15;

  item_prefix(a, sm.ipre, sm.wsum);
  const int units_per_item = a.hkv * a.n_hg;
  const int64_t N = (int64_t)units_per_item * sm.ipre[a.n_items];
  // With P <= N every workgroup's range is non-empty, so the owners of a unit
  // are consecutive workgroups (the merge kernel relies on it).
  const int P = (int)min<int64_t>(a.n_blocks, N);
  if ((int)blockIdx.x >= P) return;
  const int64_t x_end = (int64_t)(blockIdx.x + 1) * N / P;
  int64_t x = (int64_t)blockIdx.x * N / P;

  const float kscale = FP8 ? a.k_scale[0] : 1.f;
  const float vscale = FP8 ? a.v_scale[0] : 1.f;
  const float sl2 = a.scale_log2 * kscale;
  const int64_t slot_bytes = (int64_t)a.hkv * kRowBytes;

  // First item whose tile range contains x (binary search over ipre).
  int item = 0;
  {
    int lo = 0, hi = a.n_items - 1;
    while (lo < hi) {
      const int mid = (lo + hi + 1) >> 1;
      if ((int64_t)units_per_item * sm.ipre[mid] <= x) lo = mid; else hi = mid - 1;
    }
    item = lo;
  }

  while (x < x_end) {
    // ---- locate the segment: unit (item, j), tiles [t0, t1)
    while ((int64_t)units_per_item * sm.ipre[item + 1] <= x) ++item;
    const int Ti = sm.ipre[item + 1] - sm.ipre[item];
    const int64_t r = x - (int64_t)units_per_item * sm.ipre[item];
    const int j = (int)(r / Ti);
    const int t0 = (int)(r - (int64_t)j * Ti);
    const int t1 = (int)min<int64_t>(Ti, t0 + (x_end - x));
    x += t1 - t0;

    const int hk = j / a.n_hg;
    const int hg = j - hk * a.n_hg;
    const int b = a.items ? a.items[item] : item;
    const int qrow = a.q_rows ? a.q_rows[item] : b;
    const int L = item_len(a, item);
    const int hl = hg * 16 + n;
    const bool head_ok = hl < a.group;
    const int hq = hk * a.group + (head_ok ? hl : 0);
    const int64_t row = clamp_i64(a.rpi[b], 0, a.rtt_rows - 1);
    const int64_t* rtt = a.rtt + row * a.rtt_stride;
    const uint8_t* kbase = a.k_pool + (int64_t)hk * kRowBytes;
    const uint8_t* vbase = a.v_pool + (int64_t)hk * kRowBytes;

    WaveState st;
    reset_state(st);
    for (int sub = t0; sub < t1; sub += kMaxChunk / kTile) {
      const int c0 = sub * kTile;
      const int n_loc = min(L, min(t1, sub + kMaxChunk / kTile) * kTile) - c0;
      const int n_tiles = (n_loc + kTile - 1) / kTile;
      // ---- stage the slot ids (and, once per segment, the Q^T fragments)
      __syncthreads();
      for (int i = tid; i < n_loc; i += kWaves * kWave)
        sm.u.loop.slots[i] = (int32_t)pool_row(rtt[c0 + i], a.pool_slots, a.seq_override > 0);
      if (sub == t0 && w == 0) {
        const __bf16* qp = a.q + (int64_t)qrow * a.q_stride + (int64_t)hq * kD;
#pragma unroll
        for (int kk = 0; kk < 8; ++kk) {
          const int d0 = FP8 ? (64 * (kk >> 1) + 16 * g + 8 * (kk & 1)) : (32 * kk + 8 * g);
          sm.qfrag[kk][lane] = head_ok ? ld_g16(qp + d0) : u32x4{0u, 0u, 0u, 0u};
        }
      }
      __syncthreads();

      // ---- this wave's tiles (it = w, w+4, ...): K of the next tile is issued
      // once this tile's K is staged, V of the next tile once PV has consumed
      // this tile's V. The steady-state loop always has a next tile; the last
      // tile is peeled so every wait count is exact.
      int it = w;
      if (it < n_tiles) {
        u32x4 qf[8];
#pragma unroll
        for (int kk = 0; kk < 8; ++kk) qf[kk] = sm.qfrag[kk][lane];
        KBuf<FP8> kb;
        VBuf<FP8> vb;
        const int32_t* slots = sm.u.loop.slots;
        u32x4* ks = sm.u.loop.kstage[w];
        issue_k<FP8>(kb, slots, it, n_loc, g, n, kbase, slot_bytes);
        issue_v<FP8>(vb, slots, it, n_loc, g, n, vbase, slot_bytes);
        for (; it + kWaves < n_tiles; it += kWaves) {
          stage_k<FP8>(kb, ks, g, n);
          // Scheduling barriers keep each prefetch where it is: the scheduler
          // would otherwise sink it to just before its consumer.
          __builtin_amdgcn_sched_barrier(0);
          issue_k<FP8>(kb, slots, it + kWaves, n_loc, g, n, kbase, slot_bytes);
          __builtin_amdgcn_sched_barrier(0);
          const u32x2 pt = qk_softmax<FP8>(ks, qf, it, n_loc, g, n, sl2, st);
          pv<FP8>(vb, pt, st);
          __builtin_amdgcn_sched_barrier(0);
          issue_v<FP8>(vb, slots, it + kWaves, n_loc, g, n, vbase, slot_bytes);
          __builtin_amdgcn_sched_barrier(0);
        }
        stage_k<FP8>(kb, ks, g, n);
        const u32x2 pt = qk_softmax<FP8>(ks, qf, it, n_loc, g, n, sl2, st);
        pv<FP8>(vb, pt, st);
      }
    }

    // Row sums were accumulated per lane group; the 4 groups share one head.
    st.l += __shfl_xor(st.l, 16, kWave);
    st.l += __shfl_xor(st.l, 32, kWave);
    block_merge(sm.u.merge, w, lane, st);

    if (w == 0) {
      if (t0 == 0 && t1 == Ti) {
        const uint32_t m = head_ok ? write_output<FP8>(a, qrow, hq, g, st, vscale) : 0u;
        amax_commit(a.amax, m);
      } else if (n < min(a.group, 16)) {
        // Partial of unit u = item * units_per_item + j from this workgroup.
        const int64_t part = (int64_t)blockIdx.x + (int64_t)item * units_per_item + j;
        float* po = a.ws_o + ((part * 16 + n) * 4 + g) * 64;
#pragma unroll
        for (int i = 0; i < kAcc; ++i) reinterpret_cast<f32x4*>(po)[i] = st.acc[i];
        if (g == 0) {
          a.ws_ml[(part * 16 + n) * 2 + 0] = st.m;
          a.ws_ml[(part * 16 + n) * 2 + 1] = st.l;
        }
      }
    }
  }
}

// Merges the partials of every unit owned by more than one workgroup of the
// streaming kernel; one workgroup per unit. Units of an empty request (L = 0)
// get zeros, as the reference's fully masked scaled_dot_product_attention
// returns them (torch's safe softmax: a row with no visible key is all zeros).
template <bool FP8>
__global__ void __launch_bounds__(kWaves * kWave)
decode_merge_kernel(DecodeArgs a) {
  __shared__ StateSlot slots[2];
  __shared__ int32_t red[2][kWaves];
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int w = wave_id();
  const int g = lane >> 4;
  const int n = lane & 15;

  const int units_per_item = a.hkv * a.n_hg;
  const int u = blockIdx.x;
  const int item = u / units_per_item;
  const int j = u - item * units_per_item;

  // Tiles before this item and in total (block reductions over items).
  int before = 0, total = 0;
  for (int i = tid; i < a.n_items; i += kWaves * kWave) {
    const int t = item_tiles(a, i);
    total += t;
    if (i < item) before += t;
  }
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) {
    before += __shfl_xor(before, off, kWave);
    total += __shfl_xor(total, off, kWave);
  }
  if (lane == 0) {
    red[0][w] = before;
    red[1][w] = total;
  }
  __syncthreads();
  before = red[0][0] + red[0][1] + red[0][2] + red[0][3];
  total = red[1][0] + red[1][1] + red[1][2] + red[1][3];

  const int hk = j / a.n_hg;
  const int hg = j - hk * a.n_hg;
  const int qrow = a.q_rows ? a.q_rows[item] : (a.items ? a.items[item] : item);
  const int hl = hg * 16 + n;
  const bool head_ok = hl < a.group;
  const int hq = hk * a.group + (head_ok ? hl : 0);
  const float vscale = FP8 ? a.v_scale[0] : 1.f;
  const int Ti = item_tiles(a, item);

  WaveState st;
  reset_state(st);
  if (Ti == 0) {
    // An empty context (seq_len 0) is a row of zeros (the reference's fully
    // masked attention); padding entries write nothing.
    if (w == 0) {
      uint32_t m = 0;
      if (head_ok && !item_is_padding(a, item)) {
        st.m = 0.f;
        st.l = 1.f;   // O = 0
        m = write_output<FP8>(a, qrow, hq, g, st, 1.f);
      }
      amax_commit(a.amax, m);
    }
    return;
  }
  const int64_t N = (int64_t)units_per_item * total;
  const int64_t p = (int64_t)units_per_item * before + (int64_t)j * Ti;
  const int P = (int)min<int64_t>(a.n_blocks, N);   // as in the streaming kernel
  const int b0 = owner_of(p, N, P);
  const int b1 = owner_of(p + Ti - 1, N, P);
  if (b0 == b1) return;  // written directly by the streaming kernel

  if (n < min(a.group, 16)) {
    for (int bb = b0 + w; bb <= b1; bb += kWaves) {
      const int64_t pp = (int64_t)bb + u;
      const float* po = a.ws_o + ((pp * 16 + n) * 4 + g) * 64;
      f32x4 acc2[kAcc];
#pragma unroll
      for (int i = 0; i < kAcc; ++i) acc2[i] = reinterpret_cast<const f32x4*>(po)[i];
      merge_into(st, a.ws_ml[(pp * 16 + n) * 2 + 0], a.ws_ml[(pp * 16 + n) * 2 + 1], acc2);
    }
  }
  block_merge(slots, w, lane, st);
  if (w == 0) {
    const uint32_t m = head_ok ? write_output<FP8>(a, qrow, hq, g, st, vscale) : 0u;
    amax_commit(a.amax, m);
  }
}

}  // namespace


int make_decode_plan(int32_t n_items, int32_t num_q_heads, int32_t num_kv_heads,
                     int32_t head_dim, int32_t max_seq_len, int32_t num_workgroups,
                     DecodePlan* p) {
  (void)max_seq_len;
  if (n_items < 0) return fail(TF_ERR_INVALID, "decode: n_items=%d", n_items);
  if (n_items > kMaxItems)
    return fail(TF_ERR_UNSUPPORTED, "decode: %d requests in one call (at most %d)", n_items,
                kMaxItems);
  if (num_kv_heads <= 0 || num_q_heads <= 0 || num_q_heads % num_kv_heads)
    return fail(TF_ERR_INVALID, "decode: num_q_heads=%d not a multiple of num_kv_heads=%d",
                num_q_heads, num_kv_heads);
  if (num_workgroups < 0) return fail(TF_ERR_INVALID, "decode: num_workgroups=%d", num_workgroups);
  if (head_dim != kD) {
    // Other head dims run the one-wave-per-row kernel (attn_generic.hip),
    // which needs no workspace.
    if (!generic_head_dim(head_dim))
      return fail(TF_ERR_UNSUPPORTED,
                  "decode: head_dim=%d (a multiple of 8 between 8 and %d)", head_dim, kD);
    *p = DecodePlan{};
    p->generic = true;
    return TF_OK;
  }
  const int32_t group = num_q_heads / num_kv_heads;
  p->n_hgroups = (group + 15) / 16;
  p->gmax = group < 16 ? group : 16;
  p->n_units = (int64_t)n_items * num_kv_heads * p->n_hgroups;
  // One persistent workgroup (4 waves) per CU measured fastest on MI355X.
  p->generic = false;
  p->n_blocks = num_workgroups > 0 ? num_workgroups : device_cu_count();
  const int64_t parts = p->n_units + p->n_blocks;
  p->ml_bytes = (parts * 16 * 2 * 4 + 255) / 256 * 256;
  p->o_bytes = parts * 16 * (int64_t)kD * 4;
  p->total_bytes = p->ml_bytes + p->o_bytes;
  return TF_OK;
}

}  // namespace tfa

namespace tfa {
namespace {

enum : int { kPhasePartial = 1, kPhaseMerge = 2 };

int decode_launch(const void* q, int64_t q_row_stride, const void* k_pool, const void* v_pool,
                  int64_t pool_slots, int32_t kv_dtype, const float* k_scale,
                  const float* v_scale, const int64_t* req_to_token, int64_t rtt_rows,
                  int64_t rtt_row_stride, int64_t rtt_cols, const int64_t* req_pool_indices,
                  const int64_t* seq_lens, int32_t seq_len_override, const int32_t* items,
                  const int32_t* q_rows, int32_t n_items, int32_t num_q_heads,
                  int32_t num_kv_heads, int32_t head_dim, float scale, void* out,
                  int64_t out_row_stride, void* workspace, int64_t workspace_bytes,
                  int32_t max_seq_len, int32_t num_workgroups, const void* gate,
                  int64_t gate_row_stride, int64_t gate_head_stride, uint32_t* out_amax,
                  tf_stream_t stream, int phases) {
  clear_error();
  DecodePlan p;
  int rc = make_decode_plan(n_items, num_q_heads, num_kv_heads, head_dim, max_seq_len,
                            num_workgroups, &p);
  if (rc != TF_OK) return rc;
  if (n_items == 0) return TF_OK;
  if (kv_dtype != TF_DTYPE_BF16 && kv_dtype != TF_DTYPE_FP8_E4M3)
    return fail(TF_ERR_UNSUPPORTED, "decode: kv_dtype=%d", kv_dtype);
  if (!q || !k_pool || !v_pool || !req_to_token || !req_pool_indices || !out)
    return fail(TF_ERR_INVALID, "decode: null pointer argument");
  if (!seq_lens && seq_len_override <= 0)
    return fail(TF_ERR_INVALID, "decode: seq_lens is null and no override");
  if (kv_dtype == TF_DTYPE_FP8_E4M3 && (!k_scale || !v_scale))
    return fail(TF_ERR_INVALID, "decode: fp8 pool needs k_scale and v_scale");
  if (pool_slots < 1 || pool_slots > INT32_MAX || rtt_rows < 1 || rtt_cols < 1 ||
      rtt_row_stride < rtt_cols)
    return fail(TF_ERR_INVALID, "decode: bad pool/req_to_token extents");
  if (!aligned16(q) || !aligned16(out) || !aligned16(k_pool) || !aligned16(v_pool) ||
      (q_row_stride * 2) % 16 || (out_row_stride * 2) % 16)
    return fail(TF_ERR_INVALID, "decode: q/out/pools must be 16-byte aligned");
  if (q_row_stride < (int64_t)num_q_heads * head_dim ||
      out_row_stride < (int64_t)num_q_heads * head_dim)
    return fail(TF_ERR_INVALID, "decode: row stride smaller than num_q_heads*head_dim");
  if (gate && (!aligned16(gate) || gate_row_stride % 8 || gate_head_stride % 8 ||
               gate_head_stride < head_dim))
    return fail(TF_ERR_INVALID, "decode: gate must be 16-byte aligned with strides of 8 elements");
  if (p.total_bytes > 0 &&
      (!workspace || workspace_bytes < p.total_bytes || !aligned16(workspace)))
    return fail(TF_ERR_INVALID, "decode: workspace needs %lld bytes, got %lld",
                (long long)p.total_bytes, (long long)workspace_bytes);
  if (p.n_units > INT32_MAX) return fail(TF_ERR_INVALID, "decode: too many units");
  if (p.generic) {   // head_dim != 256: everything happens in the "partial" phase
    if (!(phases & kPhasePartial)) return TF_OK;
    GenericAttnArgs g{};
    g.q = static_cast<const __bf16*>(q);
    g.q_stride = q_row_stride;
    g.k_pool = static_cast<const uint8_t*>(k_pool);
    g.v_pool = static_cast<const uint8_t*>(v_pool);
    g.pool_slots = pool_slots;
    g.fp8 = kv_dtype == TF_DTYPE_FP8_E4M3;
    g.k_scale = k_scale;
    g.v_scale = v_scale;
    g.rtt = req_to_token;
    g.rtt_rows = rtt_rows;
    g.rtt_stride = rtt_row_stride;
    g.rtt_cols = rtt_cols;
    g.rpi = req_pool_indices;
    g.seq_lens = seq_lens;
    g.seq_override = seq_len_override;
    g.items = items;
    g.q_rows = q_rows;
    g.work = nullptr;
    g.n_rows = n_items;
    g.hq = num_q_heads;
    g.hkv = num_kv_heads;
    g.head_dim = head_dim;
    g.scale_log2 = scale * kLog2e;
    g.out = static_cast<__bf16*>(out);
    g.out_stride = out_row_stride;
    g.gate = static_cast<const __bf16*>(gate);
    g.gate_stride = gate_row_stride;
    g.gate_hstride = gate_head_stride;
    g.amax = out_amax;
    return launch_generic_attn(g, reinterpret_cast<hipStream_t>(stream));
  }

  DecodeArgs a;
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
  a.items = items;
  a.q_rows = q_rows;
  a.n_items = n_items;
  a.hkv = num_kv_heads;
  a.group = num_q_heads / num_kv_heads;
  a.n_hg = p.n_hgroups;
  a.scale_log2 = scale * kLog2e;
  a.out = static_cast<__bf16*>(out);
  a.out_stride = out_row_stride;
  a.gate = static_cast<const __bf16*>(gate);
  a.gate_stride = gate_row_stride;
  a.gate_hstride = gate_head_stride;
  a.amax = out_amax;
  char* ws = static_cast<char*>(workspace);
  a.ws_ml = reinterpret_cast<float*>(ws);
  a.ws_o = reinterpret_cast<float*>(ws + p.ml_bytes);
  a.n_blocks = p.n_blocks;

  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  const dim3 block(kWaves * kWave);
  const bool fp8 = kv_dtype == TF_DTYPE_FP8_E4M3;
  if (phases & kPhasePartial) {
    if (fp8)
      hipLaunchKernelGGL(decode_kernel<true>, dim3((unsigned)p.n_blocks), block, 0, s, a);
    else
      hipLaunchKernelGGL(decode_kernel<false>, dim3((unsigned)p.n_blocks), block, 0, s, a);
    rc = launch_status("tf_attn_decode partial launch");
    if (rc != TF_OK) return rc;
  }
  if (phases & kPhaseMerge) {
    if (fp8)
      hipLaunchKernelGGL(decode_merge_kernel<true>, dim3((unsigned)p.n_units), block, 0, s, a);
    else
      hipLaunchKernelGGL(decode_merge_kernel<false>, dim3((unsigned)p.n_units), block, 0, s, a);
    rc = launch_status("tf_attn_decode merge launch");
  }
  return rc;
}

}  // namespace
}  // namespace tfa

#define TF_DECODE_PARAMS                                                                    \
  const void *q, int64_t q_row_stride, const void *k_pool, const void *v_pool,            \
      int64_t pool_slots, int32_t kv_dtype, const float *k_scale, const float *v_scale,    \
      const int64_t *req_to_token, int64_t rtt_rows, int64_t rtt_row_stride,               \
      int64_t rtt_cols, const int64_t *req_pool_indices, const int64_t *seq_lens,          \
      int32_t seq_len_override, const int32_t *items, const int32_t *q_rows,               \
      int32_t n_items, int32_t num_q_heads, int32_t num_kv_heads, int32_t head_dim,        \
      float scale, void *out, int64_t out_row_stride, void *workspace,                     \
      int64_t workspace_bytes, int32_t max_seq_len, int32_t num_workgroups,                \
      const void *gate, int64_t gate_row_stride, int64_t gate_head_stride,                 \
      uint32_t *out_amax, tf_stream_t stream
#define TF_DECODE_ARGS                                                                      \
  q, q_row_stride, k_pool, v_pool, pool_slots, kv_dtype, k_scale, v_scale, req_to_token,   \
      rtt_rows, rtt_row_stride, rtt_cols, req_pool_indices, seq_lens, seq_len_override,    \
      items, q_rows, n_items, num_q_heads, num_kv_heads, head_dim, scale, out,             \
      out_row_stride, workspace, workspace_bytes, max_seq_len, num_workgroups, gate,       \
      gate_row_stride, gate_head_stride, out_amax, stream

extern "C" {

int64_t tf_attn_decode_workspace_bytes(int32_t n_items, int32_t num_q_heads,
                                       int32_t num_kv_heads, int32_t head_dim,
                                       int32_t max_seq_len, int32_t num_workgroups) {
  tfa::clear_error();
  tfa::DecodePlan p;
  const int rc = tfa::make_decode_plan(n_items, num_q_heads, num_kv_heads, head_dim,
                                       max_seq_len, num_workgroups, &p);
  if (rc != TF_OK) return rc;
  return p.total_bytes;
}

int32_t tf_attn_decode(TF_DECODE_PARAMS) {
  return tfa::decode_launch(TF_DECODE_ARGS, tfa::kPhasePartial | tfa::kPhaseMerge);
}

int32_t tf_attn_decode_partial(TF_DECODE_PARAMS) {
  return tfa::decode_launch(TF_DECODE_ARGS, tfa::kPhasePartial);
}

int32_t tf_attn_decode_merge(TF_DECODE_PARAMS) {
  return tfa::decode_launch(TF_DECODE_ARGS, tfa::kPhaseMerge);
}

}  // extern "C"

// ------------------------------------------------------------ no-allocation decode
// tf_attn_decode for callers that cannot allocate device memory: the split
// partials live in this library-owned array instead of a caller workspace.
// Every GPU the library runs on holds its own copy from module load until the
// process ends; all calls on one GPU share it (the partials need no
// initialisation: every one the merge reads was written earlier in the same
// call), so calls that overlap in time on one GPU race.
static constexpr int64_t kNoAllocScratchBytes = 32LL << 20;
static __device__ __align__(256) uint8_t scratch[kNoAllocScratchBytes];

namespace tfa {
namespace {

constexpr int kMaxDevices = 64;

// The device address of `scratch` on the current device, looked up once per
// device (the host-side name is only a handle for the lookup; passing it to a
// kernel would fault).
int noalloc_scratch(hipStream_t stream, void** ptr) {
  static std::mutex mu;
  static void* cache[kMaxDevices];
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return fail(TF_ERR_HIP, "decode_noalloc: hipGetDevice: %s",
                                   hipGetErrorString(e));
  if (dev < 0 || dev >= kMaxDevices)
    return fail(TF_ERR_UNSUPPORTED, "decode_noalloc: device %d", dev);
  if (stream) {
    hipDevice_t sdev = -1;
    e = hipStreamGetDevice(stream, &sdev);
    if (e != hipSuccess)
      return fail(TF_ERR_HIP, "decode_noalloc: hipStreamGetDevice: %s", hipGetErrorString(e));
    if (sdev != dev)
      return fail(TF_ERR_INVALID, "decode_noalloc: the stream is on device %d, device %d is "
                  "current (make the stream's device current)", (int)sdev, dev);
  }
  std::lock_guard<std::mutex> lock(mu);
  if (!cache[dev]) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p)
      return fail(TF_ERR_HIP, "decode_noalloc: hipGetSymbolAddress(scratch): %s",
                  hipGetErrorString(e));
    cache[dev] = p;
  }
  *ptr = cache[dev];
  return TF_OK;
}

}  // namespace
}  // namespace tfa

extern "C" int32_t tf_attn_decode_noalloc(
    const void* q, int64_t q_row_stride, const void* k_pool, const void* v_pool,
    int64_t pool_slots, int32_t kv_dtype, const float* k_scale, const float* v_scale,
    const int64_t* req_to_token, int64_t rtt_rows, int64_t rtt_row_stride, int64_t rtt_cols,
    const int64_t* req_pool_indices, const int64_t* seq_lens, int32_t seq_len_override,
    const int32_t* items, const int32_t* q_rows, int32_t n_items, int32_t num_q_heads,
    int32_t num_kv_heads, int32_t head_dim, float scale, void* out, int64_t out_row_stride,
    int32_t max_seq_len, int32_t num_workgroups, const void* gate, int64_t gate_row_stride,
    int64_t gate_head_stride, uint32_t* out_amax, tf_stream_t stream) {
  using namespace tfa;
  clear_error();
  DecodePlan p;
  const int rc = make_decode_plan(n_items, num_q_heads, num_kv_heads, head_dim, max_seq_len,
                                  num_workgroups, &p);
  if (rc != TF_OK) return rc;
  if (p.total_bytes > kNoAllocScratchBytes)
    return fail(TF_ERR_UNSUPPORTED,
                "decode_noalloc: this call needs %lld bytes of split scratch, the static buffer "
                "holds %lld (fewer requests or workgroups per call, or tf_attn_decode with a "
                "workspace)", (long long)p.total_bytes, (long long)kNoAllocScratchBytes);
  void* ws = nullptr;
  const int rc2 = noalloc_scratch(reinterpret_cast<hipStream_t>(stream), &ws);
  if (rc2 != TF_OK) return rc2;
  void* workspace = ws;
  const int64_t workspace_bytes = kNoAllocScratchBytes;
  return decode_launch(TF_DECODE_ARGS, kPhasePartial | kPhaseMerge);
}
