// Split-K decode attention over the req_to_token -> KV-pool slot indirection.
//
// Replaces the reference's pure-decode branch (qwen3_8/full_attention.py:215-242):
// gather of req_to_token[r, :L] rows, GQA repeat_interleave, length mask and
// SDPA, here fused into one HBM-streaming pass with no padded or expanded copy.
//
// Work decomposition
//   unit  = (request item, kv head, group of <= 16 q heads sharing that kv head)
//   block = (unit, split): `chunk` consecutive context tokens; 4 waves take
//           interleaved 16-token tiles of the chunk.
//   A block keeps the whole GQA head group together, so each K/V row read from
//   HBM feeds all of the group's q heads.
// Block prologue: the chunk's slot ids (int64 req_to_token entries, clamped to
// the pool) are staged in LDS with coalesced loads, and the group's Q^T MFMA
// fragments are staged in LDS once.
// Per 16-token tile a wave
//   * loads each lane's K slice straight into MFMA A-operand registers
//     (16-byte loads, 64 contiguous bytes of a row per 4 lanes) and its V slice
//     (four token rows x 16 bytes per lane); the next tile's loads are always in
//     flight while the current tile computes (register double buffering),
//   * S^T[token, head] = K * Q^T with v_mfma_f32_16x16x32_bf16 (heads padded to 16),
//   * online softmax per head (lane-local scores, two xor-shuffles for the max),
//   * O^T[dim, head] += V^T * P^T with v_mfma_f32_16x16x16_bf16, V^T built in
//     registers with v_perm_b32 (fp8: byte permutes + v_cvt_scalef32_pk_bf16_fp8).
//   Every per-head quantity (max, sum, rescale factor, 64 output dims) is then
//   lane-local: lane (g, n) owns head n, dims {128s + 32g + 8r + e} (bf16) or
//   {64g + 16r + e} (fp8).
// Merging
//   waves of a block merge pairwise through LDS in the same lane layout; a block
//   that is the only split of its unit writes bf16 output directly, otherwise it
//   stores an fp32 partial (O, max, sum). A second, small kernel merges the
//   partials of multi-split units (one workgroup per unit). Keeping the merge in
//   its own launch avoids device-scope fences in the streaming kernel: on gfx950
//   those write back and invalidate the whole L2 of the XCD.
#include <math.h>

#include "tf_common.h"
#include "tf_internal.h"

namespace tfa {
namespace {

constexpr int kD = 256;         // head_dim (Qwen3.8: 256)
constexpr int kWaves = 4;
constexpr int kTile = 16;       // tokens per wave iteration
constexpr int kAcc = 16;        // f32x4 accumulators per lane (64 output dims)
constexpr int kMaxChunk = 4096; // slot ids staged in LDS per block

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
  int32_t hkv, group, n_hg;
  float scale_log2;
  __bf16* out;
  int64_t out_stride;
  float* ws_ml;
  float* ws_o;
  int32_t chunk, max_splits;
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

struct DecodeSmem {
  union {
    int32_t slots[kMaxChunk];   // main loop: slot id of each chunk token
    StateSlot merge[2];         // epilogue: wave-state exchange
  } u;
  u32x4 qfrag[8][kWave];        // Q^T B-operand fragments, lane-major
};

template <bool FP8>
struct TileBuf {
  u32x4 k[FP8 ? 4 : 8];
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

template <bool FP8>
__device__ __forceinline__ void write_output(const DecodeArgs& a, int qrow, int hq, int g,
                                             const WaveState& st, float vscale) {
  const float inv = vscale / st.l;
  __bf16* o = a.out + (int64_t)qrow * a.out_stride + (int64_t)hq * kD;
  if (FP8) {
#pragma unroll
    for (int r = 0; r < 4; ++r) {
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        u32x4 v;
#pragma unroll
        for (int k = 0; k < 4; ++k)
          v[k] = pack_bf16(st.acc[8 * h + 2 * k][r] * inv, st.acc[8 * h + 2 * k + 1][r] * inv);
        *reinterpret_cast<u32x4*>(o + 64 * g + 16 * r + 8 * h) = v;
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
        *reinterpret_cast<u32x4*>(o + 128 * s + 32 * g + 8 * r) = v;
      }
    }
  }
}

// Issues the global loads of tile `it` (tokens it*16 .. it*16+15 of the chunk,
// clamped to the chunk's last token so every address is a valid row).
template <bool FP8>
__device__ __forceinline__ void issue_tile(TileBuf<FP8>& tb, const int32_t* slots, int it,
                                           int n_loc, int g, int n, const uint8_t* kbase,
                                           const uint8_t* vbase, int64_t slot_bytes) {
  const int last = n_loc - 1;
  const int t0 = it * kTile;
  const int64_t ks = slots[min(t0 + n, last)];
  const uint8_t* kp = kbase + ks * slot_bytes;
#pragma unroll
  for (int u = 0; u < (FP8 ? 4 : 8); ++u) tb.k[u] = ld_g16(kp + 64 * u + 16 * g);
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int64_t vs = slots[min(t0 + 4 * g + j, last)];
    const uint8_t* vp = vbase + vs * slot_bytes;
#pragma unroll
    for (int s = 0; s < (FP8 ? 1 : 2); ++s) tb.v[j][s] = ld_g16(vp + 16 * n + 256 * s);
  }
}

template <bool FP8>
__device__ __forceinline__ void compute_tile(const TileBuf<FP8>& tb, const u32x4 (*qfrag)[kWave],
                                             int it, int n_loc, int g, int lane, float sl2,
                                             WaveState& st) {
  // ---- S^T = K Q^T
  f32x4 sacc = {0.f, 0.f, 0.f, 0.f};
  if (FP8) {
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      sacc = mfma_16x16x32(e4m3x8_to_bf16x8(tb.k[u][0], tb.k[u][1]), qfrag[2 * u][lane], sacc);
      sacc = mfma_16x16x32(e4m3x8_to_bf16x8(tb.k[u][2], tb.k[u][3]), qfrag[2 * u + 1][lane],
                           sacc);
    }
  } else {
#pragma unroll
    for (int kk = 0; kk < 8; ++kk) sacc = mfma_16x16x32(tb.k[kk], qfrag[kk][lane], sacc);
  }

  // ---- online softmax for head n over chunk tokens it*16 + 4g + r
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

  // ---- O^T += V^T P^T
  const u32x2 pt = {pack_bf16(p[0], p[1]), pack_bf16(p[2], p[3])};
  if (FP8) {
#pragma unroll
    for (int e = 0; e < 16; e += 2) {
      const int dw = e >> 2;
      const uint32_t b0 = e & 3;
      const uint32_t sel = b0 | ((4 + b0) << 8) | ((b0 + 1) << 16) | ((5 + b0) << 24);
      const uint32_t x = __builtin_amdgcn_perm(tb.v[1][0][dw], tb.v[0][0][dw], sel);
      const uint32_t y = __builtin_amdgcn_perm(tb.v[3][0][dw], tb.v[2][0][dw], sel);
      const u32x2 va = {e4m3x2_to_bf16x2<false>(x), e4m3x2_to_bf16x2<false>(y)};
      const u32x2 vb = {e4m3x2_to_bf16x2<true>(x), e4m3x2_to_bf16x2<true>(y)};
      st.acc[e] = mfma_16x16x16(va, pt, st.acc[e]);
      st.acc[e + 1] = mfma_16x16x16(vb, pt, st.acc[e + 1]);
    }
  } else {
#pragma unroll
    for (int s = 0; s < 2; ++s) {
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const int dw = e >> 1;
        const int hi = e & 1;
        const u32x2 va = {pair_sel(tb.v[1][s][dw], tb.v[0][s][dw], hi),
                          pair_sel(tb.v[3][s][dw], tb.v[2][s][dw], hi)};
        st.acc[8 * s + e] = mfma_16x16x16(va, pt, st.acc[8 * s + e]);
      }
    }
  }
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

  const int per_item = a.hkv * a.n_hg;
  const int split = blockIdx.x % a.max_splits;
  const int unit = blockIdx.x / a.max_splits;
  const int item = unit / per_item;
  const int rem = unit - item * per_item;
  const int hk = rem / a.n_hg;
  const int hg = rem - hk * a.n_hg;
  const int b = a.items ? a.items[item] : item;
  const int qrow = a.q_rows ? a.q_rows[item] : b;

  int64_t len = a.seq_override > 0 ? (int64_t)a.seq_override : a.seq_lens[b];
  if (len > a.rtt_cols) len = a.rtt_cols;
  const int L = (int)len;
  const int hl = hg * 16 + n;             // head within the kv group
  const bool head_ok = hl < a.group;
  const int hq = hk * a.group + (head_ok ? hl : 0);

  if (L <= 0) {
    // Every key masked: the reference's softmax yields NaN.
    if (split == 0 && w == 0 && head_ok) {
      WaveState st;
      st.m = 0.f;
      st.l = __builtin_nanf("");
#pragma unroll
      for (int i = 0; i < kAcc; ++i) st.acc[i] = f32x4{0.f, 0.f, 0.f, 0.f};
      write_output<FP8>(a, qrow, hq, g, st, 1.f);
    }
    return;
  }
  const int n_split = (L + a.chunk - 1) / a.chunk;
  if (split >= n_split) return;
  const int c0 = split * a.chunk;
  const int n_loc = min(L, c0 + a.chunk) - c0;
  const int n_tiles = (n_loc + kTile - 1) / kTile;

  // ---- prologue: slot ids of the chunk and the Q^T fragments into LDS
  {
    const int64_t row = clamp_i64(a.rpi[b], 0, a.rtt_rows - 1);
    const int64_t* rtt = a.rtt + row * a.rtt_stride + c0;
    for (int i = tid; i < n_loc; i += kWaves * kWave)
      sm.u.slots[i] = (int32_t)clamp_i64(rtt[i], 0, a.pool_slots - 1);
    if (w == 0) {
      const __bf16* qp = a.q + (int64_t)qrow * a.q_stride + (int64_t)hq * kD;
#pragma unroll
      for (int kk = 0; kk < 8; ++kk) {
        const int d0 = FP8 ? (64 * (kk >> 1) + 16 * g + 8 * (kk & 1)) : (32 * kk + 8 * g);
        sm.qfrag[kk][lane] = head_ok ? ld_g16(qp + d0) : u32x4{0u, 0u, 0u, 0u};
      }
    }
  }
  const float kscale = FP8 ? a.k_scale[0] : 1.f;
  const float vscale = FP8 ? a.v_scale[0] : 1.f;
  const float sl2 = a.scale_log2 * kscale;
  const uint8_t* kbase = a.k_pool + (int64_t)hk * kRowBytes;
  const uint8_t* vbase = a.v_pool + (int64_t)hk * kRowBytes;
  const int64_t slot_bytes = (int64_t)a.hkv * kRowBytes;
  __syncthreads();

  WaveState st;
  st.m = -INFINITY;
  st.l = 0.f;
#pragma unroll
  for (int i = 0; i < kAcc; ++i) st.acc[i] = f32x4{0.f, 0.f, 0.f, 0.f};

  // ---- main loop: the next tile's loads are issued before the current tile
  // computes. Issues are unconditional (clamped rows) so the wait counts are
  // exact; a past-the-end issue re-reads cached rows of the chunk's last token.
  int it = w;
  if (it < n_tiles) {
    TileBuf<FP8> A, B;
    issue_tile<FP8>(A, sm.u.slots, it, n_loc, g, n, kbase, vbase, slot_bytes);
    for (;;) {
      issue_tile<FP8>(B, sm.u.slots, it + kWaves, n_loc, g, n, kbase, vbase, slot_bytes);
      compute_tile<FP8>(A, sm.qfrag, it, n_loc, g, lane, sl2, st);
      if (it + kWaves >= n_tiles) break;
      issue_tile<FP8>(A, sm.u.slots, it + 2 * kWaves, n_loc, g, n, kbase, vbase, slot_bytes);
      compute_tile<FP8>(B, sm.qfrag, it + kWaves, n_loc, g, lane, sl2, st);
      if (it + 2 * kWaves >= n_tiles) break;
      it += 2 * kWaves;
    }
  }

  // Row sums were accumulated per lane group; the 4 groups share one head.
  st.l += __shfl_xor(st.l, 16, kWave);
  st.l += __shfl_xor(st.l, 32, kWave);

  block_merge(sm.u.merge, w, lane, st);

  const int gmax = min(a.group, 16);
  if (n_split == 1) {
    if (w == 0 && head_ok) write_output<FP8>(a, qrow, hq, g, st, vscale);
    return;
  }

  // ---- multi-split: publish this block's fp32 partial (lane layout) for the
  // merge kernel. Partial p of unit u: O at ws_o[((p*16 + head)*4 + g)*64 ..],
  // (max, sum) at ws_ml[(p*16 + head)*2 ..], p = u * max_splits + split.
  if (w == 0 && n < gmax) {
    const int64_t part = (int64_t)unit * a.max_splits + split;
    float* po = a.ws_o + ((part * 16 + n) * 4 + g) * 64;
#pragma unroll
    for (int i = 0; i < kAcc; ++i) reinterpret_cast<f32x4*>(po)[i] = st.acc[i];
    if (g == 0) {
      a.ws_ml[(part * 16 + n) * 2 + 0] = st.m;
      a.ws_ml[(part * 16 + n) * 2 + 1] = st.l;
    }
  }
}

// Merges the split partials of every unit that has more than one split; one
// workgroup per unit, waves take splits w, w+4, ... and tree-merge through LDS.
template <bool FP8>
__global__ void __launch_bounds__(kWaves * kWave)
decode_merge_kernel(DecodeArgs a) {
  __shared__ StateSlot slots[2];
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int w = wave_id();
  const int g = lane >> 4;
  const int n = lane & 15;

  const int unit = blockIdx.x;
  const int per_item = a.hkv * a.n_hg;
  const int item = unit / per_item;
  const int rem = unit - item * per_item;
  const int hk = rem / a.n_hg;
  const int hg = rem - hk * a.n_hg;
  const int b = a.items ? a.items[item] : item;
  const int qrow = a.q_rows ? a.q_rows[item] : b;
  int64_t len = a.seq_override > 0 ? (int64_t)a.seq_override : a.seq_lens[b];
  if (len > a.rtt_cols) len = a.rtt_cols;
  const int L = (int)len;
  const int n_split = L > 0 ? (L + a.chunk - 1) / a.chunk : 0;
  if (n_split <= 1) return;  // written directly by the split kernel
  const int hl = hg * 16 + n;
  const bool head_ok = hl < a.group;
  const int hq = hk * a.group + (head_ok ? hl : 0);
  const int gmax = min(a.group, 16);
  const float vscale = FP8 ? a.v_scale[0] : 1.f;

  WaveState st;
  st.m = -INFINITY;
  st.l = 0.f;
#pragma unroll
  for (int i = 0; i < kAcc; ++i) st.acc[i] = f32x4{0.f, 0.f, 0.f, 0.f};
  if (n < gmax) {
    for (int sp = w; sp < n_split; sp += kWaves) {
      const int64_t pp = (int64_t)unit * a.max_splits + sp;
      const float* po = a.ws_o + ((pp * 16 + n) * 4 + g) * 64;
      f32x4 acc2[kAcc];
#pragma unroll
      for (int i = 0; i < kAcc; ++i) acc2[i] = reinterpret_cast<const f32x4*>(po)[i];
      merge_into(st, a.ws_ml[(pp * 16 + n) * 2 + 0], a.ws_ml[(pp * 16 + n) * 2 + 1], acc2);
    }
  }
  block_merge(slots, w, lane, st);
  if (w == 0 && head_ok) write_output<FP8>(a, qrow, hq, g, st, vscale);
}

}  // namespace

int make_decode_plan(int32_t n_items, int32_t num_q_heads, int32_t num_kv_heads,
                     int32_t head_dim, int32_t max_seq_len, int32_t chunk_tokens,
                     DecodePlan* p) {
  if (n_items < 0) return fail(TF_ERR_INVALID, "decode: n_items=%d", n_items);
  if (num_kv_heads <= 0 || num_q_heads <= 0 || num_q_heads % num_kv_heads)
    return fail(TF_ERR_INVALID, "decode: num_q_heads=%d not a multiple of num_kv_heads=%d",
                num_q_heads, num_kv_heads);
  if (head_dim != kD)
    return fail(TF_ERR_UNSUPPORTED, "decode: head_dim=%d (only %d is built)", head_dim, kD);
  if (max_seq_len < 1) max_seq_len = 1;
  if (chunk_tokens < 0 || chunk_tokens % 64 || chunk_tokens > kMaxChunk)
    return fail(TF_ERR_INVALID, "decode: chunk_tokens=%d must be a multiple of 64 <= %d",
                chunk_tokens, kMaxChunk);
  const int32_t group = num_q_heads / num_kv_heads;
  p->n_hgroups = (group + 15) / 16;
  p->gmax = group < 16 ? group : 16;
  p->n_units = (int64_t)n_items * num_kv_heads * p->n_hgroups;
  int32_t chunk = chunk_tokens;
  if (chunk == 0) {
    // Aim for ~8 workgroups per CU on a 256-CU part; chunks of 256..4096 tokens.
    const int64_t units = p->n_units > 0 ? p->n_units : 1;
    int64_t want = (2048 + units - 1) / units;
    if (want < 1) want = 1;
    int64_t c = ((int64_t)max_seq_len + want - 1) / want;
    c = (c + 63) / 64 * 64;
    const int64_t fit = ((int64_t)max_seq_len + 63) / 64 * 64;
    int64_t lo = 256;
    if (lo > fit) lo = fit;
    if (c < lo) c = lo;
    if (c > kMaxChunk) c = kMaxChunk;
    chunk = (int32_t)c;
  }
  p->chunk = chunk;
  p->max_splits = (max_seq_len + chunk - 1) / chunk;
  const int64_t parts = p->n_units * p->max_splits;
  p->ml_bytes = (parts * 16 * 2 * 4 + 255) / 256 * 256;
  p->o_bytes = parts * 16 * (int64_t)kD * 4;
  p->total_bytes = p->max_splits > 1 ? p->ml_bytes + p->o_bytes : 0;
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
                  int32_t max_seq_len, int32_t chunk_tokens, tf_stream_t stream, int phases) {
  clear_error();
  DecodePlan p;
  int rc = make_decode_plan(n_items, num_q_heads, num_kv_heads, head_dim, max_seq_len,
                            chunk_tokens, &p);
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
  if (p.total_bytes > 0 &&
      (!workspace || workspace_bytes < p.total_bytes || !aligned16(workspace)))
    return fail(TF_ERR_INVALID, "decode: workspace needs %lld bytes, got %lld",
                (long long)p.total_bytes, (long long)workspace_bytes);
  const int64_t grid = p.n_units * p.max_splits;
  if (grid > INT32_MAX) return fail(TF_ERR_INVALID, "decode: grid too large");

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
  a.hkv = num_kv_heads;
  a.group = num_q_heads / num_kv_heads;
  a.n_hg = p.n_hgroups;
  a.scale_log2 = scale * kLog2e;
  a.out = static_cast<__bf16*>(out);
  a.out_stride = out_row_stride;
  char* ws = static_cast<char*>(workspace);
  a.ws_ml = p.total_bytes ? reinterpret_cast<float*>(ws) : nullptr;
  a.ws_o = p.total_bytes ? reinterpret_cast<float*>(ws + p.ml_bytes) : nullptr;
  a.chunk = p.chunk;
  a.max_splits = p.max_splits;

  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  const dim3 block(kWaves * kWave);
  const bool fp8 = kv_dtype == TF_DTYPE_FP8_E4M3;
  if (phases & kPhasePartial) {
    if (fp8)
      hipLaunchKernelGGL(decode_kernel<true>, dim3((unsigned)grid), block, 0, s, a);
    else
      hipLaunchKernelGGL(decode_kernel<false>, dim3((unsigned)grid), block, 0, s, a);
    rc = launch_status("tf_attn_decode partial launch");
    if (rc != TF_OK) return rc;
  }
  if ((phases & kPhaseMerge) && p.max_splits > 1) {
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
      int64_t workspace_bytes, int32_t max_seq_len, int32_t chunk_tokens,                  \
      tf_stream_t stream
#define TF_DECODE_ARGS                                                                      \
  q, q_row_stride, k_pool, v_pool, pool_slots, kv_dtype, k_scale, v_scale, req_to_token,   \
      rtt_rows, rtt_row_stride, rtt_cols, req_pool_indices, seq_lens, seq_len_override,    \
      items, q_rows, n_items, num_q_heads, num_kv_heads, head_dim, scale, out,             \
      out_row_stride, workspace, workspace_bytes, max_seq_len, chunk_tokens, stream

extern "C" {

int64_t tf_attn_decode_workspace_bytes(int32_t n_items, int32_t num_q_heads,
                                       int32_t num_kv_heads, int32_t head_dim,
                                       int32_t max_seq_len, int32_t chunk_tokens) {
  tfa::clear_error();
  tfa::DecodePlan p;
  const int rc = tfa::make_decode_plan(n_items, num_q_heads, num_kv_heads, head_dim,
                                       max_seq_len, chunk_tokens, &p);
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
