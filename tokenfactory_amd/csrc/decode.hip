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
// Per 16-token tile a wave
//   * reads the 16 slot ids (lane n <- req_to_token[row, t0 + n]) one tile ahead,
//   * loads each lane's K slice straight into MFMA A-operand registers
//     (16-byte loads, 64 contiguous bytes per row per instruction) and its V
//     slice (four token rows x 16 bytes),
//   * S^T[token, head] = K * Q^T with v_mfma_f32_16x16x32_bf16 (Q is the
//     register-resident B operand, heads padded to 16),
//   * online softmax per head (lane-local scores, two xor-shuffles for the max),
//   * O^T[dim, head] += V^T * P^T with v_mfma_f32_16x16x16_bf16, V^T built in
//     registers with v_perm_b32 (fp8: byte permutes + v_cvt_scalef32_pk_bf16_fp8).
//   Every per-head quantity (max, sum, rescale factor, 64 output dims) is then
//   lane-local: lane (g, n) owns head n, dims {128s + 32g + 8r + e} (bf16) or
//   {64g + 16r + e} (fp8).
// Merging
//   waves of a block merge pairwise through LDS in the same lane layout; a block
//   that is the only split of its unit writes bf16 output directly, otherwise it
//   stores an fp32 partial (O, max, sum) and bumps the unit's arrival counter; the
//   last block to arrive merges all partials and resets the counter to zero.
#include <math.h>

#include "tf_common.h"
#include "tf_internal.h"

namespace tfa {
namespace {

constexpr int kD = 256;       // head_dim (Qwen3.8: 256)
constexpr int kWaves = 4;
constexpr int kTile = 16;     // tokens per wave iteration
constexpr int kAcc = 16;      // f32x4 accumulators per lane (64 output dims)

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
  int32_t* ws_cnt;
  float* ws_ml;
  float* ws_o;
  int32_t chunk, max_splits;
};

struct WaveState {
  float m, l;
  f32x4 acc[kAcc];
};

// Output dim of accumulator element (i, r) for lane group g.
template <bool FP8>
__device__ __forceinline__ int acc_dim(int i, int r, int g) {
  if (FP8) return 64 * g + 16 * r + i;            // i = e (0..15)
  return 128 * (i >> 3) + 32 * g + 8 * r + (i & 7);  // i = s*8 + e
}

__device__ __forceinline__ void merge_into(WaveState& st, float m2, float l2, const f32x4* acc2) {
  const float M = fmaxf(st.m, m2);
  const float a1 = (st.m == -INFINITY) ? 0.f : fast_exp2(st.m - M);
  const float a2 = (m2 == -INFINITY) ? 0.f : fast_exp2(m2 - M);
  st.l = st.l * a1 + l2 * a2;
#pragma unroll
  for (int i = 0; i < kAcc; ++i) st.acc[i] = st.acc[i] * a1 + acc2[i] * a2;
  st.m = M;
}

// LDS slot for one wave's state, element-major so lanes hit consecutive banks.
struct StateSlot {
  f32x4 acc[kAcc][kWave];
  float m[kWave];
  float l[kWave];
};

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

template <bool FP8>
__global__ void __launch_bounds__(kWaves * kWave)
decode_kernel(DecodeArgs a) {
  constexpr int kRowBytes = FP8 ? kD : 2 * kD;
  __shared__ StateSlot slots[2];
  __shared__ int s_last;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int w = tid >> 6;
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
  const int c1 = min(L, c0 + a.chunk);
  const int n_tiles = (c1 - c0 + kTile - 1) / kTile;

  const int64_t row = clamp_i64(a.rpi[b], 0, a.rtt_rows - 1);
  const int64_t* rtt = a.rtt + row * a.rtt_stride;
  const float kscale = FP8 ? a.k_scale[0] : 1.f;
  const float vscale = FP8 ? a.v_scale[0] : 1.f;
  const float sl2 = a.scale_log2 * kscale;

  // Q^T fragments: lane (g, n) holds q[head n][dims of k-step kk].
  u32x4 qf[8];
  {
    const __bf16* qp = a.q + (int64_t)qrow * a.q_stride + (int64_t)hq * kD;
#pragma unroll
    for (int kk = 0; kk < 8; ++kk) {
      const int d0 = FP8 ? (64 * (kk >> 1) + 16 * g + 8 * (kk & 1)) : (32 * kk + 8 * g);
      qf[kk] = head_ok ? ld_g16(qp + d0) : u32x4{0u, 0u, 0u, 0u};
    }
  }

  const uint8_t* kbase = a.k_pool + (int64_t)hk * kRowBytes;
  const uint8_t* vbase = a.v_pool + (int64_t)hk * kRowBytes;
  const int64_t slot_bytes = (int64_t)a.hkv * kRowBytes;

  WaveState st;
  st.m = -INFINITY;
  st.l = 0.f;
#pragma unroll
  for (int i = 0; i < kAcc; ++i) st.acc[i] = f32x4{0.f, 0.f, 0.f, 0.f};

  int it = w;
  int64_t slot_next = 0;
  if (it < n_tiles) slot_next = rtt[min(c0 + it * kTile + n, c1 - 1)];

  for (; it < n_tiles; it += kWaves) {
    const int t0 = c0 + it * kTile;
    const int slot = (int)clamp_i64(slot_next, 0, a.pool_slots - 1);
    if (it + kWaves < n_tiles) slot_next = rtt[min(t0 + kWaves * kTile + n, c1 - 1)];
    int vslot[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) vslot[j] = __shfl(slot, 4 * g + j, kWave);

    // ---- loads: K row of token t0 + n, V rows of tokens t0 + 4g + j
    const uint8_t* kp = kbase + (int64_t)slot * slot_bytes;
    constexpr int kKL = FP8 ? 4 : 8;
    u32x4 kr[kKL];
#pragma unroll
    for (int u = 0; u < kKL; ++u) kr[u] = ld_g16(kp + 64 * u + 16 * g);
    constexpr int kVL = FP8 ? 1 : 2;
    u32x4 vr[4][kVL];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const uint8_t* vp = vbase + (int64_t)vslot[j] * slot_bytes;
#pragma unroll
      for (int s = 0; s < kVL; ++s) vr[j][s] = ld_g16(vp + 16 * n + 256 * s);
    }

    // ---- S^T = K Q^T
    f32x4 sacc = {0.f, 0.f, 0.f, 0.f};
    if (FP8) {
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        sacc = mfma_16x16x32(e4m3x8_to_bf16x8(kr[u][0], kr[u][1]), qf[2 * u], sacc);
        sacc = mfma_16x16x32(e4m3x8_to_bf16x8(kr[u][2], kr[u][3]), qf[2 * u + 1], sacc);
      }
    } else {
#pragma unroll
      for (int kk = 0; kk < 8; ++kk) sacc = mfma_16x16x32(kr[kk], qf[kk], sacc);
    }

    // ---- online softmax for head n over tokens t0 + 4g + r
    float sc[4];
    float mx = -INFINITY;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int t = t0 + 4 * g + r;
      sc[r] = (t < c1) ? sacc[r] * sl2 : -INFINITY;
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
        const uint32_t x = __builtin_amdgcn_perm(vr[1][0][dw], vr[0][0][dw], sel);
        const uint32_t y = __builtin_amdgcn_perm(vr[3][0][dw], vr[2][0][dw], sel);
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
          const u32x2 va = {pair_sel(vr[1][s][dw], vr[0][s][dw], hi),
                            pair_sel(vr[3][s][dw], vr[2][s][dw], hi)};
          st.acc[8 * s + e] = mfma_16x16x16(va, pt, st.acc[8 * s + e]);
        }
      }
    }
  }

  // Row sums were accumulated per lane group; the 4 groups share one head.
  st.l += __shfl_xor(st.l, 16, kWave);
  st.l += __shfl_xor(st.l, 32, kWave);

  block_merge(slots, w, lane, st);

  const int gmax = min(a.group, 16);
  if (n_split == 1) {
    if (w == 0 && head_ok) write_output<FP8>(a, qrow, hq, g, st, vscale);
    return;
  }

  // ---- multi-split: publish this block's partial, last arrival merges.
  const int64_t part = (int64_t)unit * a.max_splits + split;
  if (w == 0 && n < gmax) {
    float* po = a.ws_o + ((part * 16 + n) * 4 + g) * 64;
#pragma unroll
    for (int i = 0; i < kAcc; ++i) reinterpret_cast<f32x4*>(po)[i] = st.acc[i];
    if (g == 0) {
      a.ws_ml[(part * 16 + n) * 2 + 0] = st.m;
      a.ws_ml[(part * 16 + n) * 2 + 1] = st.l;
    }
  }
  __threadfence();
  __syncthreads();
  if (tid == 0) {
    const int prev = atomicAdd(&a.ws_cnt[unit], 1);
    s_last = (prev == n_split - 1);
  }
  __syncthreads();
  if (!s_last) return;
  __threadfence();

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
  if (tid == 0) a.ws_cnt[unit] = 0;
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
  if (chunk_tokens < 0 || chunk_tokens % 64)
    return fail(TF_ERR_INVALID, "decode: chunk_tokens=%d must be a multiple of 64", chunk_tokens);
  const int32_t group = num_q_heads / num_kv_heads;
  p->n_hgroups = (group + 15) / 16;
  p->gmax = group < 16 ? group : 16;
  p->n_units = (int64_t)n_items * num_kv_heads * p->n_hgroups;
  int32_t chunk = chunk_tokens;
  if (chunk == 0) {
    // Aim for ~8 workgroups per CU on a 256-CU part; keep chunks between
    // 256 and 8192 tokens and at most 64 splits per unit.
    const int64_t units = p->n_units > 0 ? p->n_units : 1;
    int64_t want = (2048 + units - 1) / units;
    if (want < 1) want = 1;
    int64_t c = ((int64_t)max_seq_len + want - 1) / want;
    c = (c + 63) / 64 * 64;
    const int64_t floor64 = ((int64_t)max_seq_len + 63) / 64 * 64;
    int64_t lo = 256;
    if (lo > floor64) lo = floor64;
    if (c < lo) c = lo;
    if (c > 8192) c = 8192;
    while ((max_seq_len + c - 1) / c > 64) c += 64;
    chunk = (int32_t)c;
  }
  p->chunk = chunk;
  p->max_splits = (max_seq_len + chunk - 1) / chunk;
  const int64_t parts = p->n_units * p->max_splits;
  p->cnt_bytes = (p->n_units * 4 + 255) / 256 * 256;
  p->ml_bytes = (parts * 16 * 2 * 4 + 255) / 256 * 256;
  p->o_bytes = parts * 16 * (int64_t)kD * 4;
  p->total_bytes = p->max_splits > 1 ? p->cnt_bytes + p->ml_bytes + p->o_bytes : 0;
  return TF_OK;
}

}  // namespace tfa

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

int32_t tf_attn_decode(const void* q, int64_t q_row_stride, const void* k_pool,
                       const void* v_pool, int64_t pool_slots, int32_t kv_dtype,
                       const float* k_scale, const float* v_scale,
                       const int64_t* req_to_token, int64_t rtt_rows,
                       int64_t rtt_row_stride, int64_t rtt_cols,
                       const int64_t* req_pool_indices, const int64_t* seq_lens,
                       int32_t seq_len_override, const int32_t* items,
                       const int32_t* q_rows, int32_t n_items, int32_t num_q_heads,
                       int32_t num_kv_heads, int32_t head_dim, float scale, void* out,
                       int64_t out_row_stride, void* workspace, int64_t workspace_bytes,
                       int32_t max_seq_len, int32_t chunk_tokens, tf_stream_t stream) {
  using namespace tfa;
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
  if (p.total_bytes > 0 && (!workspace || workspace_bytes < p.total_bytes || !aligned16(workspace)))
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
  a.ws_cnt = p.total_bytes ? reinterpret_cast<int32_t*>(ws) : nullptr;
  a.ws_ml = p.total_bytes ? reinterpret_cast<float*>(ws + p.cnt_bytes) : nullptr;
  a.ws_o = p.total_bytes ? reinterpret_cast<float*>(ws + p.cnt_bytes + p.ml_bytes) : nullptr;
  a.chunk = p.chunk;
  a.max_splits = p.max_splits;

  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  if (kv_dtype == TF_DTYPE_FP8_E4M3)
    hipLaunchKernelGGL(decode_kernel<true>, dim3((unsigned)grid), dim3(kWaves * kWave), 0, s, a);
  else
    hipLaunchKernelGGL(decode_kernel<false>, dim3((unsigned)grid), dim3(kWaves * kWave), 0, s, a);
  return launch_status("tf_attn_decode launch");
}

}  // extern "C"
