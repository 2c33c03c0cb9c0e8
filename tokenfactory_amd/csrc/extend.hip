// Causal prefill / extend attention over cached prefix + new tokens (bf16 MFMA).
//
// Replaces the reference's extend / mixed branch (qwen3_8/full_attention.py:244-283)
// and the ext_len > 1 case of its bsz == 1 branch (:179-213).  The reference
// pads queries to [B, max_ext, Hq, D], gathers and GQA-expands the whole padded
// context and runs a dense masked SDPA; here each request is processed at its
// own length and nothing is padded or expanded.
//
// Work item (from tf_attn_plan_extend): (request b, kv head hk, row0).  The
// rows of a (b, hk) pair are the ext_b * G flattened (token t, q head h) pairs
// of the kv head's q-head group, row = t * G + h; an item covers 128 of them
// (32 per wave), so all G heads of a GQA group share every K/V tile.
// Row (t, h) attends to context positions 0 .. P + t, P = L - ext.
//
// Per 64-key tile (LDS double-buffered, one barrier per tile):
//   * the next tile's K and V rows are gathered with coalesced 16-byte loads
//     (slot ids come from an LDS slot buffer refilled 1024 keys at a time)
//     before the current tile's MFMAs are issued;
//   * K lands in LDS row-major with chunk c of key k at k*32 + (c ^ (k & 31));
//     V is transposed in registers (8 keys x 8 dims per thread) and lands as
//     V^T rows of 64 keys in the order the PV operand wants, chunk-swizzled;
//   * each wave computes, with v_mfma_f32_32x32x16_bf16,
//       S^T[key, row] = K * Q^T   (Q^T register-resident, K from LDS),
//       the online softmax per row (a row's 64 keys live in lanes n and n + 32),
//       O^T[dim, row] += V^T * P^T (V^T from LDS, P^T straight from S^T),
//     so each lane owns one row: its max, sum and 128 of its output dims.
#include <math.h>

#include "tf_common.h"
#include "tf_internal.h"

namespace tfa {
namespace {

constexpr int kD = 256;
constexpr int kWaves = 4;
constexpr int kThreads = kWaves * kWave;
constexpr int kRowsPerWave = 32;
constexpr int kBN = 64;                     // keys per tile
constexpr int kKChunks = 32;                // 16-byte chunks per K row (512 B)
constexpr int kVChunks = kBN / 8;           // 16-byte chunks per V^T row (64 keys)
constexpr int kSlotChunk = 1024;            // keys per slot-buffer refill
constexpr int kTilesPerSlotChunk = kSlotChunk / kBN;

struct ExtendArgs {
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
  const int32_t* work;
  int32_t hkv, group;
  float scale_log2;
  __bf16* out;
  int64_t out_stride;
};

struct ExtendSmem {
  u32x4 k[2][kBN * kKChunks];      // 2 x 32 KB
  u32x4 vt[2][kD * kVChunks];      // 2 x 32 KB
  int32_t slots[2][kSlotChunk];    // 2 x 4 KB
};

// Key (0..63 within the tile) stored at V^T position p: within each 16-key
// group st, position 8g + j holds key 16st + 8(j/4) + 4g + (j%4), the order of
// the P^T operand taken from the S^T accumulator layout.
__device__ __forceinline__ int key_at_pos(int p) {
  const int st = p >> 4, g = (p >> 3) & 1, j = p & 7;
  return 16 * st + 8 * (j >> 2) + 4 * g + (j & 3);
}

__device__ __forceinline__ int vt_swz(int row) { return (row ^ (row >> 3)) & 7; }

// Registers holding one tile's gathered rows for this thread.
//  K: key 8i + tid/32 (i = 0..7), chunk tid%32 (16 bytes of 32 dims; fp8 half rows)
//  V: keys key_at_pos(8pc + j) (pc = tid/32, j = 0..7), dims 8c..8c+7 (c = tid%32)
template <bool FP8>
struct TileRegs {
  u32x4 k[8];
  u32x4 v[8];   // fp8: 8 bytes per key in .xy
};

template <bool FP8>
__device__ __forceinline__ void issue_tile(const ExtendArgs& a, const int32_t* slots, int key0,
                                           int kend, int hk, int tid, TileRegs<FP8>& r) {
  constexpr int kRowBytes = FP8 ? kD : 2 * kD;
  const int64_t slot_bytes = (int64_t)a.hkv * kRowBytes;
  const uint8_t* kb = a.k_pool + (int64_t)hk * kRowBytes;
  const uint8_t* vb = a.v_pool + (int64_t)hk * kRowBytes;
  const int c = tid & 31;
  const int grp = tid >> 5;
  // Keys past the needed range read the last needed key (valid rows; masked).
  // Key k's slot id sits at slots[k % 2048] (two 1024-key halves).
  const int last = kend - 1;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const int key = min(key0 + 8 * i + grp, last);
    const int64_t s = slots[key & (2 * kSlotChunk - 1)];
    if (FP8) {
      // fp8 rows are 256 B: chunk c covers dims 16(c/2) .. in two halves of 8 B.
      const u32x2 x = ld_g8(kb + s * slot_bytes + 8 * c);
      r.k[i] = u32x4{x[0], x[1], 0u, 0u};
    } else {
      r.k[i] = ld_g16(kb + s * slot_bytes + 16 * c);
    }
  }
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const int key = min(key0 + key_at_pos(8 * grp + j), last);
    const int64_t s = slots[key & (2 * kSlotChunk - 1)];
    if (FP8) {
      const u32x2 x = ld_g8(vb + s * slot_bytes + 8 * c);
      r.v[j] = u32x4{x[0], x[1], 0u, 0u};
    } else {
      r.v[j] = ld_g16(vb + s * slot_bytes + 16 * c);
    }
  }
}

template <bool FP8>
__device__ __forceinline__ void store_tile(u32x4* ks, u32x4* vts, int tid,
                                           const TileRegs<FP8>& r) {
  const int c = tid & 31;
  const int grp = tid >> 5;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const int key = 8 * i + grp;
    u32x4 v = r.k[i];
    if (FP8) {
      // 8 fp8 = dims 8c..8c+7 -> one bf16 chunk (chunk index c).
      v = e4m3x8_to_bf16x8(r.k[i][0], r.k[i][1]);
    }
    ks[key * kKChunks + (c ^ (key & 31))] = v;
  }
  // V: 8 keys (position chunk grp) x 8 dims (8c .. 8c+7) -> 8 V^T rows.
  u32x4 in[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) in[j] = FP8 ? e4m3x8_to_bf16x8(r.v[j][0], r.v[j][1]) : r.v[j];
#pragma unroll
  for (int d = 0; d < 8; ++d) {
    const int dw = d >> 1, hi = d & 1;
    u32x4 o;
#pragma unroll
    for (int w = 0; w < 4; ++w) o[w] = pair_sel(in[2 * w + 1][dw], in[2 * w][dw], hi);
    const int row = 8 * c + d;
    vts[row * kVChunks + (grp ^ vt_swz(row))] = o;
  }
}

// Refills slot buffer (chunk & 1) with the slot ids of keys
// [chunk*1024, chunk*1024 + 1024) clamped to the needed range.
__device__ __forceinline__ void stage_slots(const ExtendArgs& a, const int64_t* rtt, int chunk,
                                            int kend, int tid, int32_t* buf) {
  const int k0 = chunk * kSlotChunk;
  for (int i = tid; i < kSlotChunk; i += kThreads) {
    const int key = min(k0 + i, kend - 1);
    buf[i] = (int32_t)clamp_i64(rtt[key], 0, a.pool_slots - 1);
  }
}

template <bool FP8>
__global__ void __launch_bounds__(kThreads)
extend_kernel(ExtendArgs a) {
  __shared__ __attribute__((aligned(16))) ExtendSmem sm;

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

  int64_t len = a.seq_override > 0 ? (int64_t)a.seq_override : a.seq_lens[b];
  if (len > a.rtt_cols) len = a.rtt_cols;
  const int L = (int)len;
  const int P = L - ext;
  const int rows_total = ext * G;
  if (L <= 0) return;

  const int64_t rrow = clamp_i64(a.rpi[b], 0, a.rtt_rows - 1);
  const int64_t* rtt = a.rtt + rrow * a.rtt_stride;

  // This lane's row.
  const int rho = row0 + kRowsPerWave * w + n;
  const bool row_ok = rho < rows_total;
  const int t = row_ok ? rho / G : ext - 1;
  const int h = row_ok ? rho - t * G : 0;
  const int limit = P + t;  // last visible key

  // Block / wave key extents.
  const int blk_last_row = min(row0 + kWaves * kRowsPerWave, rows_total) - 1;
  const int kend = min(L, P + blk_last_row / G + 1);   // keys [0, kend) are needed
  if (kend <= 0) return;
  const int n_tiles = (kend + kBN - 1) / kBN;
  const int w_first = row0 + kRowsPerWave * w;
  const int w_last = min(w_first + kRowsPerWave, rows_total) - 1;
  const bool wave_active = w_first < rows_total;
  const int w_kend = wave_active ? P + w_last / G + 1 : 0;
  const int w_full = wave_active ? P + w_first / G + 1 : 0;  // keys < w_full: no mask

  const float kscale = FP8 ? a.k_scale[0] : 1.f;
  const float vscale = FP8 ? a.v_scale[0] : 1.f;
  const float sl2 = a.scale_log2 * kscale;

  // Q^T fragments: lane (g, n) holds q[row n][16 kk + 8 g .. +8].  Padding
  // lanes (row_ok false) load a valid row and never write their result.
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

  // ---- prologue: slots of chunk 0, tile 0 into stage 0
  stage_slots(a, rtt, 0, kend, tid, sm.slots[0]);
  __syncthreads();
  TileRegs<FP8> regs;
  issue_tile<FP8>(a, &sm.slots[0][0], 0, kend, hk, tid, regs);
  store_tile<FP8>(sm.k[0], sm.vt[0], tid, regs);
  __syncthreads();

  for (int tile = 0; tile < n_tiles; ++tile) {
    const int k0 = tile * kBN;
    const int st = tile & 1;
    const bool has_next = tile + 1 < n_tiles;
    // Refill the other slot buffer half-way through a slot chunk (visible to
    // every thread after this tile's barrier, long before it is needed).
    if ((tile % kTilesPerSlotChunk) == kTilesPerSlotChunk / 2 &&
        (tile / kTilesPerSlotChunk + 1) * kSlotChunk < kend) {
      const int nc = tile / kTilesPerSlotChunk + 1;
      stage_slots(a, rtt, nc, kend, tid, sm.slots[nc & 1]);
    }
    if (has_next) issue_tile<FP8>(a, &sm.slots[0][0], k0 + kBN, kend, hk, tid, regs);
    __builtin_amdgcn_sched_barrier(0);

    if (wave_active && k0 < w_kend) {
      const u32x4* ks = sm.k[st];
      const u32x4* vts = sm.vt[st];
      // ---- S^T = K Q^T: two 32-key halves; lane holds keys 8(r/4) + 4g + r%4
      f32x16 s[2];
#pragma unroll
      for (int hh = 0; hh < 2; ++hh) {
        s[hh] = f32x16{};
        const int key = 32 * hh + n;
#pragma unroll
        for (int kk = 0; kk < 16; ++kk)
          s[hh] = mfma_32x32x16(ks[key * kKChunks + ((2 * kk + g) ^ (key & 31))], qf[kk], s[hh]);
      }
      const bool need_mask = (k0 + kBN) > w_full;
      float mx = -INFINITY;
#pragma unroll
      for (int hh = 0; hh < 2; ++hh) {
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          float v = s[hh][r] * sl2;
          if (need_mask) {
            const int key = k0 + 32 * hh + 8 * (r >> 2) + 4 * g + (r & 3);
            if (key > limit) v = -INFINITY;
          }
          s[hh][r] = v;
          mx = fmaxf(mx, v);
        }
      }
      mx = wave_max_xor(mx, 32);
      const float mnew = fmaxf(m, mx);
      const float alpha = fast_exp2(m - mnew);
      float psum = 0.f;
#pragma unroll
      for (int hh = 0; hh < 2; ++hh) {
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          s[hh][r] = fast_exp2(s[hh][r] - mnew);
          psum += s[hh][r];
        }
      }
      l = l * alpha + psum;
      m = mnew;
      if (__ballot(alpha != 1.f)) {
#pragma unroll
        for (int i = 0; i < 8; ++i) acc[i] *= alpha;
      }

      // ---- O^T += V^T P^T over four 16-key steps
      u32x4 pt[4];
#pragma unroll
      for (int q4 = 0; q4 < 4; ++q4) {
        const int hh = q4 >> 1, o = 8 * (q4 & 1);
#pragma unroll
        for (int k = 0; k < 4; ++k)
          pt[q4][k] = pack_bf16(s[hh][o + 2 * k], s[hh][o + 2 * k + 1]);
      }
#pragma unroll
      for (int mt = 0; mt < 8; ++mt) {
        const int row = 32 * mt + n;
#pragma unroll
        for (int q4 = 0; q4 < 4; ++q4)
          acc[mt] = mfma_32x32x16(vts[row * kVChunks + ((2 * q4 + g) ^ vt_swz(row))], pt[q4],
                                  acc[mt]);
      }
    }
    __builtin_amdgcn_sched_barrier(0);
    if (has_next) store_tile<FP8>(sm.k[st ^ 1], sm.vt[st ^ 1], tid, regs);
    __syncthreads();
  }

  if (!row_ok) return;
  l += __shfl_xor(l, 32, kWave);
  const float inv = vscale / l;
  __bf16* o = a.out + (int64_t)(q_start + t) * a.out_stride + (int64_t)(hk * G + h) * kD;
#pragma unroll
  for (int mt = 0; mt < 8; ++mt) {
#pragma unroll
    for (int rq = 0; rq < 4; ++rq) {
      const u32x2 v = {pack_bf16(acc[mt][4 * rq + 0] * inv, acc[mt][4 * rq + 1] * inv),
                       pack_bf16(acc[mt][4 * rq + 2] * inv, acc[mt][4 * rq + 3] * inv)};
      *reinterpret_cast<u32x2*>(o + 32 * mt + 8 * rq + 4 * g) = v;
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
                                  int64_t out_row_stride, tf_stream_t stream) {
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
  if (pool_slots < 1 || rtt_rows < 1 || rtt_cols < 1 || rtt_row_stride < rtt_cols)
    return fail(TF_ERR_INVALID, "extend: bad pool/req_to_token extents");
  if (!aligned16(q) || !aligned16(out) || !aligned16(k_pool) || !aligned16(v_pool) ||
      (q_row_stride * 2) % 16 || (out_row_stride * 2) % 16 || !aligned16(work))
    return fail(TF_ERR_INVALID, "extend: q/out/pools/work must be 16-byte aligned");
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

  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  if (kv_dtype == TF_DTYPE_FP8_E4M3)
    hipLaunchKernelGGL(extend_kernel<true>, dim3((unsigned)n_work), dim3(kThreads), 0, s, a);
  else
    hipLaunchKernelGGL(extend_kernel<false>, dim3((unsigned)n_work), dim3(kThreads), 0, s, a);
  return launch_status("tf_attn_extend launch");
}
