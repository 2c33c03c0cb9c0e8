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
// Per 32-key tile the workgroup
//   * gathers the 32 K rows (slot ids from req_to_token) into LDS row-major,
//   * gathers the 32 V rows, transposes 4x8 blocks in registers and stores V^T
//     (dim-major, keys in the order the PV operand wants) into LDS,
// and each wave computes, with v_mfma_f32_32x32x16_bf16,
//   S^T[key, row] = K * Q^T   (Q^T register-resident, K from LDS),
//   online softmax per row (the 32 keys of a row live in lanes n and n + 32),
//   O^T[dim, row] += V^T * P^T (V^T from LDS, P^T from the S^T registers),
// so each lane owns one row: its max, sum and 128 of its output dims.
// The next tile's global loads are issued before the current tile's MFMAs.
#include <math.h>

#include "tf_common.h"
#include "tf_internal.h"

namespace tfa {
namespace {

constexpr int kD = 256;
constexpr int kWaves = 4;
constexpr int kRowsPerWave = 32;
constexpr int kBN = 32;                    // keys per tile
constexpr int kKStride = 2 * kD + 16;      // LDS bytes per K row (padded)
constexpr int kVStride = 2 * kBN + 16;     // LDS bytes per V^T row (padded)
constexpr int kKTile = kBN * kKStride;     // 16896
constexpr int kVTile = kD * kVStride;      // 20480

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

// Key position (within a 32-key tile) held at V^T LDS position `pos`:
// within each 16-key half, 4-key blocks [0,1,2,3] sit at [0,2,1,3].
__device__ __forceinline__ int vt_pos_block(int key_block) {
  const int half = key_block >> 2;
  const int q = key_block & 3;
  return 4 * half + (((q & 1) << 1) | (q >> 1));
}

template <bool FP8>
struct TileRegs {
  // K: bf16 -> 4 x 16B chunks; fp8 -> 2 x 16B chunks (16 e4m3 each).
  u32x4 k[FP8 ? 2 : 4];
  // V: 4 keys x 8 dims: bf16 16B per key; fp8 8B per key (stored in .xy).
  u32x4 v[4];
};

template <bool FP8>
__device__ __forceinline__ void load_tile(const ExtendArgs& a, const int64_t* rtt, int L, int hk,
                                          int k0, int tid, TileRegs<FP8>& r) {
  constexpr int kRowBytes = FP8 ? kD : 2 * kD;
  const int64_t slot_bytes = (int64_t)a.hkv * kRowBytes;
  const uint8_t* kb = a.k_pool + (int64_t)hk * kRowBytes;
  const uint8_t* vb = a.v_pool + (int64_t)hk * kRowBytes;
  const int last = L - 1;
#pragma unroll
  for (int it = 0; it < (FP8 ? 2 : 4); ++it) {
    const int key = FP8 ? (it * 16 + (tid >> 4)) : (it * 8 + (tid >> 5));
    const int c = FP8 ? (tid & 15) : (tid & 31);
    const int64_t slot = clamp_i64(rtt[min(k0 + key, last)], 0, a.pool_slots - 1);
    r.k[it] = ld_g16(kb + slot * slot_bytes + 16 * c);
  }
  const int kg = tid >> 5;
  const int c = tid & 31;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const int64_t slot = clamp_i64(rtt[min(k0 + 4 * kg + e, last)], 0, a.pool_slots - 1);
    const uint8_t* vp = vb + slot * slot_bytes;
    if (FP8) {
      const u32x2 x = ld_g8(vp + 8 * c);
      r.v[e] = u32x4{x[0], x[1], 0u, 0u};
    } else {
      r.v[e] = ld_g16(vp + 16 * c);
    }
  }
}

template <bool FP8>
__device__ __forceinline__ void store_tile(char* kt, char* vt, int tid, const TileRegs<FP8>& r) {
#pragma unroll
  for (int it = 0; it < (FP8 ? 2 : 4); ++it) {
    if (FP8) {
      const int key = it * 16 + (tid >> 4);
      const int c = tid & 15;
      char* p = kt + key * kKStride + 32 * c;
      st_s16(p, e4m3x8_to_bf16x8(r.k[it][0], r.k[it][1]));
      st_s16(p + 16, e4m3x8_to_bf16x8(r.k[it][2], r.k[it][3]));
    } else {
      const int key = it * 8 + (tid >> 5);
      const int c = tid & 31;
      st_s16(kt + key * kKStride + 16 * c, r.k[it]);
    }
  }
  const int kg = tid >> 5;
  const int c = tid & 31;
  u32x4 v[4];
#pragma unroll
  for (int e = 0; e < 4; ++e) v[e] = FP8 ? e4m3x8_to_bf16x8(r.v[e][0], r.v[e][1]) : r.v[e];
  char* base = vt + 8 * vt_pos_block(kg);
#pragma unroll
  for (int d = 0; d < 8; ++d) {
    const int dw = d >> 1;
    const int hi = d & 1;
    const u32x2 x = {pair_sel(v[1][dw], v[0][dw], hi), pair_sel(v[3][dw], v[2][dw], hi)};
    st_s8(base + (8 * c + d) * kVStride, x);
  }
}

template <bool FP8>
__global__ void __launch_bounds__(kWaves * kWave)
extend_kernel(ExtendArgs a) {
  __shared__ __attribute__((aligned(16))) char smem[kKTile + kVTile];
  char* kt = smem;
  char* vt = smem + kKTile;

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
  const int kend = P + blk_last_row / G + 1;  // keys [0, kend) are needed
  const int n_tiles = (kend + kBN - 1) / kBN;
  const int w_first = row0 + kRowsPerWave * w;
  const int w_last = min(w_first + kRowsPerWave, rows_total) - 1;
  const bool wave_active = w_first < rows_total;
  const int w_kend = wave_active ? P + w_last / G + 1 : 0;
  const int w_full = wave_active ? P + w_first / G + 1 : 0;  // keys < w_full: no mask

  const float kscale = FP8 ? a.k_scale[0] : 1.f;
  const float vscale = FP8 ? a.v_scale[0] : 1.f;
  const float sl2 = a.scale_log2 * kscale;

  // Q^T fragments: lane (g, n) holds q[row n][16 kk + 8 g .. +8].
  u32x4 qf[16];
  {
    const __bf16* qp = a.q + (int64_t)(q_start + t) * a.q_stride + (int64_t)(hk * G + h) * kD;
#pragma unroll
    for (int kk = 0; kk < 16; ++kk)
      qf[kk] = row_ok ? ld_g16(qp + 16 * kk + 8 * g) : u32x4{0u, 0u, 0u, 0u};
  }

  float m = -INFINITY;
  float l = 0.f;
  f32x16 acc[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) acc[i] = f32x16{};

  TileRegs<FP8> regs;
  load_tile<FP8>(a, rtt, L, hk, 0, tid, regs);

  for (int tile = 0; tile < n_tiles; ++tile) {
    const int k0 = tile * kBN;
    __syncthreads();  // previous tile's LDS reads are done
    store_tile<FP8>(kt, vt, tid, regs);
    __syncthreads();
    if (tile + 1 < n_tiles) load_tile<FP8>(a, rtt, L, hk, k0 + kBN, tid, regs);

    if (!wave_active || k0 >= w_kend) continue;

    // ---- S^T = K Q^T : lane holds keys 8(r/4) + 4g + r%4 of row n
    f32x16 s = {};
#pragma unroll
    for (int kk = 0; kk < 16; ++kk) {
      const u32x4 kf = ld_s16(kt + n * kKStride + 32 * kk + 16 * g);
      s = mfma_32x32x16(kf, qf[kk], s);
    }
    const bool need_mask = (k0 + kBN) > w_full;
    float mx = -INFINITY;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      float v = s[r] * sl2;
      if (need_mask) {
        const int key = k0 + 8 * (r >> 2) + 4 * g + (r & 3);
        if (key > limit) v = -INFINITY;
      }
      s[r] = v;
      mx = fmaxf(mx, v);
    }
    mx = wave_max_xor(mx, 32);
    const float mnew = fmaxf(m, mx);
    const float alpha = fast_exp2(m - mnew);
    float psum = 0.f;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      s[r] = fast_exp2(s[r] - mnew);
      psum += s[r];
    }
    l = l * alpha + psum;
    m = mnew;
    if (__ballot(alpha != 1.f)) {
#pragma unroll
      for (int i = 0; i < 8; ++i) acc[i] *= alpha;
    }

    // ---- O^T += V^T P^T
    u32x4 pt[2];
#pragma unroll
    for (int st = 0; st < 2; ++st)
#pragma unroll
      for (int k = 0; k < 4; ++k) pt[st][k] = pack_bf16(s[8 * st + 2 * k], s[8 * st + 2 * k + 1]);
#pragma unroll
    for (int mt = 0; mt < 8; ++mt) {
#pragma unroll
      for (int st = 0; st < 2; ++st) {
        const u32x4 vf = ld_s16(vt + (32 * mt + n) * kVStride + 32 * st + 16 * g);
        acc[mt] = mfma_32x32x16(vf, pt[st], acc[mt]);
      }
    }
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
    hipLaunchKernelGGL(extend_kernel<true>, dim3((unsigned)n_work), dim3(kWaves * kWave), 0, s, a);
  else
    hipLaunchKernelGGL(extend_kernel<false>, dim3((unsigned)n_work), dim3(kWaves * kWave), 0, s, a);
  return launch_status("tf_attn_extend launch");
}
