// Fused q/k RMSNorm + partial (M-)RoPE + KV scatter-write.
//
// Replaces, in one pass over the projection outputs, the reference's
//   q = q_norm(q); k = k_norm(k)                 (qwen3_8/full_attention.py:141-142,
//                                                  qwen3_8/rms_norm.py:19-24)
//   q, k = rotary_emb(q, k, positions)           (:143, qwen3_8/rotary_embedding.py:46-95)
//   layer_k_buffer[out_cache_loc] = k; ... = v   (:146-149)
// which are four-plus separate PyTorch ops with a full HBM round trip each.
//
// One workgroup per token; rows are the token's Hq q heads, then its Hkv k
// heads, then its Hkv v heads; a wavefront works on two rows at a time, lane l
// of each half holding elements 8l .. 8l+7 (16-byte loads and stores).
//   q / k rows: x32 = float(x); r = rsqrt(sum(x32^2) / D + eps);
//               y = bf16(w * (x32 * r))                       (rms_norm.py:19-24)
//               for e < rotary_dim, with h = rotary_dim / 2, i = e mod h:
//                 c = bf16(cos(pos_i * inv_freq[i])), s = bf16(sin(...)),
//                 rot = e < h ? -y[e + h] : y[e - h],
//                 y'  = bf16(bf16(y c) + bf16(rot s))         (rotary_embedding.py:84-91)
//               i.e. the rounding steps of the reference's bf16 tensor ops.
//   v rows:     copied.
// M-RoPE (positions [3, T]): frequency i takes its position from row
//   interleaved: 1 if i % 3 == 1 and i < 3 s1, 2 if i % 3 == 2 and i < 3 s2, else 0
//   sectioned:   0 for i < s0, 1 for i < s0 + s1, else 2   (rotary_embedding.py:46-70).
// q rows go to q_out; k / v rows to the pool slot out_cache_loc[t] (bf16, or
// fp8-e4m3 as e4m3(clamp(x / scale, +-448)) with round to nearest even).
// The only difference from the reference's op sequence is the summation order
// of the 256 squares, which can move a normalised value by one bf16 ulp.
#include <math.h>

#include "tf_common.h"
#include "tf_internal.h"

namespace tfa {
namespace {

constexpr int kD = 256;
constexpr int kThreads = 256;
constexpr int kWaves = kThreads / kWave;

struct PrepArgs {
  const __bf16* q;
  int64_t q_tok, q_head;
  const __bf16* k;
  int64_t k_tok;
  const __bf16* v;
  int64_t v_tok;
  int64_t n_tokens;
  int32_t hq, hkv;
  const float* qw;
  const float* kw;
  float eps;
  const int64_t* pos;
  int32_t pos_rows;
  int64_t pos_stride;
  const float* inv_freq;
  int32_t rotary_dim;
  int32_t sec0, sec1, sec2;
  int32_t interleaved;
  __bf16* q_out;
  int64_t q_out_tok;
  const int64_t* loc;
  uint8_t* k_pool;
  uint8_t* v_pool;
  int64_t pool_slots;
  int32_t fp8;
  const float* k_scale;
  const float* v_scale;
};

__device__ __forceinline__ float bf16r(float x) { return (float)(__bf16)x; }

__device__ __forceinline__ float sat448(float x) {
  return x != x ? x : fminf(fmaxf(x, -448.f), 448.f);
}

__device__ __forceinline__ int mrope_row(const PrepArgs& a, int i) {
  if (a.pos_rows == 1) return 0;
  if (a.interleaved) {
    if (i % 3 == 1 && i < 3 * a.sec1) return 1;
    if (i % 3 == 2 && i < 3 * a.sec2) return 2;
    return 0;
  }
  return i < a.sec0 ? 0 : (i < a.sec0 + a.sec1 ? 1 : 2);
}

// One workgroup per token: the bf16 cos / sin of the token's rotary_dim / 2
// frequencies are computed once into LDS; each wave instruction then covers two
// rows (lanes 0-31 and 32-63, 16 bytes = 8 elements per lane), and the 4 waves
// take the token's rows in pairs, all loads of a group issued before use.
constexpr int kRowGroup = 4;   // row pairs per wave in flight

__device__ __forceinline__ const __bf16* row_ptr(const PrepArgs& a, int64_t t, int r) {
  if (r < a.hq) return a.q + t * a.q_tok + (int64_t)r * a.q_head;
  if (r < a.hq + a.hkv) return a.k + t * a.k_tok + (int64_t)(r - a.hq) * kD;
  return a.v + t * a.v_tok + (int64_t)(r - a.hq - a.hkv) * kD;
}

__global__ void __launch_bounds__(kThreads)
qk_prep_kernel(PrepArgs a) {
  // Every product below is rounded (to fp32, or to bf16 where the reference
  // rounds) before it is added: no fused multiply-adds, which would skip the
  // reference's intermediate bf16 rounding of y c and rot s.
#pragma clang fp contract(off)
  __shared__ float cs[2][kD / 2];
  const int lane = threadIdx.x & 63;
  const int l = lane & 31;            // 8 elements 8l .. 8l + 7 of the row
  const int half = lane >> 5;         // which row of the pair
  const int w = wave_id();
  const int64_t t = blockIdx.x;
  const int rows = a.hq + 2 * a.hkv;
  const int h = a.rotary_dim >> 1;

  // First group's loads go out before the cos / sin work.
  u32x4 raw[kRowGroup];
  auto load_group = [&](int g0) {
#pragma unroll
    for (int k = 0; k < kRowGroup; ++k) {
      const int r = 2 * (g0 + kWaves * k) + half;
      if (r < rows) raw[k] = ld_g16(row_ptr(a, t, r) + 8 * l);
    }
  };
  load_group(w);
  for (int i = threadIdx.x; i < h; i += kThreads) {
    const float pf = (float)a.pos[(int64_t)mrope_row(a, i) * a.pos_stride + t];
    const float ang = pf * a.inv_freq[i];
    cs[0][i] = bf16r(cosf(ang));
    cs[1][i] = bf16r(sinf(ang));
  }
  __syncthreads();

  const int64_t slot = a.loc[t];
  const bool slot_ok = slot >= 0 && slot < a.pool_slots;
  const int hl = h >> 3;                        // lanes per rotary half
  const bool rot_lane = l < 2 * hl;
  const int partner = (half << 5) + (l < hl ? l + hl : l - hl);

  for (int g0 = w; 2 * g0 < rows; g0 += kWaves * kRowGroup) {
    if (g0 != w) load_group(g0);
#pragma unroll
    for (int k = 0; k < kRowGroup; ++k) {
      const int r = 2 * (g0 + kWaves * k) + half;
      // Both halves of a wave run the shuffles below together; a half past
      // the last row computes on stale data and stores nothing.
      if (2 * (g0 + kWaves * k) >= rows) break;
      const bool live = r < rows;
      const int kind = !live ? 2 : (r < a.hq ? 0 : (r < a.hq + a.hkv ? 1 : 2));
      const int head = kind == 0 ? r : (kind == 1 ? r - a.hq : r - a.hq - a.hkv);
      float x[8];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        x[2 * j] = __uint_as_float(raw[k][j] << 16);
        x[2 * j + 1] = __uint_as_float(raw[k][j] & 0xffff0000u);
      }
      // q / k rows: RMSNorm then partial RoPE (v rows pass through; the
      // shuffles are executed by every lane so both halves stay converged).
      float ss = 0.f;
#pragma unroll
      for (int j = 0; j < 8; ++j) ss += x[j] * x[j];
#pragma unroll
      for (int m = 16; m >= 1; m >>= 1) ss += __shfl_xor(ss, m, kWave);
      if (kind != 2) {
        const float rs = rsqrtf(ss / (float)kD + a.eps);
        const float* wt = (kind == 0 ? a.qw : a.kw) + 8 * l;
        const f32x4 w0 = *reinterpret_cast<const f32x4*>(wt);
        const f32x4 w1 = *reinterpret_cast<const f32x4*>(wt + 4);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          x[j] = bf16r(w0[j] * (x[j] * rs));
          x[4 + j] = bf16r(w1[j] * (x[4 + j] * rs));
        }
      }
      float p[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) p[j] = __shfl(x[j], rot_lane ? partner : lane, kWave);
      if (kind != 2 && rot_lane) {
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          const int e = 8 * l + j;
          const int i = e < h ? e : e - h;
          const float rot = e < h ? -p[j] : p[j];
          x[j] = bf16r(bf16r(x[j] * cs[0][i]) + bf16r(rot * cs[1][i]));
        }
      }
      if (!live) continue;
      u32x4 o;
#pragma unroll
      for (int j = 0; j < 4; ++j) o[j] = pack_bf16(x[2 * j], x[2 * j + 1]);
      if (kind == 0) {
        *reinterpret_cast<u32x4*>(a.q_out + t * a.q_out_tok + (int64_t)head * kD + 8 * l) = o;
        continue;
      }
      if (!slot_ok) continue;
      uint8_t* pool = kind == 1 ? a.k_pool : a.v_pool;
      const int64_t base = (slot * a.hkv + head) * kD + 8 * l;  // element index
      if (!a.fp8) {
        *reinterpret_cast<u32x4*>(pool + base * 2) = o;
      } else {
        const float sc = kind == 1 ? a.k_scale[0] : a.v_scale[0];
        u32x2 f;
#pragma unroll
        for (int j = 0; j < 2; ++j) {
          uint32_t b4 = __builtin_amdgcn_cvt_pk_fp8_f32(sat448(x[4 * j] / sc),
                                                        sat448(x[4 * j + 1] / sc), 0u, false);
          f[j] = __builtin_amdgcn_cvt_pk_fp8_f32(sat448(x[4 * j + 2] / sc),
                                                 sat448(x[4 * j + 3] / sc), b4, true);
        }
        *reinterpret_cast<u32x2*>(pool + base) = f;
      }
    }
  }
}

}  // namespace
}  // namespace tfa

extern "C" int32_t tf_qk_norm_rope_kv_write(
    const void* q, int64_t q_token_stride, int64_t q_head_stride,
    const void* k, int64_t k_token_stride, const void* v, int64_t v_token_stride,
    int64_t n_tokens, int32_t num_q_heads, int32_t num_kv_heads, int32_t head_dim,
    const float* q_norm_weight, const float* k_norm_weight, float eps,
    const int64_t* positions, int32_t position_rows, int64_t position_row_stride,
    const float* inv_freq, int32_t rotary_dim, int32_t mrope_section0,
    int32_t mrope_section1, int32_t mrope_section2, int32_t mrope_interleaved,
    void* q_out, int64_t q_out_token_stride, const int64_t* out_cache_loc, void* k_pool,
    void* v_pool, int64_t pool_slots, int32_t kv_dtype, const float* k_scale,
    const float* v_scale, tf_stream_t stream) {
  using namespace tfa;
  clear_error();
  if (n_tokens < 0) return fail(TF_ERR_INVALID, "qk_prep: n_tokens=%lld", (long long)n_tokens);
  if (head_dim != kD)
    return fail(TF_ERR_UNSUPPORTED, "qk_prep: head_dim=%d (only %d is built)", head_dim, kD);
  if (num_q_heads <= 0 || num_kv_heads <= 0)
    return fail(TF_ERR_INVALID, "qk_prep: heads %d/%d", num_q_heads, num_kv_heads);
  if (rotary_dim < 0 || rotary_dim > head_dim || rotary_dim % 16)
    return fail(TF_ERR_UNSUPPORTED, "qk_prep: rotary_dim=%d (multiple of 16, <= head_dim)",
                rotary_dim);
  if (position_rows != 1 && position_rows != 3)
    return fail(TF_ERR_INVALID, "qk_prep: position_rows=%d (1 or 3)", position_rows);
  if (position_rows == 3 && (mrope_section0 < 0 || mrope_section1 < 0 || mrope_section2 < 0 ||
                             2 * (mrope_section0 + mrope_section1 + mrope_section2) != rotary_dim))
    return fail(TF_ERR_INVALID, "qk_prep: mrope sections %d+%d+%d must sum to rotary_dim/2",
                mrope_section0, mrope_section1, mrope_section2);
  if (kv_dtype != TF_DTYPE_BF16 && kv_dtype != TF_DTYPE_FP8_E4M3)
    return fail(TF_ERR_UNSUPPORTED, "qk_prep: kv_dtype=%d", kv_dtype);
  if (n_tokens == 0) return TF_OK;
  if (!q || !k || !v || !q_norm_weight || !k_norm_weight || !out_cache_loc || !k_pool ||
      !v_pool || !q_out || (rotary_dim > 0 && (!positions || !inv_freq)))
    return fail(TF_ERR_INVALID, "qk_prep: null pointer argument");
  if (kv_dtype == TF_DTYPE_FP8_E4M3 && (!k_scale || !v_scale))
    return fail(TF_ERR_INVALID, "qk_prep: fp8 pool needs k_scale and v_scale");
  if (!aligned16(q) || !aligned16(k) || !aligned16(v) || !aligned16(q_out) ||
      !aligned16(q_norm_weight) || !aligned16(k_norm_weight) || (q_token_stride % 8) ||
      (q_head_stride % 8) || (k_token_stride % 8) || (v_token_stride % 8) ||
      (q_out_token_stride % 8))
    return fail(TF_ERR_INVALID, "qk_prep: rows and weights must be 16-byte aligned");
  if (q_head_stride < head_dim || k_token_stride < (int64_t)num_kv_heads * head_dim ||
      v_token_stride < (int64_t)num_kv_heads * head_dim ||
      q_out_token_stride < (int64_t)num_q_heads * head_dim ||
      q_token_stride < (int64_t)(num_q_heads - 1) * q_head_stride + head_dim)
    return fail(TF_ERR_INVALID, "qk_prep: strides overlap rows");
  if (pool_slots < 1) return fail(TF_ERR_INVALID, "qk_prep: pool_slots=%lld", (long long)pool_slots);

  PrepArgs a;
  a.q = static_cast<const __bf16*>(q);
  a.q_tok = q_token_stride;
  a.q_head = q_head_stride;
  a.k = static_cast<const __bf16*>(k);
  a.k_tok = k_token_stride;
  a.v = static_cast<const __bf16*>(v);
  a.v_tok = v_token_stride;
  a.n_tokens = n_tokens;
  a.hq = num_q_heads;
  a.hkv = num_kv_heads;
  a.qw = q_norm_weight;
  a.kw = k_norm_weight;
  a.eps = eps;
  a.pos = positions;
  a.pos_rows = position_rows;
  a.pos_stride = position_row_stride;
  a.inv_freq = inv_freq;
  a.rotary_dim = rotary_dim;
  a.sec0 = mrope_section0;
  a.sec1 = mrope_section1;
  a.sec2 = mrope_section2;
  a.interleaved = mrope_interleaved;
  a.q_out = static_cast<__bf16*>(q_out);
  a.q_out_tok = q_out_token_stride;
  a.loc = out_cache_loc;
  a.k_pool = static_cast<uint8_t*>(k_pool);
  a.v_pool = static_cast<uint8_t*>(v_pool);
  a.pool_slots = pool_slots;
  a.fp8 = kv_dtype == TF_DTYPE_FP8_E4M3;
  a.k_scale = k_scale;
  a.v_scale = v_scale;

  if (n_tokens > 0x7fffffff) return fail(TF_ERR_INVALID, "qk_prep: too many tokens");
  hipLaunchKernelGGL(qk_prep_kernel, dim3((unsigned)n_tokens), dim3(kThreads), 0,
                     reinterpret_cast<hipStream_t>(stream), a);
  return launch_status("tf_qk_norm_rope_kv_write launch");
}
