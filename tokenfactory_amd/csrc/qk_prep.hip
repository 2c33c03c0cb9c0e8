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

// One wave per token, four waves per workgroup.  A token's rows (Hq q heads,
// then Hkv k heads, then Hkv v heads) are taken 8 at a time ("groups"): lane l
// works on row 8g + l / 8 and, in load j (j = 0..3), on the 8 elements
// 64 j + 8 (l % 8) .. +7 of it, so one 16-byte load per lane covers 8 rows and
// a row's sum of squares is reduced over 8 lanes with three DPP steps.  The
// rotary part of every row (its first rotary_dim elements) then fills whole
// loads, so the RoPE arithmetic runs on full waves; the rotate-half partner
// of a chunk comes from a wave-private LDS copy of the normalised rows.  The
// bf16 cos / sin of the token's rotary_dim / 2 frequencies are computed once
// per token (one sincos per lane) into a wave-private LDS table.  The loads of
// two groups (8 KB) are issued before either is used; the projection rows are
// read once and the outputs written once, so both go through non-temporal
// accesses (streaming, no cache reuse: 147 -> 136 us on a 20k-token step).
constexpr int kGroupsInFlight = 2;
constexpr int kChunks = kD / 8;                 // 16-byte chunks per row

struct PrepSmem {
  float w[2][kD];                                 // q_norm, k_norm weights
  float tab[kWaves][2][kD / 2];                   // bf16 cos, sin per frequency
  u32x4 rows[kWaves][8][kChunks];                 // normalised rows (RoPE partners)
};

__device__ __forceinline__ const __bf16* row_ptr(const PrepArgs& a, int64_t t, int r) {
  if (r < a.hq) return a.q + t * a.q_tok + (int64_t)r * a.q_head;
  if (r < a.hq + a.hkv) return a.k + t * a.k_tok + (int64_t)(r - a.hq) * kD;
  return a.v + t * a.v_tok + (int64_t)(r - a.hq - a.hkv) * kD;
}

__device__ __forceinline__ void unpack8(const u32x4& r, float (&x)[8]) {
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    x[2 * k] = __uint_as_float(r[k] << 16);
    x[2 * k + 1] = __uint_as_float(r[k] & 0xffff0000u);
  }
}

__device__ __forceinline__ u32x4 pack8(const float (&x)[8]) {
  u32x4 o;
#pragma unroll
  for (int k = 0; k < 4; ++k) o[k] = pack_bf16(x[2 * k], x[2 * k + 1]);
  return o;
}

__global__ void __launch_bounds__(kThreads)
qk_prep_kernel(PrepArgs a) {
  // Every product below is rounded (to fp32, or to bf16 where the reference
  // rounds) before it is added: no fused multiply-adds, which would skip the
  // reference's intermediate bf16 rounding of y c and rot s.
#pragma clang fp contract(off)
  __shared__ PrepSmem sm;
  const int lane = threadIdx.x & 63;
  const int w = wave_id();
  const int rsub = lane >> 3;         // row of the group
  const int col = lane & 7;           // chunk column: chunk 8 j + col in load j
  const int rows = a.hq + 2 * a.hkv;
  const int n_groups = (rows + 7) >> 3;
  const int h = a.rotary_dim >> 1;
  const int hc = h >> 3;              // rotary chunks per half
  const int rot_loads = (a.rotary_dim + 63) >> 6;

  for (int i = threadIdx.x; i < 2 * kD; i += kThreads)
    sm.w[i / kD][i % kD] = (i < kD ? a.qw : a.kw)[i % kD];
  __syncthreads();

  for (int64_t t = (int64_t)blockIdx.x * kWaves + w; t < a.n_tokens;
       t += (int64_t)gridDim.x * kWaves) {
    const int64_t slot = a.loc[t];
    const bool slot_ok = slot >= 0 && slot < a.pool_slots;
    for (int g0 = 0; g0 < n_groups; g0 += kGroupsInFlight) {
      u32x4 raw[kGroupsInFlight][4];
#pragma unroll
      for (int gi = 0; gi < kGroupsInFlight; ++gi) {
        const int r = 8 * (g0 + gi) + rsub;
        if (g0 + gi < n_groups && r < rows) {
          const __bf16* src = row_ptr(a, t, r) + 8 * col;
#pragma unroll
          for (int j = 0; j < 4; ++j) raw[gi][j] = ld_nt16(src + 64 * j);
        }
      }
      if (g0 == 0) {
        // The token's cos / sin table, while the loads are in flight.
        for (int i = lane; i < h; i += kWave) {
          const float pf = (float)a.pos[(int64_t)mrope_row(a, i) * a.pos_stride + t];
          float sn, cs;
          sincosf(pf * a.inv_freq[i], &sn, &cs);
          sm.tab[w][0][i] = bf16r(cs);
          sm.tab[w][1][i] = bf16r(sn);
        }
      }
#pragma unroll
      for (int gi = 0; gi < kGroupsInFlight; ++gi) {
        if (g0 + gi >= n_groups) break;
        const int r = 8 * (g0 + gi) + rsub;
        const bool live = r < rows;
        const int kind = !live ? 2 : (r < a.hq ? 0 : (r < a.hq + a.hkv ? 1 : 2));
        const int head = kind == 0 ? r : (kind == 1 ? r - a.hq : r - a.hq - a.hkv);
        u32x4 o[4];
        if (kind == 2) {
#pragma unroll
          for (int j = 0; j < 4; ++j) o[j] = raw[gi][j];
        } else {
          float x[4][8];
          float ss = 0.f;
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            unpack8(raw[gi][j], x[j]);
#pragma unroll
            for (int k = 0; k < 8; ++k) ss += x[j][k] * x[j][k];
          }
          ss = row_sum8(ss);
          const float rs = rsqrtf(ss / (float)kD + a.eps);
          const float* wt = sm.w[kind] + 8 * col;
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            const f32x4 w0 = *reinterpret_cast<const f32x4*>(wt + 64 * j);
            const f32x4 w1 = *reinterpret_cast<const f32x4*>(wt + 64 * j + 4);
#pragma unroll
            for (int k = 0; k < 4; ++k) {
              x[j][k] = bf16r(w0[k] * (x[j][k] * rs));
              x[j][4 + k] = bf16r(w1[k] * (x[j][4 + k] * rs));
            }
            o[j] = pack8(x[j]);
          }
          // RoPE on the rotary chunks: chunk c pairs with c + hc (c < hc) or
          // c - hc, element 8c + k with frequency (8c + k) mod h.
          if (rot_loads > 0) {
#pragma unroll
            for (int j = 0; j < 4; ++j)
              if (j < rot_loads && 8 * j + col < 2 * hc) sm.rows[w][rsub][8 * j + col] = o[j];
#pragma unroll
            for (int j = 0; j < 4; ++j) {
              const int c = 8 * j + col;
              if (j < rot_loads && c < 2 * hc) {
                const bool lo = c < hc;
                float pv[8];
                unpack8(sm.rows[w][rsub][lo ? c + hc : c - hc], pv);
                const int i0 = 8 * (lo ? c : c - hc);
                const f32x4 c0 = *reinterpret_cast<const f32x4*>(&sm.tab[w][0][i0]);
                const f32x4 c1 = *reinterpret_cast<const f32x4*>(&sm.tab[w][0][i0 + 4]);
                const f32x4 s0 = *reinterpret_cast<const f32x4*>(&sm.tab[w][1][i0]);
                const f32x4 s1 = *reinterpret_cast<const f32x4*>(&sm.tab[w][1][i0 + 4]);
#pragma unroll
                for (int k = 0; k < 8; ++k) {
                  const float cv = k < 4 ? c0[k] : c1[k - 4];
                  const float sv = k < 4 ? s0[k] : s1[k - 4];
                  const float rot = lo ? -pv[k] : pv[k];
                  x[j][k] = bf16r(bf16r(x[j][k] * cv) + bf16r(rot * sv));
                }
                o[j] = pack8(x[j]);
              }
            }
          }
        }
        if (!live) continue;
        if (kind == 0) {
          __bf16* dst = a.q_out + t * a.q_out_tok + (int64_t)head * kD + 8 * col;
#pragma unroll
          for (int j = 0; j < 4; ++j)
            __builtin_nontemporal_store(o[j], reinterpret_cast<u32x4*>(dst + 64 * j));
          continue;
        }
        if (!slot_ok) continue;
        uint8_t* pool = kind == 1 ? a.k_pool : a.v_pool;
        const int64_t base = (slot * a.hkv + head) * kD + 8 * col;   // element index
        if (!a.fp8) {
#pragma unroll
          for (int j = 0; j < 4; ++j)
            __builtin_nontemporal_store(o[j], reinterpret_cast<u32x4*>(pool + (base + 64 * j) * 2));
        } else {
          const float sc = kind == 1 ? a.k_scale[0] : a.v_scale[0];
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            float x[8];
            unpack8(o[j], x);
            u32x2 f;
#pragma unroll
            for (int q = 0; q < 2; ++q) {
              const uint32_t b4 = __builtin_amdgcn_cvt_pk_fp8_f32(
                  sat448(x[4 * q] / sc), sat448(x[4 * q + 1] / sc), 0u, false);
              f[q] = __builtin_amdgcn_cvt_pk_fp8_f32(sat448(x[4 * q + 2] / sc),
                                                     sat448(x[4 * q + 3] / sc), b4, true);
            }
            __builtin_nontemporal_store(f, reinterpret_cast<u32x2*>(pool + base + 64 * j));
          }
        }
      }
    }
  }
}

// head_dim other than 256 (a multiple of 8, at most 256): one wave per (token,
// row), lane l holding elements l, l + 64, ...; the rotate-half partner comes
// from a wave-private LDS copy of the normalised row and each rotary element's
// cos / sin is evaluated where it is used.  Same rounding steps as above.
constexpr int kGenRowMax = 256;

__global__ void __launch_bounds__(kThreads)
qk_prep_generic_kernel(PrepArgs a, int D) {
#pragma clang fp contract(off)
  __shared__ float rowbuf[kWaves][kGenRowMax];
  const int lane = threadIdx.x & 63;
  const int w = threadIdx.x / kWave;
  const int rows = a.hq + 2 * a.hkv;
  const int64_t wid = (int64_t)blockIdx.x * kWaves + w;
  if (wid >= a.n_tokens * rows) return;
  const int64_t t = wid / rows;
  const int r = (int)(wid - t * rows);
  const int kind = r < a.hq ? 0 : (r < a.hq + a.hkv ? 1 : 2);
  const int head = kind == 0 ? r : (kind == 1 ? r - a.hq : r - a.hq - a.hkv);
  const __bf16* src = kind == 0 ? a.q + t * a.q_tok + (int64_t)head * a.q_head
                                : (kind == 1 ? a.k + t * a.k_tok : a.v + t * a.v_tok) +
                                      (int64_t)head * D;
  const int h = a.rotary_dim >> 1;
  float y[kGenRowMax / kWave];
#pragma unroll
  for (int i = 0; i < kGenRowMax / kWave; ++i) {
    const int e = lane + kWave * i;
    y[i] = e < D ? (float)src[e] : 0.f;
  }
  if (kind != 2) {
    float ss = 0.f;
#pragma unroll
    for (int i = 0; i < kGenRowMax / kWave; ++i) ss += y[i] * y[i];
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) ss += __shfl_xor(ss, m, kWave);
    const float rs = rsqrtf(ss / (float)D + a.eps);
    const float* wt = kind == 0 ? a.qw : a.kw;
#pragma unroll
    for (int i = 0; i < kGenRowMax / kWave; ++i) {
      const int e = lane + kWave * i;
      if (e < D) y[i] = bf16r(wt[e] * (y[i] * rs));
    }
    if (h > 0) {
#pragma unroll
      for (int i = 0; i < kGenRowMax / kWave; ++i) {
        const int e = lane + kWave * i;
        if (e < D) rowbuf[w][e] = y[i];
      }
#pragma unroll
      for (int i = 0; i < kGenRowMax / kWave; ++i) {
        const int e = lane + kWave * i;
        if (e < 2 * h) {
          const int f = e < h ? e : e - h;
          const float pf = (float)a.pos[(int64_t)mrope_row(a, f) * a.pos_stride + t];
          float sn, cs;
          sincosf(pf * a.inv_freq[f], &sn, &cs);
          const float rot = e < h ? -rowbuf[w][e + h] : rowbuf[w][e - h];
          y[i] = bf16r(bf16r(y[i] * bf16r(cs)) + bf16r(rot * bf16r(sn)));
        }
      }
    }
  }
  if (kind == 0) {
    __bf16* dst = a.q_out + t * a.q_out_tok + (int64_t)head * D;
#pragma unroll
    for (int i = 0; i < kGenRowMax / kWave; ++i) {
      const int e = lane + kWave * i;
      if (e < D) dst[e] = (__bf16)y[i];
    }
    return;
  }
  const int64_t slot = a.loc[t];
  if (slot < 0 || slot >= a.pool_slots) return;
  const int64_t base = (slot * a.hkv + head) * D;   // element index
  uint8_t* pool = kind == 1 ? a.k_pool : a.v_pool;
  const float sc = a.fp8 ? (kind == 1 ? a.k_scale[0] : a.v_scale[0]) : 1.f;
#pragma unroll
  for (int i = 0; i < kGenRowMax / kWave; ++i) {
    const int e = lane + kWave * i;
    if (e >= D) continue;
    if (a.fp8) {
      pool[base + e] = (uint8_t)(__builtin_amdgcn_cvt_pk_fp8_f32(sat448(y[i] / sc), 0.f, 0u,
                                                                 false) & 0xffu);
    } else {
      reinterpret_cast<__bf16*>(pool)[base + e] = (__bf16)y[i];
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
  if (head_dim < 8 || head_dim > kD || head_dim % 8)
    return fail(TF_ERR_UNSUPPORTED, "qk_prep: head_dim=%d (a multiple of 8 up to %d)", head_dim,
                kD);
  if (num_q_heads <= 0 || num_kv_heads <= 0)
    return fail(TF_ERR_INVALID, "qk_prep: heads %d/%d", num_q_heads, num_kv_heads);
  if (rotary_dim < 0 || rotary_dim > head_dim || rotary_dim % 2 ||
      (head_dim == kD && rotary_dim % 16))
    return fail(TF_ERR_UNSUPPORTED,
                "qk_prep: rotary_dim=%d (even, <= head_dim; a multiple of 16 for head_dim %d)",
                rotary_dim, kD);
  if (position_rows != 1 && position_rows != 3)
    return fail(TF_ERR_INVALID, "qk_prep: position_rows=%d (1 or 3)", position_rows);
  // Sectioned M-RoPE splits the frequencies into the three sections
  // (rotary_embedding.py:64-70 splits them, so they must add up); the
  // interleaved layout takes any sections (:58-63).
  if (position_rows == 3 &&
      (mrope_section0 < 0 || mrope_section1 < 0 || mrope_section2 < 0 ||
       (!mrope_interleaved &&
        2 * (mrope_section0 + mrope_section1 + mrope_section2) != rotary_dim)))
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

  if (head_dim != kD) {   // one wave per (token, row)
    const int64_t waves = n_tokens * (num_q_heads + 2 * num_kv_heads);
    const int64_t gblocks = (waves + kWaves - 1) / kWaves;
    if (gblocks > INT32_MAX) return fail(TF_ERR_INVALID, "qk_prep: too many tokens");
    hipLaunchKernelGGL(qk_prep_generic_kernel, dim3((unsigned)gblocks), dim3(kThreads), 0,
                       reinterpret_cast<hipStream_t>(stream), a, (int)head_dim);
    return launch_status("tf_qk_norm_rope_kv_write launch");
  }
  // One token per wave, four per workgroup.
  const int64_t blocks = (n_tokens + kWaves - 1) / kWaves;
  if (blocks > INT32_MAX) return fail(TF_ERR_INVALID, "qk_prep: too many tokens");
  hipLaunchKernelGGL(qk_prep_kernel, dim3((unsigned)blocks), dim3(kThreads), 0,
                     reinterpret_cast<hipStream_t>(stream), a);
  return launch_status("tf_qk_norm_rope_kv_write launch");
}
