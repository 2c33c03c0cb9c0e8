// KV scatter-write into the slot pool and the padded slot gather.
//
// tf_kv_write replaces layer_k_buffer[out_cache_loc] = k (and v)
// (qwen3_8/full_attention.py:146-149); for an fp8-e4m3 pool it quantises with
// the per-tensor scale on the way in.  tf_gather_kv is the batched branches'
// gather pool[req_to_token[req_pool_indices, :L].clamp(min=0)]
// (qwen3_8/full_attention.py:216-220), used to check the kernels' gather
// bit-exactly.  Both move whole 16-byte pieces per thread; rows are contiguous
// (one slot = num_kv_heads * head_dim elements).
#include "tf_common.h"
#include "tf_internal.h"

namespace tfa {
namespace {

constexpr int kThreads = 256;

// Clamp to +-448, letting NaN through (as torch.clamp does).
__device__ __forceinline__ float sat448(float x) {
  return x != x ? x : fminf(fmaxf(x, -448.f), 448.f);
}

// fp32 -> e4m3 byte: clamp to +-448 then round to nearest even (gfx950 OCP cvt).
__device__ __forceinline__ uint32_t e4m3x4(float a, float b, float c, float d) {
  a = sat448(a);
  b = sat448(b);
  c = sat448(c);
  d = sat448(d);
  uint32_t r = __builtin_amdgcn_cvt_pk_fp8_f32(a, b, 0u, false);
  r = __builtin_amdgcn_cvt_pk_fp8_f32(c, d, r, true);
  return r;
}

__device__ __forceinline__ float bf16_bits_to_f32(uint32_t half_bits) {
  return __uint_as_float(half_bits << 16);
}

// One thread = 8 consecutive elements of one (token, kv-head-row) source row.
template <int SRC, int DST>
__global__ void __launch_bounds__(kThreads)
kv_write_kernel(const uint8_t* __restrict__ k, const uint8_t* __restrict__ v,
                int64_t src_stride, const int64_t* __restrict__ loc, int64_t n_tokens,
                uint8_t* __restrict__ kp, uint8_t* __restrict__ vp, int64_t pool_slots,
                const float* __restrict__ k_scale, const float* __restrict__ v_scale,
                int64_t row_elems) {
  const int64_t per_tok = row_elems / 8;
  const int64_t idx = (int64_t)blockIdx.x * kThreads + threadIdx.x;
  const int64_t total = n_tokens * per_tok * 2;
  if (idx >= total) return;
  const int which = (int)(idx / (n_tokens * per_tok));  // 0 = K, 1 = V
  const int64_t rem = idx - (int64_t)which * n_tokens * per_tok;
  const int64_t tok = rem / per_tok;
  const int64_t piece = rem - tok * per_tok;
  const int64_t slot = loc[tok];
  if (slot < 0 || slot >= pool_slots) return;
  const uint8_t* src = (which ? v : k);
  uint8_t* dst = (which ? vp : kp);
  constexpr int kSrcBytes = SRC == DT_FP32 ? 4 : 2;
  const uint8_t* s = src + (tok * src_stride + piece * 8) * kSrcBytes;
  float x[8];
  if (SRC == DT_FP32) {
    const f32x4 a = *reinterpret_cast<const f32x4*>(s);
    const f32x4 b = *reinterpret_cast<const f32x4*>(s + 16);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      x[i] = a[i];
      x[4 + i] = b[i];
    }
  } else {
    const u32x4 a = ld_g16(s);
    if (DST == DT_BF16) {  // bf16 -> bf16: bit copy
      *reinterpret_cast<u32x4*>(dst + (slot * row_elems + piece * 8) * 2) = a;
      return;
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      x[2 * i] = bf16_bits_to_f32(a[i] & 0xffffu);
      x[2 * i + 1] = bf16_bits_to_f32(a[i] >> 16);
    }
  }
  if (DST == DT_BF16) {
    u32x4 o;
#pragma unroll
    for (int i = 0; i < 4; ++i) o[i] = pack_bf16(x[2 * i], x[2 * i + 1]);
    *reinterpret_cast<u32x4*>(dst + (slot * row_elems + piece * 8) * 2) = o;
  } else {
    const float sc = which ? v_scale[0] : k_scale[0];
    u32x2 o;
    o[0] = e4m3x4(x[0] / sc, x[1] / sc, x[2] / sc, x[3] / sc);
    o[1] = e4m3x4(x[4] / sc, x[5] / sc, x[6] / sc, x[7] / sc);
    *reinterpret_cast<u32x2*>(dst + slot * row_elems + piece * 8) = o;
  }
}

__global__ void __launch_bounds__(kThreads)
gather_kernel(const uint8_t* __restrict__ pool, int64_t pool_slots, int64_t row_bytes,
              const int64_t* __restrict__ rtt, int64_t rtt_rows, int64_t rtt_stride,
              int64_t rtt_cols, const int64_t* __restrict__ rpi, int32_t max_len,
              int64_t n_pieces, uint8_t* __restrict__ out) {
  const int64_t idx = (int64_t)blockIdx.x * kThreads + threadIdx.x;
  const int64_t per_row = row_bytes / 16;
  if (idx >= n_pieces) return;
  const int64_t row_id = idx / per_row;       // b * max_len + t
  const int64_t piece = idx - row_id * per_row;
  const int64_t b = row_id / max_len;
  const int64_t t = row_id - b * max_len;
  const int64_t r = clamp_i64(rpi[b], 0, rtt_rows - 1);
  int64_t slot = t < rtt_cols ? rtt[r * rtt_stride + t] : 0;
  if (slot < 0) slot = 0;
  if (slot >= pool_slots) slot = pool_slots - 1;
  *reinterpret_cast<u32x4*>(out + row_id * row_bytes + piece * 16) =
      ld_g16(pool + slot * row_bytes + piece * 16);
}

}  // namespace
}  // namespace tfa

extern "C" {

int32_t tf_kv_write(const void* k, const void* v, int64_t src_row_stride, int32_t src_dtype,
                    const int64_t* out_cache_loc, int64_t n_tokens, void* k_pool, void* v_pool,
                    int64_t pool_slots, int32_t kv_dtype, const float* k_scale,
                    const float* v_scale, int32_t num_kv_heads, int32_t head_dim,
                    tf_stream_t stream) {
  using namespace tfa;
  clear_error();
  if (n_tokens < 0) return fail(TF_ERR_INVALID, "kv_write: n_tokens=%lld", (long long)n_tokens);
  if (n_tokens == 0) return TF_OK;
  if (!k || !v || !out_cache_loc || !k_pool || !v_pool)
    return fail(TF_ERR_INVALID, "kv_write: null pointer argument");
  if (num_kv_heads <= 0 || head_dim <= 0 || head_dim % 8)
    return fail(TF_ERR_INVALID, "kv_write: head_dim=%d must be a positive multiple of 8", head_dim);
  if (src_dtype != TF_DTYPE_BF16 && src_dtype != TF_DTYPE_FP32)
    return fail(TF_ERR_UNSUPPORTED, "kv_write: src_dtype=%d", src_dtype);
  if (kv_dtype != TF_DTYPE_BF16 && kv_dtype != TF_DTYPE_FP8_E4M3)
    return fail(TF_ERR_UNSUPPORTED, "kv_write: kv_dtype=%d", kv_dtype);
  if (kv_dtype == TF_DTYPE_FP8_E4M3 && (!k_scale || !v_scale))
    return fail(TF_ERR_INVALID, "kv_write: fp8 pool needs k_scale and v_scale");
  const int64_t row_elems = (int64_t)num_kv_heads * head_dim;
  const int src_bytes = src_dtype == TF_DTYPE_FP32 ? 4 : 2;
  if (src_row_stride < row_elems || (src_row_stride * src_bytes) % 16 || !aligned16(k) ||
      !aligned16(v) || !aligned16(k_pool) || !aligned16(v_pool))
    return fail(TF_ERR_INVALID, "kv_write: sources and pools must be 16-byte aligned rows");
  const int64_t total = n_tokens * (row_elems / 8) * 2;
  const int64_t blocks = (total + kThreads - 1) / kThreads;
  if (blocks > INT32_MAX) return fail(TF_ERR_INVALID, "kv_write: too many tokens");
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  const uint8_t* kk = static_cast<const uint8_t*>(k);
  const uint8_t* vv = static_cast<const uint8_t*>(v);
  uint8_t* kp = static_cast<uint8_t*>(k_pool);
  uint8_t* vp = static_cast<uint8_t*>(v_pool);
#define TF_KVW(S, D)                                                                      \
  hipLaunchKernelGGL((kv_write_kernel<S, D>), dim3((unsigned)blocks), dim3(kThreads), 0, s, \
                     kk, vv, src_row_stride, out_cache_loc, n_tokens, kp, vp, pool_slots,  \
                     k_scale, v_scale, row_elems)
  if (src_dtype == TF_DTYPE_BF16 && kv_dtype == TF_DTYPE_BF16) TF_KVW(DT_BF16, DT_BF16);
  else if (src_dtype == TF_DTYPE_BF16) TF_KVW(DT_BF16, DT_FP8_E4M3);
  else if (kv_dtype == TF_DTYPE_BF16) TF_KVW(DT_FP32, DT_BF16);
  else TF_KVW(DT_FP32, DT_FP8_E4M3);
#undef TF_KVW
  return launch_status("tf_kv_write launch");
}

int32_t tf_gather_kv(const void* pool, int32_t kv_dtype, int64_t pool_slots, int64_t row_elems,
                     const int64_t* req_to_token, int64_t rtt_rows, int64_t rtt_row_stride,
                     int64_t rtt_cols, const int64_t* req_pool_indices, int32_t batch_size,
                     int32_t max_len, void* out, tf_stream_t stream) {
  using namespace tfa;
  clear_error();
  if (batch_size < 0 || max_len < 0) return fail(TF_ERR_INVALID, "gather: negative extent");
  if (batch_size == 0 || max_len == 0) return TF_OK;
  if (!pool || !req_to_token || !req_pool_indices || !out)
    return fail(TF_ERR_INVALID, "gather: null pointer argument");
  int eb;
  if (kv_dtype == TF_DTYPE_BF16) eb = 2;
  else if (kv_dtype == TF_DTYPE_FP8_E4M3) eb = 1;
  else if (kv_dtype == TF_DTYPE_FP32) eb = 4;
  else return fail(TF_ERR_UNSUPPORTED, "gather: kv_dtype=%d", kv_dtype);
  const int64_t row_bytes = row_elems * eb;
  if (row_elems <= 0 || row_bytes % 16 || pool_slots < 1 || rtt_rows < 1 || rtt_cols < 1 ||
      rtt_row_stride < rtt_cols || !aligned16(pool) || !aligned16(out))
    return fail(TF_ERR_INVALID, "gather: rows must be 16-byte multiples and aligned");
  const int64_t n_pieces = (int64_t)batch_size * max_len * (row_bytes / 16);
  const int64_t blocks = (n_pieces + kThreads - 1) / kThreads;
  if (blocks > INT32_MAX) return fail(TF_ERR_INVALID, "gather: too large");
  hipLaunchKernelGGL(gather_kernel, dim3((unsigned)blocks), dim3(kThreads), 0,
                     reinterpret_cast<hipStream_t>(stream), static_cast<const uint8_t*>(pool),
                     pool_slots, row_bytes, req_to_token, rtt_rows, rtt_row_stride, rtt_cols,
                     req_pool_indices, max_len, n_pieces, static_cast<uint8_t*>(out));
  return launch_status("tf_gather_kv launch");
}

}  // extern "C"
