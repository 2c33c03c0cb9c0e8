// Gated DeltaNet decode step: the linear-attention layers' one-token update.
//
// Replaces Qwen3_8LinearAttention._batched_decode_step
// (qwen3_8/linear_attention.py:244-298) and the gated RMSNorm after it
// (:325, qwen3_8/rms_norm_gated.py:26-40), for a batch whose requests all
// extend by one token.  Per request b (state slot r = req_indices[b]):
//   causal conv:  y_c = bf16(silu(bf16(sum_i w[c][i] * [state_c, qkv_c][i])))
//                 state_c <- [state_c[1:], qkv_c]                     (:258-269)
//   q, k, v = split(y); q = normalize(q) * dk^-0.5, k = normalize(k)  (:279-280)
//   per value head h (key head h / (Hv / Hk), repeat_interleave):    (:281-297)
//     alpha = exp(-exp(A_log) * softplus(a + dt_bias)), beta = sigmoid(b)
//     S = alpha * S;  delta = beta * (v - S^T k);  S += k delta^T;  o = S^T q
//   out = bf16(norm_w * (o / rms(o)) * silu(z)) per head, o rounded to bf16
//   first                                                 (rms_norm_gated.py:26-40)
// The recurrent state S[slot][h] is a 128 x 128 fp32 matrix (key rows, value
// columns) updated in place; the conv state is bf16 [slot][channel][3].
//
// Two launches.  gdn_conv_kernel: one thread per (request, channel) runs the
// conv step, writes the bf16 SiLU output to a workspace row and shifts the conv
// state.  gdn_recur_kernel: one 256-thread workgroup per (request, value head)
// normalises its q / k from the workspace, streams the head's 64 KB state
// through registers once (thread t holds columns 4 (t % 32) .. + 3 of rows
// t / 32 + 8 i), reduces S^T k and S^T q over the rows through LDS and applies
// the gated norm to the whole head.  HBM-bound: 128 KB of state traffic per
// value head and request.
#include <math.h>

#include "tf_common.h"
#include "tf_internal.h"

namespace tfa {
namespace {

constexpr int kDk = 128;
constexpr int kDv = 128;
constexpr int kThreads = 256;
constexpr int kRowGroups = kThreads / 32;   // 8 row groups of 16 rows

struct GdnArgs {
  const uint16_t* qkv;   // bf16 [B, conv_dim]
  int64_t qkv_rs;
  const uint16_t* a;     // bf16 [B, Hv]
  const uint16_t* b;
  int64_t ab_rs;
  const uint16_t* z;     // bf16 [B, Hv * Dv]
  int64_t z_rs;
  const float* conv_w;   // fp32 [conv_dim, 4]
  const float* a_log;    // fp32 [Hv]
  const float* dt_bias;  // fp32 [Hv]
  const float* norm_w;   // fp32 [Hv * Dv]
  float eps;
  uint16_t* conv_state;  // bf16 [slots, conv_dim, 3]
  int64_t conv_ss;
  float* ssm;            // fp32 [slots, Hv, Dk, Dv]
  int64_t ssm_ss;
  const int64_t* req;
  int64_t n_slots;
  int32_t batch, hv, vpk, key_dim, conv_dim;
  uint16_t* ws;          // bf16 [B, conv_dim]: conv + SiLU outputs
  uint16_t* out;         // bf16 [B, Hv * Dv]
  int64_t out_rs;
  uint16_t* core;        // optional bf16 [B, Hv * Dv]: o before the norm
  int64_t core_rs;
};

__device__ __forceinline__ float bf(uint16_t u) { return __uint_as_float((uint32_t)u << 16); }
__device__ __forceinline__ uint16_t to_bf(float x) {
  return (uint16_t)(pack_bf16(x, 0.f) & 0xffffu);
}
__device__ __forceinline__ float round_bf(float x) { return bf(to_bf(x)); }

// Sum over the 128 threads 0..127 (waves 0 and 1); every thread gets it.
__device__ __forceinline__ float sum128(float v, float* red) {
#pragma unroll
  for (int d = 32; d >= 1; d >>= 1) v += __shfl_xor(v, d, kWave);
  const int w = threadIdx.x / kWave;
  if ((threadIdx.x & (kWave - 1)) == 0) red[w] = v;
  __syncthreads();
  const float s = red[0] + red[1];
  __syncthreads();
  return s;
}

__global__ void __launch_bounds__(kThreads) gdn_conv_kernel(GdnArgs a) {
  const int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x;
  const int bi = (int)(i / a.conv_dim), c = (int)(i - (int64_t)bi * a.conv_dim);
  if (bi >= a.batch) return;
  const int64_t r = a.req[bi];
  if (r < 0 || r >= a.n_slots) return;
  uint16_t* st = a.conv_state + r * a.conv_ss + 3 * (int64_t)c;
  const uint16_t x0 = st[0], x1 = st[1], x2 = st[2];
  const uint16_t x3 = a.qkv[bi * a.qkv_rs + c];
  const f32x4 w = *reinterpret_cast<const f32x4*>(a.conv_w + 4 * (int64_t)c);
  const float acc = w[0] * bf(x0) + w[1] * bf(x1) + w[2] * bf(x2) + w[3] * bf(x3);
  const float y = round_bf(acc);                               // conv1d output (bf16)
  a.ws[(int64_t)bi * a.conv_dim + c] = to_bf(y / (1.f + expf(-y)));   // F.silu on bf16
  st[0] = x1;
  st[1] = x2;
  st[2] = x3;
}

__global__ void __launch_bounds__(kThreads) gdn_recur_kernel(GdnArgs a) {
  __shared__ float s_q[kDk], s_k[kDk];
  __shared__ float s_red[kRowGroups][kDv];
  __shared__ float s_sum[4];
  const int bi = blockIdx.x / a.hv, h = blockIdx.x % a.hv;
  const int hk = h / a.vpk;
  const int t = threadIdx.x;
  const int64_t r = a.req[bi];
  if (r < 0 || r >= a.n_slots) return;   // a slot outside the pool: no work, no output
  const uint16_t* y = a.ws + (int64_t)bi * a.conv_dim;

  // The state loads go out first; q / k normalisation runs under their latency.
  const int d0 = 4 * (t & 31), g = t >> 5;
  float* S = a.ssm + r * a.ssm_ss + (int64_t)h * kDk * kDv;
  f32x4 s[16];
#pragma unroll
  for (int i = 0; i < 16; ++i)
    s[i] = *reinterpret_cast<const f32x4*>(S + (g + kRowGroups * i) * kDv + d0);

  // q = normalize(q) * dk^-0.5, k = normalize(k)  (F.normalize, eps 1e-12)
  {
    const float x = bf(t < kDk ? y[hk * kDk + t] : y[a.key_dim + hk * kDk + (t - kDk)]);
    float v = x * x;
#pragma unroll
    for (int d = 32; d >= 1; d >>= 1) v += __shfl_xor(v, d, kWave);
    if ((t & (kWave - 1)) == 0) s_sum[t / kWave] = v;
    __syncthreads();
    const float n = sqrtf(t < kDk ? s_sum[0] + s_sum[1] : s_sum[2] + s_sum[3]);
    const float xn = x / fmaxf(n, 1e-12f);
    if (t < kDk)
      s_q[t] = xn * 0.08838834764831845f;   // 128 ** -0.5
    else
      s_k[t - kDk] = xn;
    __syncthreads();
  }

  const float x = bf(a.a[bi * a.ab_rs + h]) + a.dt_bias[h];
  const float sp = x > 20.f ? x : log1pf(expf(x));           // F.softplus
  const float alpha = expf(-expf(a.a_log[h]) * sp);
  const float beta = 1.f / (1.f + expf(-bf(a.b[bi * a.ab_rs + h])));

  f32x4 vp = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const int k = g + kRowGroups * i;
    s[i] *= alpha;
    vp += s[i] * s_k[k];
  }
  *reinterpret_cast<f32x4*>(&s_red[g][d0]) = vp;
  __syncthreads();
  const uint16_t* vrow = y + 2 * a.key_dim + h * kDv + d0;
  f32x4 delta;
#pragma unroll
  for (int c = 0; c < 4; ++c) {
    float v_pred = 0.f;
#pragma unroll
    for (int q = 0; q < kRowGroups; ++q) v_pred += s_red[q][d0 + c];
    delta[c] = beta * (bf(vrow[c]) - v_pred);
  }
  __syncthreads();
  f32x4 op = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const int k = g + kRowGroups * i;
    s[i] += s_k[k] * delta;
    *reinterpret_cast<f32x4*>(S + k * kDv + d0) = s[i];
    op += s[i] * s_q[k];
  }
  *reinterpret_cast<f32x4*>(&s_red[g][d0]) = op;
  __syncthreads();
  float o = 0.f;
  if (t < kDv) {
#pragma unroll
    for (int q = 0; q < kRowGroups; ++q) o += s_red[q][t];
    o = round_bf(o);                               // .to(orig_dtype)
    if (a.core) a.core[bi * a.core_rs + h * kDv + t] = to_bf(o);
  }
  const float var = sum128(t < kDv ? o * o : 0.f, s_sum) / (float)kDv;
  if (t < kDv) {
    const float xn = o * rsqrtf(var + a.eps);
    const float zz = bf(a.z[bi * a.z_rs + h * kDv + t]);
    const float out = a.norm_w[h * kDv + t] * xn * (zz / (1.f + expf(-zz)));
    a.out[bi * a.out_rs + h * kDv + t] = to_bf(out);
  }
}

}  // namespace
}  // namespace tfa

extern "C" {

int64_t tf_gdn_decode_workspace_bytes(int32_t batch_size, int32_t num_k_heads,
                                      int32_t num_v_heads) {
  tfa::clear_error();
  if (batch_size < 0 || num_k_heads <= 0 || num_v_heads <= 0)
    return tfa::fail(TF_ERR_INVALID, "gdn_decode_workspace_bytes: bad arguments");
  const int64_t conv_dim = 2LL * num_k_heads * tfa::kDk + (int64_t)num_v_heads * tfa::kDv;
  return (int64_t)batch_size * conv_dim * 2;
}

int32_t tf_gdn_decode(const void* qkv, int64_t qkv_row_stride, const void* a, const void* b,
                      int64_t ab_row_stride, const void* z, int64_t z_row_stride,
                      const float* conv_weight, const float* a_log, const float* dt_bias,
                      const float* norm_weight, float eps, void* conv_state,
                      int64_t conv_slot_stride, float* ssm_state, int64_t ssm_slot_stride,
                      const int64_t* req_indices, int32_t batch_size, int64_t n_slots,
                      int32_t num_k_heads, int32_t num_v_heads, int32_t head_k_dim,
                      int32_t head_v_dim, int32_t conv_kernel, void* out,
                      int64_t out_row_stride, void* core_out, int64_t core_row_stride,
                      void* workspace, int64_t workspace_bytes, tf_stream_t stream) {
  using namespace tfa;
  clear_error();
  if (head_k_dim != kDk || head_v_dim != kDv || conv_kernel != 4)
    return fail(TF_ERR_UNSUPPORTED,
                "gdn_decode: head_k_dim=%d head_v_dim=%d conv_kernel=%d (128 / 128 / 4 only)",
                head_k_dim, head_v_dim, conv_kernel);
  if (num_k_heads <= 0 || num_v_heads <= 0 || num_v_heads % num_k_heads)
    return fail(TF_ERR_INVALID, "gdn_decode: %d value heads over %d key heads", num_v_heads,
                num_k_heads);
  if (batch_size < 0 || n_slots <= 0)
    return fail(TF_ERR_INVALID, "gdn_decode: batch_size=%d n_slots=%lld", batch_size,
                (long long)n_slots);
  if (batch_size == 0) return TF_OK;
  const int64_t key_dim = (int64_t)num_k_heads * kDk, value_dim = (int64_t)num_v_heads * kDv;
  const int64_t conv_dim = 2 * key_dim + value_dim;
  if (!qkv || !a || !b || !z || !conv_weight || !a_log || !dt_bias || !norm_weight ||
      !conv_state || !ssm_state || !req_indices || !out || !workspace)
    return fail(TF_ERR_INVALID, "gdn_decode: null pointer");
  if (workspace_bytes < (int64_t)batch_size * conv_dim * 2 ||
      (reinterpret_cast<uintptr_t>(workspace) & 1u))
    return fail(TF_ERR_INVALID, "gdn_decode: workspace of %lld bytes (needs %lld)",
                (long long)workspace_bytes, (long long)(batch_size * conv_dim * 2));
  if (qkv_row_stride < conv_dim || ab_row_stride < num_v_heads || z_row_stride < value_dim ||
      out_row_stride < value_dim || (core_out && core_row_stride < value_dim) ||
      conv_slot_stride < 3 * conv_dim || ssm_slot_stride < value_dim * kDk)
    return fail(TF_ERR_INVALID, "gdn_decode: a row or slot stride is too small");
  if (!aligned16(conv_weight) || !aligned16(ssm_state) || ssm_slot_stride % 4)
    return fail(TF_ERR_INVALID, "gdn_decode: conv_weight / ssm_state must be 16-byte aligned");
  if ((int64_t)batch_size * conv_dim > INT32_MAX)
    return fail(TF_ERR_UNSUPPORTED, "gdn_decode: batch too large");
  GdnArgs g;
  g.qkv = static_cast<const uint16_t*>(qkv);
  g.qkv_rs = qkv_row_stride;
  g.a = static_cast<const uint16_t*>(a);
  g.b = static_cast<const uint16_t*>(b);
  g.ab_rs = ab_row_stride;
  g.z = static_cast<const uint16_t*>(z);
  g.z_rs = z_row_stride;
  g.conv_w = conv_weight;
  g.a_log = a_log;
  g.dt_bias = dt_bias;
  g.norm_w = norm_weight;
  g.eps = eps;
  g.conv_state = static_cast<uint16_t*>(conv_state);
  g.conv_ss = conv_slot_stride;
  g.ssm = ssm_state;
  g.ssm_ss = ssm_slot_stride;
  g.req = req_indices;
  g.n_slots = n_slots;
  g.batch = batch_size;
  g.hv = num_v_heads;
  g.vpk = num_v_heads / num_k_heads;
  g.key_dim = (int32_t)key_dim;
  g.conv_dim = (int32_t)conv_dim;
  g.ws = static_cast<uint16_t*>(workspace);
  g.out = static_cast<uint16_t*>(out);
  g.out_rs = out_row_stride;
  g.core = static_cast<uint16_t*>(core_out);
  g.core_rs = core_row_stride;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  const int64_t n_conv = (int64_t)batch_size * conv_dim;
  hipLaunchKernelGGL(gdn_conv_kernel, dim3((n_conv + kThreads - 1) / kThreads), dim3(kThreads),
                     0, s, g);
  hipLaunchKernelGGL(gdn_recur_kernel, dim3((int64_t)batch_size * num_v_heads), dim3(kThreads), 0,
                     s, g);
  return launch_status("tf_gdn_decode launch");
}

}  // extern "C"
