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
// Two launches.  gdn_conv_kernel: one thread per (request, 4 channels) runs the
// conv step, writes the bf16 SiLU outputs to a workspace row and shifts the
// conv state; the first Hv threads of a request also form the value heads'
// gates (log alpha, beta) into the workspace.  gdn_recur_kernel: one 256-thread
// workgroup per (request, value head) normalises its q / k from the workspace,
// streams the head's 64 KB state through registers once with nontemporal
// loads and stores (thread t holds columns 4 (t % 32) .. + 3 of rows
// t / 32 + 8 i), reduces S^T k and S^T q over the rows through LDS and applies
// the gated norm to the whole head.  HBM-bound: 128 KB of state traffic per
// value head and request.
#include <math.h>

#include <algorithm>

#include <mutex>

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
  int32_t hk;
  int32_t dk, dv;        // head dims (128 / 128 on the tuned kernels)
  float qscale;          // dk^-0.5 as fp32 (the other-dims kernel)
  uint16_t* wqk;         // extend: bf16 [rows, Hk, 4, 128] normalised q (hi, lo parts) then k
  float* wg;             // extend: fp32 [rows, Hv, 2] g = log alpha, beta
  int32_t* owner;        // extend: int32 [rows] request of each token row (-1: none / skipped)
  uint16_t* silu_tab;    // extend: bf16 SiLU of the bf16 values 2^-25 <= |y| < 2^7
  float* wrec;           // extend: fp32 [chunk slots, Hv, 2304] chunk records
  const int32_t* tok;    // extend: request b owns token rows tok[b] .. tok[b + 1] - 1
  int32_t rows;          // token rows of qkv / a / b / z / out (offsets are clamped to it)
  uint16_t* ws;          // bf16 [rows, conv_dim]: conv + SiLU outputs
  uint16_t* out;         // bf16 [B, Hv * Dv]
  int64_t out_rs;
  uint16_t* core;        // optional bf16 [B, Hv * Dv]: o before the norm
  int64_t core_rs;
};

typedef float f32x2 __attribute__((ext_vector_type(2)));

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

// Four channels c .. c + 3 of one request per thread (conv_dim is a multiple
// of 4): 8-byte accesses to the conv state, qkv and the workspace when all
// three are 8-byte aligned, per channel otherwise; the arithmetic is the same.
__device__ __forceinline__ float conv_tap4(const f32x4& w, uint16_t x0, uint16_t x1,
                                           uint16_t x2, uint16_t x3) {
  const float acc = w[0] * bf(x0) + w[1] * bf(x1) + w[2] * bf(x2) + w[3] * bf(x3);
  const float y = round_bf(acc);                               // conv1d output (bf16)
  return y / (1.f + expf(-y));                                 // F.silu
}

__global__ void __launch_bounds__(kThreads) gdn_conv_kernel(GdnArgs a) {
  const int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x;
  const int per_req = a.conv_dim >> 2;
  const int bi = (int)(i / per_req), c = 4 * (int)(i - (int64_t)bi * per_req);
  if (bi >= a.batch) return;
  const int64_t r = a.req[bi];
  if (r < 0 || r >= a.n_slots) return;
  if (c / 4 < a.hv) {
    // the gates of value head h = c / 4 for the recurrence: g = log alpha, beta
    const int h = c / 4;
    const float xa = bf(a.a[bi * a.ab_rs + h]) + a.dt_bias[h];
    const float sp = xa > 20.f ? xa : log1pf(expf(xa));        // F.softplus
    *reinterpret_cast<f32x2*>(a.wg + ((int64_t)bi * a.hv + h) * 2) =
        f32x2{-expf(a.a_log[h]) * sp, 1.f / (1.f + expf(-bf(a.b[bi * a.ab_rs + h])))};
  }
  uint16_t* st = a.conv_state + r * a.conv_ss + 3 * (int64_t)c;
  const uint16_t* xin = a.qkv + bi * a.qkv_rs + c;
  uint16_t* yo = a.ws + (int64_t)bi * a.conv_dim + c;
  f32x4 w[4];
#pragma unroll
  for (int e = 0; e < 4; ++e) w[e] = *reinterpret_cast<const f32x4*>(a.conv_w + 4 * (int64_t)(c + e));
  if (((reinterpret_cast<uintptr_t>(st) | reinterpret_cast<uintptr_t>(xin) |
        reinterpret_cast<uintptr_t>(yo)) & 7u) == 0) {
    // taps of channel e: state elements 3e .. 3e + 2, then qkv element e
    uint16_t x[16];
#pragma unroll
    for (int j = 0; j < 3; ++j) {
      const u32x2 v = reinterpret_cast<const u32x2*>(st)[j];
      x[4 * j] = (uint16_t)v[0];
      x[4 * j + 1] = (uint16_t)(v[0] >> 16);
      x[4 * j + 2] = (uint16_t)v[1];
      x[4 * j + 3] = (uint16_t)(v[1] >> 16);
    }
    const u32x2 q = *reinterpret_cast<const u32x2*>(xin);
    x[12] = (uint16_t)q[0];
    x[13] = (uint16_t)(q[0] >> 16);
    x[14] = (uint16_t)q[1];
    x[15] = (uint16_t)(q[1] >> 16);
    uint16_t yv[4], ns[12];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      yv[e] = to_bf(conv_tap4(w[e], x[3 * e], x[3 * e + 1], x[3 * e + 2], x[12 + e]));
      ns[3 * e] = x[3 * e + 1];
      ns[3 * e + 1] = x[3 * e + 2];
      ns[3 * e + 2] = x[12 + e];
    }
    *reinterpret_cast<u32x2*>(yo) =
        u32x2{yv[0] | ((uint32_t)yv[1] << 16), yv[2] | ((uint32_t)yv[3] << 16)};
#pragma unroll
    for (int j = 0; j < 3; ++j)
      reinterpret_cast<u32x2*>(st)[j] =
          u32x2{ns[4 * j] | ((uint32_t)ns[4 * j + 1] << 16),
                ns[4 * j + 2] | ((uint32_t)ns[4 * j + 3] << 16)};
    return;
  }
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    uint16_t* se = st + 3 * e;
    const uint16_t x0 = se[0], x1 = se[1], x2 = se[2], x3 = xin[e];
    yo[e] = to_bf(conv_tap4(w[e], x0, x1, x2, x3));
    se[0] = x1;
    se[1] = x2;
    se[2] = x3;
  }
}

__global__ void __launch_bounds__(kThreads) gdn_recur_kernel(GdnArgs a) {
  __shared__ float s_q[kDk], s_k[kDk];
  __shared__ float s_red[kRowGroups][kDv];
  __shared__ float s_sum[4];
  const int bi = blockIdx.x / a.hv, h = blockIdx.x % a.hv;
  const int hk = h / a.vpk;
  const int t = threadIdx.x;
  const int64_t r = a.req[bi];
  if (r < 0 || r >= a.n_slots) {
    // A slot outside the pool: no state is read or written and the request's
    // output row reads as zeros (extend: gdn_norm_ext_kernel writes them).
    if (!a.tok && t < kDv) {
      a.out[(int64_t)bi * a.out_rs + h * kDv + t] = 0;
      if (a.core) a.core[(int64_t)bi * a.core_rs + h * kDv + t] = 0;
    }
    return;
  }
  // Decode: request bi is row bi.  Extend (token offsets given): this kernel
  // takes the requests that extend by exactly one token, at their row.
  int row = bi;
  if (a.tok) {
    const int t0 = min(max(a.tok[bi], 0), a.rows);
    if (min(max(a.tok[bi + 1], 0), a.rows) != t0 + 1) return;
    row = t0;
  }
  const uint16_t* y = a.ws + (int64_t)row * a.conv_dim;

  // The state loads go out first; q / k normalisation runs under their latency.
  // The state is read and written once per step, so both go nontemporal.
  const int d0 = 4 * (t & 31), g = t >> 5;
  float* S = a.ssm + r * a.ssm_ss + (int64_t)h * kDk * kDv;
  f32x4 s[16];
#pragma unroll
  for (int i = 0; i < 16; ++i)
    s[i] = __builtin_nontemporal_load(
        reinterpret_cast<const f32x4*>(S + (g + kRowGroups * i) * kDv + d0));

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

  // gates from the conv kernel (decode) or the q/k kernel (extend)
  const f32x2 gt = *reinterpret_cast<const f32x2*>(a.wg + ((int64_t)row * a.hv + h) * 2);
  const float alpha = expf(gt[0]), beta = gt[1];

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
    __builtin_nontemporal_store(s[i], reinterpret_cast<f32x4*>(S + k * kDv + d0));
    op += s[i] * s_q[k];
  }
  *reinterpret_cast<f32x4*>(&s_red[g][d0]) = op;
  __syncthreads();
  float o = 0.f;
  if (t < kDv) {
#pragma unroll
    for (int q = 0; q < kRowGroups; ++q) o += s_red[q][t];
    o = round_bf(o);                               // .to(orig_dtype)
    if (a.core) a.core[row * a.core_rs + h * kDv + t] = to_bf(o);
  }
  const float var = sum128(t < kDv ? o * o : 0.f, s_sum) / (float)kDv;
  if (t < kDv) {
    const float xn = o * rsqrtf(var + a.eps);
    const float zz = bf(a.z[row * a.z_rs + h * kDv + t]);
    const float out = a.norm_w[h * kDv + t] * xn * (zz / (1.f + expf(-zz)));
    a.out[row * a.out_rs + h * kDv + t] = to_bf(out);
  }
}

// ---------------------------------------------------------------- extend
// Requests with several new tokens (the reference's per-request loop,
// linear_attention.py:328-364): the conv runs over the flattened batch in
// parallel (kConvTokens rows x kConvCh channels per thread, inputs before a
// request's first row taken from its conv state, which the q / k kernel
// shifts afterwards); per 32-token chunk the WY quantities are prepared for all
// chunks at once; then one workgroup per (request, value head) carries the
// head's state in MFMA accumulators from the first chunk to the last (one state
// read and one write per request and head) and applies the gated norm to the
// rows as they come out.  This is the reference's chunked WY update (:194-242)
// with 32-token chunks; the chunk length does not change the result.  The
// one-token requests of the batch take gdn_recur_kernel, on a second stream
// beside the chunked pass (tf_gdn_extend).

constexpr int kConvTokens = 8;    // tokens per thread in the extend conv

// The conv output y is a bf16 value, so bf16(silu(y)) is a function of 16
// bits.  The extend conv looks it up for 2^-25 <= |y| < 2^7 (biased exponents
// kSiluELo .. kSiluELo + 31, both signs: 8192 entries) and computes it for
// the rest; the table holds what silu_bf16 computes, so both agree bit for bit.
constexpr int kSiluELo = 102;
constexpr int kSiluTab = 8192;

__device__ __forceinline__ uint16_t silu_bf16(float y) {
  return to_bf(y / (1.f + expf(-y)));   // F.silu (accurate exp: q / k / v feed everything)
}
__device__ __forceinline__ uint32_t silu_lookup(float y, const uint16_t* tab) {
  const uint32_t u = __float_as_uint(y) >> 16;   // y's bf16 bits
  const uint32_t e = ((u >> 7) & 0xffu) - kSiluELo;
  if (e < 32u) return tab[((u >> 15) << 12) | (e << 7) | (u & 127u)];
  return silu_bf16(y);
}

// owner[tt] = the request whose rows hold tt, or -1 when none does or the
// request's slot is outside the pool (those rows are skipped everywhere).
// Threads 0 .. kSiluTab - 1 also fill the SiLU table.
__global__ void __launch_bounds__(kThreads) gdn_owner_kernel(GdnArgs a) {
  const int tt = blockIdx.x * kThreads + threadIdx.x;
  if (tt < kSiluTab) {
    const uint32_t u = ((uint32_t)(tt >> 12) << 15) | ((uint32_t)(kSiluELo + ((tt >> 7) & 31)) << 7) |
                       (uint32_t)(tt & 127);
    a.silu_tab[tt] = silu_bf16(__uint_as_float(u << 16));
  }
  if (tt >= a.rows) return;
  int lo = 0, hi = a.batch - 1;
  while (lo < hi) {
    const int mid = (lo + hi + 1) >> 1;
    if (min(max(a.tok[mid], 0), a.rows) <= tt) lo = mid; else hi = mid - 1;
  }
  const int t0 = min(max(a.tok[lo], 0), a.rows), t1 = min(max(a.tok[lo + 1], 0), a.rows);
  const int64_t r = a.req[lo];
  a.owner[tt] = tt >= t0 && tt < t1 && r >= 0 && r < a.n_slots ? lo : -1;
}

constexpr int kConvCh = 4;   // channels per thread in the extend conv

// Conv + SiLU of kConvTokens consecutive token rows for kConvCh channels per
// thread (grid: channel blocks x a stride of kConvTokens-row blocks over the
// flattened batch; the SiLU table is copied to LDS once per workgroup).
// Each token's window takes the inputs before its request's first token from
// the request's conv state, which this kernel only reads; gdn_qk_ext_kernel
// (head dims 128) or gdn_conv_state_kernel shifts it afterwards.  Rows of
// requests whose slot is outside the pool are skipped.
constexpr int kConvRowWgs = 192;   // workgroups per channel block (row-block stride)

__global__ void __launch_bounds__(kThreads) gdn_conv_ext_kernel(GdnArgs a) {
  __shared__ __attribute__((aligned(16))) uint16_t tab[kSiluTab];
  for (int i = threadIdx.x; i < kSiluTab / 8; i += kThreads)
    reinterpret_cast<u32x4*>(tab)[i] = reinterpret_cast<const u32x4*>(a.silu_tab)[i];
  __syncthreads();
  const int c = kConvCh * (blockIdx.x * kThreads + threadIdx.x);
  if (c >= a.conv_dim) return;
  f32x4 w[kConvCh];
#pragma unroll
  for (int e = 0; e < kConvCh; ++e)
    w[e] = *reinterpret_cast<const f32x4*>(a.conv_w + 4 * (int64_t)(c + e));
  for (int tb = blockIdx.y * kConvTokens; tb < a.rows; tb += gridDim.y * kConvTokens) {
    u32x2 x[kConvTokens + 3];   // rows tb - 3 .. tb + kConvTokens - 1 (0 outside [0, rows))
#pragma unroll
    for (int i = 0; i < kConvTokens + 3; ++i) {
      const int tt = tb - 3 + i;
      x[i] = tt >= 0 && tt < a.rows ? *reinterpret_cast<const u32x2*>(a.qkv + tt * a.qkv_rs + c)
                                    : u32x2{0u, 0u};
    }
    // Most row blocks lie inside one in-pool request, at least 3 rows past its
    // first: then every input is a qkv row (workgroup-uniform test).
    const int tl = min(tb + kConvTokens, a.rows) - 1;
    const int ob = a.owner[tb];
    if (ob >= 0 && a.owner[tl] == ob && tb - 3 >= min(max(a.tok[ob], 0), a.rows)) {
#pragma unroll
      for (int i = 0; i < kConvTokens; ++i) {
        if (tb + i > tl) break;
        uint32_t y[kConvCh];
#pragma unroll
        for (int e = 0; e < kConvCh; ++e) {
          float in[4];
#pragma unroll
          for (int k = 0; k < 4; ++k) {
            const uint32_t pr = x[i + k][e >> 1];
            in[k] = (e & 1) ? bf16_hi(pr) : bf16_lo(pr);
          }
          y[e] = silu_lookup(
              round_bf(w[e][0] * in[0] + w[e][1] * in[1] + w[e][2] * in[2] + w[e][3] * in[3]), tab);
        }
        *reinterpret_cast<u32x2*>(a.ws + (int64_t)(tb + i) * a.conv_dim + c) =
            u32x2{y[0] | (y[1] << 16), y[2] | (y[3] << 16)};
      }
      continue;
    }
#pragma unroll
    for (int i = 0; i < kConvTokens; ++i) {
      const int tt = tb + i;
      if (tt >= a.rows) break;
      const int bi = a.owner[tt];
      if (bi < 0) continue;
      const int t0 = min(max(a.tok[bi], 0), a.rows);
      const int64_t r = a.req[bi];
      const uint16_t* st = a.conv_state + r * a.conv_ss + 3 * (int64_t)c;
      uint32_t y[kConvCh];
#pragma unroll
      for (int e = 0; e < kConvCh; ++e) {
        float in[4];
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          const int p = tt - 3 + k;   // input position; before t0 it is in the conv state
          const uint32_t pr = x[i + k][e >> 1];
          in[k] = p >= t0 ? ((e & 1) ? bf16_hi(pr) : bf16_lo(pr)) : bf(st[3 * e + p - t0 + 3]);
        }
        y[e] = silu_lookup(
            round_bf(w[e][0] * in[0] + w[e][1] * in[1] + w[e][2] * in[2] + w[e][3] * in[3]), tab);
      }
      *reinterpret_cast<u32x2*>(a.ws + (int64_t)tt * a.conv_dim + c) =
          u32x2{y[0] | (y[1] << 16), y[2] | (y[3] << 16)};
    }
  }
}

// Conv state <- the last 3 inputs of each request (after gdn_conv_ext_kernel
// has read the old state).
__device__ __forceinline__ void conv_state_shift(const GdnArgs& a, int bi, int c) {
  const int64_t r = a.req[bi];
  if (r < 0 || r >= a.n_slots) return;
  const int t0 = min(max(a.tok[bi], 0), a.rows), t1 = min(max(a.tok[bi + 1], t0), a.rows);
  uint16_t* st = a.conv_state + r * a.conv_ss + 3 * (int64_t)c;
  uint16_t x[3];
#pragma unroll
  for (int i = 0; i < 3; ++i) {
    const int tt = t1 - 3 + i;           // position in [state, tokens]
    x[i] = tt >= t0 ? a.qkv[tt * a.qkv_rs + c] : st[tt - t0 + 3];
  }
#pragma unroll
  for (int i = 0; i < 3; ++i) st[i] = x[i];
}

__global__ void __launch_bounds__(kThreads) gdn_conv_state_kernel(GdnArgs a) {
  const int c = blockIdx.x * kThreads + threadIdx.x;
  if (c < a.conv_dim) conv_state_shift(a, blockIdx.y, c);
}

// Zeros of token row tok (a row of no request or of an out-of-pool slot).
__device__ __forceinline__ void zero_row(const GdnArgs& a, int64_t tok, int i0, int step) {
  for (int d = 4 * i0; d < a.hv * a.dv; d += 4 * step) {
    *reinterpret_cast<u32x2*>(a.out + tok * a.out_rs + d) = u32x2{0u, 0u};
    if (a.core) *reinterpret_cast<u32x2*>(a.core + tok * a.core_rs + d) = u32x2{0u, 0u};
  }
}

// Per (token, key head): q / k of the head normalised (F.normalize, eps
// 1e-12; q also scaled by dk^-0.5) as fp32, and per value head of the group
// the log-decay g = log alpha and beta.  None of it depends on the state,
// so it runs for all tokens in parallel ahead of the recurrence.
__global__ void __launch_bounds__(kThreads) gdn_qk_ext_kernel(GdnArgs a) {
  // One half-wave per (token, key head): lane l of it normalises dims 4 l ..
  // 4 l + 3 of q and of k, each norm a 32-lane reduction (grid: token rows x
  // blocks of 8 key heads); the first block of each token also forms the
  // value heads' gates.
  const int tok = blockIdx.x;
  const int lane = threadIdx.x & (kWave - 1);
  const int hk = blockIdx.y * (2 * kThreads / kWave) + 2 * wave_id() + (lane >> 5);
  const bool act = hk < a.hk;
  const int d = 4 * (lane & 31);
  {
    const uint16_t* y = a.ws + (int64_t)tok * a.conv_dim + (act ? hk : 0) * kDk + d;
    const u32x2 qv = *reinterpret_cast<const u32x2*>(y);
    const u32x2 kv = *reinterpret_cast<const u32x2*>(y + a.key_dim);
    const float q[4] = {bf16_lo(qv[0]), bf16_hi(qv[0]), bf16_lo(qv[1]), bf16_hi(qv[1])};
    const float k[4] = {bf16_lo(kv[0]), bf16_hi(kv[0]), bf16_lo(kv[1]), bf16_hi(kv[1])};
    float sq = 0.f, sk = 0.f;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      sq += q[e] * q[e];
      sk += k[e] * k[e];
    }
#pragma unroll
    for (int m = 16; m >= 1; m >>= 1) {
      sq += __shfl_xor(sq, m, kWave);
      sk += __shfl_xor(sk, m, kWave);
    }
    if (act) {
      const float nq = fmaxf(sqrtf(sq), 1e-12f), nk = fmaxf(sqrtf(sk), 1e-12f);
      float qn[4], kn[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        qn[e] = q[e] / nq * 0.08838834764831845f;   // q x 128 ** -0.5
        kn[e] = k[e] / nk;
      }
      // q, then k, each as bf16 high parts and the bf16 rounding of the
      // remainders (the two MFMA operand halves)
      uint32_t* q32 = reinterpret_cast<uint32_t*>(a.wqk + ((int64_t)tok * a.hk + hk) * (4 * kDk));
      const int i = d / 2;   // dword of dims d, d + 1
      const uint32_t qh0 = pack_bf16(qn[0], qn[1]), qh1 = pack_bf16(qn[2], qn[3]);
      const uint32_t kh0 = pack_bf16(kn[0], kn[1]), kh1 = pack_bf16(kn[2], kn[3]);
      *reinterpret_cast<u32x2*>(q32 + i) = u32x2{qh0, qh1};
      *reinterpret_cast<u32x2*>(q32 + kDk / 2 + i) =
          u32x2{pack_bf16(qn[0] - bf16_lo(qh0), qn[1] - bf16_hi(qh0)),
                pack_bf16(qn[2] - bf16_lo(qh1), qn[3] - bf16_hi(qh1))};
      *reinterpret_cast<u32x2*>(q32 + kDk + i) = u32x2{kh0, kh1};
      *reinterpret_cast<u32x2*>(q32 + 3 * kDk / 2 + i) =
          u32x2{pack_bf16(kn[0] - bf16_lo(kh0), kn[1] - bf16_hi(kh0)),
                pack_bf16(kn[2] - bf16_lo(kh1), kn[3] - bf16_hi(kh1))};
    }
  }
  if (blockIdx.y != 0) return;
  for (int h = threadIdx.x; h < a.hv; h += kThreads) {
    const float xa = bf(a.a[tok * a.ab_rs + h]) + a.dt_bias[h];
    const float sp = xa > 20.f ? xa : log1pf(expf(xa));        // F.softplus
    float* gt = a.wg + ((int64_t)tok * a.hv + h) * 2;
    gt[0] = -expf(a.a_log[h]) * sp;                            // g = log alpha
    gt[1] = 1.f / (1.f + expf(-bf(a.b[tok * a.ab_rs + h])));
  }
  // Two small jobs that only need the conv's reads of the old conv states to
  // be done: zero rows of skipped token rows, and shift the conv states
  // (every request's last 3 inputs), strided over the first blocks.
  if (a.owner[tok] < 0) zero_row(a, tok, threadIdx.x, kThreads);
  const int64_t n_shift = (int64_t)a.batch * a.conv_dim;
  for (int64_t i = (int64_t)tok * kThreads + threadIdx.x; i < n_shift;
       i += (int64_t)gridDim.x * kThreads)
    conv_state_shift(a, (int)(i / a.conv_dim), (int)(i % a.conv_dim));
}

// global_load_lds_dwordx4 with a scalar base and a 32-bit lane offset: lane
// l's 16 bytes land at LDS address M0 + 16 l.  The compiler does not
// count these loads: readers wait with an explicit s_waitcnt vmcnt and a
// barrier.
__device__ __forceinline__ uint32_t lds_addr(const void* p) {
  return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void*)p;
}
__device__ __forceinline__ void dma16(const void* sbase, uint32_t voff, uint32_t lds) {
  asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, %1"
               :: "v"(voff), "s"(sbase), "s"(lds) : "m0");
}

// ---------------------------------------------------------------- chunked recurrence
// The delta rule over a chunk of C = 32 consecutive tokens of one request and
// value head, with S0 the state before the chunk, g_t = log alpha_t and
// gamma_t = g_0 + ... + g_t (t, s index the chunk's tokens):
//   A[t][s]  = beta_t e^(gamma_t - gamma_s) k_t.k_s   for s < t, else 0
//   T        = (I + A)^-1                           (unit lower triangular)
//   X        = diag(beta) (V - diag(e^gamma) K S0)
//   Delta    = T X
//   O        = diag(e^gamma) Q S0 + Bm Delta,   Bm[t][s] = e^(gamma_t - gamma_s) q_t.k_s (s <= t)
//   S        = e^(gamma_C) S0 + K^T diag(e^(gamma_C - gamma)) Delta
// This is the reference's chunk-wise WY form (linear_attention.py:194-242,
// there with 64-token chunks) and, like it, equals the token recurrence
// (:278-298) in exact arithmetic.  A chunk's tail past the request's last
// token is padded with neutral tokens (g = 0, beta = 0), which leave S and
// every real row unchanged.
//
// Two launches.  gdn_chunk_prep_kernel computes everything that does not
// depend on S - T, Bm, e^gamma, e^(gamma_C - gamma), beta - for every chunk
// of every request in parallel into a 9 KB record per (chunk, value head).
// gdn_chunk_ext_kernel then carries S through a request's chunks, one
// 512-thread workgroup per (request, value head) whose state wave w (0-3) owns
// state columns
// 32 w .. + 31 as four 32 x 32 MFMA accumulator tiles (lane (g, n) = (lane /
// 32, lane % 32): rows 32 ti + 8 (r / 4) + 4 g + r % 4 of column 32 w + n), so
// the state update is an MFMA into S and the products with S read it as an
// MFMA operand in place.  Every product runs on v_mfma_f32_32x32x16_bf16 with
// both fp32 operands split into bf16 high and low parts (hi*hi + hi*lo +
// lo*hi, about 2^-17 relative error, fp32 accumulation); q and k arrive
// already split (gdn_qk_ext_kernel).  Chunk records are numbered
// floor(t0_b / 32) + b + ci for chunk ci of request b (first token row t0_b),
// which is unique and below n_tokens / 32 + B.  Four helper waves of the same
// workgroup load the chunks and apply the gated norm to the output rows
// (gdn_chunk_ext_kernel), so the state waves' time per chunk is the
// recurrence's alone.
constexpr int kChunk = 32;
constexpr int kRec = 2304;     // floats per chunk record: T, Bm, e^gamma, e^(gC - gamma), beta
constexpr int kRecT = 0, kRecB = 1024, kRecC = 2048, kRecD = 2080, kRecBeta = 2112;

__device__ __forceinline__ int clamp_row(const GdnArgs& a, int b) {
  return min(max(a.tok[b], 0), a.rows);
}
__device__ __forceinline__ int chunk_key(const GdnArgs& a, int b) {
  return clamp_row(a, b) / kChunk + b;
}
// Token of accumulator register r of lane half g (rows of a 32 x 32 C tile).
__device__ __forceinline__ int c_row(int r, int g) { return 8 * (r >> 2) + 4 * g + (r & 3); }

// Eight fp32 values -> bf16 high parts and the bf16 rounding of the
// remainders, two per dword, element order kept.
__device__ __forceinline__ void split8(const f32x4& x0, const f32x4& x1, u32x4& hi, u32x4& lo) {
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    hi[i] = pack_bf16(x0[2 * i], x0[2 * i + 1]);
    lo[i] = pack_bf16(x0[2 * i] - bf16_lo(hi[i]), x0[2 * i + 1] - bf16_hi(hi[i]));
    hi[2 + i] = pack_bf16(x1[2 * i], x1[2 * i + 1]);
    lo[2 + i] = pack_bf16(x1[2 * i] - bf16_lo(hi[2 + i]), x1[2 * i + 1] - bf16_hi(hi[2 + i]));
  }
}
__device__ __forceinline__ void split16(const f32x16& x, int r0, u32x4& hi, u32x4& lo) {
  split8(f32x4{x[r0], x[r0 + 1], x[r0 + 2], x[r0 + 3]},
         f32x4{x[r0 + 4], x[r0 + 5], x[r0 + 6], x[r0 + 7]}, hi, lo);
}
// c + a b with a = ah + al, b = bh + bl (the al bl term is below fp32 rounding).
__device__ __forceinline__ f32x16 mma3(f32x16 c, const u32x4& ah, const u32x4& al,
                                       const u32x4& bh, const u32x4& bl) {
  c = mfma_32x32x16(al, bh, c);
  c = mfma_32x32x16(ah, bl, c);
  return mfma_32x32x16(ah, bh, c);
}

// ---- prep: one workgroup per (chunk record slot, key head)
struct PrepSmem {
  float kk[kChunk][kChunk + 1];    // k_t . k_s
  float qq[kChunk][kChunk + 1];    // q_t . k_s
  float am[4][kChunk][36];         // A of the value head each half-wave solves (16-B rows)
};

__global__ void __launch_bounds__(kThreads, 4) gdn_chunk_prep_kernel(GdnArgs a) {
  __shared__ __attribute__((aligned(16))) PrepSmem sm;
  const int slot = blockIdx.x, hk = blockIdx.y;
  const int lane = threadIdx.x & (kWave - 1), w = wave_id();
  const int g = lane >> 5, n = lane & 31;
  int lo = 0, hi = a.batch - 1;   // the request: last b with chunk_key(b) <= slot
  while (lo < hi) {
    const int mid = (lo + hi + 1) >> 1;
    if (chunk_key(a, mid) <= slot) lo = mid; else hi = mid - 1;
  }
  const int b = lo;
  const int t0 = clamp_row(a, b), t1 = max(clamp_row(a, b + 1), t0);
  const int64_t r = a.req[b];
  const int ci = slot - chunk_key(a, b);
  if (r < 0 || r >= a.n_slots || t1 - t0 < 2 || ci < 0 || ci >= (t1 - t0 + kChunk - 1) / kChunk)
    return;
  const int tb = t0 + kChunk * ci, ntok = min(kChunk, t1 - tb), last = t1 - 1;

  if (w < 2) {   // K K^T (wave 0), Q K^T (wave 1): rows t = lane n, dims 16 ks + 8 g .. + 7
    // operands straight from the split q / k rows (L2-resident): per token
    // 64 16-byte chunks, q hi, q lo, k hi, k lo
    const u32x4* row = reinterpret_cast<const u32x4*>(
        reinterpret_cast<const uint8_t*>(a.wqk) + ((int64_t)min(tb + n, last) * a.hk + hk) * 1024);
    const int xo = w == 0 ? 32 : 0;
    u32x4 xh[8], xl[8], kh[8], kl[8];
#pragma unroll
    for (int ks = 0; ks < 8; ++ks) {
      const int ch = 2 * ks + g;
      xh[ks] = row[xo + ch];
      xl[ks] = row[xo + 16 + ch];
      kh[ks] = row[32 + ch];
      kl[ks] = row[48 + ch];
    }
    f32x16 acc = {};
#pragma unroll
    for (int ks = 0; ks < 8; ++ks) acc = mma3(acc, xh[ks], xl[ks], kh[ks], kl[ks]);
    float (*M)[kChunk + 1] = w == 0 ? sm.kk : sm.qq;
#pragma unroll
    for (int rr = 0; rr < 16; ++rr) M[c_row(rr, g)][n] = acc[rr];
  }
  __syncthreads();

  // Each half-wave of waves 0 and 1 takes one value head (lanes n of half g);
  // four heads per pass.
  for (int v0 = 2 * w; w < 2 && v0 < a.vpk; v0 += 4) {
    const int v = v0 + g;
    const bool act = v < a.vpk;
    const int h = hk * a.vpk + min(v, a.vpk - 1);
    float* rec = a.wrec + ((int64_t)slot * a.hv + h) * kRec;
    const float2 gbv = *reinterpret_cast<const float2*>(a.wg + ((int64_t)min(tb + n, last) * a.hv + h) * 2);
    const float gn = n < ntok ? gbv.x : 0.f, bn = n < ntok ? gbv.y : 0.f;
    float x = gn;   // gamma_n: inclusive scan over the chunk
#pragma unroll
    for (int off = 1; off < kChunk; off <<= 1) {
      const float y = __shfl_up(x, off, 32);
      if (n >= off) x += y;
    }
    const float gc = __shfl(x, kChunk - 1, 32);
    float (*A)[36] = sm.am[2 * w + g];
    if (act) {
      rec[kRecC + n] = __expf(x);
      rec[kRecD + n] = __expf(gc - x);
      rec[kRecBeta + n] = bn;
    }
    // lane n = column s: A[t][s] into LDS, Bm[t][s] into the record
#pragma unroll
    for (int t = 0; t < kChunk; ++t) {
      const float gt = __shfl(x, t, 32), bt = __shfl(bn, t, 32);
      const float e = __expf(fminf(gt - x, 0.f));
      if (act) {
        A[t][n] = n < t ? bt * e * sm.kk[t][n] : 0.f;
        rec[kRecB + t * kChunk + n] = n <= t ? e * sm.qq[t][n] : 0.f;
      }
    }
    // this wave's writes of A before its reads (one wave: no barrier needed)
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    if (act) {      // T = (I + A)^-1 by forward substitution, lane n owns column n;
                    // each row's sum in four interleaved partial sums (shorter FMA chains)
      float tc[kChunk];
#pragma unroll
      for (int t = 0; t < kChunk; ++t) {
        float acc[4] = {t == n ? 1.f : 0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int s4 = 0; s4 < t; s4 += 4) {
          const f32x4 ar = *reinterpret_cast<const f32x4*>(&A[t][s4]);
#pragma unroll
          for (int e = 0; e < 4; ++e)
            if (s4 + e < t) acc[e] = fmaf(-ar[e], tc[s4 + e], acc[e]);
        }
        tc[t] = (acc[0] + acc[1]) + (acc[2] + acc[3]);
        __builtin_amdgcn_sched_barrier(0);
      }
#pragma unroll
      for (int t = 0; t < kChunk; ++t) rec[kRecT + t * kChunk + n] = tc[t];
    }
  }
}

// ---- the recurrence: one workgroup per (request, value head)
struct ChunkIn {
  uint32_t q[kChunk][128];   // 512 B per token: 16-B chunks 0-15 hi, 16-31 lo; chunk c of
  uint32_t k[kChunk][128];   //   either half stored at c ^ (t & 15) of that half
  uint16_t v[kChunk][kDv];   // 8 KB
  float rec[kRec];           // 9 KB: the chunk's record
};

// Dims d0 .. d0 + 3 and d0 + 8 .. d0 + 11 (d0 a multiple of 4, d0 % 8 < 4) of
// swizzled row t, high and low parts, as two MFMA operands.
__device__ __forceinline__ void row8(const uint32_t (*rows)[128], int t, int d0, u32x4& hi,
                                     u32x4& lo) {
  const uint32_t* row = rows[t];
  const int c = d0 >> 3, e = (d0 & 7) >> 1;   // 16-B chunk, dword within it
  const int p0 = 4 * ((c) ^ (t & 15)) + e, p1 = 4 * ((c + 1) ^ (t & 15)) + e;
  const u32x2 h0 = *reinterpret_cast<const u32x2*>(row + p0);
  const u32x2 h1 = *reinterpret_cast<const u32x2*>(row + p1);
  const u32x2 l0 = *reinterpret_cast<const u32x2*>(row + 64 + p0);
  const u32x2 l1 = *reinterpret_cast<const u32x2*>(row + 64 + p1);
  hi = u32x4{h0[0], h0[1], h1[0], h1[1]};
  lo = u32x4{l0[0], l0[1], l1[0], l1[1]};
}
typedef short i16x4_t __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) i16x4_t lds_i16x4;
constexpr int kChunkThreads = 2 * kThreads;   // 4 recurrence waves + 4 helper waves

// Waves 0-3 carry the state through the chunks (the MFMA work above, nothing
// else); waves 4-7, the helpers, share their SIMDs and keep the inputs ahead
// of them: while the state waves work on chunk ci, the helpers move chunk
// ci + 1 into LDS and apply the gated norm to the rows of chunk ci - 1.  The
// state update reads k transposed straight from the token-major rows
// (ds_read_b64_tr_b16).  One barrier per chunk
// hands the buffers over (chunk inputs and the output tile are
// double-buffered by chunk parity).
__global__ void __launch_bounds__(kChunkThreads) gdn_chunk_ext_kernel(GdnArgs a) {
  __shared__ __attribute__((aligned(16))) ChunkIn sm[2];
  // A chunk's recurrence output (o rounded to bf16), token-major, and the
  // head's norm weights.
  __shared__ __attribute__((aligned(16))) uint16_t otile[2][kChunk][kDv];
  __shared__ __attribute__((aligned(16))) float nw[kDv];
  const int bi = blockIdx.x / a.hv, h = blockIdx.x % a.hv;
  const int hk = h / a.vpk;
  const int lane = threadIdx.x & (kWave - 1), wv = wave_id();
  const bool helper = wv >= 4;
  const int w = wv & 3;                            // wave within its group
  const int ht = threadIdx.x & (kThreads - 1);     // thread within its group
  const int g = lane >> 5, n = lane & 31;
  const int64_t r = a.req[bi];
  if (r < 0 || r >= a.n_slots) return;
  const int t0 = clamp_row(a, bi), t1 = max(clamp_row(a, bi + 1), t0);
  if (t1 - t0 < 2) return;   // one-token requests: gdn_recur_kernel
  const int last = t1 - 1;
  const int nchunks = (t1 - t0 + kChunk - 1) / kChunk;

  // The 64 KB state goes through LDS (the chunk buffers, not yet in use) so
  // that the global accesses are coalesced 16-byte ones and each lane reads
  // its 64 values at immediate offsets from one LDS address.
  float* S = a.ssm + r * a.ssm_ss + (int64_t)h * kDk * kDv;
  float* stage = reinterpret_cast<float*>(&sm[0]);
  static_assert(sizeof(sm) >= kDk * kDv * 4, "state staging");
#pragma unroll
  for (int i = 0; i < kDk * kDv / 4 / kChunkThreads; ++i) {
    const int q = i * kChunkThreads + threadIdx.x;
    reinterpret_cast<f32x4*>(stage)[q] = reinterpret_cast<const f32x4*>(S)[q];
  }
  nw[threadIdx.x & (kDv - 1)] = a.norm_w[h * kDv + (threadIdx.x & (kDv - 1))];   // 4 writers each
  __syncthreads();

  if (!helper) {
    const int j = 32 * w + n;   // this lane's state column
    f32x16 st[4];
    {
      const float* my = stage + 4 * g * kDv + j;
#pragma unroll
      for (int ti = 0; ti < 4; ++ti)
#pragma unroll
        for (int rr = 0; rr < 16; ++rr)
          st[ti][rr] = my[(32 * ti + 8 * (rr >> 2) + (rr & 3)) * kDv];
    }
    __syncthreads();   // the staging area is free for chunk 0

    for (int ci = 0; ci < nchunks; ++ci) {
      const ChunkIn& I = sm[ci & 1];
      __syncthreads();   // chunk ci is in; its output tile is free

      // P = K S0 and R = Q S0 over the state rows (k index 8 g + jj <-> state
      // row 32 ti + 16 hh + 8 (jj / 4) + 4 g + jj % 4)
      // (two accumulators each for P and R, one per half of the state rows:
      // four independent MFMA chains)
      // (step (ti, hh) + 1's operands are read from LDS while step (ti, hh)'s
      // MFMAs run)
      f32x16 Pp[2] = {{}, {}}, Rp[2] = {{}, {}};
      u32x4 op[2][4];
      auto read_ops = [&](int step, u32x4 (&o)[4]) __attribute__((always_inline)) {
        const int d0 = 32 * (step >> 1) + 16 * (step & 1) + 4 * g;
        row8(I.k, n, d0, o[0], o[1]);
        row8(I.q, n, d0, o[2], o[3]);
      };
      // (and step + 1's state operand is split while step's MFMAs run)
      u32x4 sh[2], sl[2];
      read_ops(0, op[0]);
      split16(st[0], 0, sh[0], sl[0]);
#pragma unroll
      for (int step = 0; step < 8; ++step) {
        const int ti = step >> 1;
        if (step + 1 < 8) read_ops(step + 1, op[(step + 1) & 1]);
        __builtin_amdgcn_sched_barrier(0);
        const u32x4(&o)[4] = op[step & 1];
        Pp[ti >> 1] = mma3(Pp[ti >> 1], o[0], o[1], sh[step & 1], sl[step & 1]);
        Rp[ti >> 1] = mma3(Rp[ti >> 1], o[2], o[3], sh[step & 1], sl[step & 1]);
        if (step + 1 < 8)
          split16(st[(step + 1) >> 1], 8 * ((step + 1) & 1), sh[(step + 1) & 1], sl[(step + 1) & 1]);
#pragma unroll
        for (int q = 0; q < 6; ++q) {
          __builtin_amdgcn_sched_group_barrier(0x8, 1, 0);   // 1 MFMA
          __builtin_amdgcn_sched_group_barrier(0x2, 4, 0);   // 4 VALU
        }
        __builtin_amdgcn_sched_barrier(0);
      }
      const f32x16 P = Pp[0] + Pp[1], R = Rp[0] + Rp[1];
      // X = beta (v - e^gamma P); Delta = T X (k index 8 g + jj <-> token
      // 16 hh + 8 (jj / 4) + 4 g + jj % 4)
      f32x16 X;
#pragma unroll
      for (int rr = 0; rr < 16; ++rr) {
        const int t = c_row(rr, g);
        X[rr] = I.rec[kRecBeta + t] * (bf(I.v[t][j]) - I.rec[kRecC + t] * P[rr]);
      }
      // (T and Bm arrive split into bf16 high / low operand halves: split_tb)
      f32x16 Dp[2];
#pragma unroll
      for (int hh = 0; hh < 2; ++hh) {
        u32x4 xh, xl;
        split16(X, 8 * hh, xh, xl);
        const u32x4* tp =
            reinterpret_cast<const u32x4*>(&I.rec[kRecT + n * kChunk + 16 * hh + 8 * g]);
        Dp[hh] = mma3(f32x16{}, tp[0], tp[1], xh, xl);
      }
      f32x16 D = Dp[0] + Dp[1];
      // O = e^gamma R + Bm Delta -> the recurrence output rows of this chunk
      u32x4 dh[2], dl[2];
      split16(D, 0, dh[0], dl[0]);
      split16(D, 8, dh[1], dl[1]);
      f32x16 Op[2];
#pragma unroll
      for (int hh = 0; hh < 2; ++hh) {
        const u32x4* bp =
            reinterpret_cast<const u32x4*>(&I.rec[kRecB + n * kChunk + 16 * hh + 8 * g]);
        Op[hh] = mma3(f32x16{}, bp[0], bp[1], dh[hh], dl[hh]);
      }
      const f32x16 O = Op[0] + Op[1];
#pragma unroll
      for (int rr = 0; rr < 16; ++rr) {
        const int t = c_row(rr, g);
        otile[ci & 1][t][j] = to_bf(fmaf(I.rec[kRecC + t], R[rr], O[rr]));   // .to(orig_dtype)
      }
      // S = e^(gamma_C) S0 + K^T (diag(e^(gamma_C - gamma)) Delta)
#pragma unroll
      for (int rr = 0; rr < 16; ++rr) D[rr] *= I.rec[kRecD + c_row(rr, g)];
      split16(D, 0, dh[0], dl[0]);
      split16(D, 8, dh[1], dl[1]);
      const float cC = I.rec[kRecC + kChunk - 1];
      // A operand: K^T row i = 32 ti + n at tokens s(jj) as for Delta, read
      // from the token-major k rows with ds_read_b64_tr_b16, which hands lane
      // i of each 16-lane group element i % 4 of the 8 bytes addressed by lane
      // 4 k + (i % 16) / 4 as its element k: lane L addresses token
      // 16 hh + 4 g + (L % 16) / 4 (+ 8), dims 32 ti + 16 ((L / 16) % 2) +
      // 4 (L % 4) .. + 3 (step (ti, hh) + 1's read while step (ti, hh)'s
      // MFMAs run)
      u32x4 ka[2][2];
      const int tq = (lane & 15) >> 2, dq = 16 * ((lane >> 4) & 1) + 4 * (lane & 3);
      auto read_kt = [&](int step, u32x4 (&o)[2]) __attribute__((always_inline)) {
        const int d = 32 * (step >> 1) + dq, c = d >> 3, e = (d & 7) >> 1;
        const int t0 = 16 * (step & 1) + 4 * g + tq, t1 = t0 + 8;
        const uint32_t* a0 = &I.k[t0][4 * (c ^ (t0 & 15)) + e];
        const uint32_t* a1 = &I.k[t1][4 * (c ^ (t1 & 15)) + e];
        auto tr = [](const uint32_t* p) __attribute__((always_inline)) {
          return __builtin_bit_cast(u32x2, __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                                               (lds_i16x4*)(const_cast<uint32_t*>(p))));
        };
        const u32x2 h0 = tr(a0), h1 = tr(a1), l0 = tr(a0 + 64), l1 = tr(a1 + 64);
        o[0] = u32x4{h0[0], h0[1], h1[0], h1[1]};
        o[1] = u32x4{l0[0], l0[1], l1[0], l1[1]};
      };
      read_kt(0, ka[0]);
#pragma unroll
      for (int step = 0; step < 8; ++step) {
        const int ti = step >> 1, hh = step & 1;
        if (step + 1 < 8) read_kt(step + 1, ka[(step + 1) & 1]);
        __builtin_amdgcn_sched_barrier(0);
        if (hh == 0) st[ti] *= cC;
        st[ti] = mma3(st[ti], ka[step & 1][0], ka[step & 1][1], dh[hh], dl[hh]);
        __builtin_amdgcn_sched_barrier(0);
      }
    }
    __syncthreads();   // the last chunk's output tile is complete
    float* mine = stage + 4 * g * kDv + j;   // the chunk buffers are no longer read
#pragma unroll
    for (int ti = 0; ti < 4; ++ti)
#pragma unroll
      for (int rr = 0; rr < 16; ++rr)
        mine[(32 * ti + 8 * (rr >> 2) + (rr & 3)) * kDv] = st[ti][rr];
  } else {
    const int key0 = chunk_key(a, bi);
    // Chunk ci into buffer bf (tokens past the last one re-read the last
    // token; the record gives them beta = 0 and g = 0).  Helper wave w moves q
    // and k rows 8 w .. 8 w + 7 (4 + 4 instructions, two rows each), V rows
    // 8 w .. + 7 (2) and 3 KB of the record (waves 0-2 of the helpers).
    const uint8_t* qk_base = reinterpret_cast<const uint8_t*>(a.wqk) + (int64_t)hk * 1024;
    const uint8_t* v_base =
        reinterpret_cast<const uint8_t*>(a.ws) + ((int64_t)2 * a.key_dim + h * kDv) * 2;
    const uint8_t* rec_base = reinterpret_cast<const uint8_t*>(a.wrec) + (int64_t)h * kRec * 4;
    auto issue = [&](int ci) __attribute__((always_inline)) {
      const int tb = t0 + kChunk * ci;
      ChunkIn& I = sm[ci & 1];
#pragma unroll
      for (int p = 0; p < 4; ++p) {
        const int t = 8 * w + 2 * p + g;
        const uint32_t row = (uint32_t)min(tb + t, last) * (uint32_t)a.hk * 1024u;
        const uint32_t cpos = (uint32_t)((n & 16) | ((n & 15) ^ (t & 15))) * 16u;
        dma16(qk_base, row + cpos, lds_addr(&I.q[8 * w + 2 * p][0]));
        dma16(qk_base, row + 512u + cpos, lds_addr(&I.k[8 * w + 2 * p][0]));
      }
#pragma unroll
      for (int p = 0; p < 2; ++p) {
        const int t = 8 * w + 4 * p + (lane >> 4);
        dma16(v_base,
              (uint32_t)min(tb + t, last) * (uint32_t)a.conv_dim * 2u + 16u * (lane & 15),
              lds_addr(&I.v[8 * w + 4 * p][0]));
      }
      if (w < 3) {
        const uint32_t rec = (uint32_t)(key0 + ci) * (uint32_t)a.hv * (uint32_t)(kRec * 4);
#pragma unroll
        for (int p = 0; p < 3; ++p)
          dma16(rec_base, rec + 1024u * (3 * w + p) + 16u * lane,
                lds_addr(&I.rec[256 * (3 * w + p)]));
      }
    };
    // T and Bm of chunk ci (fp32 rows of 32) split in place into the state
    // waves' MFMA operand halves: block b of 16 floats (row n, half hh of T
    // for b < 64, of Bm after) becomes, for g = 0 and 1, the bf16 high parts
    // of columns 16 hh + 4 g + {0..3, 8..11} (16 bytes) and then the bf16
    // roundings of their remainders (16 bytes).  Lane l of helper wave w < 3
    // takes block 48 w + l: the record floats 768 w .. 768 w + 767 that this
    // wave's own DMA brought in, so its vmcnt wait covers them.
    auto split_tb = [&](int ci) __attribute__((always_inline)) {
      const int b = 48 * w + lane;
      if (w >= 3 || lane >= 48 || b >= 2 * 2 * kChunk) return;
      static_assert(kRecT == 0 && kRecB == 2 * kChunk * 16, "record layout");
      float* blk = &sm[ci & 1].rec[16 * b];
      const f32x4 x0 = *reinterpret_cast<const f32x4*>(blk);
      const f32x4 x1 = *reinterpret_cast<const f32x4*>(blk + 4);
      const f32x4 x2 = *reinterpret_cast<const f32x4*>(blk + 8);
      const f32x4 x3 = *reinterpret_cast<const f32x4*>(blk + 12);
      u32x4 h0, l0, h1, l1;
      split8(x0, x2, h0, l0);
      split8(x1, x3, h1, l1);
      u32x4* out = reinterpret_cast<u32x4*>(blk);
      out[0] = h0;
      out[1] = l0;
      out[2] = h1;
      out[3] = l1;
    };
    // Gated RMSNorm (rms_norm_gated.py:26-40) of chunk cj's rows: helper
    // thread (token, part) = (ht / 8, ht % 8) takes dims 16 part .. + 15 of
    // one row (the row's sum of squares is an 8-lane sum) with its z values
    // in zr, loaded a chunk ahead; out = bf16(norm_w * (o / rms(o)) *
    // silu(z)) with silu(z) = z / (1 + e^-z) from the hardware exp2 and
    // reciprocal (about 1 ulp each in fp32, below the bf16 rounding of the
    // output), and core_out gets o.
    const int te = ht >> 3, c0 = 16 * (ht & 7);
    u32x2 zr[4], zn[4];
    auto load_z = [&](int cj) __attribute__((always_inline)) {
      const int row = min(t0 + kChunk * cj + te, last);
      const uint16_t* zrow = a.z + (int64_t)row * a.z_rs + h * kDv + c0;
#pragma unroll
      for (int e = 0; e < 4; ++e) zn[e] = *reinterpret_cast<const u32x2*>(zrow + 4 * e);
    };
    auto norm_rows = [&](int cj) __attribute__((always_inline)) {
      const int row = t0 + kChunk * cj + te;
      const u32x4 ob[2] = {*reinterpret_cast<const u32x4*>(&otile[cj & 1][te][c0]),
                           *reinterpret_cast<const u32x4*>(&otile[cj & 1][te][c0 + 8])};
      float ss = 0.f;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const uint32_t wd = ob[e >> 2][e & 3];
        ss = fmaf(bf16_lo(wd), bf16_lo(wd), ss);
        ss = fmaf(bf16_hi(wd), bf16_hi(wd), ss);
      }
      ss = row_sum8(ss);
      if (row > last) return;   // padding of the request's last chunk
      const float inv = rsqrtf(ss / (float)kDv + a.eps);
      uint16_t* orow = a.out + (int64_t)row * a.out_rs + h * kDv + c0;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const uint32_t o01 = ob[e >> 1][2 * (e & 1)], o23 = ob[e >> 1][2 * (e & 1) + 1];
        const float o[4] = {bf16_lo(o01), bf16_hi(o01), bf16_lo(o23), bf16_hi(o23)};
        const float z[4] = {bf16_lo(zr[e][0]), bf16_hi(zr[e][0]), bf16_lo(zr[e][1]),
                            bf16_hi(zr[e][1])};
        const f32x4 wn = *reinterpret_cast<const f32x4*>(&nw[c0 + 4 * e]);
        float y[4];
#pragma unroll
        for (int k = 0; k < 4; ++k)
          y[k] = wn[k] * (o[k] * inv) *
                 (z[k] * __builtin_amdgcn_rcpf(1.f + __builtin_amdgcn_exp2f(-z[k] * kLog2e)));
        *reinterpret_cast<u32x2*>(orow + 4 * e) =
            u32x2{pack_bf16(y[0], y[1]), pack_bf16(y[2], y[3])};
        if (a.core)
          *reinterpret_cast<u32x2*>(a.core + (int64_t)row * a.core_rs + h * kDv + c0 + 4 * e) =
              u32x2{o01, o23};
      }
    };

    __syncthreads();   // the state waves have read the staging area
    issue(0);
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    split_tb(0);
    for (int ci = 0; ci < nchunks; ++ci) {
      __syncthreads();   // the state waves start chunk ci and are done with chunk ci - 1
      load_z(ci);
      if (ci + 1 < nchunks) issue(ci + 1);
      if (ci > 0) norm_rows(ci - 1);
#pragma unroll
      for (int e = 0; e < 4; ++e) zr[e] = zn[e];
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");   // chunk ci + 1 has landed
      if (ci + 1 < nchunks) split_tb(ci + 1);
    }
    __syncthreads();   // the last chunk's output tile is complete
    norm_rows(nchunks - 1);
  }
  __syncthreads();   // the final state is staged
#pragma unroll
  for (int i = 0; i < kDk * kDv / 4 / kChunkThreads; ++i) {
    const int q = i * kChunkThreads + threadIdx.x;
    reinterpret_cast<f32x4*>(S)[q] = reinterpret_cast<const f32x4*>(stage)[q];
  }
}

// ---------------------------------------------------------------- other head dims
// Head dims other than 128 (the reference's own test models use 16): one wave
// per (request, value head) carries the head's dk x dv state in registers,
// lane j holding value column j (dk, dv <= 64), through the request's token
// rows one at a time: the delta rule of linear_attention.py:278-298 (for a
// prefill the reference's chunk-wise form, :194-242, which equals it up to
// fp32 rounding), with q / k normalised (:171-172) and the gated norm
// (rms_norm_gated.py:26-40) in the same wave.  Conv outputs come from
// gdn_conv_kernel (decode: row = request) or gdn_conv_ext_kernel (extend).
// Decode: a request whose slot is outside the pool gets zero rows here;
// extend: gdn_qk_ext_kernel / gdn_zero_ext_kernel write them.
constexpr int kGenD = 64;
constexpr int kGenWaves = kThreads / kWave;

__device__ __forceinline__ float wave_sum_all(float v) {
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) v += __shfl_xor(v, m, kWave);
  return v;
}

__global__ void __launch_bounds__(kThreads) gdn_generic_kernel(GdnArgs a) {
  __shared__ float qk_all[kGenWaves][2][kGenD];   // this wave's normalised q, k
  const int wv = threadIdx.x / kWave, lane = threadIdx.x & (kWave - 1);
  const int64_t item = (int64_t)blockIdx.x * kGenWaves + wv;
  if (item >= (int64_t)a.batch * a.hv) return;
  const int bi = (int)(item / a.hv), h = (int)(item % a.hv);
  const int hk = h / a.vpk;
  const int dk = a.dk, dv = a.dv;
  const bool col = lane < dv;
  const int64_t r = a.req[bi];
  if (r < 0 || r >= a.n_slots) {
    if (!a.tok && col) {
      a.out[(int64_t)bi * a.out_rs + h * dv + lane] = 0;
      if (a.core) a.core[(int64_t)bi * a.core_rs + h * dv + lane] = 0;
    }
    return;
  }
  int t0 = bi, t1 = bi + 1;
  if (a.tok) {
    t0 = min(max(a.tok[bi], 0), a.rows);
    t1 = max(min(max(a.tok[bi + 1], 0), a.rows), t0);
  }
  float (*qk)[kGenD] = qk_all[wv];
  qk[0][lane] = 0.f;   // entries dk .. 63 stay zero: they add nothing below
  qk[1][lane] = 0.f;
  float* S = a.ssm + r * a.ssm_ss + (int64_t)h * dk * dv;
  float s[kGenD];
#pragma unroll
  for (int k = 0; k < kGenD; ++k) s[k] = (col && k < dk) ? S[k * dv + lane] : 0.f;
  for (int row = t0; row < t1; ++row) {
    const uint16_t* y = a.ws + (int64_t)row * a.conv_dim;
    const float qv = lane < dk ? bf(y[hk * dk + lane]) : 0.f;
    const float kv = lane < dk ? bf(y[a.key_dim + hk * dk + lane]) : 0.f;
    const float nq = sqrtf(wave_sum_all(qv * qv)), nk = sqrtf(wave_sum_all(kv * kv));
    if (lane < dk) {   // F.normalize (eps 1e-12), q also times dk^-0.5
      qk[0][lane] = qv / fmaxf(nq, 1e-12f) * a.qscale;
      qk[1][lane] = kv / fmaxf(nk, 1e-12f);
    }
    wave_lds_sync();   // every lane reads every entry below
    const float x = bf(a.a[(int64_t)row * a.ab_rs + h]) + a.dt_bias[h];
    const float sp = x > 20.f ? x : log1pf(expf(x));           // F.softplus
    const float alpha = expf(-expf(a.a_log[h]) * sp);
    const float beta = 1.f / (1.f + expf(-bf(a.b[(int64_t)row * a.ab_rs + h])));
    const float v = col ? bf(y[2 * a.key_dim + h * dv + lane]) : 0.f;
    float vp = 0.f;
#pragma unroll
    for (int k = 0; k < kGenD; ++k) {
      s[k] *= alpha;
      vp += s[k] * qk[1][k];
    }
    const float delta = beta * (v - vp);
    float o = 0.f;
#pragma unroll
    for (int k = 0; k < kGenD; ++k) {
      s[k] += qk[1][k] * delta;
      o += s[k] * qk[0][k];
    }
    o = round_bf(o);                                            // .to(orig_dtype)
    if (col && a.core) a.core[(int64_t)row * a.core_rs + h * dv + lane] = to_bf(o);
    const float var = wave_sum_all(col ? o * o : 0.f) / (float)dv;
    if (col) {
      const float zz = bf(a.z[(int64_t)row * a.z_rs + h * dv + lane]);
      const float xn = o * rsqrtf(var + a.eps);
      a.out[(int64_t)row * a.out_rs + h * dv + lane] =
          to_bf(a.norm_w[h * dv + lane] * xn * (zz / (1.f + expf(-zz))));
    }
    wave_lds_sync();   // the reads above finish before the next row overwrites qk
  }
#pragma unroll
  for (int k = 0; k < kGenD; ++k)
    if (col && k < dk) S[k * dv + lane] = s[k];
}

// Rows that no request owns, or whose request's slot is outside the pool,
// read as zeros in out and core_out; gdn_recur_kernel and gdn_chunk_ext_kernel
// write every other row.  One wave per row.
constexpr int kZeroRows = kThreads / kWave;   // rows per workgroup

__global__ void __launch_bounds__(kThreads) gdn_zero_ext_kernel(GdnArgs a) {
  const int64_t tok = (int64_t)blockIdx.x * kZeroRows + wave_id();
  if (tok >= a.rows || a.owner[tok] >= 0) return;
  zero_row(a, tok, threadIdx.x & (kWave - 1), kWave);
}

}  // namespace

// Decode workspace: bf16 conv outputs [B, conv_dim], then the fp32 gates
// (log alpha, beta) [B, Hv, 2].
inline int64_t gdn_dec_ws_bytes(int64_t batch, int64_t conv_dim, int32_t hv) {
  return batch * (conv_dim * 2 + (int64_t)hv * 8);
}
}  // namespace tfa

extern "C" {

int64_t tf_gdn_decode_workspace_bytes(int32_t batch_size, int32_t num_k_heads,
                                      int32_t num_v_heads) {
  tfa::clear_error();
  if (batch_size < 0 || num_k_heads <= 0 || num_v_heads <= 0)
    return tfa::fail(TF_ERR_INVALID, "gdn_decode_workspace_bytes: bad arguments");
  const int64_t conv_dim = 2LL * num_k_heads * tfa::kDk + (int64_t)num_v_heads * tfa::kDv;
  return tfa::gdn_dec_ws_bytes(batch_size, conv_dim, num_v_heads);
}

namespace tfa {
// Extend workspace bytes per token row: conv outputs (bf16), normalised q / k
// (bf16 high and low parts), gates (fp32) and the row's request (int32).
int64_t gdn_ext_row_bytes(int32_t hk, int32_t hv) {
  const int64_t conv_dim = 2LL * hk * kDk + (int64_t)hv * kDv;
  return conv_dim * 2 + (int64_t)hk * 4 * kDk * 2 + (int64_t)hv * 2 * 4 + 4;
}
// Chunk-record slots: chunk ci of request b is slot floor(t0_b / 32) + b + ci.
int64_t gdn_chunk_slots(int64_t n_tokens, int32_t batch) { return n_tokens / kChunk + batch + 1; }
// Per-token rows (16-byte aligned), then the chunk records, then the SiLU table.
int64_t gdn_ext_ws_bytes(int64_t n_tokens, int32_t batch, int32_t hk, int32_t hv) {
  return ((n_tokens * gdn_ext_row_bytes(hk, hv) + 64) & ~15LL) +
         gdn_chunk_slots(n_tokens, batch) * hv * kRec * 4 + kSiluTab * 2;
}
}  // namespace tfa

namespace {

// Validates the arguments shared by the decode and extend entry points and
// fills the kernel arguments; rows = tokens (extend) or requests (decode).
int32_t gdn_setup(const char* fn, const void* qkv, int64_t qkv_row_stride, const void* a,
                  const void* b, int64_t ab_row_stride, const void* z, int64_t z_row_stride,
                  const float* conv_weight, const float* a_log, const float* dt_bias,
                  const float* norm_weight, float eps, void* conv_state,
                  int64_t conv_slot_stride, float* ssm_state, int64_t ssm_slot_stride,
                  const int64_t* req_indices, int32_t batch_size, int64_t rows, int64_t n_slots,
                  int32_t num_k_heads, int32_t num_v_heads, int32_t head_k_dim,
                  int32_t head_v_dim, int32_t conv_kernel, void* out, int64_t out_row_stride,
                  void* core_out, int64_t core_row_stride, void* workspace,
                  int64_t workspace_bytes, tfa::GdnArgs* g) {
  using namespace tfa;
  const bool tuned = head_k_dim == kDk && head_v_dim == kDv;
  const bool other = head_k_dim >= 4 && head_k_dim <= kGenD && head_k_dim % 4 == 0 &&
                     head_v_dim >= 4 && head_v_dim <= kGenD && head_v_dim % 4 == 0;
  if ((!tuned && !other) || conv_kernel != 4)
    return fail(TF_ERR_UNSUPPORTED,
                "%s: head_k_dim=%d head_v_dim=%d conv_kernel=%d (128 / 128, or multiples of 4 "
                "up to %d; conv kernel 4)", fn, head_k_dim, head_v_dim, conv_kernel, kGenD);
  if (num_k_heads <= 0 || num_v_heads <= 0 || num_v_heads % num_k_heads)
    return fail(TF_ERR_INVALID, "%s: %d value heads over %d key heads", fn, num_v_heads,
                num_k_heads);
  if (batch_size < 0 || n_slots <= 0 || rows < 0)
    return fail(TF_ERR_INVALID, "%s: batch_size=%d n_slots=%lld", fn, batch_size,
                (long long)n_slots);
  const int64_t key_dim = (int64_t)num_k_heads * head_k_dim;
  const int64_t value_dim = (int64_t)num_v_heads * head_v_dim;
  const int64_t conv_dim = 2 * key_dim + value_dim;
  if (!qkv || !a || !b || !z || !conv_weight || !a_log || !dt_bias || !norm_weight ||
      !conv_state || !ssm_state || !req_indices || !out || !workspace)
    return fail(TF_ERR_INVALID, "%s: null pointer", fn);
  if (workspace_bytes < rows * conv_dim * 2 || (reinterpret_cast<uintptr_t>(workspace) & 1u))
    return fail(TF_ERR_INVALID, "%s: workspace of %lld bytes (needs %lld)", fn,
                (long long)workspace_bytes, (long long)(rows * conv_dim * 2));
  if (qkv_row_stride < conv_dim || ab_row_stride < num_v_heads || z_row_stride < value_dim ||
      out_row_stride < value_dim || (core_out && core_row_stride < value_dim) ||
      conv_slot_stride < 3 * conv_dim || ssm_slot_stride < value_dim * head_k_dim)
    return fail(TF_ERR_INVALID, "%s: a row or slot stride is too small", fn);
  if (!aligned16(conv_weight) || !aligned16(ssm_state) || ssm_slot_stride % 4)
    return fail(TF_ERR_INVALID, "%s: conv_weight / ssm_state must be 16-byte aligned", fn);
  if (rows * conv_dim > INT32_MAX || rows * qkv_row_stride > INT64_MAX / 4)
    return fail(TF_ERR_UNSUPPORTED, "%s: too many rows", fn);
  g->qkv = static_cast<const uint16_t*>(qkv);
  g->qkv_rs = qkv_row_stride;
  g->a = static_cast<const uint16_t*>(a);
  g->b = static_cast<const uint16_t*>(b);
  g->ab_rs = ab_row_stride;
  g->z = static_cast<const uint16_t*>(z);
  g->z_rs = z_row_stride;
  g->conv_w = conv_weight;
  g->a_log = a_log;
  g->dt_bias = dt_bias;
  g->norm_w = norm_weight;
  g->eps = eps;
  g->conv_state = static_cast<uint16_t*>(conv_state);
  g->conv_ss = conv_slot_stride;
  g->ssm = ssm_state;
  g->ssm_ss = ssm_slot_stride;
  g->req = req_indices;
  g->n_slots = n_slots;
  g->batch = batch_size;
  g->hv = num_v_heads;
  g->vpk = num_v_heads / num_k_heads;
  g->key_dim = (int32_t)key_dim;
  g->conv_dim = (int32_t)conv_dim;
  g->tok = nullptr;
  g->rows = (int32_t)rows;
  g->hk = num_k_heads;
  g->dk = head_k_dim;
  g->dv = head_v_dim;
  g->qscale = (float)(1.0 / sqrt((double)head_k_dim));
  g->wqk = nullptr;
  g->wg = nullptr;
  g->owner = nullptr;
  g->silu_tab = nullptr;
  g->wrec = nullptr;
  g->ws = static_cast<uint16_t*>(workspace);
  g->out = static_cast<uint16_t*>(out);
  g->out_rs = out_row_stride;
  g->core = static_cast<uint16_t*>(core_out);
  g->core_rs = core_row_stride;
  return TF_OK;
}

// A second stream per device for tf_gdn_extend: the one-token requests'
// recurrence runs there beside the chunked pass.  That pass holds one
// workgroup per (multi-token request, value head) for the whole extend at a
// small share of the HBM bandwidth, so the HBM-bound one-token updates fit
// beside it (they touch other state slots and output rows, so the two need
// no order between them).  The stream and its fork / join events are made on
// the first call that is not under graph capture, and only calls that are not
// under capture use them; `mu` keeps the fork .. join sequences of concurrent
// callers apart.
struct SideLane {
  std::mutex mu;
  hipStream_t stream = nullptr;
  hipEvent_t fork = nullptr, join = nullptr;
  bool ready = false;
};
constexpr int kLaneDevices = 64;
SideLane g_lanes[kLaneDevices];

// The lane of the stream's device, or nullptr when there is none to use (a
// first call under capture, an unknown device or a creation error: the caller
// then launches everything on its own stream).  Clears the HIP error of a
// failed query, so the caller checks its own launches before calling this.
SideLane* side_lane(hipStream_t s) {
  int dev = -1;
  if (s) {
    hipDevice_t d = -1;
    if (hipStreamGetDevice(s, &d) != hipSuccess) {
      (void)hipGetLastError();
      return nullptr;
    }
    dev = d;
  } else if (hipGetDevice(&dev) != hipSuccess) {
    (void)hipGetLastError();
    return nullptr;
  }
  if (dev < 0 || dev >= kLaneDevices) return nullptr;
  SideLane& L = g_lanes[dev];
  std::lock_guard<std::mutex> lock(L.mu);
  if (L.ready) return &L;
  hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
  int cur = -1;
  if (hipStreamIsCapturing(s, &cs) != hipSuccess || cs != hipStreamCaptureStatusNone ||
      hipGetDevice(&cur) != hipSuccess || (cur != dev && hipSetDevice(dev) != hipSuccess)) {
    (void)hipGetLastError();
    return nullptr;
  }
  const bool ok = hipStreamCreateWithFlags(&L.stream, hipStreamNonBlocking) == hipSuccess &&
                  hipEventCreateWithFlags(&L.fork, hipEventDisableTiming) == hipSuccess &&
                  hipEventCreateWithFlags(&L.join, hipEventDisableTiming) == hipSuccess;
  if (!ok) {
    if (L.join) (void)hipEventDestroy(L.join);
    if (L.fork) (void)hipEventDestroy(L.fork);
    if (L.stream) (void)hipStreamDestroy(L.stream);
    L.stream = nullptr;
    L.fork = L.join = nullptr;
  }
  if (cur != dev) (void)hipSetDevice(cur);
  (void)hipGetLastError();
  L.ready = ok;
  return ok ? &L : nullptr;
}

int32_t side_failure(const char* what, hipError_t e) {
  (void)hipGetLastError();
  return tfa::fail(TF_ERR_HIP, "tf_gdn_extend: %s: %s", what, hipGetErrorString(e));
}

}  // namespace

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
  if (batch_size == 0) return TF_OK;
  GdnArgs g;
  const int32_t rc = gdn_setup(
      "gdn_decode", qkv, qkv_row_stride, a, b, ab_row_stride, z, z_row_stride, conv_weight,
      a_log, dt_bias, norm_weight, eps, conv_state, conv_slot_stride, ssm_state,
      ssm_slot_stride, req_indices, batch_size, batch_size, n_slots, num_k_heads, num_v_heads,
      head_k_dim, head_v_dim, conv_kernel, out, out_row_stride, core_out, core_row_stride,
      workspace, workspace_bytes, &g);
  if (rc != TF_OK) return rc;
  const int64_t need = gdn_dec_ws_bytes(batch_size, g.conv_dim, num_v_heads);
  if (workspace_bytes < need || (reinterpret_cast<uintptr_t>(workspace) & 15u))
    return fail(TF_ERR_INVALID, "gdn_decode: workspace of %lld bytes (needs %lld, 16-byte aligned)",
                (long long)workspace_bytes, (long long)need);
  g.wg = reinterpret_cast<float*>(static_cast<uint8_t*>(workspace) +
                                  (int64_t)batch_size * g.conv_dim * 2);
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  const int64_t n_conv = (int64_t)batch_size * (g.conv_dim / 4);   // 4 channels per thread
  hipLaunchKernelGGL(gdn_conv_kernel, dim3((n_conv + kThreads - 1) / kThreads), dim3(kThreads),
                     0, s, g);
  if (g.dk != kDk)
    hipLaunchKernelGGL(gdn_generic_kernel,
                       dim3((uint32_t)(((int64_t)batch_size * num_v_heads + kGenWaves - 1) /
                                       kGenWaves)),
                       dim3(kThreads), 0, s, g);
  else
    hipLaunchKernelGGL(gdn_recur_kernel, dim3((int64_t)batch_size * num_v_heads), dim3(kThreads),
                       0, s, g);
  return launch_status("tf_gdn_decode launch");
}

int64_t tf_gdn_extend_workspace_bytes(int64_t n_tokens, int32_t batch_size,
                                      int32_t num_k_heads, int32_t num_v_heads) {
  tfa::clear_error();
  if (n_tokens < 0 || batch_size < 0 || num_k_heads <= 0 || num_v_heads <= 0)
    return tfa::fail(TF_ERR_INVALID, "gdn_extend_workspace_bytes: bad arguments");
  return tfa::gdn_ext_ws_bytes(n_tokens, batch_size, num_k_heads, num_v_heads);
}

int32_t tf_gdn_extend(const void* qkv, int64_t qkv_row_stride, const void* a, const void* b,
                      int64_t ab_row_stride, const void* z, int64_t z_row_stride,
                      const float* conv_weight, const float* a_log, const float* dt_bias,
                      const float* norm_weight, float eps, void* conv_state,
                      int64_t conv_slot_stride, float* ssm_state, int64_t ssm_slot_stride,
                      const int64_t* req_indices, const int32_t* token_offsets,
                      int32_t batch_size, int64_t n_tokens, int32_t max_extend_len,
                      int64_t n_slots,
                      int32_t num_k_heads, int32_t num_v_heads, int32_t head_k_dim,
                      int32_t head_v_dim, int32_t conv_kernel, void* out,
                      int64_t out_row_stride, void* core_out, int64_t core_row_stride,
                      void* workspace, int64_t workspace_bytes, tf_stream_t stream) {
  using namespace tfa;
  clear_error();
  if (batch_size == 0 || n_tokens == 0) return TF_OK;
  if (!token_offsets) return fail(TF_ERR_INVALID, "gdn_extend: null token_offsets");
  if (max_extend_len < 0 || max_extend_len > n_tokens)
    return fail(TF_ERR_INVALID, "gdn_extend: max_extend_len=%d", max_extend_len);
  if (batch_size > 65535) return fail(TF_ERR_UNSUPPORTED, "gdn_extend: batch_size > 65535");
  GdnArgs g;
  const int32_t rc = gdn_setup(
      "gdn_extend", qkv, qkv_row_stride, a, b, ab_row_stride, z, z_row_stride, conv_weight,
      a_log, dt_bias, norm_weight, eps, conv_state, conv_slot_stride, ssm_state,
      ssm_slot_stride, req_indices, batch_size, n_tokens, n_slots, num_k_heads, num_v_heads,
      head_k_dim, head_v_dim, conv_kernel, out, out_row_stride, core_out, core_row_stride,
      workspace, workspace_bytes, &g);
  if (rc != TF_OK) return rc;
  const int64_t need = gdn_ext_ws_bytes(n_tokens, batch_size, num_k_heads, num_v_heads);
  if (workspace_bytes < need || (reinterpret_cast<uintptr_t>(workspace) & 15u))
    return fail(TF_ERR_INVALID, "gdn_extend: workspace of %lld bytes (needs %lld, 16-byte aligned)",
                (long long)workspace_bytes, (long long)need);
  const int64_t n_slots_rec = gdn_chunk_slots(n_tokens, batch_size);
  if (n_tokens > 65535LL * kConvTokens || n_tokens * num_k_heads * 4 * kDk * 2 > UINT32_MAX ||
      n_tokens * g.conv_dim * 2 > UINT32_MAX || n_tokens * num_v_heads * 8 > UINT32_MAX ||
      n_slots_rec * num_v_heads * kRec * 4 > UINT32_MAX || z_row_stride * 2 * kChunk > UINT32_MAX)
    return fail(TF_ERR_UNSUPPORTED, "gdn_extend: too many tokens (32-bit staging offsets)");
  if ((reinterpret_cast<uintptr_t>(qkv) & 7u) || qkv_row_stride % 4 ||
      (reinterpret_cast<uintptr_t>(z) & 7u) || z_row_stride % 4 ||
      (reinterpret_cast<uintptr_t>(out) & 7u) || out_row_stride % 4 ||
      (core_out && ((reinterpret_cast<uintptr_t>(core_out) & 7u) || core_row_stride % 4)) ||
      !aligned16(norm_weight))
    return fail(TF_ERR_INVALID,
                "gdn_extend: qkv, z, out and core_out must be 8-byte aligned with row strides "
                "that are multiples of 4; norm_weight 16-byte aligned");
  g.tok = token_offsets;
  uint8_t* w = static_cast<uint8_t*>(workspace);
  const int64_t conv_bytes = n_tokens * g.conv_dim * 2;
  const int64_t qk_bytes = n_tokens * num_k_heads * 4 * kDk * 2;
  const int64_t gate_bytes = n_tokens * num_v_heads * 2 * 4;
  g.wqk = reinterpret_cast<uint16_t*>(w + ((conv_bytes + 15) & ~15LL));
  g.wg = reinterpret_cast<float*>(reinterpret_cast<uint8_t*>(g.wqk) + qk_bytes);
  g.owner = reinterpret_cast<int32_t*>(reinterpret_cast<uint8_t*>(g.wg) + gate_bytes);
  g.wrec = reinterpret_cast<float*>(w + ((n_tokens * gdn_ext_row_bytes(num_k_heads, num_v_heads) +
                                          64) & ~15LL));
  g.silu_tab = reinterpret_cast<uint16_t*>(g.wrec + n_slots_rec * num_v_heads * kRec);
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  const uint32_t cblocks = (g.conv_dim + kThreads - 1) / kThreads;
  const uint32_t tblocks = (uint32_t)((n_tokens + kConvTokens - 1) / kConvTokens);
  hipLaunchKernelGGL(gdn_owner_kernel,
                     dim3((uint32_t)((std::max<int64_t>(n_tokens, kSiluTab) + kThreads - 1) /
                                     kThreads)),
                     dim3(kThreads), 0, s, g);
  hipLaunchKernelGGL(gdn_conv_ext_kernel,
                     dim3((g.conv_dim / kConvCh + kThreads - 1) / kThreads,
                          std::min<uint32_t>(tblocks, kConvRowWgs)),
                     dim3(kThreads), 0, s, g);
  if (g.dk != kDk) {   // other head dims: every request's rows in one wave per value head
    hipLaunchKernelGGL(gdn_conv_state_kernel, dim3(cblocks, batch_size), dim3(kThreads), 0, s,
                       g);
    hipLaunchKernelGGL(gdn_generic_kernel,
                       dim3((uint32_t)(((int64_t)batch_size * num_v_heads + kGenWaves - 1) /
                                       kGenWaves)),
                       dim3(kThreads), 0, s, g);
    hipLaunchKernelGGL(gdn_zero_ext_kernel,
                       dim3((uint32_t)((n_tokens + kZeroRows - 1) / kZeroRows)), dim3(kThreads),
                       0, s, g);
    return launch_status("tf_gdn_extend launch");
  }
  hipLaunchKernelGGL(gdn_qk_ext_kernel,
                     dim3((uint32_t)n_tokens,
                          (num_k_heads + 2 * kThreads / kWave - 1) / (2 * kThreads / kWave)),
                     dim3(kThreads), 0, s, g);
  hipLaunchKernelGGL(gdn_chunk_prep_kernel, dim3((uint32_t)n_slots_rec, num_k_heads),
                     dim3(kThreads), 0, s, g);
  const int32_t pre = launch_status("tf_gdn_extend launch");
  if (pre != TF_OK) return pre;
  // The one-token recurrence on the side stream, beside the chunked pass,
  // when the batch can hold both kinds of request; it needs only the conv
  // outputs, and the caller's stream waits for it before the call's end.
  // A call under graph capture keeps everything on the caller's stream: the
  // side stream, once joined into a capture, would stay in capture mode until
  // that capture ends, and an eager call from another thread would then
  // launch onto it.
  hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
  const bool capturing =
      hipStreamIsCapturing(s, &cs) != hipSuccess || cs != hipStreamCaptureStatusNone;
  (void)hipGetLastError();
  SideLane* lane =
      (!capturing && max_extend_len > 1 && batch_size > 1) ? side_lane(s) : nullptr;
  std::unique_lock<std::mutex> held;
  hipStream_t rs = s;
  if (lane) {
    held = std::unique_lock<std::mutex>(lane->mu);
    hipError_t e = hipEventRecord(lane->fork, s);
    if (e == hipSuccess) e = hipStreamWaitEvent(lane->stream, lane->fork, 0);
    if (e != hipSuccess) return side_failure("fork to the side stream", e);
    rs = lane->stream;
  }
  hipLaunchKernelGGL(gdn_recur_kernel, dim3((int64_t)batch_size * num_v_heads), dim3(kThreads), 0,
                     rs, g);
  if (lane) {
    const hipError_t e = hipEventRecord(lane->join, rs);
    if (e != hipSuccess) return side_failure("join event", e);
  }
  hipLaunchKernelGGL(gdn_chunk_ext_kernel, dim3((int64_t)batch_size * num_v_heads),
                     dim3(kChunkThreads), 0, s, g);
  if (lane) {
    const hipError_t e = hipStreamWaitEvent(s, lane->join, 0);
    if (e != hipSuccess) return side_failure("join with the side stream", e);
  }
  return launch_status("tf_gdn_extend launch");
}

}  // extern "C"
