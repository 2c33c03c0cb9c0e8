// Slot attention for head dims other than 256: decode and extend rows of any
// head_dim that is a multiple of 8, up to 256 (the reference's own test
// configurations use head_dim 32).  tf_attn_decode / tf_attn_extend route
// here when head_dim != 256; the 256-dim kernels (decode.hip, extend.hip) are
// the tuned paths of the 27B model.
//
// Same semantics as those kernels (qwen3_8/full_attention.py:163-283): row
// (token t, q head h) of request b attends to context positions 0 .. P + t,
// P = L_b - ext_b, q head h reads kv head h / G, slot ids come from
// req_to_token (negative ids index from the pool's end in a bsz == 1 call,
// then every id is clamped into the pool), fp8-e4m3 pools are read with their
// per-tensor scales, and the optional output gate is applied to the rounded
// output as bf16(bf16(o) * bf16(silu(g))).
//
// One wave per query row.  Keys go 64 at a time: lane j scores key k0 + j
// against the whole q row (held by every lane as packed bf16), the wave takes
// the tile's max and sum, and each lane accumulates two output dims (2l, 2l + 1,
// and 128 + 2l, 129 + 2l for head_dim > 128) over the tile's keys in fp32.
#include <math.h>

#include "tf_common.h"
#include "tf_internal.h"

namespace tfa {

namespace {

constexpr int kGenWaves = 4;
constexpr int kGenThreads = kGenWaves * kWave;
constexpr int kGenMaxD = 256;

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) v += __shfl_xor(v, m, kWave);
  return v;
}
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) v = fmaxf(v, __shfl_xor(v, m, kWave));
  return v;
}

// 8 elements of a K or V row (bf16, or e4m3 when FP8) at element offset e.
template <bool FP8>
__device__ __forceinline__ void load8(const uint8_t* row, int e, float (&x)[8]) {
  if (FP8) {
    const u32x2 r = *reinterpret_cast<const u32x2*>(row + e);
    const u32x4 b = e4m3x8_to_bf16x8(r[0], r[1]);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      x[2 * i] = __uint_as_float(b[i] << 16);
      x[2 * i + 1] = __uint_as_float(b[i] & 0xffff0000u);
    }
  } else {
    const u32x4 r = *reinterpret_cast<const u32x4*>(row + 2 * e);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      x[2 * i] = __uint_as_float(r[i] << 16);
      x[2 * i + 1] = __uint_as_float(r[i] & 0xffff0000u);
    }
  }
}

// Two consecutive elements of a row at element offset e (e even).
template <bool FP8>
__device__ __forceinline__ void load2(const uint8_t* row, int e, float& x0, float& x1) {
  if (FP8) {
    const uint32_t b = e4m3x2_to_bf16x2<false>(*reinterpret_cast<const uint16_t*>(row + e));
    x0 = __uint_as_float(b << 16);
    x1 = __uint_as_float(b & 0xffff0000u);
  } else {
    const uint32_t r = *reinterpret_cast<const uint32_t*>(row + 2 * e);
    x0 = __uint_as_float(r << 16);
    x1 = __uint_as_float(r & 0xffff0000u);
  }
}

template <bool FP8>
__global__ void __launch_bounds__(kGenThreads) generic_attn_kernel(GenericAttnArgs a) {
  const int lane = threadIdx.x & (kWave - 1);
  const int64_t wid = (int64_t)blockIdx.x * kGenWaves + threadIdx.x / kWave;
  const int G = a.hq / a.hkv;
  const int D = a.head_dim;

  // This wave's query row.
  int b, h, hk;
  int64_t qrow, limit, L;
  if (a.work) {   // extend: work entry wid / 256, row (wid % 256) of it
    const int64_t e = wid / kExtendItemRows;
    if (e >= a.n_rows) return;
    const int32_t* wk = a.work + 8 * e;
    const int ext = wk[4];
    if (ext <= 0) return;                      // padding entry of a device-built list
    const int r = wk[2] + (int)(wid % kExtendItemRows);
    if (r >= ext * G) return;
    b = wk[0];
    hk = wk[1];
    const int t = r / G;
    h = hk * G + r % G;
    qrow = (int64_t)wk[3] + t;
    L = a.seq_override > 0 ? (int64_t)a.seq_override : a.seq_lens[b];
    if (L > a.rtt_cols) L = a.rtt_cols;
    limit = L - ext + t;                       // last visible key
  } else {        // decode: item wid / hq, head wid % hq
    const int64_t i = wid / a.hq;
    if (i >= a.n_rows) return;
    b = a.items ? a.items[i] : (int)i;
    if (b < 0) return;                         // padding item
    qrow = a.q_rows ? a.q_rows[i] : b;
    h = (int)(wid % a.hq);
    hk = h / G;
    L = a.seq_override > 0 ? (int64_t)a.seq_override : a.seq_lens[b];
    if (L > a.rtt_cols) L = a.rtt_cols;
    limit = L - 1;
  }
  // A row with no visible key (a decode item with seq_len 0, an extend row
  // past a too-short context) is all zeros, as the reference's fully masked
  // scaled_dot_product_attention returns it and as the tuned kernels write it.
  const int64_t nkeys = limit + 1;

  const int64_t rrow = clamp_i64(a.rpi[b], 0, a.rtt_rows - 1);
  const int64_t* rtt = a.rtt + rrow * a.rtt_stride;
  const bool wrap = a.seq_override > 0;
  const int esz = FP8 ? 1 : 2;
  const int64_t row_bytes = (int64_t)a.hkv * D * esz;
  const uint8_t* kbase = a.k_pool + (int64_t)hk * D * esz;
  const uint8_t* vbase = a.v_pool + (int64_t)hk * D * esz;

  // q row, packed bf16, in this wave's LDS row (every lane reads the same
  // word: a broadcast).  Only this wave touches it; wave_lds_sync orders
  // every lane's writes before any lane's reads.
  __shared__ uint32_t qs_all[kGenWaves][kGenMaxD / 2];
  uint32_t* q = qs_all[threadIdx.x / kWave];
  const uint32_t* qp =
      reinterpret_cast<const uint32_t*>(a.q + qrow * a.q_stride + (int64_t)h * D);
  for (int i = lane; i < D / 2; i += kWave) q[i] = qp[i];
  wave_lds_sync();

  const float sl2 = a.scale_log2 * (FP8 ? a.k_scale[0] : 1.f);
  float m = -INFINITY, l = 0.f;
  float acc[4] = {0.f, 0.f, 0.f, 0.f};   // dims 2l, 2l + 1, 128 + 2l, 129 + 2l
  const int d0 = 2 * lane, d1 = 128 + 2 * lane;

  for (int64_t k0 = 0; k0 < nkeys; k0 += kWave) {
    const int64_t k = k0 + lane;
    const bool live = k < nkeys;
    const int64_t slot = live ? pool_row(rtt[k], a.pool_slots, wrap) : 0;
    float s = -INFINITY;
    if (live) {
      const uint8_t* kr = kbase + slot * row_bytes;
      float dot = 0.f;
      for (int e = 0; e < D; e += 8) {
        float x[8];
        load8<FP8>(kr, e, x);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const uint32_t qq = q[(e >> 1) + i];
          dot = fmaf(__uint_as_float(qq << 16), x[2 * i], dot);
          dot = fmaf(__uint_as_float(qq & 0xffff0000u), x[2 * i + 1], dot);
        }
      }
      s = dot * sl2;
    }
    const float mt = wave_max(s);
    const float mnew = fmaxf(m, mt);           // finite: key k0 is live
    const float alpha = exp2f(m - mnew);
    const float p = live ? exp2f(s - mnew) : 0.f;
    l = l * alpha + wave_sum(p);
#pragma unroll
    for (int i = 0; i < 4; ++i) acc[i] *= alpha;
    m = mnew;
    const int n = (int)min<int64_t>(kWave, nkeys - k0);
    for (int j = 0; j < n; ++j) {
      const float pj = __shfl(p, j, kWave);
      const int64_t sj = __shfl(slot, j, kWave);
      const uint8_t* vr = vbase + sj * row_bytes;
      if (d0 < D) {
        float x0, x1;
        load2<FP8>(vr, d0, x0, x1);
        acc[0] = fmaf(pj, x0, acc[0]);
        acc[1] = fmaf(pj, x1, acc[1]);
      }
      if (d1 < D) {
        float x0, x1;
        load2<FP8>(vr, d1, x0, x1);
        acc[2] = fmaf(pj, x0, acc[2]);
        acc[3] = fmaf(pj, x1, acc[3]);
      }
    }
  }

  const float inv = nkeys > 0 ? (FP8 ? a.v_scale[0] : 1.f) / l : 0.f;
  __bf16* orow = a.out + qrow * a.out_stride + (int64_t)h * D;
  const __bf16* grow = a.gate ? a.gate + qrow * a.gate_stride + (int64_t)h * a.gate_hstride
                              : nullptr;
  uint32_t omax = 0;
#pragma unroll
  for (int u = 0; u < 2; ++u) {
    const int d = u ? d1 : d0;
    if (d >= D) continue;
    uint32_t o = pack_bf16(acc[2 * u] * inv, acc[2 * u + 1] * inv);
    if (grow) o = gate_pair(o, *reinterpret_cast<const uint32_t*>(grow + d));
    omax = max(omax, max(o & 0x7fffu, (o >> 16) & 0x7fffu));
    *reinterpret_cast<uint32_t*>(orow + d) = o;
  }
  amax_commit(a.amax, omax);
}

}  // namespace

bool generic_head_dim(int32_t head_dim) {
  return head_dim != 256 && head_dim >= 8 && head_dim <= kGenMaxD && head_dim % 8 == 0;
}

int launch_generic_attn(const GenericAttnArgs& a, hipStream_t stream) {
  const int64_t waves = a.work ? (int64_t)a.n_rows * kExtendItemRows : (int64_t)a.n_rows * a.hq;
  const int64_t blocks = (waves + kGenWaves - 1) / kGenWaves;
  if (blocks <= 0) return TF_OK;
  if (blocks > INT32_MAX) return fail(TF_ERR_INVALID, "attention: too many rows");
  if (a.fp8)
    hipLaunchKernelGGL(generic_attn_kernel<true>, dim3((unsigned)blocks), dim3(kGenThreads), 0,
                       stream, a);
  else
    hipLaunchKernelGGL(generic_attn_kernel<false>, dim3((unsigned)blocks), dim3(kGenThreads), 0,
                       stream, a);
  return launch_status("generic attention launch");
}

}  // namespace tfa
