// Device-side planning of one attention step: the extend work list of
// tf_attn_plan_extend and the decode item list of tf_attn_plan_decode_items,
// built on the GPU from the device extend_lens, so a step needs no host loop
// and no host->device copy and can be captured in a HIP graph.
//
// The host-side bookkeeping this replaces is the reference's per-step index
// work around the extend branch (qwen3_8/full_attention.py:250-265: q_start
// prefix sums and the per-request row split) and the caller's per-step host
// metadata (engine/model_runner.py:108-188).  The lists are identical to the
// host planners' (same order: largest extend first, later row tiles first, kv
// heads inner) and are padded to capacities the host knows without reading
// device memory:
//   work:  kv_heads * (ceil(T * G / 256) + B) entries, padding {0,0,0,0,0,...}
//          (ext 0: the extend kernels skip it);
//   decode items: B entries, padding -1 (the decode kernels skip it).
#include "tf_common.h"
#include "tf_internal.h"

namespace tfa {
namespace {

constexpr int kPlanMaxBatch = 4096;
constexpr int kPlanThreads = 1024;
constexpr int kPlanPer = kPlanMaxBatch / kPlanThreads;   // requests per thread

struct PlanArgs {
  const int64_t* ext;
  int32_t batch, hkv, group, dec_to_dec;
  int32_t* work;
  int32_t work_cap;
  int32_t* dec_items;
  int32_t* dec_rows;
  int32_t dec_cap;
  int32_t* status;
};

struct PlanSmem {
  int32_t ext[kPlanMaxBatch];        // extend length per request (0 if absent)
  int32_t qs[kPlanMaxBatch];         // first q row of each request
  int32_t order[kPlanMaxBatch];      // extend requests, largest first
  int32_t off[kPlanMaxBatch + 1];    // first work entry of the request at rank r
  int64_t wsum[kPlanThreads / kWave];
};

// Exclusive block-wide prefix sum of one value per thread; returns the prefix
// and sets total.  All threads must call it.
__device__ int64_t block_scan(int64_t v, int64_t* wsum, int64_t& total) {
  const int lane = threadIdx.x & (kWave - 1);
  const int w = threadIdx.x / kWave;
  int64_t x = v;
#pragma unroll
  for (int d = 1; d < kWave; d <<= 1) {
    const int64_t y = __shfl_up(x, d, kWave);
    if (lane >= d) x += y;
  }
  __syncthreads();
  if (lane == kWave - 1) wsum[w] = x;
  __syncthreads();
  int64_t before = 0;
  total = 0;
  for (int k = 0; k < kPlanThreads / kWave; ++k) {
    if (k < w) before += wsum[k];
    total += wsum[k];
  }
  return before + x - v;
}

__global__ void __launch_bounds__(kPlanThreads) plan_kernel(PlanArgs a) {
  __shared__ PlanSmem sm;
  const int tid = threadIdx.x;
  const int G = a.group;

  // Requests tid * kPlanPer + k: lengths, q_start, decode / extend roles.
  int32_t e[kPlanPer];
  bool bad = false;
  int64_t tok = 0;
#pragma unroll
  for (int k = 0; k < kPlanPer; ++k) {
    const int b = tid * kPlanPer + k;
    int64_t x = b < a.batch ? a.ext[b] : 0;
    if (b < a.batch && (x < 1 || x > INT32_MAX)) {
      bad = true;
      x = 0;
    }
    e[k] = (int32_t)x;
    tok += x;
  }
  int64_t total_tok;
  int64_t q0 = block_scan(tok, sm.wsum, total_tok);
  int64_t q_start[kPlanPer];
  int ndec = 0, next = 0;
#pragma unroll
  for (int k = 0; k < kPlanPer; ++k) {
    q_start[k] = q0;
    sm.qs[tid * kPlanPer + k] = (int32_t)min<int64_t>(q0, INT32_MAX);
    q0 += e[k];
    const bool dec = e[k] == 1 && a.dec_to_dec;
    const bool ext = e[k] >= 1 && !dec;
    sm.ext[tid * kPlanPer + k] = ext ? e[k] : 0;
    ndec += dec;
    next += ext;
  }

  // Decode items in request order.
  int64_t n_dec64, n_ext64;
  int64_t d0 = block_scan(ndec, sm.wsum, n_dec64);
#pragma unroll
  for (int k = 0; k < kPlanPer; ++k) {
    if (e[k] == 1 && a.dec_to_dec) {
      if (d0 < a.dec_cap) {
        a.dec_items[d0] = tid * kPlanPer + k;
        a.dec_rows[d0] = (int32_t)q_start[k];
      }
      ++d0;
    }
  }
  (void)block_scan(next, sm.wsum, n_ext64);
  __syncthreads();   // sm.ext complete

  // Rank of each extend request: larger extend first, then request order.
#pragma unroll
  for (int k = 0; k < kPlanPer; ++k) {
    const int b = tid * kPlanPer + k;
    const int x = sm.ext[b];
    if (x == 0) continue;
    int rank = 0;
    for (int c = 0; c < a.batch; ++c) {
      const int y = sm.ext[c];
      rank += (y > x) || (y == x && y != 0 && c < b);
    }
    sm.order[rank] = b;
  }
  __syncthreads();

  // Work entries per rank: kv_heads x row tiles of the request.
  int64_t cnt = 0;
  int32_t n_r[kPlanPer];
#pragma unroll
  for (int k = 0; k < kPlanPer; ++k) {
    const int r = tid * kPlanPer + k;
    n_r[k] = 0;
    if (r < n_ext64) {
      const int64_t rows = (int64_t)sm.ext[sm.order[r]] * G;
      n_r[k] = (int32_t)(a.hkv * ((rows + kExtendItemRows - 1) / kExtendItemRows));
    }
    cnt += n_r[k];
  }
  int64_t n_work64;
  int64_t w0 = block_scan(cnt, sm.wsum, n_work64);
#pragma unroll
  for (int k = 0; k < kPlanPer; ++k) {
    sm.off[tid * kPlanPer + k] = (int32_t)min<int64_t>(w0, INT32_MAX);
    w0 += n_r[k];
  }
  if (tid == 0) sm.off[kPlanMaxBatch] = (int32_t)min<int64_t>(n_work64, INT32_MAX);
  __syncthreads();

  // Entries, one thread each: rank by binary search over the offsets, then
  // (tile from the last, kv head inner) within the request.  Entries past the
  // real ones are padding (ext 0).
  const int n_work = (int)min<int64_t>(n_work64, a.work_cap);
  for (int idx = tid; idx < a.work_cap; idx += kPlanThreads) {
    int32_t* wk = a.work + 8 * (int64_t)idx;
    int32_t v[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    if (idx < n_work) {
      int lo = 0, hi = (int)n_ext64 - 1;   // last rank with off <= idx
      while (lo < hi) {
        const int mid = (lo + hi + 1) >> 1;
        if (sm.off[mid] <= idx) lo = mid; else hi = mid - 1;
      }
      const int b = sm.order[lo];
      const int x = sm.ext[b];
      const int tiles = (int)(((int64_t)x * G + kExtendItemRows - 1) / kExtendItemRows);
      const int j = idx - sm.off[lo];
      const int t = tiles - 1 - j / a.hkv;
      v[0] = b;
      v[1] = j % a.hkv;
      v[2] = t * kExtendItemRows;
      v[3] = sm.qs[b];
      v[4] = x;
    }
#pragma unroll
    for (int q = 0; q < 8; ++q) wk[q] = v[q];
  }
  for (int i = (int)min<int64_t>(n_dec64, a.dec_cap) + tid; i < a.dec_cap; i += kPlanThreads) {
    a.dec_items[i] = -1;
    a.dec_rows[i] = 0;
  }
  const bool any_bad = __syncthreads_or(bad);
  if (tid == 0) {
    a.status[0] = (int32_t)min<int64_t>(n_work64, INT32_MAX);
    a.status[1] = (int32_t)n_dec64;
    a.status[2] = (any_bad ? 2 : 0) | (n_work64 > a.work_cap || n_dec64 > a.dec_cap ? 1 : 0);
  }
}

}  // namespace
}  // namespace tfa

extern "C" {

int64_t tf_attn_plan_device_capacity(int64_t total_tokens, int32_t batch_size,
                                     int32_t num_q_heads, int32_t num_kv_heads) {
  tfa::clear_error();
  if (total_tokens < 0 || batch_size < 0 || num_kv_heads <= 0 || num_q_heads <= 0 ||
      num_q_heads % num_kv_heads)
    return tfa::fail(TF_ERR_INVALID, "plan_device_capacity: bad arguments");
  const int64_t g = num_q_heads / num_kv_heads;
  return (int64_t)num_kv_heads *
         ((total_tokens * g + tfa::kExtendItemRows - 1) / tfa::kExtendItemRows + batch_size);
}

int32_t tf_attn_plan_device(const int64_t* extend_lens, int32_t batch_size,
                            int32_t num_q_heads, int32_t num_kv_heads,
                            int32_t decode_to_decode_kernel, int32_t* work,
                            int32_t work_capacity, int32_t* dec_items, int32_t* dec_rows,
                            int32_t dec_capacity, int32_t* status, tf_stream_t stream) {
  using namespace tfa;
  clear_error();
  if (batch_size < 0 || batch_size > kPlanMaxBatch)
    return fail(TF_ERR_UNSUPPORTED, "plan_device: batch_size=%d (at most %d)", batch_size,
                kPlanMaxBatch);
  if (num_kv_heads <= 0 || num_q_heads <= 0 || num_q_heads % num_kv_heads)
    return fail(TF_ERR_INVALID, "plan_device: heads %d/%d", num_q_heads, num_kv_heads);
  if (work_capacity < 0 || dec_capacity < 0 || !status ||
      (batch_size > 0 && !extend_lens) || (work_capacity > 0 && !work) ||
      (dec_capacity > 0 && (!dec_items || !dec_rows)))
    return fail(TF_ERR_INVALID, "plan_device: null pointer or negative capacity");
  PlanArgs a;
  a.ext = extend_lens;
  a.batch = batch_size;
  a.hkv = num_kv_heads;
  a.group = num_q_heads / num_kv_heads;
  a.dec_to_dec = decode_to_decode_kernel ? 1 : 0;
  a.work = work;
  a.work_cap = work_capacity;
  a.dec_items = dec_items;
  a.dec_rows = dec_rows;
  a.dec_cap = dec_capacity;
  a.status = status;
  hipLaunchKernelGGL(plan_kernel, dim3(1), dim3(kPlanThreads), 0,
                     reinterpret_cast<hipStream_t>(stream), a);
  return launch_status("tf_attn_plan_device launch");
}

}  // extern "C"
