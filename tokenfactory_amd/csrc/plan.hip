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

// ---------------------------------------------------------------------------
// req_to_token sync: the per-step incremental update of the resident device
// req_to_token table (engine/model_runner.py:147-167) as one kernel.  Request
// b of the batch owns two runs of flat elements, its rewritten prefix positions
// [patch_from, prefix) read from patch_vals, then its new positions
// [prefix, seq) read from out_cache_loc; every workgroup scans the run lengths
// of the whole batch into LDS and then takes flat elements in a grid-stride
// loop, finding each element's request by binary search.
constexpr int kSyncMaxBatch = kPlanMaxBatch;

struct SyncArgs {
  int64_t* table;
  int64_t rows, stride, cols;
  const int64_t* rpi;
  const int64_t* prefix;
  const int64_t* seq;
  const int64_t* loc;
  int64_t loc_len;
  const int64_t* pfrom;   // NULL: no rewritten prefixes
  const int64_t* poff;
  const int64_t* pvals;
  int64_t pvals_len;
  int32_t batch;
};

struct SyncSmem {
  int64_t flat[kSyncMaxBatch + 1];   // first flat element of request b
  int64_t loc[kSyncMaxBatch];        // first out_cache_loc entry of request b
  int64_t wsum[kPlanThreads / kWave];
};

// What request b writes.  A request whose row or range is outside the table
// (row outside [0, rows), not 0 <= prefix <= seq <= cols) writes nothing and
// takes no out_cache_loc entries; a patch run outside [0, prefix) or past the
// end of patch_vals is dropped.
struct SyncReq {
  int64_t row, prefix, pfrom, poff, n_patch, n_new;
};

__device__ __forceinline__ SyncReq sync_req(const SyncArgs& a, int b) {
  SyncReq q{0, 0, 0, 0, 0, 0};
  const int64_t r = a.rpi[b], p = a.prefix[b], s = a.seq[b];
  if (r < 0 || r >= a.rows || p < 0 || p > s || s > a.cols) return q;
  q.row = r;
  q.prefix = p;
  q.n_new = s - p;
  if (a.pfrom) {
    const int64_t f = a.pfrom[b], o = a.poff[b];
    if (f >= 0 && f < p && o >= 0 && o <= a.pvals_len - (p - f)) {
      q.pfrom = f;
      q.poff = o;
      q.n_patch = p - f;
    }
  }
  return q;
}

__global__ void __launch_bounds__(kPlanThreads) rtt_sync_kernel(SyncArgs a) {
  __shared__ SyncSmem sm;
  const int tid = threadIdx.x;
  int64_t n_el[kPlanPer], n_loc[kPlanPer];
  int64_t el = 0, lc = 0;
#pragma unroll
  for (int k = 0; k < kPlanPer; ++k) {
    const int b = tid * kPlanPer + k;
    n_el[k] = n_loc[k] = 0;
    if (b < a.batch) {
      const SyncReq q = sync_req(a, b);
      n_el[k] = q.n_patch + q.n_new;
      n_loc[k] = q.n_new;
    }
    el += n_el[k];
    lc += n_loc[k];
  }
  int64_t total, total_loc;
  int64_t e0 = block_scan(el, sm.wsum, total);
  int64_t l0 = block_scan(lc, sm.wsum, total_loc);
#pragma unroll
  for (int k = 0; k < kPlanPer; ++k) {
    sm.flat[tid * kPlanPer + k] = e0;
    sm.loc[tid * kPlanPer + k] = l0;
    e0 += n_el[k];
    l0 += n_loc[k];
  }
  if (tid == 0) sm.flat[kSyncMaxBatch] = total;
  __syncthreads();

  const int64_t step = (int64_t)gridDim.x * kPlanThreads;
  for (int64_t idx = (int64_t)blockIdx.x * kPlanThreads + tid; idx < total; idx += step) {
    int lo = 0, hi = a.batch - 1;   // last request with flat <= idx
    while (lo < hi) {
      const int mid = (lo + hi + 1) >> 1;
      if (sm.flat[mid] <= idx) lo = mid; else hi = mid - 1;
    }
    const SyncReq q = sync_req(a, lo);
    const int64_t j = idx - sm.flat[lo];
    int64_t pos, val;
    if (j < q.n_patch) {
      pos = q.pfrom + j;
      val = a.pvals[q.poff + j];
    } else {
      const int64_t li = sm.loc[lo] + (j - q.n_patch);
      if (li >= a.loc_len) continue;
      pos = q.prefix + (j - q.n_patch);
      val = a.loc[li];
    }
    a.table[q.row * a.stride + pos] = val;
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

int32_t tf_req_to_token_sync(int64_t* req_to_token, int64_t rtt_rows, int64_t rtt_row_stride,
                             int64_t rtt_cols, const int64_t* req_pool_indices,
                             const int64_t* prefix_lens, const int64_t* seq_lens,
                             const int64_t* out_cache_loc, int64_t out_cache_loc_len,
                             const int64_t* patch_from, const int64_t* patch_offsets,
                             const int64_t* patch_vals, int64_t patch_vals_len,
                             int32_t batch_size, int32_t num_workgroups, tf_stream_t stream) {
  using namespace tfa;
  clear_error();
  if (batch_size < 0 || batch_size > kSyncMaxBatch)
    return fail(TF_ERR_UNSUPPORTED, "req_to_token_sync: batch_size=%d (at most %d)",
                batch_size, kSyncMaxBatch);
  if (num_workgroups < 0 || num_workgroups > 4096)
    return fail(TF_ERR_INVALID, "req_to_token_sync: num_workgroups=%d", num_workgroups);
  if (batch_size == 0) return TF_OK;
  if (!req_to_token || !req_pool_indices || !prefix_lens || !seq_lens)
    return fail(TF_ERR_INVALID, "req_to_token_sync: null pointer argument");
  if (rtt_rows < 1 || rtt_cols < 1 || rtt_row_stride < rtt_cols)
    return fail(TF_ERR_INVALID, "req_to_token_sync: table %lld x %lld, row stride %lld",
                (long long)rtt_rows, (long long)rtt_cols, (long long)rtt_row_stride);
  if (out_cache_loc_len < 0 || (out_cache_loc_len > 0 && !out_cache_loc))
    return fail(TF_ERR_INVALID, "req_to_token_sync: out_cache_loc of %lld entries",
                (long long)out_cache_loc_len);
  const bool patches = patch_from || patch_offsets || patch_vals;
  if (patches && (!patch_from || !patch_offsets || (patch_vals_len > 0 && !patch_vals)))
    return fail(TF_ERR_INVALID,
                "req_to_token_sync: patch_from, patch_offsets and patch_vals go together");
  if (patch_vals_len < 0)
    return fail(TF_ERR_INVALID, "req_to_token_sync: patch_vals_len=%lld",
                (long long)patch_vals_len);
  SyncArgs a;
  a.table = req_to_token;
  a.rows = rtt_rows;
  a.stride = rtt_row_stride;
  a.cols = rtt_cols;
  a.rpi = req_pool_indices;
  a.prefix = prefix_lens;
  a.seq = seq_lens;
  a.loc = out_cache_loc;
  a.loc_len = out_cache_loc_len;
  a.pfrom = patches ? patch_from : nullptr;
  a.poff = patches ? patch_offsets : nullptr;
  a.pvals = patches ? patch_vals : nullptr;
  a.pvals_len = patches ? patch_vals_len : 0;
  a.batch = batch_size;
  hipLaunchKernelGGL(rtt_sync_kernel, dim3(num_workgroups ? num_workgroups : 64),
                     dim3(kPlanThreads), 0, reinterpret_cast<hipStream_t>(stream), a);
  return launch_status("tf_req_to_token_sync launch");
}

}  // extern "C"
