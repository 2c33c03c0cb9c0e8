// Library-wide C-ABI plumbing: version, thread-local error text, host planners.
#include <stdarg.h>
#include <stdio.h>
#include <string.h>

#include <algorithm>
#include <mutex>
#include <vector>

#include "tf_internal.h"

namespace tfa {

static thread_local char g_err[512];

int fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
  return code;
}

void clear_error() { g_err[0] = '\0'; }

int launch_status(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(TF_ERR_HIP, "%s: %s", what, hipGetErrorString(e));
  return TF_OK;
}

int device_cu_count() {
  static int cached[64];
  static std::mutex mu;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  std::lock_guard<std::mutex> lock(mu);
  if (cached[dev] == 0) {
    int cus = 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
        cus <= 0)
      cus = 256;
    cached[dev] = cus;
  }
  return cached[dev];
}

}  // namespace tfa

extern "C" {

int32_t tf_attn_abi_version(void) { return 12; }

const char* tf_attn_last_error(void) { return tfa::g_err; }

int32_t tf_attn_plan_decode_items(const int64_t* extend_lens, int32_t batch_size,
                                  int32_t* items, int32_t* q_rows, int32_t capacity) {
  tfa::clear_error();
  if (batch_size < 0 || (batch_size > 0 && !extend_lens))
    return tfa::fail(TF_ERR_INVALID, "plan_decode_items: bad batch");
  int64_t start = 0;
  int32_t n = 0;
  for (int32_t b = 0; b < batch_size; ++b) {
    const int64_t e = extend_lens[b];
    if (e < 1) return tfa::fail(TF_ERR_INVALID, "plan_decode_items: extend_lens[%d]=%lld < 1",
                                b, (long long)e);
    if (e == 1) {
      if (items && q_rows) {
        if (n >= capacity)
          return tfa::fail(TF_ERR_INVALID, "plan_decode_items: capacity %d", capacity);
        items[n] = b;
        q_rows[n] = (int32_t)start;
      }
      ++n;
    }
    start += e;
    if (start > INT32_MAX) return tfa::fail(TF_ERR_INVALID, "plan_decode_items: too many tokens");
  }
  return n;
}

// Extend items hold kExtendItemRows flattened (token, q-head-of-group) rows.
int32_t tf_attn_plan_extend(const int64_t* extend_lens, int32_t batch_size,
                            int32_t num_q_heads, int32_t num_kv_heads,
                            int32_t decode_to_decode_kernel, int32_t* work,
                            int32_t capacity) {
  tfa::clear_error();
  if (batch_size < 0 || (batch_size > 0 && !extend_lens))
    return tfa::fail(TF_ERR_INVALID, "plan_extend: bad batch");
  if (num_kv_heads <= 0 || num_q_heads <= 0 || num_q_heads % num_kv_heads)
    return tfa::fail(TF_ERR_INVALID, "plan_extend: heads %d/%d", num_q_heads, num_kv_heads);
  const int64_t group = num_q_heads / num_kv_heads;
  const int64_t tile_rows = tfa::kExtendItemRows;

  std::vector<int64_t> q_start(batch_size);
  std::vector<int32_t> order;
  int64_t start = 0;
  for (int32_t b = 0; b < batch_size; ++b) {
    const int64_t e = extend_lens[b];
    if (e < 1) return tfa::fail(TF_ERR_INVALID, "plan_extend: extend_lens[%d]=%lld < 1",
                                b, (long long)e);
    q_start[b] = start;
    start += e;
    if (start > INT32_MAX) return tfa::fail(TF_ERR_INVALID, "plan_extend: too many tokens");
    if (e == 1 && decode_to_decode_kernel) continue;
    order.push_back(b);
  }
  // Largest extend first: its tiles see the most keys.
  std::stable_sort(order.begin(), order.end(), [&](int32_t x, int32_t y) {
    return extend_lens[x] > extend_lens[y];
  });
  int64_t n = 0;
  for (int32_t b : order) {
    const int64_t rows = extend_lens[b] * group;
    const int64_t tiles = (rows + tile_rows - 1) / tile_rows;
    for (int64_t t = tiles - 1; t >= 0; --t) {
      for (int32_t h = 0; h < num_kv_heads; ++h) {
        if (!work) {  // counting pass
          ++n;
          continue;
        }
        if (n >= capacity) return tfa::fail(TF_ERR_INVALID, "plan_extend: capacity %d", capacity);
        int32_t* w = work + 8 * n;
        w[0] = b;
        w[1] = h;
        w[2] = (int32_t)(t * tile_rows);
        w[3] = (int32_t)q_start[b];
        w[4] = (int32_t)extend_lens[b];
        w[5] = 0;
        w[6] = 0;
        w[7] = 0;
        ++n;
      }
    }
  }
  return (int32_t)n;
}

}  // extern "C"
