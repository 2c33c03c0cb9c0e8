// Host-side helpers shared by the C-ABI translation units.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "tf_attn.h"

namespace tfa {

// Records a formatted message for tf_attn_last_error() and returns `code`.
int fail(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
// Clears the thread's last error.
void clear_error();
// Maps the most recent launch status to TF_OK / TF_ERR_HIP.
int launch_status(const char* what);
// Compute units of the current device (cached per device; 256 if the query fails).
int device_cu_count();

inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }
inline bool aligned8(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 7u) == 0; }

// Decode plan shared by the launcher and the workspace-size query.
struct DecodePlan {
  int32_t n_blocks;     // workgroups of the streaming kernel (1 per CU by default)
  int32_t n_hgroups;    // ceil(group / 16)
  int32_t gmax;         // min(group, 16)
  int64_t n_units;      // items * kv_heads * n_hgroups
  int64_t ml_bytes, o_bytes, total_bytes;  // split partials: (max, sum) and O
  bool generic;         // head_dim != 256: the one-wave-per-row kernel, no workspace
};
int make_decode_plan(int32_t n_items, int32_t num_q_heads, int32_t num_kv_heads,
                     int32_t head_dim, int32_t max_seq_len, int32_t num_workgroups,
                     DecodePlan* plan);

// Extend kernel arguments (validated by tf_attn_extend).  Work items cover
// kExtendItemRows flattened (token, q-head-of-group) rows each.
constexpr int kExtendItemRows = 256;
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
  const __bf16* gate;             // optional output gate (NULL: none)
  int64_t gate_stride, gate_hstride;
  uint32_t* amax;                 // optional: raised to max |out| (bf16 bits)
};

// Slot attention for head dims other than 256 (attn_generic.hip): one wave per
// query row.  work != NULL: the rows of n_rows extend work entries; else the
// Hq rows of n_rows decode items (items / q_rows as in tf_attn_decode).
struct GenericAttnArgs {
  const __bf16* q;
  int64_t q_stride;
  const uint8_t* k_pool;
  const uint8_t* v_pool;
  int64_t pool_slots;
  int32_t fp8;
  const float* k_scale;
  const float* v_scale;
  const int64_t* rtt;
  int64_t rtt_rows, rtt_stride, rtt_cols;
  const int64_t* rpi;
  const int64_t* seq_lens;
  int32_t seq_override;
  const int32_t* items;
  const int32_t* q_rows;
  const int32_t* work;
  int32_t n_rows;
  int32_t hq, hkv, head_dim;
  float scale_log2;
  __bf16* out;
  int64_t out_stride;
  const __bf16* gate;
  int64_t gate_stride, gate_hstride;
  uint32_t* amax;   // optional: raised to max |out| (bf16 bits)
};
// head_dim handled by the generic kernel: a multiple of 8 in [8, 256], not 256.
bool generic_head_dim(int32_t head_dim);
int launch_generic_attn(const GenericAttnArgs& a, hipStream_t stream);

}  // namespace tfa
