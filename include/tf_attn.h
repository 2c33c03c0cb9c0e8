/*
 * tf_attn.h - C ABI of libtf_attn.so, the MI355X (gfx950) full-attention path.
 *
 * Drop-in boundary: the Python method
 *   Qwen3_8FullAttention._slot_based_attention(q, layer_k_buffer,
 *                                              layer_v_buffer, batch)
 * (reference qwen3_8/full_attention.py:163-283) and the KV write just before it
 * (qwen3_8/full_attention.py:146-149).  The reference has no FFI: its host
 * side calls these entry points through ctypes (tokenfactory_amd/_native.py).
 *
 * Conventions
 *  - Every pointer argument is a device pointer unless stated otherwise; the
 *    library never allocates, frees or retains device memory.
 *  - Index tensors keep the reference's dtype: int64 (req_to_token,
 *    req_pool_indices, seq_lens, out_cache_loc; ForwardBatch,
 *    qwen3_8/forward_batch.py:19-31).  Work lists made by the planners are int32.
 *  - KV pools are one layer's [pool_slots, num_kv_heads, head_dim] block
 *    (qwen3_8/hybrid_cache_pool.py:48-61, accessor :106-109), row-major, in bf16 or in
 *    OCP fp8-e4m3 with per-tensor fp32 scales (k_scale / v_scale, device
 *    scalars; ignored for bf16).  Slot 0 is the padding slot
 *    (token_to_kv_pool.py:20-23); req_to_token holds -1 for empty positions
 *    (req_to_token_pool.py:13-16).  Slot ids read from req_to_token are clamped
 *    into [0, pool_slots) so a bad id cannot fault the GPU.
 *  - head_dim: 256 runs the tuned kernels (the 27B model); any other multiple
 *    of 8 up to 256 runs one-wave-per-row kernels with the same semantics (the
 *    reference's test configurations use 32); others are TF_ERR_UNSUPPORTED.
 *    Decode at head_dim != 256 needs no workspace (the size query returns 0).
 *  - q / out are [T, num_q_heads, head_dim] bf16 with a free token stride
 *    (q_row_stride / out_row_stride, in elements); heads and dims are dense.
 *  - q head h reads kv head h / (num_q_heads / num_kv_heads)
 *    (repeat_interleave semantics, qwen3_8/full_attention.py:191-193).
 *  - Request b of the batch owns context positions [0, L_b) with
 *    L_b = seq_lens[b] (or seq_len_override when > 0: the reference's bsz == 1
 *    branch takes L from max_seq_len, full_attention.py:186), of which the last
 *    ext_b are new; new token t attends to positions 0 .. L_b - ext_b + t
 *    (full_attention.py:200-208, 234-238, 266-278).
 *  - Work is enqueued on `stream` (NULL = the null stream); no call
 *    synchronises the device.
 *  - Return value: TF_OK (0) or a negative TF_ERR_* code; tf_attn_last_error()
 *    then describes the failure (thread-local string).
 */
#ifndef TF_ATTN_H_
#define TF_ATTN_H_

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct ihipStream_t* tf_stream_t; /* hipStream_t */

enum {
  TF_DTYPE_BF16 = 0,
  TF_DTYPE_FP8_E4M3 = 1,
  TF_DTYPE_FP32 = 2
};

enum {
  TF_OK = 0,
  TF_ERR_INVALID = -1,     /* bad shape, size, pointer or alignment */
  TF_ERR_UNSUPPORTED = -2, /* valid but not implemented (head_dim, dtype, group) */
  TF_ERR_HIP = -3          /* a HIP runtime call failed */
};

/* Integer ABI revision; bumped whenever a signature below changes or one is added. */
int32_t tf_attn_abi_version(void);

/* Message for the last non-zero return on the calling thread ("" if none). */
const char* tf_attn_last_error(void);

/* ------------------------------------------------------------------ decode
 * Decode attention: one new token per request (ext_b == 1).
 * Replaces the pure-decode branch, full_attention.py:215-242, and the
 * ext_len == 1 case of the bsz == 1 branch, full_attention.py:179-213.
 *
 * Processes n_items requests.  Item i is batch entry items[i] (or i when
 * items is NULL) and reads / writes query row q_rows[i] (or items[i] / i when
 * q_rows is NULL) of q and out; items[i] < 0 is a padding entry (no work, no
 * output), as tf_attn_plan_device writes them.
 *
 * The streaming kernel runs a persistent grid of num_workgroups workgroups
 * (0 = one per compute unit) that split the (request, kv head, 16-token tile)
 * work evenly, whatever the length mix; a request's kv head that spans several
 * workgroups leaves fp32 partials that the merge phase combines.  Beside an
 * extend launch on another stream, three per compute unit fill the CUs the
 * extend kernel frees sooner (the Python side's choice for mixed steps).  The
 * grid fixes where partials are cut, so results depend on it in the last bits.
 * At most 2048 requests per call.
 * workspace: device scratch of tf_attn_decode_workspace_bytes(...) bytes (no
 * initialisation needed) holding the partials between the two phases.  Calls
 * that overlap in time must not share a workspace.
 * max_seq_len: an upper bound of every L_b processed (host int, as
 * ForwardBatch.max_seq_len); kept for the caller's bookkeeping.
 *
 * gate (optional, NULL = none): bf16 output gate, element (row, head, dim) at
 * gate + row * gate_row_stride + head * gate_head_stride + dim (16-byte aligned,
 * strides multiples of 8 elements).  With a gate the kernels write
 * bf16(bf16(attn) * bf16(silu(gate))), the module's
 * `attn_output * F.silu(gate)` (full_attention.py:157-159) fused into the
 * output write; the gate of the reference is the second half of each head's
 * q projection, so a strided view of it is passed as is.
 *
 * out_amax (optional, NULL = none): a device uint32 that each call raises to
 * the largest bf16 bit pattern of |o| over the outputs it writes (sign bit
 * cleared, so the integer order is the float order and NaN sorts above inf),
 * with device-scope atomics: the per-tensor amax that the dynamic FP8
 * quantisation of the following o_proj needs (fp8_triton.py:128), folded into
 * the output write.  The caller sets it (normally to 0) before the step; calls
 * that write parts of one output tensor (decode and extend of a mixed step,
 * on one stream or two) may share it.  tf_fp8_act_quant_amax consumes it.
 *
 * tf_attn_decode runs both phases.  tf_attn_decode_partial runs the
 * HBM-streaming split kernel only (requests that fit one split get their final
 * output, the others leave partials in the workspace); tf_attn_decode_merge then
 * combines the partials.  Calling the two phases back to back with identical
 * arguments is exactly tf_attn_decode; the split lets a caller time the
 * streaming kernel alone or merge partials computed elsewhere.
 */
int64_t tf_attn_decode_workspace_bytes(int32_t n_items, int32_t num_q_heads,
                                       int32_t num_kv_heads, int32_t head_dim,
                                       int32_t max_seq_len, int32_t num_workgroups);

int32_t tf_attn_decode(const void* q, int64_t q_row_stride,
                       const void* k_pool, const void* v_pool, int64_t pool_slots,
                       int32_t kv_dtype, const float* k_scale, const float* v_scale,
                       const int64_t* req_to_token, int64_t rtt_rows,
                       int64_t rtt_row_stride, int64_t rtt_cols,
                       const int64_t* req_pool_indices, const int64_t* seq_lens,
                       int32_t seq_len_override,
                       const int32_t* items, const int32_t* q_rows, int32_t n_items,
                       int32_t num_q_heads, int32_t num_kv_heads, int32_t head_dim,
                       float scale, void* out, int64_t out_row_stride,
                       void* workspace, int64_t workspace_bytes,
                       int32_t max_seq_len, int32_t num_workgroups,
                       const void* gate, int64_t gate_row_stride, int64_t gate_head_stride,
                       uint32_t* out_amax, tf_stream_t stream);

int32_t tf_attn_decode_partial(const void* q, int64_t q_row_stride,
                               const void* k_pool, const void* v_pool, int64_t pool_slots,
                               int32_t kv_dtype, const float* k_scale, const float* v_scale,
                               const int64_t* req_to_token, int64_t rtt_rows,
                               int64_t rtt_row_stride, int64_t rtt_cols,
                               const int64_t* req_pool_indices, const int64_t* seq_lens,
                               int32_t seq_len_override,
                               const int32_t* items, const int32_t* q_rows, int32_t n_items,
                               int32_t num_q_heads, int32_t num_kv_heads, int32_t head_dim,
                               float scale, void* out, int64_t out_row_stride,
                               void* workspace, int64_t workspace_bytes,
                               int32_t max_seq_len, int32_t num_workgroups,
                               const void* gate, int64_t gate_row_stride, int64_t gate_head_stride,
                               uint32_t* out_amax, tf_stream_t stream);

int32_t tf_attn_decode_merge(const void* q, int64_t q_row_stride,
                             const void* k_pool, const void* v_pool, int64_t pool_slots,
                             int32_t kv_dtype, const float* k_scale, const float* v_scale,
                             const int64_t* req_to_token, int64_t rtt_rows,
                             int64_t rtt_row_stride, int64_t rtt_cols,
                             const int64_t* req_pool_indices, const int64_t* seq_lens,
                             int32_t seq_len_override,
                             const int32_t* items, const int32_t* q_rows, int32_t n_items,
                             int32_t num_q_heads, int32_t num_kv_heads, int32_t head_dim,
                             float scale, void* out, int64_t out_row_stride,
                             void* workspace, int64_t workspace_bytes,
                             int32_t max_seq_len, int32_t num_workgroups,
                             const void* gate, int64_t gate_row_stride, int64_t gate_head_stride,
                             uint32_t* out_amax, tf_stream_t stream);

/* tf_attn_decode_noalloc: no counterpart in the reference.  For callers that
 * cannot allocate device memory (code under HIP graph capture, tight serving
 * loops, harnesses that forbid hipMalloc): tf_attn_decode with the same
 * arguments minus the workspace, whose split partials live instead in a
 * library-owned static device array of 32 MiB per GPU (held from library load
 * until the process ends).  It allocates nothing and calls no allocating
 * routine.  Returns TF_ERR_UNSUPPORTED when tf_attn_decode_workspace_bytes()
 * of the same arguments exceeds 32 MiB (e.g. more than ~1700 (request, kv
 * head) units with one workgroup per CU).  Every call on one GPU uses that
 * GPU's single array: calls that overlap in time on one GPU (several streams,
 * several threads) race and must be serialised by the caller.  The stream must
 * belong to the current device.  Results are bit-identical to tf_attn_decode.
 */
int32_t tf_attn_decode_noalloc(const void* q, int64_t q_row_stride,
                               const void* k_pool, const void* v_pool, int64_t pool_slots,
                               int32_t kv_dtype, const float* k_scale, const float* v_scale,
                               const int64_t* req_to_token, int64_t rtt_rows,
                               int64_t rtt_row_stride, int64_t rtt_cols,
                               const int64_t* req_pool_indices, const int64_t* seq_lens,
                               int32_t seq_len_override,
                               const int32_t* items, const int32_t* q_rows, int32_t n_items,
                               int32_t num_q_heads, int32_t num_kv_heads, int32_t head_dim,
                               float scale, void* out, int64_t out_row_stride,
                               int32_t max_seq_len, int32_t num_workgroups,
                               const void* gate, int64_t gate_row_stride,
                               int64_t gate_head_stride, uint32_t* out_amax,
                               tf_stream_t stream);

/* ------------------------------------------------------------------ extend
 * Causal prefill / extend attention over cached prefix + new tokens, bf16
 * MFMA, flash-style.  Replaces the extend / mixed branch,
 * full_attention.py:244-283, and the ext_len > 1 case of the bsz == 1 branch,
 * full_attention.py:179-213.
 *
 * work: device int32 [n_work][8] from tf_attn_plan_extend() or
 * tf_attn_plan_device(); one entry per (request, kv head, tile of 256
 * (token, q-head) rows).
 * gate, out_amax: optional output gate and output amax, as for tf_attn_decode.
 */
int32_t tf_attn_extend(const void* q, int64_t q_row_stride,
                       const void* k_pool, const void* v_pool, int64_t pool_slots,
                       int32_t kv_dtype, const float* k_scale, const float* v_scale,
                       const int64_t* req_to_token, int64_t rtt_rows,
                       int64_t rtt_row_stride, int64_t rtt_cols,
                       const int64_t* req_pool_indices, const int64_t* seq_lens,
                       int32_t seq_len_override,
                       const int32_t* work, int32_t n_work,
                       int32_t num_q_heads, int32_t num_kv_heads, int32_t head_dim,
                       float scale, void* out, int64_t out_row_stride,
                       const void* gate, int64_t gate_row_stride, int64_t gate_head_stride,
                       uint32_t* out_amax, tf_stream_t stream);

/* ------------------------------------------------------------------ planning
 * Host-side work planning (all pointers are HOST pointers; no GPU needed).
 *
 * tf_attn_plan_extend: for the requests with extend_lens[b] > 1 (all of them
 * when decode_to_decode_kernel == 0) writes extend work items
 * {b, kv_head, row0, q_start_b, ext_b, 0, 0, 0} into work (capacity entries)
 * and returns their count, or a negative error.  q_start_b is the first row of
 * request b in the flattened q (exclusive prefix sum of extend_lens, as
 * full_attention.py:250-256).  Items are ordered request by request, largest
 * extend first, kv heads inner, later (heavier) row tiles first.
 *
 * tf_attn_plan_decode_items: lists the requests with extend_lens[b] == 1 in
 * items (batch index) and q_rows (their row in q); returns the count.
 *
 * With work == NULL (or items / q_rows == NULL) the planners only count.
 */
int32_t tf_attn_plan_extend(const int64_t* extend_lens, int32_t batch_size,
                            int32_t num_q_heads, int32_t num_kv_heads,
                            int32_t decode_to_decode_kernel,
                            int32_t* work, int32_t capacity);

int32_t tf_attn_plan_decode_items(const int64_t* extend_lens, int32_t batch_size,
                                  int32_t* items, int32_t* q_rows, int32_t capacity);

/* ------------------------------------------------------------------ device-side planning
 * tf_attn_plan_device: the same two lists built on the GPU (one workgroup) from
 * DEVICE extend_lens (int64 [batch_size], batch_size <= 4096), enqueued on
 * stream, so a step needs no host loop, no host->device copy and no sync and
 * can be captured in a HIP graph (it replaces the per-step host bookkeeping
 * of full_attention.py:250-265 and engine/model_runner.py:108-188).
 * work: device int32 [work_capacity][8], filled with the entries of
 * tf_attn_plan_extend in the same order, then padding entries (ext 0) up to
 * work_capacity; launching tf_attn_extend with n_work = work_capacity is then
 * exact (padding workgroups exit at once).  dec_items / dec_rows: device int32
 * [dec_capacity], the decode items of tf_attn_plan_decode_items then -1 / 0
 * padding (tf_attn_decode* skip items < 0; pass n_items = dec_capacity).
 * status: device int32 [3] = {real work entries, real decode items, flags}
 * (flags bit 0: a capacity was too small; bit 1: an extend length outside
 * [1, 2^31)).
 * tf_attn_plan_device_capacity: num_kv_heads * (ceil(T * G / 256) + B), the
 * work entries the plan of any B requests with T tokens in total can need
 * (G = num_q_heads / num_kv_heads); dec_capacity = B suffices.
 */
int64_t tf_attn_plan_device_capacity(int64_t total_tokens, int32_t batch_size,
                                     int32_t num_q_heads, int32_t num_kv_heads);

int32_t tf_attn_plan_device(const int64_t* extend_lens, int32_t batch_size,
                            int32_t num_q_heads, int32_t num_kv_heads,
                            int32_t decode_to_decode_kernel, int32_t* work,
                            int32_t work_capacity, int32_t* dec_items, int32_t* dec_rows,
                            int32_t dec_capacity, int32_t* status, tf_stream_t stream);

/* ------------------------------------------------------------------ req_to_token sync
 * Brings the resident device req_to_token table up to date for one batch: the
 * per-step incremental sync of engine/model_runner.py:147-167, which copies
 * each request's rewritten prefix positions from the host table
 * (req_to_token_pool.py:30-35 moves dirty_from back on such a rewrite) and
 * then this step's out_cache_loc slice into the request's row.  Here the
 * whole batch is one kernel.  For request b, row r = req_pool_indices[b]:
 *   req_to_token[r, patch_from[b] : prefix_lens[b]]
 *       = patch_vals[patch_offsets[b] : patch_offsets[b] + prefix_lens[b] - patch_from[b]]
 *   req_to_token[r, prefix_lens[b] : seq_lens[b]]
 *       = out_cache_loc[o_b : o_b + seq_lens[b] - prefix_lens[b]],
 *         o_b = sum over b' < b of (seq_lens[b'] - prefix_lens[b'])
 * (the flattened order of the batch's new tokens, model_runner.py:118-135).
 * patch_from[b] >= prefix_lens[b] means no rewritten positions; patch_from,
 * patch_offsets and patch_vals may all be NULL (none in the batch).
 * req_pool_indices, prefix_lens, seq_lens, patch_from, patch_offsets: int64
 * device arrays of batch_size entries; out_cache_loc: out_cache_loc_len int64
 * entries; patch_vals: patch_vals_len int64 entries.  Rows must be distinct
 * within one call.  Every length is read from device memory, so a call with a
 * fixed batch_size can be captured in a HIP graph and replayed after the
 * arrays are refilled.  A request whose row or range lies outside the table
 * (r outside [0, rtt_rows), not 0 <= prefix <= seq <= rtt_cols) writes nothing
 * and takes no out_cache_loc entries; entries past out_cache_loc_len and patch
 * runs outside [0, prefix) or past patch_vals_len are not written.
 * At most 4096 requests per call; num_workgroups 0 = 64.
 */
int32_t tf_req_to_token_sync(int64_t* req_to_token, int64_t rtt_rows, int64_t rtt_row_stride,
                             int64_t rtt_cols, const int64_t* req_pool_indices,
                             const int64_t* prefix_lens, const int64_t* seq_lens,
                             const int64_t* out_cache_loc, int64_t out_cache_loc_len,
                             const int64_t* patch_from, const int64_t* patch_offsets,
                             const int64_t* patch_vals, int64_t patch_vals_len,
                             int32_t batch_size, int32_t num_workgroups, tf_stream_t stream);

/* ------------------------------------------------------------------ KV write
 * k_pool[out_cache_loc[t]] = k[t]; v_pool[out_cache_loc[t]] = v[t]
 * (full_attention.py:146-149).  k / v: [n_tokens, num_kv_heads, head_dim] in
 * src_dtype (bf16 or fp32) with token stride src_row_stride (elements).  For an
 * fp8 pool each element is stored as e4m3(clamp(x / scale, -448, 448)), round
 * to nearest even.  Slots outside [0, pool_slots) are skipped.
 */
int32_t tf_kv_write(const void* k, const void* v, int64_t src_row_stride,
                    int32_t src_dtype, const int64_t* out_cache_loc, int64_t n_tokens,
                    void* k_pool, void* v_pool, int64_t pool_slots, int32_t kv_dtype,
                    const float* k_scale, const float* v_scale,
                    int32_t num_kv_heads, int32_t head_dim, tf_stream_t stream);

/* ------------------------------------------------------------------ q/k prep
 * Fused q/k RMSNorm + partial (M-)RoPE + KV scatter-write, the steps right
 * before attention: q = q_norm(q), k = k_norm(k) (full_attention.py:141-142,
 * rms_norm.py:19-24), q, k = rotary_emb(q, k, positions) (:143,
 * rotary_embedding.py:46-95), layer_k_buffer[out_cache_loc] = k and the same
 * for v (:146-149), with the reference's bf16 rounding steps.
 *
 * q: bf16 rows of n_tokens x num_q_heads x head_dim at (q_token_stride,
 * q_head_stride) elements (a view of the gated q projection works as is);
 * k / v: bf16 [n_tokens, num_kv_heads, head_dim] with token strides.
 * q_norm_weight / k_norm_weight: fp32 [head_dim], 16-byte aligned.
 * positions: int64 [position_rows, *] (1 = text positions, 3 = M-RoPE),
 * rows position_row_stride elements apart. inv_freq: fp32 [rotary_dim / 2].
 * mrope_section*: the three M-RoPE sections (summing to rotary_dim / 2),
 * mrope_interleaved: 1 for the interleaved layout.
 * q_out: bf16 [n_tokens, num_q_heads, head_dim] (token stride q_out_token_stride).
 * K / V rows go to the pool like tf_kv_write (bf16, or fp8-e4m3 with
 * k_scale / v_scale); slots outside [0, pool_slots) are skipped.
 * head_dim a multiple of 8 up to 256; rotary_dim even (a multiple of 16 for
 * head_dim 256).  With 3-row positions the sections must sum to rotary_dim / 2
 * for the sectioned layout (the reference splits by them); the interleaved
 * layout takes any sections (rotary_embedding.py:58-70).
 */
int32_t tf_qk_norm_rope_kv_write(const void* q, int64_t q_token_stride, int64_t q_head_stride,
                                 const void* k, int64_t k_token_stride,
                                 const void* v, int64_t v_token_stride,
                                 int64_t n_tokens, int32_t num_q_heads, int32_t num_kv_heads,
                                 int32_t head_dim, const float* q_norm_weight,
                                 const float* k_norm_weight, float eps,
                                 const int64_t* positions, int32_t position_rows,
                                 int64_t position_row_stride, const float* inv_freq,
                                 int32_t rotary_dim, int32_t mrope_section0,
                                 int32_t mrope_section1, int32_t mrope_section2,
                                 int32_t mrope_interleaved, void* q_out,
                                 int64_t q_out_token_stride, const int64_t* out_cache_loc,
                                 void* k_pool, void* v_pool, int64_t pool_slots,
                                 int32_t kv_dtype, const float* k_scale, const float* v_scale,
                                 tf_stream_t stream);

/* ------------------------------------------------------------------ FP8 linear
 * The block-FP8 o_proj that follows the gated attention output
 * (full_attention.py:161 -> RowParallelFP8Linear, fp8_linear.py:181-201 ->
 * triton_block_fp8_linear, fp8_triton.py:107-183), as two calls.
 *
 * tf_fp8_act_quant replaces the dynamic activation quantisation of
 * fp8_triton.py:127-130:
 *   x_scale = bf16(max(max|x|, 1e-12) / 448)   (a NaN in x makes it NaN)
 *   xq      = e4m3(clamp(x / x_scale, -448, 448)), round to nearest even.
 * x: bf16 [rows, cols], cols a multiple of 8, row stride x_row_stride
 * elements (a multiple of 8), 16-byte aligned.  xq: e4m3 [rows, cols], row
 * stride xq_row_stride bytes (a multiple of 8), 8-byte aligned.  x_scale: a
 * device fp32 scalar that receives the scale.  workspace: device scratch of at
 * least TF_FP8_QUANT_WORKSPACE_BYTES bytes, 4-byte aligned (no initial
 * contents needed).
 *
 * tf_fp8_block_gemm replaces _block_fp8_gemm_kernel (fp8_triton.py:17-98):
 *   out[i, j] = bf16( sum over 128-wide K slices s of
 *                     (sum_{k in s} xq[i, k] w[j, k]) * (x_scale * w_scale[j / block_h, 128 s / block_w])
 *                     + bias[j] ),   fp32 accumulation.
 * xq: e4m3 [m, k]; w: e4m3 [n, k] (nn.Linear layout); both 16-byte aligned
 * with row strides (bytes) that are multiples of 16; k a multiple of 128.
 * w_scale: fp32 [ceil(n / block_h), ceil(k / block_w)] at the given element
 * strides (block_w a multiple of 128), or NULL for a weight without block
 * scales (weight_scale_inv None: every scale 1).  bias: bf16 [n] or NULL.
 * out: bf16 [m, n], row stride out_row_stride elements (a multiple of 4),
 * 8-byte aligned.
 * workspace (optional, NULL allowed): when m is small (up to 512) the output
 * tiles alone leave most compute units idle and the call splits K over
 * several workgroups per tile if it gets tf_fp8_block_gemm_workspace_bytes(m,
 * n, k) bytes of 16-byte aligned scratch (fp32 partials, no initialisation
 * needed; the partials are summed in a fixed order, so results do not depend
 * on timing).  Without it (or when the size query returns 0) one workgroup
 * covers each output tile.
 */
#define TF_FP8_QUANT_WORKSPACE_BYTES 4096

int32_t tf_fp8_act_quant(const void* x, int32_t x_dtype, int64_t rows, int64_t cols,
                         int64_t x_row_stride, void* xq, int64_t xq_row_stride,
                         float* x_scale, void* workspace, int64_t workspace_bytes,
                         tf_stream_t stream);

/* tf_fp8_act_quant_amax: tf_fp8_act_quant with max|x| already known, as the
 * attention entry points accumulate it in their out_amax argument over the
 * output they write (the bf16 bit pattern of |x|, sign cleared): the same
 * x_scale and xq bit for bit, one launch (the quantisation pass) instead of
 * two, no workspace.  amax_bits: device uint32, 4-byte aligned.  Replaces
 * the same lines of fp8_triton.py (127-130) for a caller whose producer
 * computed the amax (the gated attention output in front of o_proj).
 */
int32_t tf_fp8_act_quant_amax(const void* x, int32_t x_dtype, int64_t rows, int64_t cols,
                              int64_t x_row_stride, void* xq, int64_t xq_row_stride,
                              float* x_scale, const uint32_t* amax_bits, tf_stream_t stream);

int32_t tf_fp8_block_gemm(const void* xq, int64_t xq_row_stride, const float* x_scale,
                          const void* w, int64_t w_row_stride, const float* w_scale,
                          int64_t w_scale_row_stride, int64_t w_scale_col_stride,
                          int32_t block_h, int32_t block_w, const void* bias, int64_t m,
                          int64_t n, int64_t k, void* out, int64_t out_row_stride,
                          void* workspace, int64_t workspace_bytes, tf_stream_t stream);

int64_t tf_fp8_block_gemm_workspace_bytes(int64_t m, int64_t n, int64_t k);

/* ------------------------------------------------------------------ Gated DeltaNet decode
 * One-token step of the linear-attention (Gated DeltaNet) layers for a batch
 * whose requests all extend by one token: Qwen3_8LinearAttention.
 * _batched_decode_step (qwen3_8/linear_attention.py:244-298) followed by the
 * gated RMSNorm (:325, rms_norm_gated.py:26-40); out_proj is left to the caller.
 *
 * Request b reads state slot r = req_indices[b] (requests with r outside
 * [0, n_slots) leave every state untouched and get zero out / core_out rows):
 *   conv: y = bf16(silu(bf16(sum_i conv_weight[c][i] * [conv_state[r][c][0..2], qkv[b][c]][i])))
 *         conv_state[r][c] <- [conv_state[r][c][1..2], qkv[b][c]]
 *   q, k, v = split(y, [Hk*Dk, Hk*Dk, Hv*Dv]); q = normalize(q) / sqrt(Dk);
 *   k = normalize(k); value head h uses key head h / (Hv / Hk);
 *   alpha = exp(-exp(a_log[h]) * softplus(a[b][h] + dt_bias[h])), beta = sigmoid(b[b][h]);
 *   S = alpha * ssm_state[r][h]; S += k (beta (v - S^T k))^T; ssm_state[r][h] = S;
 *   o = bf16(S^T q);  out[b] = bf16(norm_weight * o / rms_head(o) * silu(z[b])).
 * qkv: bf16 [B, 2*Hk*Dk + Hv*Dv]; a, b: bf16 [B, Hv] (common row stride);
 * z: bf16 [B, Hv*Dv]; conv_weight: fp32 [conv_dim, 4] (16-byte aligned);
 * a_log, dt_bias: fp32 [Hv]; norm_weight: fp32 [Hv*Dv] (rms over Dv);
 * conv_state: bf16 [slots, conv_dim, 3]; ssm_state: fp32 [slots, Hv, Dk, Dv]
 * (16-byte aligned), both updated in place, slot strides in elements;
 * out (and the optional core_out, the pre-norm o): bf16 [B, Hv*Dv].
 * workspace: 16-byte aligned device scratch of tf_gdn_decode_workspace_bytes(B, Hk,
 * Hv) bytes (the bf16 conv outputs and the fp32 gates between the two
 * launches; no initialisation needed; sized for Dk = Dv = 128, enough for
 * every supported head dim).
 * Dk = head_k_dim, Dv = head_v_dim: 128 / 128 (the Qwen3.5 layers, on the
 * MFMA-tiled kernels), or each a multiple of 4 up to 64 (the small test
 * models, e.g. 16 / 16, on one wave per (request, value head) with the state
 * in registers, the whole call's tokens in that wave); conv_kernel = 4.
 * Requests of one call must use distinct slots.
 */
int64_t tf_gdn_decode_workspace_bytes(int32_t batch_size, int32_t num_k_heads,
                                      int32_t num_v_heads);

int32_t tf_gdn_decode(const void* qkv, int64_t qkv_row_stride, const void* a, const void* b,
                      int64_t ab_row_stride, const void* z, int64_t z_row_stride,
                      const float* conv_weight, const float* a_log, const float* dt_bias,
                      const float* norm_weight, float eps, void* conv_state,
                      int64_t conv_slot_stride, float* ssm_state, int64_t ssm_slot_stride,
                      const int64_t* req_indices, int32_t batch_size, int64_t n_slots,
                      int32_t num_k_heads, int32_t num_v_heads, int32_t head_k_dim,
                      int32_t head_v_dim, int32_t conv_kernel, void* out,
                      int64_t out_row_stride, void* core_out, int64_t core_row_stride,
                      void* workspace, int64_t workspace_bytes, tf_stream_t stream);

/* ------------------------------------------------------------------ Gated DeltaNet extend
 * The same layer for a batch with any extend lengths: the reference's
 * per-request loop (linear_attention.py:328-364: _causal_conv1d_step,
 * _gated_delta_rule_step, then the gated norm).  Request b owns the token rows
 * token_offsets[b] .. token_offsets[b + 1] - 1 of qkv, a, b, z and out
 * (device int32 [batch_size + 1], non-decreasing, clamped into [0, n_tokens]);
 * max_extend_len: the largest extend length (host int, validated only);
 * each request's conv runs over [conv_state, its tokens] and its state is
 * carried through its tokens in order.  The state update is the reference's
 * chunk-wise WY form (:194-242) with 32-token chunks (the same recurrence as
 * token by token, equal up to fp32 rounding).  Six launches: the request
 * of every token row, the conv for every (token, channel) in parallel,
 * normalised q / k and the gates for every token in parallel (with the
 * conv-state shift and zeros for the rows of no request or of an out-of-pool
 * slot), the state-independent part of every chunk in parallel, the
 * one-token requests' update (as in tf_gdn_decode) and the chunked recurrence
 * with the gated norm of its rows (one workgroup per request of two or more
 * tokens and value head, its state in registers from first chunk to last).
 * When the
 * batch can hold both kinds of request (batch_size > 1, max_extend_len > 1),
 * the one-token update of a call that is not under graph capture runs on a
 * second stream of the library's (one per device, made on the first such
 * call) that forks from `stream` after the chunk preparation and joins it
 * before the call returns; concurrent calls on one device serialise their
 * fork .. join sequences on a lock.  A call under capture launches everything
 * on `stream`, so captured and eager calls never share the second stream.  qkv, z, out and core_out must be 8-byte aligned
 * with row strides that are multiples of 4; norm_weight 16-byte aligned.  Other arguments
 * as for tf_gdn_decode, with rows = tokens; workspace:
 * tf_gdn_extend_workspace_bytes(n_tokens, batch_size, Hk, Hv) bytes, 16-byte
 * aligned.  At head dims other than 128 / 128 the call is five launches: the
 * request of every row, the conv, the conv-state shift, every request's
 * tokens in order in one wave per (request, value head), and the zero rows.
 */
int64_t tf_gdn_extend_workspace_bytes(int64_t n_tokens, int32_t batch_size,
                                      int32_t num_k_heads, int32_t num_v_heads);

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
                      void* workspace, int64_t workspace_bytes, tf_stream_t stream);

/* ------------------------------------------------------------------ gather
 * Padded slot gather of the batched branches (full_attention.py:216-220):
 * out[b, t] = pool[max(req_to_token[req_pool_indices[b], t], 0)] for
 * t < max_len, bit-exact.  out: [batch, max_len, row_elems] in the pool dtype.
 * Used to check the kernels' token-granular gather against PyTorch indexing.
 */
int32_t tf_gather_kv(const void* pool, int32_t kv_dtype, int64_t pool_slots,
                     int64_t row_elems, const int64_t* req_to_token, int64_t rtt_rows,
                     int64_t rtt_row_stride, int64_t rtt_cols,
                     const int64_t* req_pool_indices, int32_t batch_size,
                     int32_t max_len, void* out, tf_stream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* TF_ATTN_H_ */
