"""Op-for-op PyTorch restatement of the reference's slot-based attention.

TEST INFRASTRUCTURE ONLY (the checker and the timed CPU baseline); the product
path never imports it.

Follows ``Qwen3_8FullAttention._slot_based_attention`` in the reference
(``qwen3_8/full_attention.py:163-283``) step by step, with the same tensor ops
in the same order, so that timing it on the host measures the reference's CPU
path and running it in fp32 gives the parity oracle:

* ``bsz == 1`` branch (``full_attention.py:179-213``): unclamped slot gather of
  ``req_to_token[r, :max_seq_len]``, GQA ``repeat_interleave`` on the head dim,
  an additive ``0/-inf`` causal mask only when ``ext_len > 1``;
* pure-decode branch (``full_attention.py:215-242``): padded, clamped gather
  ``req_to_token[req_pool_indices, :max_seq_len].clamp(min=0)``, expand, length
  mask ``k < seq_lens[b]``;
* extend / mixed branch (``full_attention.py:244-283``): queries scattered into
  a padded ``[B, max_ext, Hq, D]`` block, mask ``k <= q_abs and k < seq_len``,
  padded query rows opened on key 0 only, result gathered back to ``[T, Hq, D]``.

The KV write (``full_attention.py:146-149``) is ``write_kv_ref``.
"""
from __future__ import annotations

from typing import Optional

import torch
import torch.nn.functional as F


def _expand_heads(x: torch.Tensor, group: int, head_dim_axis: int) -> torch.Tensor:
    """GQA expansion: kv head ``j`` is repeated ``group`` times in place, so q head
    ``h`` reads kv head ``h // group`` (``full_attention.py:191-193, 221-227``)."""
    if group > 1:
        return torch.repeat_interleave(x, group, dim=head_dim_axis)
    return x


def _single_request(q, k_buf, v_buf, batch, group, scaling):
    # full_attention.py:179-213
    if batch.req_pool_indices_list is not None:
        row = batch.req_pool_indices_list[0]
    else:
        row = int(batch.req_pool_indices[0].item())
    ext = batch.extend_lens[0]
    total = batch.max_seq_len

    slots = batch.req_to_token[row, :total]          # no clamp on this branch
    keys = _expand_heads(k_buf[slots], group, 1)      # [L, Hq, D]
    vals = _expand_heads(v_buf[slots], group, 1)

    q4 = q.transpose(0, 1).unsqueeze(0)               # [1, Hq, ext, D]
    k4 = keys.transpose(0, 1).unsqueeze(0)            # [1, Hq, L, D]
    v4 = vals.transpose(0, 1).unsqueeze(0)

    bias = None
    if ext > 1:
        qpos = torch.arange(total - ext, total, device=q.device).unsqueeze(1)
        kpos = torch.arange(total, device=q.device).unsqueeze(0)
        allowed = qpos >= kpos
        bias = torch.zeros((ext, total), dtype=q.dtype, device=q.device)
        bias = bias.masked_fill(~allowed, float("-inf"))

    res = F.scaled_dot_product_attention(q4, k4, v4, attn_mask=bias, scale=scaling)
    return res.squeeze(0).transpose(0, 1)             # [ext, Hq, D]


def _padded_kv(k_buf, v_buf, batch, group):
    # full_attention.py:215-229
    total = batch.max_seq_len
    slots = batch.req_to_token[batch.req_pool_indices, :total].clamp(min=0)
    keys = _expand_heads(k_buf[slots], group, 2)      # [B, L, Hq, D]
    vals = _expand_heads(v_buf[slots], group, 2)
    return keys.transpose(1, 2), vals.transpose(1, 2)  # [B, Hq, L, D]


def _decode(q, k4, v4, batch, scaling):
    # full_attention.py:231-242
    bsz = batch.batch_size
    total = batch.max_seq_len
    q4 = q.unsqueeze(2)                               # [B, Hq, 1, D]
    kpos = torch.arange(total, device=q.device).unsqueeze(0)
    live = kpos < batch.seq_lens.unsqueeze(1)          # [B, L]
    bias = torch.zeros((bsz, 1, 1, total), dtype=q.dtype, device=q.device)
    bias = bias.masked_fill(~live.unsqueeze(1).unsqueeze(2), float("-inf"))
    res = F.scaled_dot_product_attention(q4, k4, v4, attn_mask=bias, scale=scaling)
    return res.squeeze(2)


def _extend(q, k4, v4, batch, scaling, num_heads, head_dim):
    # full_attention.py:244-283
    bsz = batch.batch_size
    total = batch.max_seq_len
    widest = batch.max_extend_len
    ext = batch.extend_lens_tensor
    if ext is None:
        ext = torch.tensor(batch.extend_lens, dtype=torch.long, device=q.device)

    which_req = torch.repeat_interleave(torch.arange(bsz, device=q.device), ext)
    first = torch.cumsum(ext, dim=0) - ext
    within = torch.arange(q.shape[0], device=q.device) - torch.repeat_interleave(first, ext)

    qpad = torch.zeros((bsz, widest, num_heads, head_dim), dtype=q.dtype, device=q.device)
    qpad[which_req, within] = q
    q4 = qpad.transpose(1, 2)                         # [B, Hq, Le, D]

    rel = torch.arange(widest, device=q.device).view(1, widest, 1)
    absolute = (batch.seq_lens - ext).view(bsz, 1, 1) + rel
    kpos = torch.arange(total, device=q.device).view(1, 1, total)
    real_q = rel < ext.view(bsz, 1, 1)
    live_k = kpos < batch.seq_lens.view(bsz, 1, 1)
    causal = (kpos <= absolute) & live_k
    allowed = torch.where(real_q, causal, kpos == 0)   # padded rows see key 0 only

    bias = torch.zeros((bsz, 1, widest, total), dtype=q.dtype, device=q.device)
    bias = bias.masked_fill(~allowed.unsqueeze(1), float("-inf"))
    res = F.scaled_dot_product_attention(q4, k4, v4, attn_mask=bias, scale=scaling)
    return res.transpose(1, 2)[which_req, within]


def slot_based_attention_ref(
    q: torch.Tensor,
    layer_k_buffer: torch.Tensor,
    layer_v_buffer: torch.Tensor,
    batch,
    num_queries_per_kv: int,
    scaling: float,
) -> torch.Tensor:
    """Reference semantics of ``_slot_based_attention`` (``full_attention.py:163-283``).

    ``q`` is ``[T, Hq, D]``; the buffers are one layer's ``[S, Hkv, D]`` pool;
    ``batch`` is any object carrying the ``ForwardBatch`` fields
    (``qwen3_8/forward_batch.py:19-31``). Returns ``[T, Hq, D]``.
    """
    if batch.batch_size == 1:
        return _single_request(q, layer_k_buffer, layer_v_buffer, batch,
                               num_queries_per_kv, scaling)
    k4, v4 = _padded_kv(layer_k_buffer, layer_v_buffer, batch, num_queries_per_kv)
    if batch.max_extend_len == 1:
        return _decode(q, k4, v4, batch, scaling)
    return _extend(q, k4, v4, batch, scaling, q.shape[1], q.shape[2])


def gather_kv_ref(pool: torch.Tensor, req_to_token: torch.Tensor,
                  req_pool_indices: torch.Tensor, max_len: int) -> torch.Tensor:
    """The batched branch's padded slot gather (``full_attention.py:216-220``):
    ``pool[req_to_token[req_pool_indices, :max_len].clamp(min=0)]``."""
    slots = req_to_token[req_pool_indices, :max_len].clamp(min=0)
    return pool[slots]


def write_kv_ref(layer_k_buffer: torch.Tensor, layer_v_buffer: torch.Tensor,
                 out_cache_loc: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
                 k_scale: Optional[float] = None, v_scale: Optional[float] = None) -> None:
    """KV scatter-write (``full_attention.py:146-149``): ``buf[out_cache_loc] = x``.

    For an fp8-e4m3fn pool the rows are quantised first with the per-tensor
    scale (``oracle.kv_quant.quantize_e4m3``); the reference itself has no fp8 KV.
    """
    if layer_k_buffer.dtype == torch.float8_e4m3fn:
        from .kv_quant import quantize_e4m3
        layer_k_buffer[out_cache_loc] = quantize_e4m3(k, k_scale)
        layer_v_buffer[out_cache_loc] = quantize_e4m3(v, v_scale)
    else:
        layer_k_buffer[out_cache_loc] = k
        layer_v_buffer[out_cache_loc] = v
