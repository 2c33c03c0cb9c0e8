"""Runs the oracle restatement on a device workload (TEST INFRASTRUCTURE ONLY).

``reference_attention(wl)`` copies to the host only the pool rows the batch
references (renumbering ``req_to_token`` to them; ``-1`` entries stay ``-1``),
dequantises an fp8 pool with its per-tensor scales, and runs
``oracle.slot_attention.slot_based_attention_ref`` in fp32 on the CPU.
``prepare_host_inputs`` returns the same host arguments without running, for
timing the restatement as the CPU baseline.
"""
from __future__ import annotations

import torch

from .kv_quant import dequantize_e4m3
from .slot_attention import slot_based_attention_ref


class HostBatch:
    """``ForwardBatch`` fields as host tensors (attention-relevant ones)."""

    def __init__(self, batch):
        for name in ("batch_size", "extend_lens", "is_prefill", "max_seq_len",
                     "max_extend_len", "req_pool_indices_list"):
            setattr(self, name, getattr(batch, name))
        for name in ("req_pool_indices", "seq_lens", "prefix_lens", "out_cache_loc",
                     "req_to_token", "extend_lens_tensor"):
            t = getattr(batch, name)
            setattr(self, name, None if t is None else t.cpu())


def pool_rows(entries, pool_slots, single):
    """The pool row each ``req_to_token`` entry reads: the batched branches
    clamp negative entries to slot 0 (``full_attention.py:217-219``); the
    ``bsz == 1`` branch indexes the pool directly (``:188-190``), so an entry
    ``-S <= v < 0`` reads slot ``S + v`` as torch indexing does.  Entries the
    reference would reject (past the pool, or below ``-S``) are clamped into
    the pool, as the kernels do."""
    if single:
        entries = torch.where(entries < 0, entries + pool_slots, entries)
    return entries.clamp(0, pool_slots - 1)


def compact_pools(wl):
    """(k_rows, v_rows, req_to_token) restricted to the slots the batch reads;
    the returned table indexes the compacted rows (no negative entries)."""
    b = wl.batch
    width = b.max_seq_len
    sub = b.req_to_token[b.req_pool_indices, :width]
    rows = pool_rows(sub, wl.k_pool.shape[0], b.batch_size == 1)
    used, inv = torch.unique(rows, return_inverse=True)
    kp = wl.k_pool[used].cpu()
    vp = wl.v_pool[used].cpu()
    rtt = torch.full((b.batch_size, width + 1), -1, dtype=torch.long)
    rtt[:, :width] = inv.cpu()
    return kp, vp, rtt


def prepare_host_inputs(wl):
    """fp32 host (q, k_pool, v_pool, batch, group, scale) for the restatement."""
    kp, vp, rtt = compact_pools(wl)
    if kp.dtype == torch.float8_e4m3fn:
        kf = dequantize_e4m3(kp, wl.k_scale.float().cpu().item())
        vf = dequantize_e4m3(vp, wl.v_scale.float().cpu().item())
    else:
        kf, vf = kp.float(), vp.float()
    batch = HostBatch(wl.batch)
    batch.req_to_token = rtt
    batch.req_pool_indices = torch.arange(wl.batch.batch_size)
    batch.req_pool_indices_list = list(range(wl.batch.batch_size))
    return (wl.q.float().cpu(), kf, vf, batch, wl.num_q_heads // wl.num_kv_heads, wl.scale)


def reference_attention(wl):
    return slot_based_attention_ref(*prepare_host_inputs(wl))
