"""Per-step batch metadata consumed by the full-attention kernels.

Same field names, types and defaulting rules as the reference's
``ForwardBatch`` (``qwen3_8/forward_batch.py:6-45``) so that its producer
(``engine/model_runner.py:108-188``) and every consumer keep working unchanged.

What the attention path reads:

* ``batch_size``, ``req_pool_indices`` (int64 ``[B]``, row of each request in
  ``req_to_token``), ``seq_lens`` (int64 ``[B]``, prefix + new tokens);
* ``extend_lens`` (host list, new tokens per request; decode requests have 1),
  ``extend_lens_tensor`` (its device copy), ``max_seq_len``, ``max_extend_len``
  (host ints), ``req_pool_indices_list`` (host copy of ``req_pool_indices``);
* ``req_to_token`` (int64 ``[max_reqs, max_context_len]``; ``-1`` = empty) and
  ``out_cache_loc`` (int64 ``[T]``, pool slot of each new token).

``prefix_lens`` and ``is_prefill`` are carried but not read by attention (the
prefix is ``seq_lens - extend_lens``, as at ``qwen3_8/full_attention.py:267``).
"""
from __future__ import annotations

from dataclasses import dataclass
from typing import List, Optional

import torch


@dataclass
class ForwardBatch:
    batch_size: int
    req_pool_indices: torch.Tensor
    seq_lens: torch.Tensor
    prefix_lens: torch.Tensor
    extend_lens: List[int]
    out_cache_loc: torch.Tensor
    req_to_token: torch.Tensor
    is_prefill: bool = True
    # Host-side copies that spare the forward pass a device->host sync.
    max_seq_len: int = 0
    max_extend_len: int = 0
    extend_lens_tensor: Optional[torch.Tensor] = None
    req_pool_indices_list: Optional[List[int]] = None

    def __post_init__(self) -> None:
        # Defaulting order and rules follow qwen3_8/forward_batch.py:33-45.
        if self.extend_lens and self.max_extend_len == 0:
            self.max_extend_len = max(self.extend_lens)
        if self.extend_lens and self.extend_lens_tensor is None:
            self.extend_lens_tensor = torch.tensor(
                list(self.extend_lens), dtype=torch.long,
                device=self.out_cache_loc.device)
        if self.max_seq_len == 0 and self.seq_lens.numel() > 0:
            self.max_seq_len = int(self.seq_lens.max().item())
        if self.req_pool_indices_list is None and self.req_pool_indices.numel() > 0:
            self.req_pool_indices_list = [int(v) for v in self.req_pool_indices.tolist()]
