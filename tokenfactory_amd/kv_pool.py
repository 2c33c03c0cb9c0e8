"""Full-attention KV pool: the token-slot half of the reference's hybrid cache pool.

Layout as the reference (``qwen3_8/hybrid_cache_pool.py:48-61``, accessor ``:106-109``):
``k_buffer`` / ``v_buffer`` are ``[num_full_layers, max_total_tokens,
local_kv_heads, head_dim]``; ``get_full_kv_buffers(layer_idx)`` returns the
contiguous ``[S, Hkv, D]`` views of one full-attention layer, indexed by model
layer number through ``full_layer_map``. Slot 0 is the padding slot
(``token_to_kv_pool.py:20-23``).

Additions for MI355X: the pool may be stored as OCP ``float8_e4m3fn`` with one
fp32 scale per layer for K and one for V (``k_scale`` / ``v_scale``, device
tensors ``[num_full_layers]``); ``write_kv`` quantises on the way in.
A 1M-slot bf16 pool with 4 kv heads of 256 dims is 2 GiB for K plus 2 GiB for V
per layer, which the 288 GB of HBM3E holds comfortably for all 16 layers.
"""
from __future__ import annotations

from typing import Dict, Iterable, Optional, Tuple

import torch

from .attention import write_kv


class FullAttnKVPool:
    def __init__(self, full_layer_indices: Iterable[int], max_total_tokens: int,
                 num_kv_heads: int, head_dim: int, device="cuda",
                 dtype: torch.dtype = torch.bfloat16):
        if dtype not in (torch.bfloat16, torch.float8_e4m3fn, torch.float32):
            raise ValueError(f"unsupported KV dtype {dtype}")
        self.full_layer_map: Dict[int, int] = {
            layer: i for i, layer in enumerate(full_layer_indices)}
        n_layers = len(self.full_layer_map)
        self.max_total_tokens = max_total_tokens
        self.num_kv_heads = num_kv_heads
        self.head_dim = head_dim
        self.device = torch.device(device)
        self.dtype = dtype
        shape = (n_layers, max_total_tokens, num_kv_heads, head_dim)
        self.k_buffer = torch.zeros(shape, dtype=dtype, device=self.device)
        self.v_buffer = torch.zeros_like(self.k_buffer)
        self.k_scale = torch.ones(n_layers, dtype=torch.float32, device=self.device)
        self.v_scale = torch.ones(n_layers, dtype=torch.float32, device=self.device)

    @classmethod
    def from_config(cls, config, max_total_tokens: int, device="cuda",
                    dtype: torch.dtype = torch.bfloat16) -> "FullAttnKVPool":
        """Builds the pool the way ``Qwen3_8HybridCachePool`` sizes its full-attention
        part (``hybrid_cache_pool.py:36-61``, layer list from ``config.py:83-87``): full layers from ``layer_types``,
        ``max(1, num_key_value_heads // tp_size)`` local kv heads."""
        layers = [i for i, t in enumerate(config.layer_types) if t == "full_attention"]
        local_kv = max(1, config.num_key_value_heads // getattr(config, "tp_size", 1))
        return cls(layers, max_total_tokens, local_kv, config.head_dim, device, dtype)

    @property
    def is_fp8(self) -> bool:
        return self.dtype == torch.float8_e4m3fn

    def get_full_kv_buffers(self, layer_idx: int) -> Tuple[torch.Tensor, torch.Tensor]:
        i = self.full_layer_map[layer_idx]
        return self.k_buffer[i], self.v_buffer[i]

    def get_full_kv_scales(self, layer_idx: int) -> Tuple[Optional[torch.Tensor],
                                                           Optional[torch.Tensor]]:
        """Per-tensor fp32 scales of the layer (``None`` for a non-fp8 pool)."""
        if not self.is_fp8:
            return None, None
        i = self.full_layer_map[layer_idx]
        return self.k_scale[i:i + 1], self.v_scale[i:i + 1]

    def set_kv_scales(self, layer_idx: int, k_scale: float, v_scale: float) -> None:
        i = self.full_layer_map[layer_idx]
        self.k_scale[i] = float(k_scale)
        self.v_scale[i] = float(v_scale)

    def write_kv(self, layer_idx: int, out_cache_loc: torch.Tensor, k: torch.Tensor,
                 v: torch.Tensor) -> None:
        """``k_buf[out_cache_loc] = k`` (and v) for one layer (``full_attention.py:146-149``)."""
        kb, vb = self.get_full_kv_buffers(layer_idx)
        ks, vs = self.get_full_kv_scales(layer_idx)
        write_kv(kb, vb, out_cache_loc, k, v, ks, vs)
