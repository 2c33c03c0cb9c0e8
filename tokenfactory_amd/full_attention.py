"""``FullAttention``: a drop-in for the reference's ``Qwen3_8FullAttention`` module.

Keeps the reference's call signatures
``forward(hidden_states, positions, cache_pool, forward_batch)``
(``qwen3_8/full_attention.py:112-161``) and
``_slot_based_attention(q, layer_k_buffer, layer_v_buffer, batch)`` (``:163-283``),
and its per-rank head bookkeeping (``:36-52``). The hot steps run on the
gfx950 kernels: q/k norm + RoPE + the KV scatter-write (``:141-149``,
``tf_qk_norm_rope_kv_write``) and the attention itself (``tf_attn_decode`` /
``tf_attn_extend``).

q/k RMSNorm with the ``w * x`` convention (``qwen3_8/rms_norm.py:19-24``),
partial rotate-half RoPE on the first ``head_dim * partial_rotary_factor`` dims
(``qwen3_8/rotary_embedding.py:46-95``) and the KV write run as one fused
kernel (``tf_qk_norm_rope_kv_write``); ``RMSNorm`` / ``PartialRoPE`` below hold
their parameters and state the same math in PyTorch. The ``attn * silu(gate)``
output gate (``full_attention.py:157-159``) is fused into the attention
kernels' output write (the gate is passed as a strided view of the q
projection). With an FP8 ``quantization_config`` (``quant_method == "fp8"``,
``weight_block_size``; ``qwen3_8/fp8_linear.py:27-40``) the q/k/v/o
projections are ``Fp8Linear`` (dynamic e4m3 activations x block-scaled e4m3
weights on the gfx950 FP8 GEMM, like the reference's Triton path); otherwise
plain bf16 ``nn.Linear``.
"""
from __future__ import annotations

from typing import List, Optional

import torch
import torch.nn as nn

from .attention import qk_norm_rope_kv_write, slot_based_attention
from .fp8_linear import Fp8Linear


def _fp8_block_size(config):
    """``weight_block_size`` when the config asks for block-FP8 linears
    (``fp8_linear.py:27-40``), else None."""
    q = getattr(config, "quantization_config", None)
    if isinstance(q, dict) and q.get("quant_method") == "fp8":
        return tuple(q.get("weight_block_size", [128, 128]))
    return None


class RMSNorm(nn.Module):
    """fp32 RMSNorm, ``weight * x / rms(x)`` (``qwen3_8/rms_norm.py:19-24``)."""

    def __init__(self, dim: int, eps: float = 1e-6):
        super().__init__()
        self.weight = nn.Parameter(torch.ones(dim))
        self.eps = eps

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        xf = x.float()
        xf = xf * torch.rsqrt(xf.pow(2).mean(dim=-1, keepdim=True) + self.eps)
        return (self.weight.float() * xf).to(x.dtype)


class PartialRoPE(nn.Module):
    """Rotate-half RoPE on the leading ``rotary_dim`` dims; 1-D positions or
    interleaved 3-D M-RoPE positions (``qwen3_8/rotary_embedding.py:15-95``)."""

    def __init__(self, head_dim: int, partial_rotary_factor: float, rope_theta: float,
                 mrope_section: Optional[List[int]] = None, mrope_interleaved: bool = True):
        super().__init__()
        self.rotary_dim = int(head_dim * partial_rotary_factor)
        self.mrope_section = list(mrope_section or [11, 11, 10])
        self.mrope_interleaved = mrope_interleaved
        exps = torch.arange(0, self.rotary_dim, 2, dtype=torch.float32) / self.rotary_dim
        self.register_buffer("inv_freq", 1.0 / (rope_theta ** exps), persistent=False)

    def _angles(self, positions: torch.Tensor) -> torch.Tensor:
        if positions.dim() == 1:
            return positions.float()[:, None] * self.inv_freq[None, :]
        per_axis = positions.float()[:, :, None] * self.inv_freq[None, None, :]  # [3, T, R/2]
        if self.mrope_interleaved:
            ang = per_axis[0].clone()
            for axis in (1, 2):
                stop = 3 * self.mrope_section[axis]
                ang[:, axis:stop:3] = per_axis[axis, :, axis:stop:3]
            return ang
        pieces = per_axis.split(self.mrope_section, dim=-1)
        return torch.cat([p[i] for i, p in enumerate(pieces)], dim=-1)

    def forward(self, q: torch.Tensor, k: torch.Tensor, positions: torch.Tensor):
        ang = self._angles(positions)
        ang = torch.cat((ang, ang), dim=-1)
        cos = ang.cos()[:, None, :].to(q.dtype)
        sin = ang.sin()[:, None, :].to(q.dtype)
        r = self.rotary_dim

        def rot(x):
            xr, xp = x[..., :r], x[..., r:]
            half = r // 2
            turned = torch.cat((-xr[..., half:], xr[..., :half]), dim=-1)
            return torch.cat((xr * cos + turned * sin, xp), dim=-1)

        return rot(q), rot(k)


class FullAttention(nn.Module):
    """GQA full attention with output gate over a slot-indirected KV pool."""

    def __init__(self, config, layer_idx: int, dtype: torch.dtype = torch.bfloat16):
        super().__init__()
        self.layer_idx = layer_idx
        tp = getattr(config, "tp_size", 1)
        if config.num_attention_heads % tp:
            raise ValueError("num_attention_heads must divide by tp_size")
        self.head_dim = config.head_dim
        self.scaling = self.head_dim ** -0.5
        self.attn_output_gate = getattr(config, "attn_output_gate", True)
        self.num_heads = config.num_attention_heads // tp
        if config.num_key_value_heads >= tp:
            if config.num_key_value_heads % tp:
                raise ValueError("num_key_value_heads must divide by tp_size")
            self.num_kv_heads = config.num_key_value_heads // tp
        else:
            if tp % config.num_key_value_heads:
                raise ValueError("tp_size must divide by num_key_value_heads")
            self.num_kv_heads = 1
        self.num_queries_per_kv = self.num_heads // self.num_kv_heads

        hidden = config.hidden_size
        bias = getattr(config, "attention_bias", False)
        q_out = self.num_heads * self.head_dim * (2 if self.attn_output_gate else 1)
        block = _fp8_block_size(config)
        if block is not None:
            def linear(i, o):
                return Fp8Linear(i, o, bias=bias, block_size=block)
        else:
            def linear(i, o):
                return nn.Linear(i, o, bias=bias, dtype=dtype)
        kv_out = self.num_kv_heads * self.head_dim
        self.q_proj = linear(hidden, q_out)
        self.k_proj = linear(hidden, kv_out)
        self.v_proj = linear(hidden, kv_out)
        self.o_proj = linear(self.num_heads * self.head_dim, hidden)
        eps = getattr(config, "rms_norm_eps", 1e-6)
        self.q_norm = RMSNorm(self.head_dim, eps)
        self.k_norm = RMSNorm(self.head_dim, eps)
        self.rotary_emb = PartialRoPE(self.head_dim,
                                      getattr(config, "partial_rotary_factor", 0.25),
                                      getattr(config, "rope_theta", 1e7),
                                      getattr(config, "mrope_section", None),
                                      getattr(config, "mrope_interleaved", True))

    def forward(self, hidden_states: torch.Tensor, positions: torch.Tensor, cache_pool,
                forward_batch) -> torch.Tensor:
        n_tok = hidden_states.shape[0]
        if self.attn_output_gate:
            qg = self.q_proj(hidden_states).view(n_tok, self.num_heads, 2 * self.head_dim)
            q, gate = qg.chunk(2, dim=-1)   # gate stays a [T, Hq, D] view of qg
        else:
            q = self.q_proj(hidden_states).view(n_tok, self.num_heads, self.head_dim)
            gate = None
        k = self.k_proj(hidden_states).view(n_tok, self.num_kv_heads, self.head_dim)
        v = self.v_proj(hidden_states).view(n_tok, self.num_kv_heads, self.head_dim)

        k_buf, v_buf = cache_pool.get_full_kv_buffers(self.layer_idx)
        scales = (cache_pool.get_full_kv_scales(self.layer_idx)
                  if hasattr(cache_pool, "get_full_kv_scales") else (None, None))
        # q_norm / k_norm, partial RoPE and the KV write (:141-149) in one launch.
        rope = self.rotary_emb
        q = qk_norm_rope_kv_write(
            q, k, v, self.q_norm.weight, self.k_norm.weight, self.q_norm.eps, positions,
            rope.inv_freq, rope.rotary_dim, rope.mrope_section, rope.mrope_interleaved,
            k_buf, v_buf, forward_batch.out_cache_loc, *scales)

        # Attention with the output gate `attn * silu(gate)` (:150-159) fused
        # into the kernels' output write; in front of an FP8 o_proj the same
        # write also takes the per-tensor amax of the activation quantisation
        # (fp8_triton.py:128), which saves that pass a read of the output.
        fp8_out = isinstance(self.o_proj, Fp8Linear)
        amax = torch.zeros((1,), dtype=torch.int32, device=q.device) if fp8_out else None
        attn = slot_based_attention(q, k_buf, v_buf, forward_batch, scaling=self.scaling,
                                    k_scale=scales[0], v_scale=scales[1], gate=gate,
                                    out_amax=amax)
        x = attn.reshape(n_tok, self.num_heads * self.head_dim)
        return self.o_proj(x, x_amax=amax) if fp8_out else self.o_proj(x)

    def _slot_based_attention(self, q: torch.Tensor, layer_k_buffer: torch.Tensor,
                              layer_v_buffer: torch.Tensor, batch, k_scale=None,
                              v_scale=None) -> torch.Tensor:
        """The reference's ungated attention call (``:163-283``); ``forward``
        uses the same kernels with the output gate fused."""
        return slot_based_attention(q, layer_k_buffer, layer_v_buffer, batch,
                                    scaling=self.scaling, k_scale=k_scale, v_scale=v_scale)
