"""q/k RMSNorm + partial (M-)RoPE restated op for op (reference
``qwen3_8/rms_norm.py:19-24`` and ``qwen3_8/rotary_embedding.py:36-95``).

TEST INFRASTRUCTURE ONLY. The functions follow the reference's tensor ops in
its order and dtypes, so run on bf16 inputs they reproduce the reference's
bf16 rounding steps, and on fp32 inputs its fp32 CPU path. Pinned by the
golden vectors the reference module itself produced
(``tests/golden/module_golden.npz``; ``tests/test_qk_prep_oracle.py``).
"""
from __future__ import annotations

from typing import List

import torch


def rms_norm_ref(x: torch.Tensor, weight: torch.Tensor, eps: float) -> torch.Tensor:
    """``Qwen3_8RMSNorm.forward`` (rms_norm.py:19-24)."""
    orig = x.dtype
    xf = x.float()
    var = xf.pow(2).mean(dim=-1, keepdim=True)
    return (weight.float() * (xf * torch.rsqrt(var + eps))).to(orig)


def inv_freq_ref(rotary_dim: int, theta: float) -> torch.Tensor:
    """``PartialRotaryEmbedding.inv_freq`` (rotary_embedding.py:30-37)."""
    return 1.0 / (theta ** (torch.arange(0, rotary_dim, 2, dtype=torch.float32) / rotary_dim))


def _cos_sin(positions, inv_freq, mrope_section: List[int], interleaved: bool, dtype):
    """``_compute_cos_sin`` (rotary_embedding.py:46-73)."""
    if positions.ndim == 1:
        freqs = torch.outer(positions.float(), inv_freq)
    else:
        f3 = positions.float()[:, :, None] * inv_freq[None, None, :]
        if interleaved:
            freqs = f3[0].clone()
            for axis in (1, 2):
                lim = mrope_section[axis] * 3
                freqs[:, axis:lim:3] = f3[axis, :, axis:lim:3]
        else:
            freqs = torch.cat([c[i] for i, c in enumerate(f3.split(mrope_section, dim=-1))],
                              dim=-1)
    emb = torch.cat((freqs, freqs), dim=-1)
    return emb.cos().unsqueeze(1).to(dtype), emb.sin().unsqueeze(1).to(dtype)


def _rotate_half(x):
    half = x.shape[-1] // 2
    return torch.cat((-x[..., half:], x[..., :half]), dim=-1)


def rope_ref(q, k, positions, inv_freq, rotary_dim: int, mrope_section: List[int],
             interleaved: bool):
    """``PartialRotaryEmbedding.forward`` (rotary_embedding.py:75-95)."""
    cos, sin = _cos_sin(positions, inv_freq.to(q.device), mrope_section, interleaved, q.dtype)
    qr, qp = q[..., :rotary_dim], q[..., rotary_dim:]
    kr, kp = k[..., :rotary_dim], k[..., rotary_dim:]
    qr = qr * cos + _rotate_half(qr) * sin
    kr = kr * cos + _rotate_half(kr) * sin
    return torch.cat((qr, qp), dim=-1), torch.cat((kr, kp), dim=-1)


def qk_prep_ref(q, k, q_norm_w, k_norm_w, eps, positions, inv_freq, rotary_dim,
                mrope_section, interleaved):
    """``q_norm``/``k_norm`` then ``rotary_emb`` (full_attention.py:141-143)."""
    q = rms_norm_ref(q, q_norm_w, eps)
    k = rms_norm_ref(k, k_norm_w, eps)
    return rope_ref(q, k, positions, inv_freq, rotary_dim, mrope_section, interleaved)
