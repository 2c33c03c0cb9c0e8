"""fp8-e4m3fn KV quantisation with a per-tensor scale, and its dequantisation.

TEST INFRASTRUCTURE ONLY.

The reference keeps its KV pool in the activation dtype
(``qwen3_8/hybrid_cache_pool.py:48-61``); the fp8 KV variant is this build's
addition. Its convention, shared by the HIP write kernel:

* scale ``s`` is a positive fp32 per-tensor factor (``amax / 448`` for the
  synthetic workloads), stored beside the pool;
* ``q = e4m3fn(clamp(x_fp32 / s, -448, 448))`` with round-to-nearest-even
  (PyTorch's ``float8_e4m3fn`` cast), saturating instead of producing NaN;
* ``x_hat = float(q) * s``: the e4m3fn -> fp32 conversion is exact.

Attention over an fp8 pool is compared with the same attention run on the
dequantised pool ``x_hat``.
"""
from __future__ import annotations

import torch

E4M3_MAX = 448.0


def quantize_e4m3(x: torch.Tensor, scale) -> torch.Tensor:
    s = torch.as_tensor(scale, dtype=torch.float32, device=x.device)
    y = (x.float() / s).clamp(-E4M3_MAX, E4M3_MAX)
    return y.to(torch.float8_e4m3fn)


def dequantize_e4m3(q: torch.Tensor, scale) -> torch.Tensor:
    s = torch.as_tensor(scale, dtype=torch.float32, device=q.device)
    return q.float() * s


def per_tensor_scale(x: torch.Tensor) -> float:
    """``amax / 448`` (the synthetic workloads' convention)."""
    return float(x.float().abs().max()) / E4M3_MAX
