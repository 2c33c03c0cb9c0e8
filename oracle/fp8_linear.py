"""Block-FP8 linear layer (the o_proj after the gated attention output).

TEST INFRASTRUCTURE ONLY.

Restates, op for op on the CPU, the reference's Triton path for a
float8_e4m3fn weight (``Qwen3_8FP8Linear._linear_op``,
``qwen3_8/fp8_linear.py:181-201``):

* ``quantize_activations`` -- ``triton_block_fp8_linear``'s dynamic
  per-tensor activation quantisation (``qwen3_8/fp8_triton.py:127-130``):
  ``amax = x.abs().max().clamp(min=1e-12)`` and ``amax / 448`` on bf16 tensors
  (so both round to bf16), then ``e4m3(clamp(x.float() / x_scale, +-448))``;
* ``block_gemm`` -- ``_block_fp8_gemm_kernel`` (``fp8_triton.py:17-98``):
  ``acc += (xq[:, ks] @ w[:, ks]^T) * (x_scale * ws[n // block_h, k0 // block_w])``
  over ``BLOCK_K = 64`` slices ``ks`` (``fp8_triton.py:146-153``), then
  ``+ bias`` and the cast to the activation dtype. The slice products are
  formed in float64 (fp8 x fp8 products and their sums are exact there for the
  sizes used), so the result is the exactly accumulated value up to the final
  fp32 rounding; the kernel under test accumulates in fp32 in another order.
* ``dequantize_weight`` -- ``Qwen3_8FP8Linear.dequantize_weight``
  (``fp8_linear.py:74-86``), used by the closed-form pin below.

Pins (``tests/test_fp8_linear_oracle.py``): the e4m3 decode table against the
format's bit layout, round-to-nearest-even ties of the encode, the bf16
rounding of ``x_scale``; ``block_gemm`` against the dequantise-then-matmul
closed form, against explicit Python loops on tiny inputs, and against an
all-ones input whose output is ``x_scale * 128 * sum_kb ws[n // bh, kb]`` (a
transposed or shifted scale index fails it); the parameter shapes of
``Fp8Linear`` against the reference's own checkpoint-shape tests
(``tests/test_qwen3_8_model.py:48-75``, ``tests/test_tensor_parallel.py:35-60``).
"""
from __future__ import annotations

import math
from typing import Optional

import torch

FP8_MAX = 448.0
BLOCK_K = 64          # the reference kernel's K step for 128-wide scale blocks


def quantize_activations(x: torch.Tensor):
    """``(x_fp8, x_scale)`` for a 2-D bf16 tensor, as ``fp8_triton.py:127-130``."""
    x = x.cpu()
    amax = x.abs().max().clamp(min=1e-12)
    x_scale = (amax / FP8_MAX).to(torch.float32)
    x_fp8 = (x.float() / x_scale).clamp(-FP8_MAX, FP8_MAX).to(torch.float8_e4m3fn)
    return x_fp8, x_scale.reshape(1)


def block_gemm(xq: torch.Tensor, x_scale: torch.Tensor, w: torch.Tensor,
               ws: Optional[torch.Tensor], block_h: int = 128, block_w: int = 128,
               bias: Optional[torch.Tensor] = None) -> torch.Tensor:
    """fp32 ``[M, N]`` result of ``_block_fp8_gemm_kernel`` before the output cast."""
    xq, w = xq.cpu(), w.cpu()
    m, k = xq.shape
    n = w.shape[0]
    a = xq.to(torch.float64)
    b = w.to(torch.float64)
    if ws is None:                       # fp8_triton.py:132-135: one all-ones block
        ws = torch.ones((1, 1), dtype=torch.float32)
        block_h, block_w = n, k
    ws = ws.cpu().to(torch.float64)
    sx = float(x_scale.reshape(-1)[0])
    rows = torch.arange(n) // block_h
    acc = torch.zeros((m, n), dtype=torch.float64)
    for k0 in range(0, k, BLOCK_K):
        k1 = min(k0 + BLOCK_K, k)
        part = a[:, k0:k1] @ b[:, k0:k1].T
        col_scale = ws[rows, k0 // block_w] * sx
        acc += part * col_scale[None, :]
    if bias is not None:
        acc += bias.cpu().to(torch.float64)[None, :]
    return acc.to(torch.float32)


def block_fp8_linear(x: torch.Tensor, w: torch.Tensor, ws: Optional[torch.Tensor],
                     bias: Optional[torch.Tensor] = None, block_h: int = 128,
                     block_w: int = 128):
    """``(out_fp32, x_fp8, x_scale)`` of ``triton_block_fp8_linear`` on 2-D x;
    the reference's output is ``out_fp32.to(x.dtype)``."""
    xq, sx = quantize_activations(x)
    return block_gemm(xq, sx, w, ws, block_h, block_w, bias), xq, sx


def dequantize_weight(w: torch.Tensor, ws: torch.Tensor, block_h: int = 128,
                      block_w: int = 128) -> torch.Tensor:
    """float64 ``w * ws`` expanded over its blocks (``fp8_linear.py:74-86``)."""
    n, k = w.shape
    full = ws.cpu().to(torch.float64).repeat_interleave(block_h, 0).repeat_interleave(block_w, 1)
    return w.cpu().to(torch.float64) * full[:n, :k]


def quantize_weight_blocks(w: torch.Tensor, block_h: int = 128, block_w: int = 128):
    """Synthetic checkpoint weights: per-block ``scale = amax / 448`` and
    ``e4m3(w / scale)`` (the layout ``weight`` / ``weight_scale_inv`` of the
    reference's FP8 checkpoints)."""
    w = w.cpu().to(torch.float32)
    n, k = w.shape
    sh, sw = math.ceil(n / block_h), math.ceil(k / block_w)
    pad = torch.zeros((sh * block_h, sw * block_w), dtype=torch.float32)
    pad[:n, :k] = w
    blocks = pad.view(sh, block_h, sw, block_w)
    scale = blocks.abs().amax(dim=(1, 3)).clamp(min=1e-12) / FP8_MAX
    q = (blocks / scale[:, None, :, None]).clamp(-FP8_MAX, FP8_MAX)
    wq = q.view(sh * block_h, sw * block_w)[:n, :k].to(torch.float8_e4m3fn)
    return wq, scale.to(torch.float32)
