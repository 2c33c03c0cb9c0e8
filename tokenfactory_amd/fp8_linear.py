"""Block-FP8 linear layers on the gfx950 kernels.

``block_fp8_linear`` is the native counterpart of the reference's
``triton_block_fp8_linear(x, weight, weight_scale_inv, bias, block_h, block_w)``
(``qwen3_8/fp8_triton.py:107-183``): dynamic per-tensor quantisation of the
activations to e4m3 (``tf_fp8_act_quant``) followed by the block-scaled FP8
GEMM (``tf_fp8_block_gemm``), bf16 in and out.

``Fp8Linear`` mirrors ``Qwen3_8FP8Linear`` (``qwen3_8/fp8_linear.py:12-212``)
for a float8_e4m3fn weight: the same parameter and buffer names and shapes
(``weight`` ``[out, in]``, ``weight_scale_inv`` ``[ceil(out / block_h),
ceil(in / block_w)]``), ``dequantize_weight`` with the reference's
expand-and-multiply semantics, and a forward that always runs the native GEMM.
There is no non-native path: without the library every call raises.
"""
from __future__ import annotations

import contextlib
import math
from typing import Optional, Sequence

import torch
import torch.nn as nn

from . import _native

FP8_MAX = 448.0


def _ptr(t: Optional[torch.Tensor]) -> int:
    return 0 if t is None else t.data_ptr()


def _stream_ptr(stream, device) -> int:
    s = stream if stream is not None else torch.cuda.current_stream(device)
    return s.cuda_stream


def on_stream(stream):
    """Context that makes ``stream`` current (a no-op for None), so that the
    temporaries a call allocates and the torch ops it runs are ordered on the
    stream its kernels run on, and the caching allocator reuses their memory
    only after that stream is done with it."""
    return torch.cuda.stream(stream) if stream is not None else contextlib.nullcontext()


K_SLICE = 128   # the GEMM's K granularity (one weight-scale block)


def _padded_k(k: int) -> int:
    return -(-k // K_SLICE) * K_SLICE


def _pad_cols(t: torch.Tensor, cols: int) -> torch.Tensor:
    """``t`` with zero columns appended up to ``cols`` (zero e4m3 products add
    nothing to any sum)."""
    if t.shape[1] == cols:
        return t
    out = torch.zeros((t.shape[0], cols), dtype=torch.uint8, device=t.device)
    out[:, : t.shape[1]] = t.view(torch.uint8)
    return out.view(t.dtype)


def quantize_activations(x2d: torch.Tensor, stream=None, padded_cols: Optional[int] = None,
                         amax: Optional[torch.Tensor] = None):
    """Dynamic per-tensor e4m3 quantisation of a bf16 ``[rows, cols]`` matrix
    (``fp8_triton.py:127-130``). Returns ``(xq, x_scale)``: float8_e4m3fn rows
    and a 1-element fp32 tensor holding ``bf16(max(amax|x|, 1e-12) / 448)``.
    With ``padded_cols`` the rows of ``xq`` are zero-extended to that width.
    ``amax``: the max of ``|x|`` already computed by x's producer (a 1-element
    int32 device tensor holding the bf16 bit pattern, as the attention kernels'
    ``out_amax`` leaves it); the result is the same, with one launch
    (``tf_fp8_act_quant_amax``) instead of two."""
    if x2d.dtype != torch.bfloat16 or x2d.dim() != 2 or not x2d.is_cuda:
        raise ValueError("quantize_activations: x must be a 2-D bf16 CUDA tensor")
    if x2d.stride(1) != 1:
        raise ValueError("quantize_activations: x rows must be contiguous")
    rows, cols = x2d.shape
    width = cols if padded_cols is None else padded_cols
    if width < cols:
        raise ValueError("quantize_activations: padded_cols < cols")
    with on_stream(stream):
        xq = torch.empty((rows, width), dtype=torch.float8_e4m3fn, device=x2d.device)
        if width > cols:
            xq.view(torch.uint8)[:, cols:].zero_()
        scale = torch.empty((1,), dtype=torch.float32, device=x2d.device)
        if amax is not None:
            if amax.dtype != torch.int32 or amax.numel() != 1 or amax.device != x2d.device:
                raise ValueError("quantize_activations: amax must be a 1-element int32 tensor "
                                 "on x's device")
            _native.call("tf_fp8_act_quant_amax", _ptr(x2d), _native.TF_DTYPE_BF16, rows, cols,
                         x2d.stride(0), _ptr(xq), xq.stride(0), _ptr(scale), _ptr(amax),
                         _stream_ptr(stream, x2d.device))
            return xq, scale
        ws = torch.empty((_native.TF_FP8_QUANT_WORKSPACE_BYTES,), dtype=torch.uint8,
                         device=x2d.device)
        _native.call("tf_fp8_act_quant", _ptr(x2d), _native.TF_DTYPE_BF16, rows, cols,
                     x2d.stride(0), _ptr(xq), xq.stride(0), _ptr(scale), _ptr(ws), ws.numel(),
                     _stream_ptr(stream, x2d.device))
    return xq, scale


def block_fp8_gemm(xq: torch.Tensor, x_scale: torch.Tensor, weight: torch.Tensor,
                   weight_scale_inv: Optional[torch.Tensor], bias: Optional[torch.Tensor],
                   block_h: int = 128, block_w: int = 128, out: Optional[torch.Tensor] = None,
                   stream=None) -> torch.Tensor:
    """``bf16(sum_kb (xq w^T)[:, kb] * x_scale * weight_scale_inv[n // block_h,
    kb // block_w] + bias)`` (``fp8_triton.py:17-98``), fp32 accumulation.

    ``xq`` may carry zero columns beyond ``weight``'s width (up to the next
    multiple of 128); a width that is not a multiple of 128 is zero-padded
    here, since the kernel consumes K in 128-wide slices."""
    if xq.dtype != torch.float8_e4m3fn or weight.dtype != torch.float8_e4m3fn:
        raise ValueError("block_fp8_gemm: xq and weight must be float8_e4m3fn")
    if xq.dim() != 2 or weight.dim() != 2:
        raise ValueError(f"block_fp8_gemm: shapes {tuple(xq.shape)} x {tuple(weight.shape)}^T")
    k = weight.shape[1]
    kp = _padded_k(k)
    if xq.shape[1] not in (k, kp):
        raise ValueError(f"block_fp8_gemm: shapes {tuple(xq.shape)} x {tuple(weight.shape)}^T")
    if xq.stride(1) != 1 or weight.stride(1) != 1:
        raise ValueError("block_fp8_gemm: xq / weight rows must be contiguous")
    m = xq.shape[0]
    n = weight.shape[0]
    if weight_scale_inv is not None:
        if weight_scale_inv.dtype != torch.float32:
            raise ValueError("block_fp8_gemm: weight_scale_inv must be float32")
        need = (math.ceil(n / block_h), math.ceil(k / block_w))
        if tuple(weight_scale_inv.shape) != need:
            raise ValueError(f"block_fp8_gemm: weight_scale_inv {tuple(weight_scale_inv.shape)}, "
                             f"expected {need}")
    if bias is not None and (bias.dtype != torch.bfloat16 or bias.shape != (n,)
                             or bias.stride(0) != 1):
        raise ValueError("block_fp8_gemm: bias must be a contiguous bf16 [out_features]")
    if x_scale.dtype != torch.float32 or x_scale.numel() != 1:
        raise ValueError("block_fp8_gemm: x_scale must be a 1-element float32 tensor")
    if out is not None and (out.dtype != torch.bfloat16 or tuple(out.shape) != (m, n)
                            or out.stride(1) != 1):
        raise ValueError("block_fp8_gemm: out must be bf16 [m, n] with contiguous rows")
    # split-K scratch for small m (0 bytes when the call does not split)
    nbytes = _native.load().tf_fp8_block_gemm_workspace_bytes(m, n, kp) if m > 0 else 0
    if nbytes < 0:
        raise ValueError("block_fp8_gemm: bad shape")
    with on_stream(stream):
        if out is None:
            out = torch.empty((m, n), dtype=torch.bfloat16, device=xq.device)
        ws = weight_scale_inv
        if kp != k:
            xq, weight = _pad_cols(xq, kp), _pad_cols(weight, kp)
            if ws is None:        # one all-ones block over the true K (fp8_triton.py:132-135)
                block_w = kp
        scratch = torch.empty((nbytes,), dtype=torch.uint8, device=xq.device) if nbytes else None
        _native.call("tf_fp8_block_gemm", _ptr(xq), xq.stride(0), _ptr(x_scale),
                     _ptr(weight), weight.stride(0), _ptr(ws),
                     0 if ws is None else ws.stride(0), 0 if ws is None else ws.stride(1),
                     block_h, block_w, _ptr(bias), m, n, kp, _ptr(out), out.stride(0),
                     _ptr(scratch), nbytes, _stream_ptr(stream, xq.device))
    return out


def block_fp8_linear(x: torch.Tensor, weight: torch.Tensor,
                     weight_scale_inv: Optional[torch.Tensor], bias: Optional[torch.Tensor],
                     block_h: int = 128, block_w: int = 128, stream=None,
                     x_amax: Optional[torch.Tensor] = None) -> torch.Tensor:
    """Native ``triton_block_fp8_linear`` (``fp8_triton.py:107-183``): x ``[..., in]``
    bf16, weight float8_e4m3fn ``[out, in]`` -> bf16 ``[..., out]``. ``x_amax``:
    max ``|x|`` from x's producer, see ``quantize_activations``."""
    in_features = weight.shape[1]
    if x.shape[-1] != in_features:
        raise ValueError(f"block_fp8_linear: x [..., {x.shape[-1]}] vs weight in={in_features}")
    x2d = x.reshape(-1, in_features)
    if x2d.stride(1) != 1:
        x2d = x2d.contiguous()
    xq, scale = quantize_activations(x2d, stream, padded_cols=_padded_k(in_features),
                                     amax=x_amax)
    out = block_fp8_gemm(xq, scale, weight, weight_scale_inv, bias, block_h, block_w,
                         stream=stream)
    return out.reshape(*x.shape[:-1], weight.shape[0])


class Fp8Linear(nn.Module):
    """``Qwen3_8FP8Linear`` with a float8_e4m3fn weight (``fp8_linear.py:12-212``).

    ``weight``: float8_e4m3fn ``[out_features, in_features]``;
    ``weight_scale_inv``: fp32 ``[ceil(out / block_h), ceil(in / block_w)]``
    (ones at init, like the reference), ``bias``: bf16 or absent.
    """

    def __init__(self, in_features: int, out_features: int, bias: bool = False,
                 block_size: Sequence[int] = (128, 128), device=None):
        super().__init__()
        self.in_features = in_features
        self.out_features = out_features
        self.block_h, self.block_w = int(block_size[0]), int(block_size[1])
        self.weight = nn.Parameter(
            torch.zeros((out_features, in_features), dtype=torch.float8_e4m3fn, device=device),
            requires_grad=False)
        self.register_buffer("weight_scale_inv", torch.ones(
            (math.ceil(out_features / self.block_h), math.ceil(in_features / self.block_w)),
            dtype=torch.float32, device=device), persistent=True)
        if bias:
            self.bias = nn.Parameter(torch.zeros(out_features, dtype=torch.bfloat16,
                                                 device=device), requires_grad=False)
        else:
            self.register_parameter("bias", None)

    @torch.no_grad()
    def quantize_from(self, w: torch.Tensor) -> "Fp8Linear":
        """Fills ``weight`` / ``weight_scale_inv`` from a dense ``[out, in]``
        weight with per-block scales ``amax / 448`` (the checkpoint format)."""
        out_f, in_f = self.out_features, self.in_features
        bh, bw = self.block_h, self.block_w
        wf = w.to(torch.float32)
        sh, sw = self.weight_scale_inv.shape
        pad = torch.zeros((sh * bh, sw * bw), dtype=torch.float32, device=wf.device)
        pad[:out_f, :in_f] = wf
        blocks = pad.view(sh, bh, sw, bw)
        amax = blocks.abs().amax(dim=(1, 3)).clamp(min=1e-12)
        scale = amax / FP8_MAX
        q = (blocks / scale[:, None, :, None]).clamp(-FP8_MAX, FP8_MAX)
        self.weight.copy_(q.view(sh * bh, sw * bw)[:out_f, :in_f].to(torch.float8_e4m3fn))
        self.weight_scale_inv.copy_(scale)
        return self

    def dequantize_weight(self, target_dtype: torch.dtype) -> torch.Tensor:
        """``weight * repeat_interleave(weight_scale_inv)`` (``fp8_linear.py:74-86``)."""
        scale = self.weight_scale_inv.to(torch.float32)
        full = scale.repeat_interleave(self.block_h, dim=0).repeat_interleave(self.block_w, dim=1)
        full = full[: self.out_features, : self.in_features]
        return (self.weight.to(torch.float32) * full).to(target_dtype)

    def forward(self, x: torch.Tensor, x_amax: Optional[torch.Tensor] = None) -> torch.Tensor:
        """``x_amax``: optional max ``|x|`` from x's producer (see
        ``quantize_activations``); the result does not change."""
        return block_fp8_linear(x, self.weight, self.weight_scale_inv, self.bias,
                                self.block_h, self.block_w, x_amax=x_amax)

    def extra_repr(self) -> str:
        return (f"in_features={self.in_features}, out_features={self.out_features}, "
                f"bias={self.bias is not None}, block_size=({self.block_h}, {self.block_w})")
