"""Gated DeltaNet (linear-attention) decode step on the gfx950 kernel.

``gdn_decode_step`` is the native counterpart of
``Qwen3_8LinearAttention._batched_decode_step`` (``qwen3_8/linear_attention.py:244-298``)
followed by ``self.norm(attn_out, z)`` (``:325``): one fused launch
(``tf_gdn_decode``) does the causal-conv step, q/k normalisation, the gated
delta-rule state update, the readout and the gated RMSNorm, updating the
layer's conv and SSM states in place.

``LinearAttention`` mirrors ``Qwen3_8LinearAttention``'s parameters
(``:29-107``: ``in_proj_qkv``, ``in_proj_z``, ``in_proj_b``, ``in_proj_a``,
``conv1d``, ``A_log``, ``dt_bias``, ``norm.weight``, ``out_proj``) and its
``forward(hidden_states, cache_pool, forward_batch)``: all-decode batches run
``gdn_decode_step``; batches with longer extends run ``gdn_extend_step``
(``tf_gdn_extend``), the reference's per-request conv + chunked-update loop
(the same chunk-wise WY update on MFMAs, 32-token chunks, each head's state
held in registers from the first chunk to the last).
"""
from __future__ import annotations

from typing import Optional, Sequence

import torch
import torch.nn as nn

from . import _native
from .fp8_linear import Fp8Linear, on_stream

HEAD_DIM = 128      # the tuned kernels' head dims (key and value)
MAX_OTHER_HEAD_DIM = 64   # other head dims: multiples of 4 up to this (one wave per head)
CONV_KERNEL = 4


def head_dims_supported(dk: int, dv: int) -> bool:
    """Head dims the kernels take: 128 / 128, or multiples of 4 up to 64 each
    (the reference's own test models use 16)."""
    if dk == HEAD_DIM and dv == HEAD_DIM:
        return True
    return all(d % 4 == 0 and 4 <= d <= MAX_OTHER_HEAD_DIM for d in (dk, dv))


def _ptr(t: Optional[torch.Tensor]) -> int:
    return 0 if t is None else t.data_ptr()


def _rows(t: torch.Tensor, name: str) -> int:
    if t.dim() != 2 or t.stride(1) != 1:
        raise ValueError(f"gdn_decode_step: {name} must be 2-D with contiguous rows")
    return t.stride(0)


def _check_common(qkv, b, a, z, conv_weight, a_log, dt_bias, norm_weight, layer_conv_state,
                  layer_ssm_state, req_indices, num_v_heads):
    """Checks the shared arguments; returns the head dims (dk, dv) of
    ``layer_ssm_state`` [slots, Hv, Dk, Dv]."""
    for name, t, dt in (("qkv", qkv, torch.bfloat16), ("b", b, torch.bfloat16),
                        ("a", a, torch.bfloat16), ("z", z, torch.bfloat16),
                        ("conv_weight", conv_weight, torch.float32),
                        ("a_log", a_log, torch.float32), ("dt_bias", dt_bias, torch.float32),
                        ("norm_weight", norm_weight, torch.float32),
                        ("layer_conv_state", layer_conv_state, torch.bfloat16),
                        ("layer_ssm_state", layer_ssm_state, torch.float32),
                        ("req_indices", req_indices, torch.int64)):
        if t.dtype != dt or not t.is_cuda:
            raise ValueError(f"gdn step: {name} must be a {dt} CUDA tensor")
    if a.stride() != b.stride() or a.shape != b.shape:
        raise ValueError("gdn step: a and b must share shape and strides")
    for name, t in (("conv_weight", conv_weight), ("a_log", a_log), ("dt_bias", dt_bias),
                    ("norm_weight", norm_weight), ("req_indices", req_indices)):
        if not t.is_contiguous():
            raise ValueError(f"gdn step: {name} must be contiguous")
    cs, ss = layer_conv_state, layer_ssm_state
    if cs.dim() != 3 or cs.stride(2) != 1 or cs.stride(1) != CONV_KERNEL - 1:
        raise ValueError("gdn step: conv state must be [slots, conv_dim, 3] with dense rows")
    if ss.dim() != 4 or ss.shape[1] != num_v_heads or not ss[0].is_contiguous():
        raise ValueError("gdn step: ssm state must be [slots, Hv, Dk, Dv], dense per slot")
    dk, dv = int(ss.shape[2]), int(ss.shape[3])
    if not head_dims_supported(dk, dv):
        raise NotImplementedError(f"gdn step: head dims {dk} / {dv} (128 / 128, or multiples "
                                  f"of 4 up to {MAX_OTHER_HEAD_DIM})")
    return dk, dv


def gdn_decode_step(qkv: torch.Tensor, b: torch.Tensor, a: torch.Tensor, z: torch.Tensor,
                    conv_weight: torch.Tensor, a_log: torch.Tensor, dt_bias: torch.Tensor,
                    norm_weight: torch.Tensor, eps: float, layer_conv_state: torch.Tensor,
                    layer_ssm_state: torch.Tensor, req_indices: torch.Tensor,
                    num_k_heads: int, num_v_heads: int, return_core: bool = False,
                    stream=None):
    """One decode step of a Gated DeltaNet layer for B requests (one token each).

    qkv bf16 [B, 2*Hk*Dk + Hv*Dv], b / a bf16 [B, Hv], z bf16 [B, Hv*Dv];
    conv_weight fp32 [conv_dim, 4]; a_log, dt_bias fp32 [Hv]; norm_weight fp32
    [Hv*Dv]; layer_conv_state bf16 [slots, conv_dim, 3] and layer_ssm_state
    fp32 [slots, Hv, Dk, Dv] (updated in place; its shape gives the head dims);
    req_indices int64 [B] (distinct).
    Returns the normed bf16 output [B, Hv*Dv] (and the pre-norm output)."""
    bsz = qkv.shape[0]
    dk, dv = _check_common(qkv, b, a, z, conv_weight, a_log, dt_bias, norm_weight,
                           layer_conv_state, layer_ssm_state, req_indices, num_v_heads)
    value_dim = num_v_heads * dv
    cs, ss = layer_conv_state, layer_ssm_state
    s = stream if stream is not None else torch.cuda.current_stream(qkv.device)
    with on_stream(stream):
        out = torch.empty((bsz, value_dim), dtype=torch.bfloat16, device=qkv.device)
        core = torch.empty_like(out) if return_core else None
        # bf16 conv outputs [B, conv_dim], then fp32 gates [B, Hv, 2]
        ws = torch.empty(bsz * ((2 * num_k_heads * dk + value_dim) * 2 + num_v_heads * 8),
                         dtype=torch.uint8, device=qkv.device)
        _native.call("tf_gdn_decode", _ptr(qkv), _rows(qkv, "qkv"), _ptr(a), _ptr(b),
                     _rows(a, "a"), _ptr(z), _rows(z, "z"), _ptr(conv_weight), _ptr(a_log),
                     _ptr(dt_bias), _ptr(norm_weight), float(eps), _ptr(cs), cs.stride(0),
                     _ptr(ss), ss.stride(0), _ptr(req_indices), bsz, cs.shape[0], num_k_heads,
                     num_v_heads, dk, dv, CONV_KERNEL, _ptr(out), out.stride(0),
                     _ptr(core), 0 if core is None else core.stride(0), _ptr(ws),
                     ws.numel(), s.cuda_stream)
    return (out, core) if return_core else out


def gdn_extend_step(qkv: torch.Tensor, b: torch.Tensor, a: torch.Tensor, z: torch.Tensor,
                    conv_weight: torch.Tensor, a_log: torch.Tensor, dt_bias: torch.Tensor,
                    norm_weight: torch.Tensor, eps: float, layer_conv_state: torch.Tensor,
                    layer_ssm_state: torch.Tensor, req_indices: torch.Tensor,
                    extend_lens: Sequence[int], num_k_heads: int, num_v_heads: int,
                    return_core: bool = False, stream=None):
    """The layer for a batch with any extend lengths (the reference's per-request
    loop, ``linear_attention.py:328-364``): request i owns the next
    ``extend_lens[i]`` token rows of qkv / a / b / z. Same tensors as
    ``gdn_decode_step`` with rows = tokens; returns ``[T, Hv*Dv]`` bf16."""
    n_tok = qkv.shape[0]
    lens = [int(e) for e in extend_lens]
    if len(lens) != req_indices.numel() or sum(lens) != n_tok or min(lens, default=1) < 0:
        raise ValueError("gdn_extend_step: extend_lens must cover the token rows, one per request")
    dk, dv = _check_common(qkv, b, a, z, conv_weight, a_log, dt_bias, norm_weight,
                           layer_conv_state, layer_ssm_state, req_indices, num_v_heads)
    offsets = [0]
    for e in lens:
        offsets.append(offsets[-1] + e)
    value_dim = num_v_heads * dv
    ws_bytes = _native.load().tf_gdn_extend_workspace_bytes(n_tok, len(lens), num_k_heads,
                                                           num_v_heads)
    if ws_bytes < 0:
        raise ValueError("gdn_extend_step: bad head counts")
    s = stream if stream is not None else torch.cuda.current_stream(qkv.device)
    cs, ss = layer_conv_state, layer_ssm_state
    with on_stream(stream):
        tok = torch.tensor(offsets, dtype=torch.int32).to(qkv.device, non_blocking=True)
        out = torch.empty((n_tok, value_dim), dtype=torch.bfloat16, device=qkv.device)
        core = torch.empty_like(out) if return_core else None
        ws = torch.empty((max(ws_bytes, 1),), dtype=torch.uint8, device=qkv.device)
        _native.call("tf_gdn_extend", _ptr(qkv), _rows(qkv, "qkv"), _ptr(a), _ptr(b),
                     _rows(a, "a"), _ptr(z), _rows(z, "z"), _ptr(conv_weight), _ptr(a_log),
                     _ptr(dt_bias), _ptr(norm_weight), float(eps), _ptr(cs), cs.stride(0),
                     _ptr(ss), ss.stride(0), _ptr(req_indices), _ptr(tok), len(lens), n_tok,
                     max(lens), cs.shape[0], num_k_heads, num_v_heads, dk, dv,
                     CONV_KERNEL, _ptr(out), out.stride(0), _ptr(core),
                     0 if core is None else core.stride(0), _ptr(ws), ws.numel(), s.cuda_stream)
    return (out, core) if return_core else out


class LinearAttention(nn.Module):
    """Gated DeltaNet layer with ``Qwen3_8LinearAttention``'s parameter names and
    shapes (one TP rank's share; ``qwen3_8/linear_attention.py:29-107``)."""

    def __init__(self, config, layer_idx: int, dtype: torch.dtype = torch.bfloat16):
        super().__init__()
        tp = getattr(config, "tp_size", 1)
        self.layer_idx = layer_idx
        self.num_k_heads = config.linear_num_key_heads // tp
        self.num_v_heads = config.linear_num_value_heads // tp
        self.head_k_dim = config.linear_key_head_dim
        self.head_v_dim = config.linear_value_head_dim
        if (not head_dims_supported(self.head_k_dim, self.head_v_dim)
                or config.linear_conv_kernel_dim != CONV_KERNEL):
            raise NotImplementedError(
                f"LinearAttention: head dims {self.head_k_dim} / {self.head_v_dim} (128 / 128 or "
                f"multiples of 4 up to {MAX_OTHER_HEAD_DIM}) with conv kernel {CONV_KERNEL}")
        self.key_dim = self.num_k_heads * self.head_k_dim
        self.value_dim = self.num_v_heads * self.head_v_dim
        self.conv_dim = 2 * self.key_dim + self.value_dim
        self.eps = getattr(config, "rms_norm_eps", 1e-6)
        hidden = config.hidden_size
        q = getattr(config, "quantization_config", None)
        if isinstance(q, dict) and q.get("quant_method") == "fp8":
            block = tuple(q.get("weight_block_size", [128, 128]))
            self.in_proj_qkv = Fp8Linear(hidden, self.conv_dim, block_size=block)
            self.in_proj_z = Fp8Linear(hidden, self.value_dim, block_size=block)
            self.out_proj = Fp8Linear(self.value_dim, hidden, block_size=block)
        else:
            self.in_proj_qkv = nn.Linear(hidden, self.conv_dim, bias=False, dtype=dtype)
            self.in_proj_z = nn.Linear(hidden, self.value_dim, bias=False, dtype=dtype)
            self.out_proj = nn.Linear(self.value_dim, hidden, bias=False, dtype=dtype)
        self.in_proj_b = nn.Linear(hidden, self.num_v_heads, bias=False, dtype=dtype)
        self.in_proj_a = nn.Linear(hidden, self.num_v_heads, bias=False, dtype=dtype)
        self.conv1d = nn.Conv1d(self.conv_dim, self.conv_dim, kernel_size=CONV_KERNEL,
                                groups=self.conv_dim, padding=CONV_KERNEL - 1, bias=False,
                                dtype=dtype)
        self.A_log = nn.Parameter(torch.zeros(self.num_v_heads, dtype=dtype))
        self.dt_bias = nn.Parameter(torch.ones(self.num_v_heads, dtype=dtype))
        self.norm = nn.Module()
        self.norm.weight = nn.Parameter(torch.ones(self.value_dim, dtype=dtype))
        self._packed = None
        self._packed_key = None

    def _kernel_params(self):
        """fp32 copies of the conv taps, A_log, dt_bias and norm weight (exact
        for bf16 parameters), rebuilt when a parameter changes."""
        params = (self.conv1d.weight, self.A_log, self.dt_bias, self.norm.weight)
        key = tuple((p.data_ptr(), p._version, p.device) for p in params)
        if self._packed_key != key:
            self._packed = (
                self.conv1d.weight.detach().float().reshape(self.conv_dim, CONV_KERNEL).contiguous(),
                self.A_log.detach().float().contiguous(),
                self.dt_bias.detach().float().contiguous(),
                self.norm.weight.detach().float().contiguous())
            self._packed_key = key
        return self._packed

    def forward(self, hidden_states: torch.Tensor, cache_pool, forward_batch) -> torch.Tensor:
        qkv = self.in_proj_qkv(hidden_states)
        z = self.in_proj_z(hidden_states)
        b = self.in_proj_b(hidden_states)
        a = self.in_proj_a(hidden_states)
        conv_state, ssm_state = cache_pool.get_linear_states(self.layer_idx)
        conv_w, a_log, dt_bias, norm_w = self._kernel_params()
        if all(e == 1 for e in forward_batch.extend_lens):     # :316-326
            attn = gdn_decode_step(qkv, b, a, z, conv_w, a_log, dt_bias, norm_w, self.eps,
                                   conv_state, ssm_state, forward_batch.req_pool_indices,
                                   self.num_k_heads, self.num_v_heads)
        else:                                                    # :328-364
            attn = gdn_extend_step(qkv, b, a, z, conv_w, a_log, dt_bias, norm_w, self.eps,
                                   conv_state, ssm_state, forward_batch.req_pool_indices,
                                   forward_batch.extend_lens, self.num_k_heads,
                                   self.num_v_heads)
        return self.out_proj(attn)
