"""Gated DeltaNet (the linear-attention layers) on the CPU.

TEST INFRASTRUCTURE ONLY.

Restates, op for op, ``qwen3_8/linear_attention.py`` and
``qwen3_8/rms_norm_gated.py``:

* ``causal_conv_decode`` -- the conv part of ``_batched_decode_step``
  (``:258-269``): ``padded = cat(conv_state, qkv)``, depthwise conv over the 4
  taps, SiLU, state <- last 3 inputs. The reference runs ``F.conv1d`` on bf16
  tensors; GPU backends accumulate in fp32 and round once to bf16, which is
  what is restated here (then ``F.silu`` on the bf16 tensor, rounded again).
* ``causal_conv_prefill`` -- ``_causal_conv1d_step`` (``:133-152``) for one
  request's ``ext_len`` tokens, same arithmetic.
* ``delta_rule_decode`` -- the state update and readout of
  ``_batched_decode_step`` (``:278-298``) on already normalised q / k.
* ``gated_delta_rule_chunked`` -- ``_gated_delta_rule_step`` (``:154-242``):
  the chunk-wise WY form (chunk 64, ``solve_triangular``) used for prefill.
* ``rms_norm_gated`` -- ``Qwen3_8RMSNormGated.forward`` with per-head
  variance (``rms_norm_gated.py:26-40``).
* ``gdn_decode`` -- the whole decode step plus the norm, what
  ``tf_gdn_decode`` computes.

Pins (``tests/test_gdn_oracle.py``): T recurrent decode steps equal one chunked
prefill over the same T tokens (two independent formulations; T crosses the
64-token chunk boundary), the delta rule's closed form (alpha = beta = 1 and a
unit key write v into that key's row; beta = 0 only decays), the conv with a
unit last tap reproduces SiLU of the new input and shifts the state, the GVA
map against per-head runs with the key head ``h // (Hv / Hk)``, and the
gated norm's closed form on constant rows.
"""
from __future__ import annotations

import torch
import torch.nn.functional as F

DK = 128
DV = 128


def _bf16(x: torch.Tensor) -> torch.Tensor:
    return x.to(torch.bfloat16)


def conv_taps(padded: torch.Tensor, weight: torch.Tensor) -> torch.Tensor:
    """Depthwise conv of ``padded`` [..., C, 4] (bf16 values) with ``weight``
    [C, 4]: fp32 sum of the four products, rounded once to bf16, then SiLU
    (computed in fp32, rounded to bf16)."""
    y = (padded.float() * weight.float()).sum(-1)
    return F.silu(_bf16(y).float()).to(torch.bfloat16)


def causal_conv_decode(qkv: torch.Tensor, conv_state: torch.Tensor, weight: torch.Tensor):
    """``(out [B, C] bf16, new_state [B, C, 3] bf16)`` (``:258-269``)."""
    padded = torch.cat([conv_state, qkv.unsqueeze(-1)], dim=-1)   # [B, C, 4]
    return conv_taps(padded, weight), padded[:, :, 1:].clone()


def causal_conv_prefill(qkv: torch.Tensor, state: torch.Tensor, weight: torch.Tensor):
    """One request's ``ext_len`` tokens (``:133-152``): ``(out [T, C], new_state [C, 3])``."""
    padded = torch.cat([state, qkv.transpose(0, 1)], dim=-1)        # [C, 3 + T]
    t = qkv.shape[0]
    windows = torch.stack([padded[:, i:i + 4] for i in range(t)], dim=0)  # [T, C, 4]
    return conv_taps(windows, weight), padded[:, -3:].clone()


def normalize_qk(q: torch.Tensor, k: torch.Tensor):
    """``F.normalize(q.float()) * dk^-0.5`` and ``F.normalize(k.float())``
    (``:171-172``), dk = ``q.shape[-1]`` (the layer's ``head_k_dim``)."""
    qn = F.normalize(q.float(), p=2.0, dim=-1) * (q.shape[-1] ** -0.5)
    kn = F.normalize(k.float(), p=2.0, dim=-1)
    return qn, kn


def gates(a: torch.Tensor, b: torch.Tensor, a_log: torch.Tensor, dt_bias: torch.Tensor):
    """``(decay_rate, beta)`` (``:177-181``); ``alpha = exp(decay_rate)``."""
    decay = -torch.exp(a_log.float()) * F.softplus(a.float() + dt_bias.float())
    return decay, torch.sigmoid(b.float())


def delta_rule_decode(qn, kn, v, alpha, beta, state):
    """One step for every head: ``qn``, ``kn`` [H, Dk] (already expanded to the
    value heads), ``v`` [H, Dv], ``alpha``, ``beta`` [H]; ``state`` [H, Dk, Dv]
    fp32 is returned updated (``:291-297``). Returns ``(o [H, Dv], state)``."""
    s = state * alpha[:, None, None]
    v_pred = torch.einsum("hkd,hk->hd", s, kn)
    delta = beta[:, None] * (v.float() - v_pred)
    s = s + torch.einsum("hk,hd->hkd", kn, delta)
    return torch.einsum("hkd,hk->hd", s, qn), s


def gated_delta_rule_chunked(q, k, v, b, a, state, a_log, dt_bias, vpk, chunk_size=64):
    """``_gated_delta_rule_step`` for ``ext_len > 1`` (``:194-242``): q, k
    [T, Hk, Dk], v [T, Hv, Dv] (bf16 conv outputs), a, b [T, Hv]; ``state``
    [Hv, Dk, Dv] fp32 is updated in place. Returns fp32 [T, Hv, Dv]."""
    qn, kn = normalize_qk(q, k)
    q_exp = torch.repeat_interleave(qn, vpk, dim=1)
    k_exp = torch.repeat_interleave(kn, vpk, dim=1)
    v32 = v.float()
    decay_rate, beta = gates(a, b, a_log, dt_bias)
    outs = []
    for start in range(0, q.shape[0], chunk_size):
        end = min(start + chunk_size, q.shape[0])
        c = end - start
        q_h, k_h = q_exp[start:end].transpose(0, 1), k_exp[start:end].transpose(0, 1)
        v_h = v32[start:end].transpose(0, 1)
        g_h, beta_h = decay_rate[start:end].transpose(0, 1), beta[start:end].transpose(0, 1)
        gamma = torch.cumsum(g_h, dim=-1)
        diff = gamma.unsqueeze(-1) - gamma.unsqueeze(-2)
        tril = torch.tril(torch.ones((c, c), dtype=torch.bool))
        stril = torch.tril(torch.ones((c, c), dtype=torch.bool), diagonal=-1)
        gamma_tril = torch.exp(diff.masked_fill(~tril, float("-inf")))
        gamma_stril = gamma_tril.masked_fill(~stril, 0.0)
        kk = k_h @ k_h.transpose(-1, -2)
        lhs = torch.eye(c).unsqueeze(0) + beta_h.unsqueeze(-1) * gamma_stril * kk
        exp_gamma = torch.exp(gamma).unsqueeze(-1)
        rhs = beta_h.unsqueeze(-1) * (v_h - exp_gamma * (k_h @ state))
        u = torch.linalg.solve_triangular(lhs, rhs, upper=False, unitriangular=True)
        out_h = exp_gamma * (q_h @ state) + (gamma_tril * (q_h @ k_h.transpose(-1, -2))) @ u
        outs.append(out_h.transpose(0, 1))
        total = torch.exp(gamma[:, -1]).view(-1, 1, 1)
        to_end = torch.exp(gamma[:, -1:] - gamma).unsqueeze(-1)
        state.mul_(total).add_((k_h * to_end).transpose(-1, -2) @ u)
    return torch.cat(outs, dim=0)


def rms_norm_gated(x: torch.Tensor, gate: torch.Tensor, weight: torch.Tensor, eps: float,
                   head_dim: int = DV) -> torch.Tensor:
    """``Qwen3_8RMSNormGated.forward`` with ``head_dim`` (``rms_norm_gated.py:26-40``)."""
    xf = x.float()
    shape = xf.shape
    xh = xf.view(*shape[:-1], -1, head_dim)
    var = xh.pow(2).mean(dim=-1, keepdim=True)
    xn = (xh * torch.rsqrt(var + eps)).view(shape)
    return (weight.float() * xn * F.silu(gate.float())).to(x.dtype)


def gdn_decode(qkv, a, b, z, conv_weight, a_log, dt_bias, norm_weight, eps, conv_state,
               ssm_state, req_indices, num_k_heads, num_v_heads):
    """The decode step of ``tf_gdn_decode``: ``_batched_decode_step`` (``:244-298``)
    then the gated norm (``:325``). ``conv_state`` [slots, C, 3] bf16 and
    ``ssm_state`` [slots, Hv, Dk, Dv] fp32 are updated in place (CPU tensors); Dk
    and Dv are its last two extents.
    Returns ``(out, core)``: the normed bf16 output and the bf16 pre-norm output."""
    req = req_indices.cpu().long()
    dk, dv = ssm_state.shape[-2], ssm_state.shape[-1]
    key_dim = num_k_heads * dk
    conv_out, new_state = causal_conv_decode(qkv.cpu(), conv_state[req], conv_weight.cpu())
    conv_state[req] = new_state
    bsz = qkv.shape[0]
    q, k, v = conv_out.split([key_dim, key_dim, num_v_heads * dv], dim=-1)
    qn, kn = normalize_qk(q.view(bsz, num_k_heads, dk), k.view(bsz, num_k_heads, dk))
    vpk = num_v_heads // num_k_heads
    q_exp = torch.repeat_interleave(qn, vpk, dim=1)
    k_exp = torch.repeat_interleave(kn, vpk, dim=1)
    decay, beta = gates(a.cpu(), b.cpu(), a_log.cpu(), dt_bias.cpu())
    alpha = torch.exp(decay)
    outs = []
    for i in range(bsz):
        o, s = delta_rule_decode(q_exp[i], k_exp[i], v[i].view(num_v_heads, dv), alpha[i],
                                 beta[i], ssm_state[req[i]])
        ssm_state[req[i]] = s
        outs.append(o)
    core = torch.stack(outs).reshape(bsz, num_v_heads * dv).to(torch.bfloat16)
    out = rms_norm_gated(core, z.cpu(), norm_weight.cpu(), eps, head_dim=dv)
    return out, core


def gdn_extend(qkv, a, b, z, conv_weight, a_log, dt_bias, norm_weight, eps, conv_state,
               ssm_state, req_indices, extend_lens, num_k_heads, num_v_heads):
    """The reference's per-request loop for a batch with any extend lengths
    (``linear_attention.py:328-364``): ``_causal_conv1d_step`` and
    ``_gated_delta_rule_step`` (chunked WY for ``ext_len > 1``, the one-step
    formula for ``ext_len == 1``) per request, then the gated norm over all rows.
    States are updated in place (CPU tensors); head dims from ``ssm_state``'s
    last two extents. Returns ``(out, core)``."""
    dk, dv = ssm_state.shape[-2], ssm_state.shape[-1]
    key_dim = num_k_heads * dk
    vpk = num_v_heads // num_k_heads
    outs, off = [], 0
    for i, e in enumerate(extend_lens):
        r = int(req_indices[i])
        rows = slice(off, off + e)
        off += e
        conv_out, new_state = causal_conv_prefill(qkv[rows].cpu(), conv_state[r],
                                                  conv_weight.cpu())
        conv_state[r] = new_state
        q, k, v = conv_out.split([key_dim, key_dim, num_v_heads * dv], dim=-1)
        q = q.view(e, num_k_heads, dk)
        k = k.view(e, num_k_heads, dk)
        v = v.view(e, num_v_heads, dv)
        if e == 1:                           # :184-192
            qn, kn = normalize_qk(q[0], k[0])
            decay, beta = gates(a[rows].cpu()[0], b[rows].cpu()[0], a_log.cpu(), dt_bias.cpu())
            o, s = delta_rule_decode(torch.repeat_interleave(qn, vpk, 0),
                                     torch.repeat_interleave(kn, vpk, 0), v[0],
                                     torch.exp(decay), beta, ssm_state[r])
            ssm_state[r] = s
            o = o.unsqueeze(0)
        else:
            o = gated_delta_rule_chunked(q, k, v, b[rows].cpu(), a[rows].cpu(), ssm_state[r],
                                         a_log.cpu(), dt_bias.cpu(), vpk)
        outs.append(o.reshape(e, num_v_heads * dv).to(torch.bfloat16))
    core = torch.cat(outs, dim=0)
    return rms_norm_gated(core, z.cpu(), norm_weight.cpu(), eps, head_dim=dv), core

