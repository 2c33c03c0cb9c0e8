"""Pins of the Gated DeltaNet oracle (CPU only).

Each check fixes the oracle by something other than its own formula: the
chunk-wise WY prefill against the token-by-token recurrence (two independent
formulations of the same state-space update), closed forms of the delta rule,
the conv and the gated norm, and the GVA map against per-head runs.
"""
import math

import pytest
import torch
import torch.nn.functional as F

from oracle import gdn as og


def rand_inputs(t, hk, hv, seed, dk=og.DK, dv=og.DV):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn((t, hk, dk), generator=g).to(torch.bfloat16)
    k = torch.randn((t, hk, dk), generator=g).to(torch.bfloat16)
    v = torch.randn((t, hv, dv), generator=g).to(torch.bfloat16)
    a = torch.randn((t, hv), generator=g).to(torch.bfloat16)
    b = torch.randn((t, hv), generator=g).to(torch.bfloat16)
    a_log = torch.rand((hv,), generator=g) * 2 - 3          # decay rates ~ -exp(-2) * softplus
    dt_bias = torch.rand((hv,), generator=g)
    state = torch.randn((hv, dk, dv), generator=g) * 0.1
    return q, k, v, a, b, a_log, dt_bias, state


@pytest.mark.parametrize("t,chunk,dk,dv", [(5, 64, 128, 128), (64, 64, 128, 128),
                                           (70, 64, 128, 128), (70, 32, 128, 128),
                                           (33, 32, 128, 128),
                                           # the reference's test models: head dims 16
                                           (70, 64, 16, 16), (9, 64, 32, 16)])
def test_chunked_prefill_equals_recurrence(t, chunk, dk, dv):
    # chunk 64: the reference's chunk length; chunk 32: the GPU kernel's
    hk, hv = 2, 6
    q, k, v, a, b, a_log, dt_bias, s0 = rand_inputs(t, hk, hv, t, dk, dv)
    s_chunk = s0.clone()
    out_chunk = og.gated_delta_rule_chunked(q, k, v, b, a, s_chunk, a_log, dt_bias, hv // hk,
                                            chunk_size=chunk)
    s = s0.clone()
    outs = []
    for i in range(t):
        qn, kn = og.normalize_qk(q[i], k[i])
        decay, beta = og.gates(a[i], b[i], a_log, dt_bias)
        o, s = og.delta_rule_decode(torch.repeat_interleave(qn, 3, 0),
                                    torch.repeat_interleave(kn, 3, 0), v[i], torch.exp(decay),
                                    beta, s)
        outs.append(o)
    out_rec = torch.stack(outs)
    scale = float(out_rec.abs().max())
    assert torch.allclose(out_chunk, out_rec, atol=1e-4 * scale, rtol=1e-4)
    assert torch.allclose(s_chunk, s, atol=1e-4 * float(s.abs().max()), rtol=1e-4)


@pytest.mark.parametrize("dk", [16, 128])
def test_normalize_qk_closed_form(dk):
    # q is scaled by head_k_dim^-0.5 of the layer (16 in the reference's test models)
    q = torch.zeros((3, dk))
    q[0, 1] = 5.0
    q[1, dk - 1] = -0.25
    q[2] = 2.0                                   # equal entries: the unit vector dk^-0.5 * 1
    qn, kn = og.normalize_qk(q, q.clone())
    assert float(kn[0, 1]) == 1.0 and float(qn[0, 1]) == pytest.approx(dk ** -0.5, rel=1e-6)
    assert float(qn[1, dk - 1]) == pytest.approx(-(dk ** -0.5), rel=1e-6)
    assert torch.allclose(kn[2], torch.full((dk,), dk ** -0.5))
    assert torch.allclose(qn[2], torch.full((dk,), 1.0 / dk))


def test_delta_rule_closed_forms():
    hv = 3
    g = torch.Generator().manual_seed(1)
    s0 = torch.randn((hv, og.DK, og.DV), generator=g)
    v = torch.randn((hv, og.DV), generator=g)
    kn = torch.zeros((hv, og.DK))
    qn = torch.zeros((hv, og.DK))
    for h, (i, j) in enumerate([(0, 5), (17, 17), (127, 64)]):
        kn[h, i] = 1.0
        qn[h, j] = og.DK ** -0.5
    ones = torch.ones(hv)
    o, s = og.delta_rule_decode(qn, kn, v, ones, ones, s0.clone())
    for h, (i, j) in enumerate([(0, 5), (17, 17), (127, 64)]):
        want = s0[h].clone()
        want[i] = v[h]                       # the key's row now holds v (s + (v - s) in fp32)
        assert torch.allclose(s[h], want, atol=1e-6, rtol=1e-6)
        assert torch.allclose(o[h], want[j] * og.DK ** -0.5)
    # beta = 0: nothing is written, the state only decays
    alpha = torch.tensor([0.5, 0.25, 1.0])
    _, s = og.delta_rule_decode(qn, kn, v, alpha, torch.zeros(hv), s0.clone())
    assert torch.allclose(s, s0 * alpha[:, None, None])


def test_gates_special_values():
    # A_log = -inf: decay 0 (alpha 1); large a: softplus(x) = x past the threshold
    decay, beta = og.gates(torch.tensor([0.0, 30.0]), torch.tensor([0.0, 40.0]),
                           torch.tensor([float("-inf"), 0.0]), torch.tensor([0.0, 0.0]))
    assert decay[0] == 0 and float(decay[1]) == -30.0
    assert float(beta[0]) == 0.5 and float(beta[1]) == 1.0


def test_conv_unit_tap_and_state_shift():
    c = 16
    g = torch.Generator().manual_seed(2)
    qkv = torch.randn((3, c), generator=g).to(torch.bfloat16)
    st = torch.randn((3, c, 3), generator=g).to(torch.bfloat16)
    w = torch.zeros((c, 4))
    w[:, 3] = 1.0
    out, new = og.causal_conv_decode(qkv, st, w)
    assert torch.equal(out, F.silu(qkv.float()).to(torch.bfloat16))
    assert torch.equal(new[:, :, :2], st[:, :, 1:]) and torch.equal(new[:, :, 2], qkv)
    # first tap only: the oldest state entry
    w = torch.zeros((c, 4))
    w[:, 0] = 1.0
    out, _ = og.causal_conv_decode(qkv, st, w)
    assert torch.equal(out, F.silu(st[:, :, 0].float()).to(torch.bfloat16))


def test_conv_prefill_matches_decode_steps():
    c, t = 24, 7
    g = torch.Generator().manual_seed(3)
    qkv = torch.randn((t, c), generator=g).to(torch.bfloat16)
    st = torch.randn((c, 3), generator=g).to(torch.bfloat16)
    w = torch.randn((c, 4), generator=g).to(torch.bfloat16).float()
    out_p, new_p = og.causal_conv_prefill(qkv, st, w)
    s = st.unsqueeze(0)
    for i in range(t):
        o, s = og.causal_conv_decode(qkv[i:i + 1], s, w)
        assert torch.equal(o[0], out_p[i])
    assert torch.equal(s[0], new_p)


def test_gva_map_matches_per_head_runs():
    hk, hv, t = 2, 6, 9
    q, k, v, a, b, a_log, dt_bias, s0 = rand_inputs(t, hk, hv, 5)
    s_all = s0.clone()
    out_all = og.gated_delta_rule_chunked(q, k, v, b, a, s_all, a_log, dt_bias, hv // hk)
    for h in range(hv):
        kh = h // (hv // hk)                 # repeat_interleave: key head h // 3
        s_h = s0[h:h + 1].clone()
        out_h = og.gated_delta_rule_chunked(q[:, kh:kh + 1], k[:, kh:kh + 1], v[:, h:h + 1],
                                            b[:, h:h + 1], a[:, h:h + 1], s_h,
                                            a_log[h:h + 1], dt_bias[h:h + 1], 1)
        assert torch.allclose(out_h[:, 0], out_all[:, h], atol=1e-5, rtol=1e-5)
        assert torch.allclose(s_h[0], s_all[h], atol=1e-5, rtol=1e-5)


def test_rms_norm_gated_closed_form():
    x = torch.full((2, 256), 3.0)
    x[:, 128:] = -0.5
    z = torch.tensor([0.0, 2.0]).repeat_interleave(128).repeat(2, 1)
    w = torch.full((256,), 2.0)
    y = og.rms_norm_gated(x, z, w, eps=0.0)
    # per head x / rms(x) = sign(x); silu(0) = 0, silu(2) = 2 sigmoid(2)
    assert torch.all(y[:, :128] == 0)
    want = 2.0 * -1.0 * (2.0 / (1.0 + math.exp(-2.0)))
    assert torch.allclose(y[:, 128:], torch.full((2, 128), want), rtol=1e-6)
