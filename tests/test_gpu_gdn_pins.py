"""Closed forms and a cross-kernel identity of the Gated DeltaNet steps on the
HIP path (the oracle's own pins, tests/test_gdn_oracle.py, taken end to end).

* A unit key with alpha = beta = 1 writes v into that key's row of the state
  and leaves every other row bit for bit; with a one-hot query the pre-norm
  output is bf16 of that row times dk^-0.5, exactly.  Inputs: conv weights
  with only the last tap (the conv output is the input), one-hot q / k
  channels (SiLU(0) = 0, so the normalised q / k are unit vectors),
  A_log = -inf (decay 0: alpha = 1) and b = 20 (sigmoid rounds to 1 in fp32).
* b = -inf (beta = 0) only decays the state: every row is alpha * S0.
* T tokens through the extend path (32-token chunks on MFMAs) equal T decode
  steps (the recurrence kernel), state and outputs.
"""
import pytest
import torch
import torch.nn.functional as F

from oracle import gdn as og
from tests.test_gpu_gdn import check_chunked_outputs, close_fraction, make_params, make_step
from tokenfactory_amd.linear_attention import gdn_decode_step, gdn_extend_step

pytestmark = pytest.mark.gpu


def unit_case(gpu, bsz, hk, hv, b_value, seed):
    conv_dim = 2 * hk * 128 + hv * 128
    g = torch.Generator().manual_seed(seed)
    conv_w = torch.zeros((conv_dim, 4))
    conv_w[:, 3] = 1.0
    a_log = torch.full((hv,), float("-inf"))
    dt_bias = torch.rand((hv,), generator=g)
    norm_w = torch.ones(hv * 128)
    qkv = torch.zeros((bsz, conv_dim))
    hot_q = torch.randint(0, 128, (bsz, hk), generator=g)
    hot_k = torch.randint(0, 128, (bsz, hk), generator=g)
    for bi in range(bsz):
        for kh in range(hk):
            qkv[bi, kh * 128 + hot_q[bi, kh]] = 3.0
            qkv[bi, hk * 128 + kh * 128 + hot_k[bi, kh]] = 1.5
    qkv[:, 2 * hk * 128:] = torch.randn((bsz, hv * 128), generator=g)
    qkv = qkv.to(torch.bfloat16)
    a = torch.randn((bsz, hv), generator=g).to(torch.bfloat16)
    b = torch.full((bsz, hv), b_value).to(torch.bfloat16)
    z = torch.randn((bsz, hv * 128), generator=g).to(torch.bfloat16)
    cs = torch.randn((bsz + 2, conv_dim, 3), generator=g).to(torch.bfloat16).to(gpu)
    ss = (torch.randn((bsz + 2, hv, 128, 128), generator=g) * 0.5).to(gpu)
    req = torch.randperm(bsz + 2, generator=g)[:bsz].to(gpu)
    params = [p.to(gpu) for p in (conv_w, a_log, dt_bias, norm_w)]
    return qkv, a, b, z, params, cs, ss, req, hot_q, hot_k


def test_unit_key_writes_value_row(gpu):
    bsz, hk, hv = 3, 2, 6
    qkv, a, b, z, params, cs, ss, req, hot_q, hot_k = unit_case(gpu, bsz, hk, hv, 20.0, 41)
    s0 = ss.clone()
    out, core = gdn_decode_step(qkv.to(gpu), b.to(gpu), a.to(gpu), z.to(gpu), *params, 1e-6,
                                cs, ss, req, hk, hv, return_core=True)
    torch.cuda.synchronize()
    vpk = hv // hk
    v_all = F.silu(qkv[:, 2 * hk * 128:].float()).to(torch.bfloat16).float().view(bsz, hv, 128)
    for bi in range(bsz):
        r = int(req[bi])
        for h in range(hv):
            i, j = int(hot_k[bi, h // vpk]), int(hot_q[bi, h // vpk])
            s_new, s_old = ss[r, h].cpu(), s0[r, h].cpu()
            rows = torch.ones(128, dtype=torch.bool)
            rows[i] = False
            assert torch.equal(s_new[rows], s_old[rows]), f"b={bi} h={h}: rows besides {i} moved"
            # s + (v - s) in fp32 is v to within an ulp of s and v; v = bf16(silu(x))
            assert torch.allclose(s_new[i], v_all[bi, h], rtol=2 ** -8, atol=1e-6), \
                f"b={bi} h={h}: row {i} is not v"
            want = (s_new[j] * og.DK ** -0.5).to(torch.bfloat16)
            got = core[bi, h * 128:(h + 1) * 128].cpu()
            assert torch.equal(got, want), f"b={bi} h={h}: o != bf16(S[{j}] dk^-0.5)"


def test_zero_beta_only_decays(gpu):
    bsz, hk, hv = 2, 2, 4
    qkv, a, b, z, params, cs, ss, req, _, _ = unit_case(gpu, bsz, hk, hv, float("-inf"), 43)
    a_log = torch.randn((hv,), generator=torch.Generator().manual_seed(5)) - 1.0
    params[1] = a_log.to(gpu)
    s0 = ss.clone()
    gdn_decode_step(qkv.to(gpu), b.to(gpu), a.to(gpu), z.to(gpu), *params, 1e-6, cs, ss, req,
                    hk, hv)
    torch.cuda.synchronize()
    decay, _ = og.gates(a.float(), b.float(), a_log, params[2].cpu())
    alpha = torch.exp(decay)                              # [B, Hv]
    for bi in range(bsz):
        r = int(req[bi])
        for h in range(hv):
            want = s0[r, h].cpu() * alpha[bi, h]
            got = ss[r, h].cpu()
            # alpha from the oracle's gates (torch on the CPU) may differ from the
            # kernel's by an ulp or two
            assert torch.allclose(got, want, rtol=1e-6, atol=0), f"b={bi} h={h}: not alpha * S0"
            ratio = got[s0[r, h].cpu() != 0] / s0[r, h].cpu()[s0[r, h].cpu() != 0]
            assert float(ratio.max() - ratio.min()) <= 2.5e-7 * float(alpha[bi, h]), \
                f"b={bi} h={h}: rows decayed by different factors"


@pytest.mark.parametrize("t,hk,hv", [(37, 2, 6), (64, 4, 4), (5, 1, 2)])
def test_extend_equals_decode_steps(gpu, t, hk, hv):
    print(f"[gdn pins] T={t} Hk={hk} Hv={hv}", flush=True)
    bsz = 2
    conv_dim = 2 * hk * 128 + hv * 128
    g = torch.Generator().manual_seed(t + hk)
    cs0 = torch.randn((bsz + 1, conv_dim, 3), generator=g).to(torch.bfloat16).to(gpu)
    ss0 = (torch.randn((bsz + 1, hv, 128, 128), generator=g) * 0.2).to(gpu)
    req = torch.tensor([2, 0], device=gpu)
    gp = [p.to(gpu) for p in make_params(hk, hv, t)]
    qkv, a, b, z = (x.to(gpu) for x in make_step(bsz * t, hk, hv, 90 + t))
    cs_e, ss_e = cs0.clone(), ss0.clone()
    out_e, core_e = gdn_extend_step(qkv, b, a, z, *gp, 1e-6, cs_e, ss_e, req, [t, t], hk, hv,
                                    return_core=True)
    cs_d, ss_d = cs0.clone(), ss0.clone()
    outs, cores = [], []
    for i in range(t):
        rows = torch.tensor([i, t + i], device=gpu)
        o, c = gdn_decode_step(qkv[rows], b[rows], a[rows], z[rows], *gp, 1e-6, cs_d, ss_d, req,
                               hk, hv, return_core=True)
        outs.append(o)
        cores.append(c)
    torch.cuda.synchronize()
    # step i's row r is token row r * t + i
    out_d = torch.stack(outs, 1).reshape(bsz * t, -1)
    core_d = torch.stack(cores, 1).reshape(bsz * t, -1)
    assert torch.equal(cs_e, cs_d), "conv state"
    scale = float(ss0.abs().max())
    close_fraction(ss_e.cpu(), ss_d.cpu(), 2e-4 * scale, 1e-2 * scale, 1e-3, "ssm state")
    check_chunked_outputs(core_e.cpu(), core_d.cpu(), "pre-norm output", False)
    check_chunked_outputs(out_e.cpu(), out_d.cpu(), "normed output", True)
