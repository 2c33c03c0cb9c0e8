"""Gated DeltaNet at head dims other than 128 (gdn_generic_kernel).

The reference's own test models use linear-attention heads of 16
(tests/test_hybrid_radix_cache.py:142-145 of the reference: 2 key and 6 value
heads of 16, hidden 128). Checked against the oracle (``oracle/gdn.py``, whose
head dims follow the state's shape; its dk^-0.5 scale and chunked form are
pinned at dk = 16 in ``tests/test_gdn_oracle.py``) with the bars of the
128-dim tests: conv state bit-exact, slots no request uses untouched, the fp32
SSM state within 1e-5 (decode) or 2e-4 (extend: the kernel's token recurrence
against the oracle's chunked form) of its scale on all but 1e-3 of the
elements, outputs within the bf16 bar.
"""
from types import SimpleNamespace

import pytest
import torch

from oracle import gdn as og
from tests.test_gpu_gdn import check_outputs, close_fraction
from tokenfactory_amd.forward_batch import ForwardBatch
from tokenfactory_amd.linear_attention import LinearAttention, gdn_decode_step, gdn_extend_step

pytestmark = pytest.mark.gpu


def params(hk, hv, dk, dv, seed):
    g = torch.Generator().manual_seed(seed)
    conv_dim = 2 * hk * dk + hv * dv
    conv_w = (torch.randn((conv_dim, 4), generator=g) * 0.5).to(torch.bfloat16).float()
    a_log = (torch.rand((hv,), generator=g) * 2 - 2.5).to(torch.bfloat16).float()
    dt_bias = torch.rand((hv,), generator=g).to(torch.bfloat16).float()
    norm_w = (1 + 0.1 * torch.randn((hv * dv,), generator=g)).to(torch.bfloat16).float()
    return conv_w, a_log, dt_bias, norm_w


def step_inputs(rows, hk, hv, dk, dv, seed):
    g = torch.Generator().manual_seed(seed)
    qkv = torch.randn((rows, 2 * hk * dk + hv * dv), generator=g).to(torch.bfloat16)
    a = torch.randn((rows, hv), generator=g).to(torch.bfloat16)
    b = torch.randn((rows, hv), generator=g).to(torch.bfloat16)
    z = torch.randn((rows, hv * dv), generator=g).to(torch.bfloat16)
    return qkv, a, b, z


def states(n_slots, hk, hv, dk, dv, seed):
    g = torch.Generator().manual_seed(seed)
    cs = torch.randn((n_slots, 2 * hk * dk + hv * dv, 3), generator=g).to(torch.bfloat16)
    ss = torch.randn((n_slots, hv, dk, dv), generator=g) * 0.2
    return cs, ss


@pytest.mark.parametrize("bsz,hk,hv,dk,dv", [(5, 2, 6, 16, 16), (3, 2, 4, 32, 16),
                                              (4, 1, 3, 64, 64), (2, 2, 2, 4, 8)])
def test_decode_steps_match_oracle(gpu, bsz, hk, hv, dk, dv):
    what0 = f"B={bsz} Hk={hk} Hv={hv} dk={dk} dv={dv}"
    print(f"[gdn dims] decode {what0}", flush=True)
    n_slots = bsz + 3
    conv_state, ssm_state = states(n_slots, hk, hv, dk, dv, bsz + dk)
    req = torch.randperm(n_slots, generator=torch.Generator().manual_seed(dv))[:bsz]
    p = params(hk, hv, dk, dv, 7 + dk)
    cs, ss = conv_state.to(gpu), ssm_state.to(gpu)
    gp = [t.to(gpu) for t in p]
    untouched = torch.ones(n_slots, dtype=torch.bool)
    untouched[req] = False
    for step in range(3):
        qkv, a, b, z = step_inputs(bsz, hk, hv, dk, dv, 100 * step + dk)
        out, core = gdn_decode_step(qkv.to(gpu), b.to(gpu), a.to(gpu), z.to(gpu), *gp, 1e-6,
                                    cs, ss, req.to(gpu), hk, hv, return_core=True)
        want_out, want_core = og.gdn_decode(qkv, a, b, z, *p, 1e-6, conv_state, ssm_state, req,
                                            hk, hv)
        torch.cuda.synchronize()
        what = f"{what0} step {step}"
        assert torch.equal(cs.cpu(), conv_state), f"{what}: conv state"
        got = ss.cpu()
        assert torch.equal(got[untouched], ssm_state[untouched]), f"{what}: untouched slots"
        scale = float(ssm_state.abs().max())
        close_fraction(got[~untouched], ssm_state[~untouched], 1e-5 * scale, 1e-2 * scale, 1e-3,
                       f"{what}: ssm state")
        check_outputs(core.cpu(), want_core, f"{what}: pre-norm output")
        check_outputs(out.cpu(), want_out, f"{what}: normed output")


@pytest.mark.parametrize("lens,hk,hv,dk,dv", [([5, 1, 70, 3], 2, 6, 16, 16),
                                               ([40, 1, 2], 2, 4, 64, 32),
                                               ([1, 1, 1], 2, 6, 16, 16)])
def test_extend_matches_oracle(gpu, lens, hk, hv, dk, dv):
    print(f"[gdn dims] extend lens={lens} Hk={hk} Hv={hv} dk={dk} dv={dv}", flush=True)
    n_slots = len(lens) + 3
    conv_state, ssm_state = states(n_slots, hk, hv, dk, dv, sum(lens) + dk)
    req = torch.randperm(n_slots, generator=torch.Generator().manual_seed(dk))[:len(lens)]
    p = params(hk, hv, dk, dv, 3 + dv)
    cs, ss = conv_state.to(gpu), ssm_state.to(gpu)
    gp = [t.to(gpu) for t in p]
    for call, ls in enumerate((lens, [max(1, e // 2) for e in reversed(lens)])):
        qkv, a, b, z = step_inputs(sum(ls), hk, hv, dk, dv, 50 + call)
        out, core = gdn_extend_step(qkv.to(gpu), b.to(gpu), a.to(gpu), z.to(gpu), *gp, 1e-6,
                                    cs, ss, req.to(gpu), ls, hk, hv, return_core=True)
        want_out, want_core = og.gdn_extend(qkv, a, b, z, *p, 1e-6, conv_state, ssm_state, req,
                                            ls, hk, hv)
        torch.cuda.synchronize()
        what = f"lens={ls} dk={dk} dv={dv} call {call}"
        assert torch.equal(cs.cpu(), conv_state), f"{what}: conv state"
        scale = float(ssm_state.abs().max())
        close_fraction(ss.cpu(), ssm_state, 2e-4 * scale, 1e-2 * scale, 1e-3,
                       f"{what}: ssm state")
        check_outputs(core.cpu(), want_core, f"{what}: pre-norm output")
        check_outputs(out.cpu(), want_out, f"{what}: normed output")


def test_out_of_pool_slots_give_zero_rows(gpu):
    hk, hv, dk, dv, n_slots = 2, 6, 16, 16, 5
    conv_state, ssm_state = states(n_slots, hk, hv, dk, dv, 1)
    p = [t.to(gpu) for t in params(hk, hv, dk, dv, 2)]
    req = torch.tensor([-1, n_slots, 2], dtype=torch.int64, device=gpu)
    cs, ss = conv_state.to(gpu), ssm_state.to(gpu)
    qkv, a, b, z = (t.to(gpu) for t in step_inputs(3, hk, hv, dk, dv, 3))
    out, core = gdn_decode_step(qkv, b, a, z, *p, 1e-6, cs, ss, req, hk, hv, return_core=True)
    torch.cuda.synchronize()
    assert torch.equal(out[:2].cpu(), torch.zeros((2, hv * dv), dtype=torch.bfloat16))
    assert torch.equal(core[:2].cpu(), torch.zeros((2, hv * dv), dtype=torch.bfloat16))
    keep = torch.ones(n_slots, dtype=torch.bool)
    keep[2] = False
    assert torch.equal(ss.cpu()[keep], ssm_state[keep])
    lens = [4, 1, 6]
    qkv, a, b, z = (t.to(gpu) for t in step_inputs(sum(lens), hk, hv, dk, dv, 4))
    # NaNs in the memory the caching allocator hands out next, so rows the
    # kernels did not write would not read as zeros by chance
    poison = torch.full((2, sum(lens), hv * dv), float("nan"), dtype=torch.bfloat16, device=gpu)
    del poison
    out, core = gdn_extend_step(qkv, b, a, z, *p, 1e-6, cs, ss, req, lens, hk, hv,
                                return_core=True)
    torch.cuda.synchronize()
    assert torch.equal(out[:5].cpu(), torch.zeros((5, hv * dv), dtype=torch.bfloat16))
    assert torch.equal(core[:5].cpu(), torch.zeros((5, hv * dv), dtype=torch.bfloat16))
    assert torch.isfinite(out[5:].float()).all()


def test_unsupported_head_dims_are_rejected(gpu):
    hk, hv = 2, 2
    for dk, dv in ((18, 16), (16, 66), (128, 64)):
        conv_state, ssm_state = states(3, hk, hv, dk, dv, 5)
        p = [t.to(gpu) for t in params(hk, hv, dk, dv, 6)]
        qkv, a, b, z = (t.to(gpu) for t in step_inputs(2, hk, hv, dk, dv, 7))
        with pytest.raises(NotImplementedError):
            gdn_decode_step(qkv, b, a, z, *p, 1e-6, conv_state.to(gpu), ssm_state.to(gpu),
                            torch.tensor([0, 1], device=gpu), hk, hv)


class _StatePool:
    def __init__(self, cs, ss):
        self.cs, self.ss = cs, ss

    def get_linear_states(self, layer_idx):
        return self.cs, self.ss


def test_module_at_the_reference_test_config(gpu):
    """``LinearAttention`` at the reference's test model (hidden 128, 2 key and
    6 value heads of 16): forward equals its own projections -> the oracle's
    step -> out_proj, on an all-decode batch and then on a mixed batch."""
    cfg = SimpleNamespace(hidden_size=128, linear_num_key_heads=2, linear_num_value_heads=6,
                          linear_key_head_dim=16, linear_value_head_dim=16,
                          linear_conv_kernel_dim=4, rms_norm_eps=1e-6, tp_size=1)
    torch.manual_seed(0)
    mod = LinearAttention(cfg, layer_idx=0).to(gpu)
    with torch.no_grad():
        for prm in mod.parameters():
            prm.copy_((torch.randn_like(prm.float()) * 0.3).to(prm.dtype))
        mod.A_log.fill_(-1.0)
    n_slots = 7
    cs = torch.randn((n_slots, mod.conv_dim, 3)).to(torch.bfloat16)
    ss = torch.randn((n_slots, 6, 16, 16)) * 0.2
    pool = _StatePool(cs.to(gpu), ss.to(gpu))
    req = torch.tensor([5, 0, 3, 6], dtype=torch.int64)
    bsz = req.numel()
    batch = ForwardBatch(batch_size=bsz, req_pool_indices=req.to(gpu),
                         seq_lens=torch.full((bsz,), 10, device=gpu),
                         prefix_lens=torch.full((bsz,), 9, device=gpu), extend_lens=[1] * bsz,
                         out_cache_loc=torch.zeros((bsz,), dtype=torch.int64, device=gpu),
                         req_to_token=torch.zeros((n_slots, 16), dtype=torch.int64, device=gpu),
                         is_prefill=False)
    for lens in ([1] * bsz, [1, 6, 1, 3]):
        batch.extend_lens = lens
        hidden = (torch.randn((sum(lens), 128)) * 0.5).to(torch.bfloat16).to(gpu)
        with torch.no_grad():
            got = mod(hidden, pool, batch)
            qkv, z = mod.in_proj_qkv(hidden), mod.in_proj_z(hidden)
            b, a = mod.in_proj_b(hidden), mod.in_proj_a(hidden)
            conv_w, a_log, dt_bias, norm_w = (t.cpu() for t in mod._kernel_params())
            core_out, _ = og.gdn_extend(qkv.cpu(), a.cpu(), b.cpu(), z.cpu(), conv_w, a_log,
                                        dt_bias, norm_w, 1e-6, cs, ss, req, lens, 2, 6)
            want = mod.out_proj(core_out.to(gpu))
        torch.cuda.synchronize()
        assert torch.allclose(got.float(), want.float(), atol=2e-2, rtol=1e-2), f"lens={lens}"
        assert torch.equal(pool.cs.cpu(), cs), f"lens={lens}: conv state"
        scale = float(ss.abs().max())
        close_fraction(pool.ss.cpu(), ss, 2e-4 * scale, 1e-2 * scale, 1e-3,
                       f"lens={lens}: ssm state")
