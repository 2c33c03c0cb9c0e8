"""Output gate fused into the attention kernels' output write.

The module applies ``attn_output * F.silu(gate)`` on bf16 tensors after the
attention call (``full_attention.py:157-159``). With a gate the kernels round
the attention output to bf16, ``silu(gate)`` (fp32, ``x / (1 + exp(-x))``) to
bf16 and the product to bf16, which is that op sequence; the reference here is
those two PyTorch ops applied to the same kernels' ungated output. The
kernels evaluate silu with the hardware exp2 and reciprocal (about 1 ulp of
fp32 each), so bf16(silu) may differ from the exactly rounded one by one bf16
ulp when it sits at a rounding boundary; through the rounded product that is
at most 3 * 2^-8 relative. Allowed on at most 1e-3 of the elements; everything
else must be bit-identical.
"""
import pytest
import torch
import torch.nn.functional as F

from tests.helpers import small_case
from tokenfactory_amd import slot_based_attention, workloads

pytestmark = pytest.mark.gpu


def module_gate(wl, seed, scale=3.0):
    """A gate in the module's layout: the second half of each head's 2D-wide
    slice of the q projection, passed as a strided view."""
    T, H, D = wl.q.shape
    g = torch.Generator(device=wl.q.device).manual_seed(seed)
    qg = (torch.randn((T, H, 2 * D), generator=g, device=wl.q.device) * scale).to(torch.bfloat16)
    return qg[..., D:]


def attend(wl, gate=None, **kw):
    return slot_based_attention(wl.q, wl.k_pool, wl.v_pool, wl.batch, scaling=wl.scale,
                                k_scale=wl.k_scale, v_scale=wl.v_scale, gate=gate, **kw)


def assert_bits_match(got, want, what):
    got, want = got.contiguous(), want.contiguous()
    assert got.shape == want.shape and got.dtype == want.dtype == torch.bfloat16
    nan_g, nan_w = torch.isnan(got), torch.isnan(want)
    assert torch.equal(nan_g, nan_w), f"{what}: NaN positions differ"
    ok = ~nan_g
    same = got.view(torch.int16)[ok] == want.view(torch.int16)[ok]
    g, w = got[ok].float(), want[ok].float()
    n, n_off = same.numel(), int((~same).sum())
    # one bf16 ulp of silu (at most 2^-7 relative) plus the two roundings of
    # the product (2^-9 each): at most 3 * 2^-8 relative
    rel = ((g - w).abs() / w.abs().clamp_min(1e-30))[~same]
    assert n_off == 0 or float(rel.max()) <= 3 * 2.0 ** -8, \
        f"{what}: relative difference {float(rel.max()):.3e} above one ulp of silu"
    assert n_off <= max(1, n // 1000), f"{what}: {n_off} of {n} elements differ"
    print(f"[gate] {what}: {n_off} of {n} elements differ (within one ulp of silu), "
          f"the rest bit-identical", flush=True)


def check(wl, seed, what, **kw):
    print(f"[gate] {what} B={wl.batch.batch_size} ext={wl.ext_lens[:6]} L={wl.seq_lens[:6]}",
          flush=True)
    gate = module_gate(wl, seed)
    plain = attend(wl, **kw)
    fused = attend(wl, gate=gate, **kw)
    want = plain * F.silu(gate)
    torch.cuda.synchronize()
    assert_bits_match(fused, want, what)


@pytest.mark.parametrize("workgroups", [0, 1])
def test_gate_decode(gpu, workgroups):
    # workgroups=0: long contexts split over many workgroups (merge kernel
    # writes); workgroups=1: every unit is finished by its only owner.
    wl = small_case([300, 2000, 47, 1200, 9], [1] * 5, hq=24, hkv=4, d=256, seed=5,
                    device=gpu, dtype=torch.bfloat16)
    check(wl, 1, f"decode wg={workgroups}", decode_workgroups=workgroups)


def test_gate_extend(gpu):
    wl = small_case([300, 700, 64], [100, 300, 64], hq=24, hkv=4, d=256, seed=6, device=gpu,
                    dtype=torch.bfloat16)
    check(wl, 2, "extend")


def test_gate_mixed(gpu):
    wl = workloads.mixed(device=gpu, n_extend=2, extend_new=130, prefix_hi=500, n_decode=7,
                         dec_lo=1, dec_hi=1500, pool_slots=1 << 14)
    check(wl, 3, "mixed")


def test_gate_fp8_pool(gpu):
    wl = workloads.build("fp8g", [40, 300, 900], [40, 100, 1], num_q_heads=24, num_kv_heads=4,
                         head_dim=256, pool_slots=2048, device=gpu, seed=43, kv_fp8=True)
    check(wl, 4, "fp8 extend + decode")


def test_gate_special_values(gpu):
    # silu(+inf) = inf, silu(-inf) = -inf / inf = NaN, NaN stays NaN; large
    # magnitudes saturate to x and 0.
    wl = small_case([200, 150], [60, 1], hq=24, hkv=4, d=256, seed=7, device=gpu,
                    dtype=torch.bfloat16)
    gate = module_gate(wl, 5, scale=30.0)
    gate[0, 0, :4] = torch.tensor([float("inf"), float("-inf"), float("nan"), 0.0])
    gate[60, 3, 10:12] = torch.tensor([-1e30, 1e30])
    plain = attend(wl)
    fused = attend(wl, gate=gate)
    torch.cuda.synchronize()
    assert_bits_match(fused, plain * F.silu(gate), "special values")


def test_gate_layout_checks(gpu):
    wl = small_case([20], [20], hq=24, hkv=4, d=256, seed=8, device=gpu, dtype=torch.bfloat16)
    bad = torch.zeros((20, 24, 256 + 4), dtype=torch.bfloat16, device=gpu)[..., 4:]
    with pytest.raises(ValueError):
        attend(wl, gate=bad)          # 8-byte aligned start
    with pytest.raises(ValueError):
        attend(wl, gate=module_gate(wl, 1).float())
