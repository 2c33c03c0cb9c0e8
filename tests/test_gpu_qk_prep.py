"""Fused q/k RMSNorm + partial (M-)RoPE + KV write (``tf_qk_norm_rope_kv_write``)
against the oracle.

References: the oracle's op-for-op restatement run on the same bf16 inputs on
the CPU (the reference's bf16 rounding steps) and the same restatement in fp32.
* Against the bf16 restatement the kernel is bit-exact up to the summation
  order of the 256 squares of the RMSNorm (one bf16 ulp, rarely) and the last
  fp32 ulp of cos / sin (the GPU's and the CPU's libm), which can round c or s
  to the neighbouring bf16 value once in tens of thousands: every element is
  within |err| <= 1e-2 + 8e-3 |ref|, fewer than 0.5 % differ at all, and dims
  past rotary_dim differ by at most one ulp.
* Against the fp32 restatement (the bf16 pipeline's own rounding): relative
  Frobenius error <= 5e-3 and |err| <= 5e-2 + 1e-2 |ref|.
V rows are copied bit-exactly; rows whose slot is outside the pool are skipped.
"""
import pytest
import torch

from oracle.kv_quant import quantize_e4m3
from oracle.qk_prep import inv_freq_ref, qk_prep_ref
from tokenfactory_amd import qk_norm_rope_kv_write

pytestmark = pytest.mark.gpu


def _bf16_ulp_diff(a: torch.Tensor, b: torch.Tensor) -> torch.Tensor:
    ia = a.contiguous().view(torch.int16).to(torch.int32)
    ib = b.contiguous().view(torch.int16).to(torch.int32)
    # map sign-magnitude bf16 bit patterns onto a monotone integer line
    ia = torch.where(ia < 0, -32768 - ia, ia)
    ib = torch.where(ib < 0, -32768 - ib, ib)
    return (ia - ib).abs()


def _case(gpu, T, hq, hkv, mrope, interleaved=True, seed=0, rd=64, pool=200):
    g = torch.Generator(device="cpu").manual_seed(seed)
    qg = (torch.randn(T, hq, 512, generator=g) * 2).to(torch.bfloat16).to(gpu)
    q = qg[:, :, :256]                               # the q half of a gated projection
    k = (torch.randn(T, hkv, 256, generator=g) * 2).to(torch.bfloat16).to(gpu)
    v = torch.randn(T, hkv, 256, generator=g).to(torch.bfloat16).to(gpu)
    qw = (1 + 0.3 * torch.randn(256, generator=g)).to(gpu)
    kw = (1 + 0.3 * torch.randn(256, generator=g)).to(gpu)
    pos = torch.randint(0, 100000, (T,), generator=g)
    if mrope:
        pos = torch.stack([pos, pos + torch.randint(0, 50, (T,), generator=g), pos // 3])
    loc = torch.randperm(pool - 1, generator=g)[:T] + 1
    return dict(q=q, k=k, v=v, qw=qw, kw=kw, pos=pos.to(gpu), loc=loc.to(gpu), rd=rd,
                sec=[11, 11, 10] if rd == 64 else [rd // 6, rd // 6, rd // 2 - 2 * (rd // 6)],
                inter=interleaved, pool=pool)


def _run(c, gpu, kv_dtype=torch.bfloat16, scales=(None, None)):
    kp = torch.zeros(c["pool"], c["k"].shape[1], 256, device=gpu).to(kv_dtype)
    vp = torch.zeros_like(kp)
    qo = qk_norm_rope_kv_write(c["q"], c["k"], c["v"], c["qw"], c["kw"], 1e-6, c["pos"],
                               inv_freq_ref(c["rd"], 1e7), c["rd"], c["sec"], c["inter"],
                               kp, vp, c["loc"], *scales)
    torch.cuda.synchronize()
    return qo, kp, vp


def _oracle(c, device, dtype):
    q = c["q"].to(device=device, dtype=dtype)
    k = c["k"].to(device=device, dtype=dtype)
    return qk_prep_ref(q, k, c["qw"].to(device), c["kw"].to(device), 1e-6,
                       c["pos"].to(device), inv_freq_ref(c["rd"], 1e7), c["rd"], c["sec"],
                       c["inter"])


def _check_rows(got, bf, f32, rd):
    """got / bf / f32: [..., 256] kernel, bf16 restatement, fp32 restatement (CPU)."""
    got = got.cpu()
    ulp = _bf16_ulp_diff(got[..., rd:], bf[..., rd:])
    assert ulp.max().item() <= 1, f"pass-through dims: {ulp.max().item()} ulp"
    g, r = got.float(), bf.float()
    assert (g != r).float().mean().item() < 5e-3
    err = (g - r).abs()
    assert (err <= 1e-2 + 8e-3 * r.abs()).all(), err.max().item()
    e32 = (g - f32).abs()
    assert (e32.norm() / f32.norm()).item() <= 5e-3
    assert (e32 <= 5e-2 + 1e-2 * f32.abs()).all(), e32.max().item()


@pytest.mark.parametrize("T,hq,hkv,mrope,inter,rd", [
    (1, 24, 4, False, True, 64), (37, 24, 4, False, True, 64), (300, 16, 2, True, True, 64),
    (64, 8, 8, True, False, 64), (19, 6, 1, False, True, 128), (33, 4, 2, True, True, 32)])
def test_qk_prep_matches_oracle(gpu, T, hq, hkv, mrope, inter, rd):
    print(f"[qk_prep] T={T} {hq}/{hkv} mrope={mrope} interleaved={inter} rd={rd}", flush=True)
    c = _case(gpu, T, hq, hkv, mrope, inter, seed=T + hq, rd=rd, pool=max(200, 2 * T))
    qo, kp, vp = _run(c, gpu)
    loc = c["loc"]
    qb, kb = _oracle(c, "cpu", torch.bfloat16)
    qf, kf = _oracle(c, "cpu", torch.float32)
    _check_rows(qo, qb, qf, rd)
    _check_rows(kp[loc], kb, kf, rd)
    assert torch.equal(vp[loc], c["v"])
    untouched = torch.ones(kp.shape[0], dtype=torch.bool, device=gpu)
    untouched[loc] = False
    assert not kp[untouched].any() and not vp[untouched].any()


def test_qk_prep_norm_is_exact_at_position_zero(gpu):
    """cos 1 and sin 0 leave only the RMSNorm: one bf16 ulp at most, rarely."""
    c = _case(gpu, 40, 24, 4, False, seed=1)
    c["pos"] = torch.zeros_like(c["pos"])
    qo, kp, _ = _run(c, gpu)
    qb, kb = _oracle(c, "cpu", torch.bfloat16)
    for got, ref in ((qo.cpu(), qb), (kp[c["loc"]].cpu(), kb)):
        ulp = _bf16_ulp_diff(got, ref)
        assert ulp.max().item() <= 1 and (ulp > 0).float().mean().item() < 0.02


def test_qk_prep_skips_slots_outside_the_pool(gpu):
    c = _case(gpu, 8, 8, 2, False, seed=3, pool=16)
    c["loc"] = torch.tensor([1, -1, 2, 16, 3, 99, 4, 5], device=gpu)
    qo, kp, vp = _run(c, gpu)
    ok = torch.tensor([0, 2, 4, 6, 7], device=gpu)
    assert torch.equal(vp[c["loc"][ok]], c["v"][ok])
    written = torch.zeros(16, dtype=torch.bool, device=gpu)
    written[c["loc"][ok]] = True
    assert not vp[~written].any()


def test_qk_prep_fp8_pool(gpu):
    c = _case(gpu, 50, 24, 4, False, seed=9)
    ks = torch.tensor([0.02], device=gpu)
    vs = torch.tensor([0.01], device=gpu)
    qo, kp, vp = _run(c, gpu, torch.float8_e4m3fn, (ks, vs))
    loc = c["loc"]
    assert torch.equal(vp[loc].view(torch.uint8),
                       quantize_e4m3(c["v"].float(), 0.01).view(torch.uint8))
    # K: e4m3 of rows that match the bf16 restatement as above; almost every
    # code is identical and the dequantised values stay within the e4m3 step.
    _, kb = _oracle(c, "cpu", torch.bfloat16)
    ref = quantize_e4m3(kb.float(), 0.02)
    got = kp[loc].cpu()
    assert (got.view(torch.uint8) != ref.view(torch.uint8)).float().mean().item() < 0.01
    rf, gf = ref.float() * 0.02, got.float() * 0.02
    assert ((gf - rf).abs() <= 2e-2 + 0.07 * rf.abs()).all()
