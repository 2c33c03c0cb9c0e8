"""Head dims other than 256 (attn_generic.hip and the generic qk_prep kernel).

The reference's own test configurations use head_dim 32
(tests/test_hybrid_radix_cache.py:661-676 of the reference); every entry
point takes any head_dim that is a multiple of 8 up to 256. Checked against
the oracle with the same tolerances as the 256-dim kernels: attention within
2e-2 + 1e-2 |ref| elementwise and 1e-2 relative Frobenius error of the fp32
restatement (fp8 pools against the dequantised pool); the fused gate within
one ulp of silu of the unfused ops; q/k norm + RoPE within one bf16 ulp of the
oracle's bf16 op sequence (summation order) and V rows bit-exact; the module
at the reference's mini configuration against its CPU fp32 composition with
the oracle in place of the kernels.
"""
from types import SimpleNamespace

import pytest
import torch
import torch.nn.functional as F

from oracle.kv_quant import quantize_e4m3
from oracle.qk_prep import inv_freq_ref, qk_prep_ref
from oracle.slot_attention import slot_based_attention_ref
from tests.helpers import assert_attn_close, assert_empty_context_rows, restatement, small_case
from tests.test_gpu_gate import assert_bits_match, module_gate
from tokenfactory_amd import qk_norm_rope_kv_write, slot_based_attention, workloads
from tokenfactory_amd.forward_batch import ForwardBatch
from tokenfactory_amd.full_attention import FullAttention

pytestmark = pytest.mark.gpu

DIMS = [32, 64, 80, 128]


def run(wl, **kw):
    return slot_based_attention(wl.q, wl.k_pool, wl.v_pool, wl.batch, scaling=wl.scale,
                                k_scale=wl.k_scale, v_scale=wl.v_scale, **kw)


def check(wl, what):
    print(f"[head dims] {what} D={wl.head_dim} B={wl.batch.batch_size} ext={wl.ext_lens[:6]} "
          f"L={wl.seq_lens[:6]} Hq={wl.num_q_heads} Hkv={wl.num_kv_heads}", flush=True)
    out = run(wl)
    torch.cuda.synchronize()
    return assert_attn_close(out, restatement(wl), what=f"{what} D={wl.head_dim}")


@pytest.mark.parametrize("d", DIMS)
def test_decode(gpu, d):
    wl = small_case([1, 5, 64, 65, 300, 1000], [1] * 6, hq=8, hkv=2, d=d, seed=d, device=gpu,
                    dtype=torch.bfloat16)
    check(wl, "decode")


@pytest.mark.parametrize("d", DIMS)
def test_decode_empty_context_rows_are_zero(gpu, d):
    """seq_len 0: a row of zeros, as at head_dim 256 and in the reference."""
    wl = small_case([7, 300, 64], [1] * 3, hq=8, hkv=2, d=d, seed=d + 7, device=gpu,
                    dtype=torch.bfloat16)
    wl.batch.seq_lens[0] = 0
    print(f"[head dims] empty context D={d}", flush=True)
    out = run(wl)
    torch.cuda.synchronize()
    assert_empty_context_rows(out, restatement(wl), [0], what=f"seq_len 0 D={d}")


@pytest.mark.parametrize("d", DIMS)
def test_extend_and_mixed(gpu, d):
    check(small_case([70], [70], hq=4, hkv=1, d=d, seed=d + 1, device=gpu,
                     dtype=torch.bfloat16), "prefill")
    check(small_case([333 + 40], [40], hq=6, hkv=3, d=d, seed=d + 2, device=gpu,
                     dtype=torch.bfloat16), "extend over a prefix")
    check(small_case([50, 400, 7, 900, 64], [50, 1, 3, 1, 20], hq=8, hkv=2, d=d, seed=d + 3,
                     device=gpu, dtype=torch.bfloat16), "mixed")


@pytest.mark.parametrize("d", [32, 128])
def test_fp8_pool_and_bsz1_negative_entries(gpu, d):
    wl = workloads.build("fp8", [40, 300, 9], [40, 100, 1], num_q_heads=8, num_kv_heads=2,
                         head_dim=d, pool_slots=512, device=gpu, seed=d, kv_fp8=True)
    check(wl, "fp8 mixed")
    for fp8 in (False, True):
        wl = workloads.build("neg", [200], [60], num_q_heads=4, num_kv_heads=1, head_dim=d,
                             pool_slots=512, device=gpu, seed=d + 7, kv_fp8=fp8)
        wl.batch.req_to_token[wl.rows[0], [0, 90, 150]] = -1
        check(wl, "-1 entries, bsz=1" + (", fp8" if fp8 else ""))


@pytest.mark.parametrize("d", [32, 80])
def test_fused_gate(gpu, d):
    wl = small_case([50, 400, 7], [50, 1, 3], hq=8, hkv=2, d=d, seed=d + 5, device=gpu,
                    dtype=torch.bfloat16)
    gate = module_gate(wl, d)
    plain = run(wl)
    fused = run(wl, gate=gate)
    torch.cuda.synchronize()
    assert_bits_match(fused, plain * F.silu(gate), f"gate D={d}")


def test_rejects_head_dims_that_are_not_multiples_of_8(gpu):
    wl = small_case([10], [1], hq=4, hkv=1, d=36, seed=1, device=gpu, dtype=torch.bfloat16)
    with pytest.raises(NotImplementedError):
        run(wl)


def _bf16_ulp_diff(a, b):
    ia = a.contiguous().view(torch.int16).to(torch.int32)
    ib = b.contiguous().view(torch.int16).to(torch.int32)
    ia = torch.where(ia < 0, -32768 - ia, ia)
    ib = torch.where(ib < 0, -32768 - ib, ib)
    return (ia - ib).abs()


@pytest.mark.parametrize("d,rd,mrope", [(32, 8, True), (32, 32, False), (64, 16, True),
                                        (128, 32, False), (80, 40, True)])
def test_qk_prep(gpu, d, rd, mrope):
    print(f"[head dims] qk_prep D={d} rotary_dim={rd} mrope={mrope}", flush=True)
    T, hq, hkv, pool = 45, 4, 1, 128
    g = torch.Generator().manual_seed(d + rd)
    qg = (torch.randn(T, hq, 2 * d, generator=g) * 2).to(torch.bfloat16).to(gpu)
    q = qg[:, :, :d]
    k = (torch.randn(T, hkv, d, generator=g) * 2).to(torch.bfloat16).to(gpu)
    v = torch.randn(T, hkv, d, generator=g).to(torch.bfloat16).to(gpu)
    qw = (1 + 0.3 * torch.randn(d, generator=g)).to(gpu)
    kw = (1 + 0.3 * torch.randn(d, generator=g)).to(gpu)
    pos = torch.randint(0, 100000, (T,), generator=g)
    if mrope:
        pos = torch.stack([pos, pos + torch.randint(0, 50, (T,), generator=g), pos // 3])
    sec = [11, 11, 10]            # the 27B config's sections, as the mini config keeps them
    loc = (torch.randperm(pool - 1, generator=g)[:T] + 1).to(gpu)
    invf = inv_freq_ref(rd, 1e7)
    for kv_dtype in (torch.bfloat16, torch.float8_e4m3fn):
        kp = torch.zeros(pool, hkv, d, device=gpu).to(kv_dtype)
        vp = torch.zeros_like(kp)
        scales = (torch.tensor([0.02], device=gpu), torch.tensor([0.01], device=gpu)) \
            if kv_dtype == torch.float8_e4m3fn else (None, None)
        qo = qk_norm_rope_kv_write(q, k, v, qw, kw, 1e-6, pos.to(gpu), invf, rd, sec, True,
                                   kp, vp, loc, *scales)
        torch.cuda.synchronize()
        qb, kb = qk_prep_ref(q.cpu(), k.cpu(), qw.cpu(), kw.cpu(), 1e-6, pos, invf, rd, sec,
                             True)
        if kv_dtype == torch.bfloat16:
            for got, ref in ((qo.cpu(), qb), (kp[loc].cpu(), kb)):
                ulp = _bf16_ulp_diff(got, ref)
                assert ulp.max().item() <= 1 and (ulp > 0).float().mean().item() < 0.02, \
                    f"D={d}: {int((ulp > 0).sum())} elements off, max {ulp.max().item()} ulp"
            assert torch.equal(vp[loc], v)
        else:
            assert torch.equal(vp[loc].view(torch.uint8),
                               quantize_e4m3(v.float(), 0.01).view(torch.uint8))
            ref = quantize_e4m3(kb.float(), 0.02)
            got = kp[loc].cpu()
            assert (got.view(torch.uint8) != ref.view(torch.uint8)).float().mean().item() < 0.01


def _mini_config():
    """The reference's mini test configuration (tests/test_hybrid_radix_cache.py:661-676:
    hidden 128, 4 q / 1 kv heads of 32) with the 27B model's rotary settings."""
    return SimpleNamespace(hidden_size=128, num_attention_heads=4, num_key_value_heads=1,
                           head_dim=32, tp_size=1, attn_output_gate=True, attention_bias=False,
                           rms_norm_eps=1e-6, partial_rotary_factor=0.25, rope_theta=1e7,
                           mrope_section=[11, 11, 10], mrope_interleaved=True)


class _Pool:
    def __init__(self, k, v):
        self.k, self.v = k, v

    def get_full_kv_buffers(self, layer_idx):
        return self.k, self.v


def test_module_at_the_reference_mini_config(gpu):
    """FullAttention.forward (bf16 projections, the kernels) against the same
    module in fp32 on the CPU with the oracle's KV write and attention, on a
    mixed batch with 3-row M-RoPE positions."""
    cfg = _mini_config()
    torch.manual_seed(5)
    ref_mod = FullAttention(cfg, layer_idx=3, dtype=torch.float32)
    with torch.no_grad():
        for lin in (ref_mod.q_proj, ref_mod.k_proj, ref_mod.v_proj, ref_mod.o_proj):
            lin.weight.copy_((torch.randn_like(lin.weight) * lin.in_features ** -0.5)
                             .to(torch.bfloat16).float())
        ref_mod.q_norm.weight.copy_((1 + 0.3 * torch.randn(32)).to(torch.bfloat16).float())
        ref_mod.k_norm.weight.copy_((1 + 0.3 * torch.randn(32)).to(torch.bfloat16).float())
    mod = FullAttention(cfg, layer_idx=3, dtype=torch.bfloat16).to(gpu)
    with torch.no_grad():
        for name in ("q_proj", "k_proj", "v_proj", "o_proj"):
            getattr(mod, name).weight.copy_(getattr(ref_mod, name).weight)
        mod.q_norm.weight.copy_(ref_mod.q_norm.weight)
        mod.k_norm.weight.copy_(ref_mod.k_norm.weight)

    S, ctx = 256, 80
    seq, ext = [30, 50, 12], [30, 1, 4]
    T = sum(ext)
    rtt = torch.full((4, ctx), -1, dtype=torch.long)
    perm = torch.randperm(S - 1)[:sum(seq)] + 1
    o = 0
    for r, L in enumerate(seq):
        rtt[r, :L] = perm[o:o + L]
        o += L
    loc = torch.cat([rtt[r, L - e:L] for r, (L, e) in enumerate(zip(seq, ext))])
    k0 = torch.randn(S, 1, 32).to(torch.bfloat16)
    v0 = torch.randn(S, 1, 32).to(torch.bfloat16)
    hidden = torch.randn(T, 128).to(torch.bfloat16)
    base = torch.cat([torch.arange(L - e, L) for L, e in zip(seq, ext)])
    pos = torch.stack([base, base + 3, base // 2])

    def fb(device):
        return ForwardBatch(batch_size=3, req_pool_indices=torch.arange(3, device=device),
                            seq_lens=torch.tensor(seq, device=device),
                            prefix_lens=torch.tensor([L - e for L, e in zip(seq, ext)],
                                                     device=device),
                            extend_lens=list(ext), out_cache_loc=loc.to(device),
                            req_to_token=rtt.to(device), is_prefill=True)

    pool = _Pool(k0.clone().to(gpu), v0.clone().to(gpu))
    with torch.no_grad():
        out = mod(hidden.to(gpu), pos.to(gpu), pool, fb(gpu))
    torch.cuda.synchronize()

    # CPU fp32: the module's host pieces, then the oracle's write and attention.
    x = hidden.float()
    with torch.no_grad():
        q, gate = ref_mod.q_proj(x).view(T, 4, 64).chunk(2, dim=-1)
        k = ref_mod.k_proj(x).view(T, 1, 32)
        v = ref_mod.v_proj(x).view(T, 1, 32)
        q, k = ref_mod.rotary_emb(ref_mod.q_norm(q), ref_mod.k_norm(k), pos)
        kp, vp = k0.float(), v0.float()
        kp[loc], vp[loc] = k, v
        attn = slot_based_attention_ref(q, kp, vp, fb("cpu"), 4, ref_mod.scaling)
        want = ref_mod.o_proj(attn.reshape(T, -1) * F.silu(gate.reshape(T, -1)))
    assert_attn_close(pool.k[loc], k, atol=4e-2, rtol=2e-2, norm_rel=1e-2, what="mini k_written")
    err = assert_attn_close(out, want, atol=4e-2, rtol=2e-2, norm_rel=1e-2, what="mini out")
    print(f"[head dims] mini module out: max abs {err[0]:.2e}, rel-norm {err[1]:.2e}", flush=True)
