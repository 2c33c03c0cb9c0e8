"""``FullAttention.forward`` on the GPU (bf16 projections, gfx950 KV write and
attention kernels) against the reference module's fp32 outputs.

Golden vectors: ``tests/golden/module_golden.npz`` from the reference's own
``Qwen3_8FullAttention`` (mixed batch, pure decode with M-RoPE positions,
bsz == 1 extend). Inputs, weights and the pre-filled pool are bf16 values, so
the only differences are the bf16 rounding of the activations this module
keeps in bf16 (projection outputs, q/k after norm and RoPE, P in the PV
product). Tolerance: |out - ref| <= 4e-2 + 2e-2 |ref| elementwise and a
relative Frobenius error <= 1e-2, for every intermediate and the output
(measured: rel-norm 2-6e-3).
"""
import pytest
import torch

from tests import module_golden as mg
from tests.helpers import assert_attn_close
from tokenfactory_amd import full_attention as fa
from tokenfactory_amd.full_attention import FullAttention

pytestmark = pytest.mark.gpu
TOL = dict(atol=4e-2, rtol=2e-2, norm_rel=1e-2)


class _Pool:
    def __init__(self, d, device):
        self.k = mg.bf16(d["k_pool0"]).to(device=device, dtype=torch.bfloat16)
        self.v = mg.bf16(d["v_pool0"]).to(device=device, dtype=torch.bfloat16)

    def get_full_kv_buffers(self, layer_idx):
        return self.k, self.v


@pytest.mark.parametrize("name", mg.CASES)
def test_full_attention_forward_matches_reference_module(gpu, name, monkeypatch):
    d, meta = mg.load()
    print(f"[module] case={name}", flush=True)
    mod = FullAttention(mg.config(meta), layer_idx=3, dtype=torch.bfloat16).to(gpu)
    mg.load_weights(mod, d)
    pool = _Pool(d, gpu)
    captured = {}
    inner = fa.slot_based_attention

    def spy(q, kb, vb, batch, *, gate=None, **kw):
        # forward fuses the output gate into the attention call; the ungated
        # attention (the reference's intermediate) comes from a second call.
        captured["q"] = q.clone()
        captured["attn"] = inner(q, kb, vb, batch, **kw).clone()
        return inner(q, kb, vb, batch, gate=gate, **kw)

    monkeypatch.setattr(fa, "slot_based_attention", spy)
    hidden = mg.bf16(d[f"{name}_hidden"]).to(device=gpu, dtype=torch.bfloat16)
    pos = torch.from_numpy(d[f"{name}_positions"]).to(gpu)
    with torch.no_grad():
        out = mod(hidden, pos, pool, mg.batch(d, meta, name, gpu))
    torch.cuda.synchronize()
    loc = torch.from_numpy(d[f"{name}_out_cache_loc"]).to(gpu)
    for what, got in (("q", captured["q"]), ("k_written", pool.k[loc]),
                      ("v_written", pool.v[loc]), ("attn", captured["attn"]), ("out", out)):
        err = assert_attn_close(got, mg.expected(d, name, what), what=f"{name} {what}", **TOL)
        print(f"[module] {name} {what}: max abs {err[0]:.2e}, rel-norm {err[1]:.2e}", flush=True)
    # the pool outside the written slots is untouched
    keep = torch.ones(pool.k.shape[0], dtype=torch.bool, device=gpu)
    keep[loc] = False
    ref_k = mg.bf16(d["k_pool0"]).to(device=gpu, dtype=torch.bfloat16)
    assert torch.equal(pool.k[keep], ref_k[keep])


def test_full_attention_fp8_projections(gpu, monkeypatch):
    """FP8 quantization_config: q/k/v/o are block-FP8 linears. Each projection
    is checked against the oracle's block-FP8 linear on the same input (q/k/v on
    the hidden states, o_proj on the gated attention output the module feeds it)."""
    from oracle import fp8_linear as ofl
    from tokenfactory_amd.fp8_linear import Fp8Linear

    d, meta = mg.load()
    cfg = mg.config(meta)
    cfg.quantization_config = {"quant_method": "fp8", "fmt": "e4m3",
                               "activation_scheme": "dynamic", "weight_block_size": [128, 128]}
    mod = FullAttention(cfg, layer_idx=3, dtype=torch.bfloat16).to(gpu)
    for name in ("q_proj", "k_proj", "v_proj", "o_proj"):
        lin = getattr(mod, name)
        assert isinstance(lin, Fp8Linear) and lin.weight.dtype == torch.float8_e4m3fn
        lin.quantize_from(mg.bf16(d[f"w_{name}"]).to(gpu))
    pool = _Pool(d, gpu)
    seen = {}
    inner = fa.slot_based_attention

    def spy(q, kb, vb, batch, *, gate=None, **kw):
        seen["gated"] = inner(q, kb, vb, batch, gate=gate, **kw)
        return seen["gated"]

    monkeypatch.setattr(fa, "slot_based_attention", spy)
    hidden = mg.bf16(d["mixed_hidden"]).to(device=gpu, dtype=torch.bfloat16)
    pos = torch.from_numpy(d["mixed_positions"]).to(gpu)
    print("[module fp8] mixed case", flush=True)
    with torch.no_grad():
        out = mod(hidden, pos, pool, mg.batch(d, meta, "mixed", gpu))
        proj = {n: getattr(mod, n)(hidden) for n in ("q_proj", "k_proj", "v_proj")}
    torch.cuda.synchronize()
    n_tok = hidden.shape[0]
    x_o = seen["gated"].reshape(n_tok, -1)
    for name, x, got in [(n, hidden, proj[n]) for n in proj] + [("o_proj", x_o, out)]:
        lin = getattr(mod, name)
        ref, _, _ = ofl.block_fp8_linear(x.cpu(), lin.weight.cpu(), lin.weight_scale_inv.cpu())
        rms = float(ref.pow(2).mean().sqrt())
        assert torch.allclose(got.cpu().float(), ref, atol=2e-2 * rms, rtol=1e-2), name
    # forward hands o_proj the amax the attention write accumulated
    # (out_amax); the two-pass quantisation that measures it gives the same bits
    with torch.no_grad():
        assert torch.equal(out, mod.o_proj(x_o)), "o_proj with the attention's amax differs"



@pytest.mark.parametrize("name", mg.CASES)
def test_full_attention_on_fp8_kv_pool(gpu, name, monkeypatch):
    """``FullAttnKVPool.from_config`` with an fp8-e4m3 pool driving
    ``FullAttention.forward`` (the per-layer ``get_full_kv_scales`` path):

    * the pool is filled with the golden pool's rows through ``write_kv``
      (quantise-on-write): every dequantised value within half an e4m3 step
      (2^-4 relative, or 2^-10 scaled below the normal range) of the input;
    * the K / V rows the forward writes quantise the reference module's
      written K / V the same way;
    * the attention the module computes equals the oracle's attention over the
      same dequantised pool (bf16 tolerance: 2e-2 + 1e-2 |ref|, rel-norm 1e-2).
    """
    from oracle.harness import reference_attention
    from oracle.kv_quant import dequantize_e4m3
    from tokenfactory_amd import workloads
    from tokenfactory_amd.kv_pool import FullAttnKVPool

    d, meta = mg.load()
    cfg = mg.config(meta)
    cfg.layer_types = ["linear_attention"] * 3 + ["full_attention"] + ["linear_attention"] * 3 + \
        ["full_attention"]
    S = meta["pool_slots"]
    pool = FullAttnKVPool.from_config(cfg, S, device=gpu, dtype=torch.float8_e4m3fn)
    assert pool.full_layer_map == {3: 0, 7: 1} and pool.is_fp8
    assert pool.k_buffer.shape == (2, S, cfg.num_key_value_heads, cfg.head_dim)
    kf = mg.bf16(d["k_pool0"]).to(gpu)
    vf = mg.bf16(d["v_pool0"]).to(gpu)
    ks, vs = float(kf.abs().max()) / 448.0, float(vf.abs().max()) / 448.0
    pool.set_kv_scales(3, ks, vs)
    pool.write_kv(3, torch.arange(S, device=gpu), kf.to(torch.bfloat16), vf.to(torch.bfloat16))

    def within_e4m3_step(deq, x, scale, what):
        bound = torch.maximum(x.abs() * 2.0 ** -4, torch.full_like(x, scale * 2.0 ** -10))
        assert ((deq - x).abs() <= bound * 1.0001).all(), what

    kb, vb = pool.get_full_kv_buffers(3)
    k_sc, v_sc = pool.get_full_kv_scales(3)
    assert float(k_sc) == pytest.approx(ks) and float(v_sc) == pytest.approx(vs)
    within_e4m3_step(dequantize_e4m3(kb.cpu(), ks), kf.cpu(), ks, "pool K")
    within_e4m3_step(dequantize_e4m3(vb.cpu(), vs), vf.cpu(), vs, "pool V")

    mod = FullAttention(cfg, layer_idx=3, dtype=torch.bfloat16).to(gpu)
    mg.load_weights(mod, d)
    captured = {}
    inner = fa.slot_based_attention

    def spy(q, k_buf, v_buf, batch, *, gate=None, **kw):
        captured["q"] = q.clone()
        captured["attn"] = inner(q, k_buf, v_buf, batch, **kw).clone()
        return inner(q, k_buf, v_buf, batch, gate=gate, **kw)

    monkeypatch.setattr(fa, "slot_based_attention", spy)
    batch = mg.batch(d, meta, name, gpu)
    hidden = mg.bf16(d[f"{name}_hidden"]).to(device=gpu, dtype=torch.bfloat16)
    pos = torch.from_numpy(d[f"{name}_positions"]).to(gpu)
    print(f"[module fp8 pool] case={name}", flush=True)
    with torch.no_grad():
        out = mod(hidden, pos, pool, batch)
    torch.cuda.synchronize()
    assert torch.isfinite(out.float()).all()
    loc = torch.from_numpy(d[f"{name}_out_cache_loc"])
    for what, buf, sc in (("k_written", kb, ks), ("v_written", vb, vs)):
        # the write saturates at +-448 x scale (the scale came from the pool
        # before this step); the module's bf16 K differs from the fp32
        # reference by ~2^-8, on top of the quantisation step
        want = mg.expected(d, name, what).clamp(-448.0 * sc, 448.0 * sc)
        deq = dequantize_e4m3(buf.cpu()[loc], sc)
        bound = want.abs() * (2.0 ** -4 + 2.0 ** -7) + sc * 2.0 ** -9 + 1e-2
        assert ((deq - want).abs() <= bound).all(), f"{name} {what}"
    c = meta["cases"][name]
    wl = workloads.Workload(
        name=name, q=captured["q"], k_pool=kb, v_pool=vb, batch=batch, seq_lens=list(c["seq"]),
        ext_lens=list(c["ext"]), rows=list(c["req"]), num_q_heads=cfg.num_attention_heads,
        num_kv_heads=cfg.num_key_value_heads, head_dim=cfg.head_dim, scale=mod.scaling,
        k_scale=k_sc, v_scale=v_sc)
    assert_attn_close(captured["attn"], reference_attention(wl), what=f"{name} fp8-pool attention")
