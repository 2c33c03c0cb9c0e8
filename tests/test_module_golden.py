"""Module-level composition against the reference's own outputs (CPU only).

The golden vectors come from the reference's ``Qwen3_8FullAttention.forward``
(fp32, CPU, mini config: hidden 32, 4 q / 2 kv heads, head_dim 256) on a
mixed, a pure-decode (3-D M-RoPE positions) and a bsz == 1 extend batch. Here
the host-side pieces of ``tokenfactory_amd.FullAttention`` (projections, q/k
RMSNorm, partial RoPE, silu gate, o_proj) run in fp32 on the CPU with the
oracle in place of the kernels, and the oracle's attention restatement is
checked against the reference's attention output directly.
"""
import pytest
import torch
import torch.nn.functional as F

from oracle.slot_attention import slot_based_attention_ref
from tests import module_golden as mg
from tokenfactory_amd.full_attention import FullAttention

TOL = dict(atol=2e-3, rtol=2e-3)   # float16 storage of the golden outputs + fp32 op order


@pytest.fixture(scope="module")
def golden():
    d, meta = mg.load()
    mod = FullAttention(mg.config(meta), layer_idx=3, dtype=torch.float32)
    mg.load_weights(mod, d)
    return d, meta, mod


@pytest.mark.parametrize("name", mg.CASES)
def test_norm_rope_projection_match_reference(golden, name):
    d, meta, mod = golden
    hidden = mg.bf16(d[f"{name}_hidden"])
    pos = torch.from_numpy(d[f"{name}_positions"])
    T = hidden.shape[0]
    qg = mod.q_proj(hidden).view(T, mod.num_heads, 2 * mod.head_dim)
    q, _ = qg.chunk(2, dim=-1)
    k = mod.k_proj(hidden).view(T, mod.num_kv_heads, mod.head_dim)
    v = mod.v_proj(hidden).view(T, mod.num_kv_heads, mod.head_dim)
    q, k = mod.rotary_emb(mod.q_norm(q), mod.k_norm(k), pos)
    torch.testing.assert_close(q, mg.expected(d, name, "q"), **TOL)
    torch.testing.assert_close(k, mg.expected(d, name, "k_written"), **TOL)
    torch.testing.assert_close(v, mg.expected(d, name, "v_written"), **TOL)


@pytest.mark.parametrize("name", mg.CASES)
def test_oracle_attention_matches_reference_output(golden, name):
    """The oracle's restatement, fed the reference's own q and pool, reproduces
    the reference's ``_slot_based_attention`` output."""
    d, meta, mod = golden
    k = mg.bf16(d["k_pool0"])
    v = mg.bf16(d["v_pool0"])
    loc = torch.from_numpy(d[f"{name}_out_cache_loc"])
    k[loc] = mg.expected(d, name, "k_written")
    v[loc] = mg.expected(d, name, "v_written")
    out = slot_based_attention_ref(mg.expected(d, name, "q"), k, v, mg.batch(d, meta, name, "cpu"),
                                   mod.num_queries_per_kv, mod.scaling)
    torch.testing.assert_close(out, mg.expected(d, name, "attn"), **TOL)


@pytest.mark.parametrize("name", mg.CASES)
def test_gate_and_o_proj_composition_matches_reference(golden, name):
    d, meta, mod = golden
    hidden = mg.bf16(d[f"{name}_hidden"])
    T = hidden.shape[0]
    _, gate = mod.q_proj(hidden).view(T, mod.num_heads, 2 * mod.head_dim).chunk(2, dim=-1)
    attn = mg.expected(d, name, "attn").reshape(T, -1)
    out = mod.o_proj(attn * F.silu(gate.reshape(T, -1)))
    torch.testing.assert_close(out, mg.expected(d, name, "out"), **TOL)
