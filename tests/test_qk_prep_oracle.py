"""The q/k RMSNorm + partial M-RoPE oracle against the reference module's own
outputs (CPU only): fed the golden projection outputs in fp32, it must give the
q that reached the reference's attention and the K it wrote to the pool."""
import pytest
import torch

from oracle.qk_prep import inv_freq_ref, qk_prep_ref
from tests import module_golden as mg
from tokenfactory_amd.full_attention import PartialRoPE

TOL = dict(atol=2e-3, rtol=2e-3)   # float16 storage of the golden outputs


@pytest.mark.parametrize("name", mg.CASES)
def test_qk_prep_oracle_reproduces_reference_module(name):
    d, meta = mg.load()
    hidden = mg.bf16(d[f"{name}_hidden"])
    T = hidden.shape[0]
    hq, hkv, dim = meta["num_attention_heads"], meta["num_key_value_heads"], meta["head_dim"]
    q, _ = (hidden @ mg.bf16(d["w_q_proj"]).T).view(T, hq, 2 * dim).chunk(2, dim=-1)
    k = (hidden @ mg.bf16(d["w_k_proj"]).T).view(T, hkv, dim)
    rd = int(dim * meta["partial_rotary_factor"])
    qo, ko = qk_prep_ref(q, k, mg.bf16(d["w_q_norm"]), mg.bf16(d["w_k_norm"]),
                         meta["rms_norm_eps"], torch.from_numpy(d[f"{name}_positions"]),
                         inv_freq_ref(rd, meta["rope_theta"]), rd, meta["mrope_section"],
                         meta["mrope_interleaved"])
    torch.testing.assert_close(qo, mg.expected(d, name, "q"), **TOL)
    torch.testing.assert_close(ko, mg.expected(d, name, "k_written"), **TOL)


def test_inv_freq_matches_module_buffer():
    rope = PartialRoPE(256, 0.25, 1e7)
    assert torch.equal(rope.inv_freq, inv_freq_ref(64, 1e7))
