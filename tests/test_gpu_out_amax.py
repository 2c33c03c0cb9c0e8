"""``out_amax`` of the attention entry points and ``tf_fp8_act_quant_amax``.

The per-tensor amax of the dynamic FP8 quantisation in front of o_proj
(``fp8_triton.py:127-130``) is folded into the attention output write:

* the amax a call leaves equals the maximum over its output of the bf16 bit
  pattern with the sign cleared, exactly, for decode (direct write and split
  merge), extend, mixed steps on one stream and on two, fp8 pools, the fused
  output gate and head dims other than 256; calls sharing the word leave the
  larger value, and a NaN output row leaves the NaN pattern;
* ``quantize_activations`` given that amax returns the same ``xq`` and
  ``x_scale``, bit for bit, as the two-pass quantisation that measures the
  amax itself (``tf_fp8_act_quant``), which the oracle pins separately.
"""
import pytest
import torch

from tests.helpers import small_case
from tests.test_gpu_gate import module_gate
from tokenfactory_amd import fp8_linear as fl
from tokenfactory_amd import workloads
from tokenfactory_amd.attention import SlotAttentionCall

pytestmark = pytest.mark.gpu


def bits_amax(out: torch.Tensor) -> int:
    """max over out of |out| as bf16 bits (NaN patterns above inf)."""
    return int((out.contiguous().view(torch.int16).to(torch.int32) & 0x7fff).max())


def run_with_amax(wl, amax=None, **kw):
    if amax is None:
        amax = torch.zeros((1,), dtype=torch.int32, device=wl.q.device)
    call = SlotAttentionCall(wl.q, wl.k_pool, wl.v_pool, wl.batch, scaling=wl.scale,
                             k_scale=wl.k_scale, v_scale=wl.v_scale, out_amax=amax, **kw)
    out = call.run()
    torch.cuda.synchronize()
    return out, amax


def bf16_case(seq, ext, d=256, hq=24, hkv=4, seed=0, gpu="cuda"):
    return small_case(seq, ext, hq=hq, hkv=hkv, d=d, seed=seed, device=gpu,
                      dtype=torch.bfloat16)


CASES = {
    "decode": lambda g: bf16_case([1, 5, 64, 65, 300, 1000], [1] * 6, seed=1, gpu=g),
    # two long requests: their (request, kv head) units span several
    # workgroups, so the merge kernel writes the output
    "decode split": lambda g: bf16_case([20000, 30000], [1, 1], seed=2, gpu=g),
    "extend": lambda g: bf16_case([333 + 40], [40], seed=3, gpu=g),
    "mixed": lambda g: bf16_case([50, 400, 7, 900, 64], [50, 1, 3, 1, 20], seed=4, gpu=g),
    "fp8 mixed": lambda g: workloads.build("fp8", [40, 300, 9], [40, 100, 1], num_q_heads=8,
                                           num_kv_heads=2, head_dim=256, pool_slots=512,
                                           device=g, seed=5, kv_fp8=True),
    "generic d32": lambda g: bf16_case([50, 400, 7], [50, 1, 3], d=32, hq=8, hkv=2, seed=6,
                                       gpu=g),
    "generic d80 fp8": lambda g: workloads.build("fp8", [40, 300, 9], [40, 100, 1],
                                                 num_q_heads=8, num_kv_heads=2, head_dim=80,
                                                 pool_slots=512, device=g, seed=7, kv_fp8=True),
}


@pytest.mark.parametrize("name", list(CASES))
@pytest.mark.parametrize("gated", [False, True])
def test_amax_is_the_output_bit_maximum(gpu, name, gated):
    wl = CASES[name](gpu)
    print(f"[out_amax] {name} gated={gated} ext={wl.ext_lens[:6]} L={wl.seq_lens[:6]}",
          flush=True)
    gate = module_gate(wl, 11) if gated else None
    out, amax = run_with_amax(wl, gate=gate)
    want = bits_amax(out)
    assert want > 0 and int(amax.item()) == want, f"{name}: {int(amax.item()):#x} vs {want:#x}"


def test_amax_on_two_streams_and_shared_word(gpu):
    wl = CASES["mixed"](gpu)
    one, a1 = run_with_amax(wl, overlap_decode=False)
    two, a2 = run_with_amax(wl, overlap_decode=True)
    assert torch.equal(one, two) and int(a1.item()) == int(a2.item()) == bits_amax(one)
    # a second call on the same word keeps the larger of the two maxima
    small = bf16_case([1, 5], [1, 1], seed=9, gpu=gpu)
    word = torch.zeros((1,), dtype=torch.int32, device=gpu)
    o1, _ = run_with_amax(small, amax=word)
    first = int(word.item())
    o2, _ = run_with_amax(wl, amax=word)
    assert int(word.item()) == max(first, bits_amax(o2)) and first == bits_amax(o1)


def test_nan_row_sets_the_nan_pattern(gpu):
    wl = bf16_case([5, 64], [1, 1], seed=12, gpu=gpu)
    wl.q[1] = float("nan")   # NaN scores: the reference's softmax gives a NaN row
    out, amax = run_with_amax(wl)
    assert torch.isnan(out[1].float()).all() and int(amax.item()) == bits_amax(out) >= 0x7f81


def test_empty_context_row_adds_nothing_to_amax(gpu):
    wl = bf16_case([5, 64], [1, 1], seed=12, gpu=gpu)
    wl.batch.seq_lens[1] = 0   # no visible key: a row of zeros
    out, amax = run_with_amax(wl)
    assert (out[1] == 0).all() and int(amax.item()) == bits_amax(out[:1]) == bits_amax(out)


@pytest.mark.parametrize("name", ["decode", "mixed", "fp8 mixed"])
def test_quantisation_with_amax_is_bit_identical(gpu, name):
    wl = CASES[name](gpu)
    out, amax = run_with_amax(wl, gate=module_gate(wl, 13))
    x = out.reshape(out.shape[0], -1)
    xq, sx = fl.quantize_activations(x, padded_cols=x.shape[1])
    xq2, sx2 = fl.quantize_activations(x, padded_cols=x.shape[1], amax=amax)
    torch.cuda.synchronize()
    assert torch.equal(sx, sx2), f"{name}: x_scale {float(sx)} vs {float(sx2)}"
    assert torch.equal(xq.view(torch.uint8), xq2.view(torch.uint8)), f"{name}: xq differs"
    with pytest.raises(ValueError):
        fl.quantize_activations(x, amax=amax.to(torch.int64))
