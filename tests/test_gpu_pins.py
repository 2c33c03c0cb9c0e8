"""The oracle's invariant pins (tests/test_oracle_pins.py) on the HIP path.

Each pin builds its case on the CPU in fp32.  The adapter below rounds q, K
and V to bf16 in place, so the pin's closed-form expectation uses exactly the
values the kernels read, runs ``slot_based_attention`` on the GPU and returns
the bf16 output as fp32.  Head dim 256 runs the tuned decode and extend
kernels, 16 the one-wave-per-row kernel.

Tolerances: a single visible key, a dominant key and a relocation of the
slots leave nothing to round (the output is a V row, or the same computation
over moved rows), so those pins keep the oracle's own bounds.  Equal keys give
a mean of V rounded once to bf16 (half an ulp of values below 2: 4e-3); the
prefix, chunking and decode pins compare two runs whose bf16 probabilities and
outputs may round apart by an ulp (8e-3); the two-key logistic weight
carries the bf16 rounding of its probabilities (1e-2).
"""
import dataclasses

import pytest
import torch

from tests import test_oracle_pins as pins
from tokenfactory_amd import slot_based_attention
from tokenfactory_amd.forward_batch import ForwardBatch

pytestmark = pytest.mark.gpu

GPU_ATOL = {
    "pin_single_key_returns_value": None,
    "pin_equal_keys_average_visible_values": 4e-3,
    "pin_two_keys_logistic_weight": 1e-2,
    "pin_dominant_key_selects_its_value": None,
    "pin_slot_permutation_invariance": None,
    "pin_prefix_extend_equals_full_prefill_rows": 8e-3,
    "pin_chunked_extend_equals_one_shot": 8e-3,
    "pin_decode_equals_last_prefill_row": 8e-3,
}


def attn_gpu(wl):
    dev = torch.device("cuda")
    for name in ("q", "k_pool", "v_pool"):
        t = getattr(wl, name)
        t.copy_(t.to(torch.bfloat16).float())   # the pin then reads the rounded inputs
    fields = {f.name: getattr(wl.batch, f.name) for f in dataclasses.fields(wl.batch)}
    batch = ForwardBatch(**{k: v.to(dev) if isinstance(v, torch.Tensor) else v
                            for k, v in fields.items()})
    out = slot_based_attention(wl.q.to(dev, torch.bfloat16), wl.k_pool.to(dev, torch.bfloat16),
                               wl.v_pool.to(dev, torch.bfloat16), batch, scaling=wl.scale)
    torch.cuda.synchronize()
    return out.float().cpu().numpy()


def test_every_pin_has_a_gpu_tolerance():
    assert sorted(GPU_ATOL) == sorted(p.__name__ for p in pins.PINS)


@pytest.mark.parametrize("d", [256, 16])
@pytest.mark.parametrize("pin", pins.PINS, ids=lambda f: f.__name__)
def test_hip_path_satisfies_pin(gpu, pin, d):
    print(f"[pins] {pin.__name__} d={d}", flush=True)
    assert pin(attn_gpu, d=d, atol=GPU_ATOL[pin.__name__])
