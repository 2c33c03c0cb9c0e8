"""``slot_based_attention`` plans a model step once.

A model step runs every full-attention layer over one ``ForwardBatch``
(``decoder_layer.py:68-69``).  The first call made with a batch plans its work
lists on the device and keeps them on the batch; the calls of the other layers
reuse them (no further planner launch, no host planning), on the caller's
stream or on another one, and a new batch object (the next step) plans again.
Every call equals the host-planned one-stream call bit for bit: the device
plan is the host plan plus padding, and the decode launches of a mixed step
write other rows than the extend kernel.
"""
import pytest
import torch

from tests.helpers import small_case
from tokenfactory_amd import _native, slot_based_attention, workloads
from tokenfactory_amd.attention import SlotAttentionCall
from tokenfactory_amd.forward_batch import ForwardBatch

pytestmark = pytest.mark.gpu


def host_planned(wl, **kw):
    call = SlotAttentionCall(wl.q, wl.k_pool, wl.v_pool, wl.batch, scaling=wl.scale,
                             k_scale=wl.k_scale, v_scale=wl.v_scale, overlap_decode=False, **kw)
    return call.run().clone()


def next_step(batch):
    """The same lengths as a new ForwardBatch object (the next model step)."""
    return ForwardBatch(batch_size=batch.batch_size, req_pool_indices=batch.req_pool_indices,
                        seq_lens=batch.seq_lens, prefix_lens=batch.prefix_lens,
                        extend_lens=list(batch.extend_lens), out_cache_loc=batch.out_cache_loc,
                        req_to_token=batch.req_to_token, is_prefill=batch.is_prefill,
                        max_seq_len=batch.max_seq_len, max_extend_len=batch.max_extend_len,
                        req_pool_indices_list=batch.req_pool_indices_list)


CASES = {
    "mixed": lambda dev: workloads.mixed(device=dev, n_extend=3, extend_new=300, prefix_hi=900,
                                         n_decode=20, dec_lo=1, dec_hi=3000, pool_slots=1 << 16),
    "extend": lambda dev: small_case([700, 64, 300], [500, 64, 20], hq=24, hkv=4, d=256,
                                     seed=3, device=dev, dtype=torch.bfloat16),
    "bsz1": lambda dev: small_case([900], [257], hq=24, hkv=4, d=256, seed=4, device=dev,
                                   dtype=torch.bfloat16),
    "fp8": lambda dev: workloads.build("fp8sp", [40, 300, 900, 77], [40, 100, 1, 1],
                                       num_q_heads=24, num_kv_heads=4, head_dim=256,
                                       pool_slots=2048, device=dev, seed=45, kv_fp8=True),
    "head_dim_128": lambda dev: small_case([300, 50, 9], [100, 1, 9], hq=8, hkv=2, d=128,
                                           seed=5, device=dev, dtype=torch.bfloat16),
}


@pytest.mark.parametrize("case", sorted(CASES))
def test_layers_of_a_step_share_one_plan(gpu, case, monkeypatch):
    wl = CASES[case](gpu)
    print(f"[step plan] {case} ext={wl.ext_lens[:8]}", flush=True)
    want = host_planned(wl)
    launched = []
    real = _native.call

    def counting(name, *args):
        launched.append(name)
        return real(name, *args)

    monkeypatch.setattr(_native, "call", counting)

    def layer(batch):
        return slot_based_attention(wl.q, wl.k_pool, wl.v_pool, batch, scaling=wl.scale,
                                    k_scale=wl.k_scale, v_scale=wl.v_scale).clone()

    outs = [layer(wl.batch) for _ in range(4)]          # four layers of one step
    side = torch.cuda.Stream(device=gpu)
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        outs.append(layer(wl.batch))                     # a layer on another stream
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    assert launched.count("tf_attn_plan_device") == 1
    for i, out in enumerate(outs):
        assert torch.equal(out, want), f"{case}: call {i} differs from the host-planned step"

    step2 = next_step(wl.batch)
    out = layer(step2)
    torch.cuda.synchronize()
    assert launched.count("tf_attn_plan_device") == 2
    assert torch.equal(out, want)


def test_pure_decode_steps_plan_nothing(gpu, monkeypatch):
    wl = small_case([300, 2000, 47, 9], [1] * 4, hq=24, hkv=4, d=256, seed=10, device=gpu,
                    dtype=torch.bfloat16)
    want = host_planned(wl)
    launched = []
    real = _native.call
    monkeypatch.setattr(_native, "call", lambda name, *a: launched.append(name) or real(name, *a))
    out = slot_based_attention(wl.q, wl.k_pool, wl.v_pool, wl.batch, scaling=wl.scale)
    torch.cuda.synchronize()
    assert "tf_attn_plan_device" not in launched and "tf_attn_extend" not in launched
    assert torch.equal(out, want)


def test_captured_layer_call_replays_beside_eager_calls(gpu):
    """A layer call captured in a HIP graph plans inside the graph: every replay
    equals the host-planned step, and eager calls with the same batch between
    the replays (which share the batch's step plan) do too."""
    wl = CASES["mixed"](gpu)
    want = host_planned(wl)

    def layer():
        return slot_based_attention(wl.q, wl.k_pool, wl.v_pool, wl.batch, scaling=wl.scale)

    first = layer().clone()
    side = torch.cuda.Stream(device=gpu)
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        layer()                                       # warm-up outside the capture
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        captured = layer()
    torch.cuda.synchronize()
    assert torch.equal(first, want)
    for r in range(3):
        print(f"[step plan] replay {r}", flush=True)
        captured.zero_()
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(captured, want), f"replay {r}"
        eager = layer()
        torch.cuda.synchronize()
        assert torch.equal(eager, want), f"eager call after replay {r}"


def test_mixed_steps_use_three_decode_workgroups_per_cu(gpu):
    """A step with extends and decodes runs its decode kernel on three
    workgroups per CU (they fill the CUs the extend kernel frees); serial and
    overlapped calls use the same grid and give the same bits, and an explicit
    ``decode_workgroups`` or a pure decode step keeps its own grid."""
    cus = torch.cuda.get_device_properties(gpu).multi_processor_count
    wl = CASES["mixed"](gpu)
    ser = SlotAttentionCall(wl.q, wl.k_pool, wl.v_pool, wl.batch, scaling=wl.scale,
                            overlap_decode=False)
    ovl = SlotAttentionCall(wl.q, wl.k_pool, wl.v_pool, wl.batch, scaling=wl.scale,
                            overlap_decode=True)
    own = SlotAttentionCall(wl.q, wl.k_pool, wl.v_pool, wl.batch, scaling=wl.scale,
                            decode_workgroups=cus)
    assert ser.decode_workgroups == ovl.decode_workgroups == 3 * cus
    assert own.decode_workgroups == cus
    a, b = ser.run().clone(), ovl.run().clone()
    torch.cuda.synchronize()
    assert torch.equal(a, b)
    dec = small_case([300, 2000, 47, 9], [1] * 4, hq=24, hkv=4, d=256, seed=10, device=gpu,
                     dtype=torch.bfloat16)
    call = SlotAttentionCall(dec.q, dec.k_pool, dec.v_pool, dec.batch, scaling=dec.scale)
    assert call.decode_workgroups == 0
