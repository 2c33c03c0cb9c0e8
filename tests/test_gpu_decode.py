"""Split-K decode kernel vs the oracle (pure-decode and bsz == 1 branches).

Tolerance (bf16 outputs vs an fp32 reference): |out - ref| <= 2e-2 + 1e-2 |ref|
elementwise and a relative Frobenius error <= 1e-2. fp8-KV outputs are compared
with the same bounds against attention over the same KV dequantised to fp32.
"""
import numpy as np
import pytest
import torch

from tests.helpers import (assert_attn_close, assert_empty_context_rows, rebatch, restatement,
                           small_case)
from tokenfactory_amd import _native, slot_based_attention, workloads

pytestmark = pytest.mark.gpu


def run(wl, workgroups=0):
    return slot_based_attention(wl.q, wl.k_pool, wl.v_pool, wl.batch, scaling=wl.scale,
                                k_scale=wl.k_scale, v_scale=wl.v_scale,
                                decode_workgroups=workgroups)


def check(wl, workgroups=0, what=""):
    print(f"[decode] {what} B={wl.batch.batch_size} L<={wl.batch.max_seq_len} "
          f"Hq={wl.num_q_heads} Hkv={wl.num_kv_heads} workgroups={workgroups}", flush=True)
    out = run(wl, workgroups)
    torch.cuda.synchronize()
    return assert_attn_close(out, restatement(wl), what=what)


def test_reference_cpu_decode_shape_in_bf16(gpu):
    wl = workloads.build("cfg1_bf16", [128, 256, 384, 512], [1, 1, 1, 1], num_q_heads=16,
                         num_kv_heads=2, head_dim=256, pool_slots=4096, device=gpu, seed=7)
    check(wl, what="B=4 L=128..512 16/2")


@pytest.mark.parametrize("L", [1, 2, 15, 16, 17, 63, 64, 65, 1000, 4097])
def test_single_request_lengths(gpu, L):
    wl = small_case([L], [1], hq=24, hkv=4, d=256, seed=L, device=gpu, dtype=torch.bfloat16)
    check(wl, what=f"bsz1 L={L}")


@pytest.mark.parametrize("workgroups", [0, 1, 3, 7, 64, 513, 4096])
def test_balanced_split_and_merge(gpu, workgroups):
    """Any grid size: one workgroup owning every unit, workgroups straddling unit
    boundaries, and far more workgroups than tiles (empty ranges)."""
    rng = np.random.default_rng(3)
    lens = rng.integers(1, 3000, size=7).tolist()
    wl = small_case(lens, [1] * 7, hq=24, hkv=4, d=256, seed=4, device=gpu,
                    dtype=torch.bfloat16)
    check(wl, workgroups, what=f"workgroups={workgroups}")


def test_empty_and_tiny_requests(gpu):
    """L = 1 units next to long ones; many units per workgroup."""
    lens = [1, 2, 4000, 1, 17, 33, 1, 900]
    wl = small_case(lens, [1] * len(lens), hq=24, hkv=4, d=256, seed=8, device=gpu,
                    dtype=torch.bfloat16)
    for wg in (0, 5, 40):
        check(wl, wg, what=f"tiny wg={wg}")


@pytest.mark.parametrize("workgroups", [0, 3])
def test_empty_context_rows_are_zero(gpu, workgroups):
    """A request with seq_len 0 sees no key: its row is zeros, as the
    reference's fully masked attention returns it, and the other rows are
    unaffected."""
    wl = small_case([300, 40, 1000, 2], [1] * 4, hq=24, hkv=4, d=256, seed=9, device=gpu,
                    dtype=torch.bfloat16)
    wl.batch.seq_lens[1] = 0
    print(f"[decode] empty context at row 1, workgroups={workgroups}", flush=True)
    out = run(wl, workgroups)
    torch.cuda.synchronize()
    assert_empty_context_rows(out, restatement(wl), [1], what="seq_len 0")


def test_workspace_reuse_across_shapes(gpu):
    """One workspace serves calls of different shapes back to back (a small call's
    partials land where a larger call's would); each call stays correct."""
    big = small_case([3000, 2500, 17, 900], [1] * 4, hq=24, hkv=4, d=256, seed=5,
                     device=gpu, dtype=torch.bfloat16)
    small = rebatch(big, [2500, 17], [1, 1], big.q[1:3].clone(), rows=big.rows[1:3])
    for wl in (big, small, big, small):
        check(wl, 37, what="reuse")


def test_split_phases_compose_to_full_call(gpu):
    from tokenfactory_amd.attention import SlotAttentionCall
    wl = small_case([2000, 33, 4100], [1, 1, 1], hq=24, hkv=4, d=256, seed=6, device=gpu,
                    dtype=torch.bfloat16)
    call = SlotAttentionCall(wl.q, wl.k_pool, wl.v_pool, wl.batch, scaling=wl.scale,
                             decode_workgroups=29)
    full = call.run().clone()
    call.out.zero_()
    call.run_decode_partial()
    call.run_decode_merge()
    assert torch.equal(call.out, full)


@pytest.mark.parametrize("hq,hkv", [(16, 16), (8, 4), (16, 4), (24, 4), (32, 4), (16, 1),
                                    (40, 2)])
def test_group_sizes(gpu, hq, hkv):
    wl = small_case([300, 1, 77, 1500], [1] * 4, hq=hq, hkv=hkv, d=256, seed=hq + hkv,
                    device=gpu, dtype=torch.bfloat16)
    check(wl, 24, what=f"G={hq // hkv}")


def test_peaky_softmax(gpu):
    """Large-norm queries make the softmax concentrate on few keys."""
    wl = small_case([900, 2049], [1, 1], hq=24, hkv=4, d=256, seed=9, device=gpu,
                    dtype=torch.bfloat16, q_std=6.0)
    check(wl, 24, what="peaky")


def test_shared_prefix_rows_give_identical_outputs(gpu):
    """Two requests on one radix prefix with the same query.  The persistent grid
    may cut them at different tile boundaries, so only the fp32 summation order
    of their splits may differ; with one workgroup per request they are equal."""
    wl = small_case([700, 700, 420], [1, 1, 1], hq=24, hkv=4, d=256, seed=10, device=gpu,
                    dtype=torch.bfloat16, groups=[0, 0, 1], prefixes=[700, 400])
    wl.q[1] = wl.q[0]
    out = run(wl)
    assert_attn_close(out[1], out[0], atol=4e-3, rtol=4e-3, norm_rel=4e-3,
                      what="shared prefix rows")
    assert_attn_close(out, restatement(wl), what="shared prefix")
    one = run(wl, workgroups=1)
    assert torch.equal(one[0], one[1])


@pytest.mark.parametrize("lens", [[5, 700, 64], [4096, 33]])
def test_fp8_kv_decode(gpu, lens):
    wl = workloads.build("fp8", lens, [1] * len(lens), num_q_heads=24, num_kv_heads=4,
                         head_dim=256, pool_slots=sum(lens) + 100, device=gpu, seed=31,
                         kv_fp8=True)
    check(wl, 24, what="fp8")


def test_decode_rows_via_item_list(gpu):
    """Mixed-batch decode rows: the kernel reads only the listed items and their q rows."""
    wl = small_case([50, 400, 8, 1200], [3, 1, 2, 1], hq=24, hkv=4, d=256, seed=12,
                    device=gpu, dtype=torch.bfloat16)
    out = run(wl)
    ref = restatement(wl)
    assert_attn_close(out, ref, what="mixed rows")


def test_full_size_decode_b64_sampled(gpu):
    """The 64-request decode step at full size (1M-slot pool, L in [1k, 8k]); four
    requests are re-checked against the oracle on a sub-batch, and rows of the full
    output must not depend on the batch they were computed in."""
    wl = workloads.decode_b64(device=gpu)
    out = run(wl)
    torch.cuda.synchronize()
    assert torch.isfinite(out.float()).all()
    pick = [0, 17, 40, 63]
    sub = rebatch(wl, [wl.seq_lens[i] for i in pick], [1] * 4, wl.q[pick].clone(),
                  rows=[wl.rows[i] for i in pick])
    assert_attn_close(out[pick], restatement(sub), what="b64 sample")
    # The same rows computed inside a 4-request batch are split differently over
    # the workgroups; only fp32 summation order may differ.
    assert_attn_close(run(sub), out[pick], atol=4e-3, rtol=4e-3, norm_rel=4e-3,
                      what="batch composition")


@pytest.mark.parametrize("bsz", [1, 3])
def test_negative_slot_entries(gpu, bsz):
    """A -1 inside a request's req_to_token row: the bsz == 1 branch reads the
    pool's last slot (torch indexing, full_attention.py:188-190), the batched
    branch slot 0 (clamp, :217-219); the oracle follows the same rules."""
    lens = [300, 77, 1000][:bsz]
    wl = small_case(lens, [1] * bsz, hq=24, hkv=4, d=256, seed=40 + bsz, device=gpu,
                    dtype=torch.bfloat16, q_std=3.0)
    for b in range(bsz):
        wl.batch.req_to_token[wl.rows[b], [5, lens[b] // 2]] = -1
    check(wl, 0, what=f"-1 entries, bsz={bsz}")
