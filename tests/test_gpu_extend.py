"""Extend / prefill MFMA kernel (and mixed batches) vs the oracle.

Same tolerance as the decode tests: |out - ref| <= 2e-2 + 1e-2 |ref| elementwise
and relative Frobenius error <= 1e-2 against an fp32 reference; fp8-KV against
the dequantised KV.
"""
import numpy as np
import pytest
import torch

from tests.helpers import assert_attn_close, rebatch, restatement, small_case
from tokenfactory_amd import slot_based_attention, workloads

pytestmark = pytest.mark.gpu


def run(wl):
    return slot_based_attention(wl.q, wl.k_pool, wl.v_pool, wl.batch, scaling=wl.scale,
                                k_scale=wl.k_scale, v_scale=wl.v_scale)


def check(wl, what=""):
    print(f"[extend] {what} B={wl.batch.batch_size} ext={wl.ext_lens[:6]} "
          f"L={wl.seq_lens[:6]} Hq={wl.num_q_heads} Hkv={wl.num_kv_heads}", flush=True)
    out = run(wl)
    torch.cuda.synchronize()
    return assert_attn_close(out, restatement(wl), what=what)


@pytest.mark.parametrize("n", [2, 5, 21, 22, 64, 300])
def test_single_request_prefill(gpu, n):
    wl = small_case([n], [n], hq=24, hkv=4, d=256, seed=n, device=gpu, dtype=torch.bfloat16)
    check(wl, f"prefill n={n}")


@pytest.mark.parametrize("prefix,n", [(1, 2), (100, 31), (513, 64), (2000, 200)])
def test_single_request_extend_over_prefix(gpu, prefix, n):
    wl = small_case([prefix + n], [n], hq=24, hkv=4, d=256, seed=prefix, device=gpu,
                    dtype=torch.bfloat16)
    check(wl, f"extend P={prefix} n={n}")


@pytest.mark.parametrize("hq,hkv", [(16, 16), (8, 1), (24, 4), (16, 2), (12, 4)])
def test_group_sizes_and_tile_edges(gpu, hq, hkv):
    # 128 / G rows per tile: choose ext so tiles end exactly, one short and one over.
    g = hq // hkv
    exts = [max(2, 128 // g), max(2, 128 // g + 1), max(2, 256 // g - 1), 3]
    seq = [e + p for e, p in zip(exts, [0, 37, 300, 5])]
    wl = small_case(seq, exts, hq=hq, hkv=hkv, d=256, seed=g, device=gpu,
                    dtype=torch.bfloat16)
    check(wl, f"G={g}")


def test_radix_shared_prefix_groups(gpu):
    wl = workloads.extend_prefix(device=gpu, prefix_hi=600, new_lo=16, new_hi=160,
                                 pool_slots=1 << 14)
    check(wl, "shared prefixes")


def test_mixed_chunked_prefill_and_decode(gpu):
    wl = workloads.mixed(device=gpu, n_extend=3, extend_new=150, prefix_hi=700, n_decode=9,
                         dec_lo=1, dec_hi=2500, pool_slots=1 << 15)
    check(wl, "mixed")


def test_mixed_step_with_decode_on_a_second_stream(gpu):
    """A reused call with overlap_decode=True (decode launches on a second
    stream beside the extend kernel) gives the one-stream result bit for bit,
    run after run, and matches the oracle."""
    from tokenfactory_amd.attention import SlotAttentionCall
    wl = workloads.mixed(device=gpu, n_extend=3, extend_new=150, prefix_hi=700, n_decode=9,
                         dec_lo=1, dec_hi=2500, pool_slots=1 << 15)
    serial = SlotAttentionCall(wl.q, wl.k_pool, wl.v_pool, wl.batch, scaling=wl.scale,
                               overlap_decode=False).run().clone()
    call = SlotAttentionCall(wl.q, wl.k_pool, wl.v_pool, wl.batch, scaling=wl.scale,
                             overlap_decode=True)
    assert call.n_work and call.n_dec
    for _ in range(3):
        call.out.zero_()
        out = call.run()
        torch.cuda.synchronize()
        assert torch.equal(out, serial)
    assert_attn_close(out, restatement(wl), what="mixed, decode overlapped")


def test_prefix_extend_rows_equal_full_prefill(gpu):
    P, N = 300, 90
    full = small_case([P + N], [P + N], hq=24, hkv=4, d=256, seed=3, device=gpu,
                      dtype=torch.bfloat16)
    ref = run(full)
    ext = rebatch(full, [P + N], [N], full.q[P:].clone())
    got = run(ext)
    # Same math on the same rows: only the tiling of the key loop may differ.
    assert_attn_close(got, ref[P:], atol=4e-3, rtol=4e-3, norm_rel=4e-3, what="prefix==full")


def test_fp8_kv_extend(gpu):
    wl = workloads.build("fp8x", [40, 300, 9], [40, 100, 1], num_q_heads=24, num_kv_heads=4,
                         head_dim=256, pool_slots=512, device=gpu, seed=41, kv_fp8=True)
    check(wl, "fp8 extend")


def test_full_size_extend_prefix_sampled(gpu):
    """16 requests, 4 radix groups, P in [0, 4k], N in [512, 2k] at full size; two
    requests are re-checked against the oracle on a sub-batch."""
    wl = workloads.extend_prefix(device=gpu)
    out = run(wl)
    torch.cuda.synchronize()
    assert torch.isfinite(out.float()).all()
    starts = np.cumsum([0] + wl.ext_lens)
    # The two cheapest requests for the CPU oracle, one per prefix group if possible.
    pick = sorted(range(len(wl.seq_lens)), key=lambda i: wl.seq_lens[i] * wl.ext_lens[i])[:2]
    sub = rebatch(wl, [wl.seq_lens[i] for i in pick], [wl.ext_lens[i] for i in pick],
                  torch.cat([wl.q[starts[i]:starts[i + 1]] for i in pick]),
                  rows=[wl.rows[i] for i in pick])
    want = torch.cat([out[starts[i]:starts[i + 1]] for i in pick])
    assert_attn_close(want, restatement(sub), what="extend full-size sample")


@pytest.mark.parametrize("fp8", [False, True])
def test_negative_slot_entries_bsz1(gpu, fp8):
    """bsz == 1 extend over a row with -1 entries reads the pool's last slot
    there (full_attention.py:188-190), as the oracle does."""
    wl = workloads.build("neg", [400], [120], num_q_heads=24, num_kv_heads=4, head_dim=256,
                         pool_slots=1024, device=gpu, seed=44, kv_fp8=fp8)
    wl.batch.req_to_token[wl.rows[0], [0, 150, 300]] = -1
    check(wl, "-1 entries, bsz=1" + (", fp8" if fp8 else ""))
