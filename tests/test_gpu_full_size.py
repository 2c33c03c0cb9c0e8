"""The serving-step workloads at their full sizes, checked against the oracle.

The oracle is far too slow for a whole step, so each test runs the full step on
the GPU once and then checks

* sampled rows of that very output against the oracle (sub-batches that share
  the step's pools and ``req_to_token`` rows: ``rebatch`` / ``subset``), chosen
  to cover the expensive cases: the longest contexts, the rows with the most
  keys, the first rows after a prefix;
* every other row through batch-composition invariance: the same requests run
  in smaller batches (which the kernels tile and split differently) must give
  the same rows up to fp32 summation order (4e-3);
* where the step has a second launch shape (decode on a second stream), that
  it is bit-identical to the one-stream sequence.

Tolerances as everywhere: bf16 outputs within 2e-2 + 1e-2 |ref| elementwise and
a relative Frobenius error <= 1e-2 against an fp32 reference; fp8-KV outputs
against attention over the same dequantised KV with the same bounds.
"""
import numpy as np
import pytest
import torch

from tests.helpers import assert_attn_close, brute, rebatch, restatement, subset
from tokenfactory_amd import slot_based_attention, workloads
from tokenfactory_amd.attention import SlotAttentionCall

pytestmark = pytest.mark.gpu

INV = dict(atol=4e-3, rtol=4e-3, norm_rel=4e-3)   # same rows, other tiling / split


def run(wl, **kw):
    return slot_based_attention(wl.q, wl.k_pool, wl.v_pool, wl.batch, scaling=wl.scale,
                                k_scale=wl.k_scale, v_scale=wl.v_scale, **kw)


def rows_of(wl, i):
    starts = np.cumsum([0] + wl.ext_lens)
    return int(starts[i]), int(starts[i + 1])


def tail_rows(wl, i, n):
    """The last ``n`` query rows of request ``i`` as a one-request batch: its
    whole context, of which the last ``n`` positions are new."""
    a, b = rows_of(wl, i)
    return rebatch(wl, [wl.seq_lens[i]], [n], wl.q[b - n:b].clone(), rows=[wl.rows[i]])


def head_rows(wl, i, n):
    """The first ``n`` new rows of request ``i``: its prefix plus ``n`` tokens."""
    a, _ = rows_of(wl, i)
    prefix = wl.seq_lens[i] - wl.ext_lens[i]
    return rebatch(wl, [prefix + n], [n], wl.q[a:a + n].clone(), rows=[wl.rows[i]])


def test_full_size_mixed_step(gpu):
    """4 extends of 2048 tokens on U[0, 8k] prefixes + 128 decodes with contexts
    U[512, 16k] in a 2M-slot pool (KV byte offsets above 2^32), one step."""
    wl = workloads.mixed(device=gpu)
    ext_idx = [i for i, e in enumerate(wl.ext_lens) if e > 1]
    dec_idx = [i for i, e in enumerate(wl.ext_lens) if e == 1]
    print(f"[full mixed] prefixes={[wl.seq_lens[i] - wl.ext_lens[i] for i in ext_idx]} "
          f"decode L in [{min(wl.seq_lens[i] for i in dec_idx)}, "
          f"{max(wl.seq_lens[i] for i in dec_idx)}]", flush=True)
    serial = SlotAttentionCall(wl.q, wl.k_pool, wl.v_pool, wl.batch, scaling=wl.scale,
                               overlap_decode=False).run().clone()
    call = SlotAttentionCall(wl.q, wl.k_pool, wl.v_pool, wl.batch, scaling=wl.scale,
                             overlap_decode=True)
    for _ in range(2):
        call.out.zero_()
        out = call.run()
        torch.cuda.synchronize()
        assert torch.equal(out, serial), "decode on a second stream changed the result"
    assert torch.isfinite(out.float()).all()

    # Oracle: the two longest decode contexts (a batched decode sub-step).
    longest = sorted(dec_idx, key=lambda i: wl.seq_lens[i])[-2:]
    sub = subset(wl, longest)
    assert_attn_close(out[[rows_of(wl, i)[0] for i in longest]], restatement(sub),
                      what=f"mixed: decode rows L={[wl.seq_lens[i] for i in longest]}")
    # Oracle: the last 64 rows of the longest-prefix extend (the most keys) and the
    # first 64 rows of the shortest-prefix one (the causal diagonal from its start).
    far = max(ext_idx, key=lambda i: wl.seq_lens[i])
    near = min(ext_idx, key=lambda i: wl.seq_lens[i])
    _, b = rows_of(wl, far)
    assert_attn_close(out[b - 64:b], restatement(tail_rows(wl, far, 64)),
                      what=f"mixed: last rows, L={wl.seq_lens[far]}")
    a, _ = rows_of(wl, near)
    assert_attn_close(out[a:a + 64], restatement(head_rows(wl, near, 64)),
                      what=f"mixed: first rows, P={wl.seq_lens[near] - 2048}")

    # Every row: the extends alone and the decodes alone give the same rows.
    ext_only = run(subset(wl, ext_idx))
    dec_only = run(subset(wl, dec_idx))
    torch.cuda.synchronize()
    ext_rows = torch.cat([torch.arange(*rows_of(wl, i)) for i in ext_idx]).to(gpu)
    dec_rows = torch.tensor([rows_of(wl, i)[0] for i in dec_idx], device=gpu)
    assert_attn_close(out[ext_rows], ext_only, what="mixed: extend rows vs extend-only step",
                      **INV)
    assert_attn_close(out[dec_rows], dec_only, what="mixed: decode rows vs decode-only step",
                      **INV)


def test_full_size_fp8_128k_decode(gpu):
    """8 requests of 131072 tokens over an fp8-e4m3 pool with per-tensor scales:
    two requests against float64 attention over the dequantised KV (one request
    at a time: the op-for-op restatement would materialise ~6 GB of expanded K),
    and every row against the same requests decoded in smaller batches."""
    wl = workloads.decode_fp8_128k(device=gpu)
    print(f"[full fp8 128k] B={wl.batch.batch_size} L={wl.seq_lens[0]}", flush=True)
    out = run(wl)
    torch.cuda.synchronize()
    assert torch.isfinite(out.float()).all()
    for i in (0, 5):
        one = subset(wl, [i])
        want = torch.from_numpy(brute(one, dense=True)).float()
        assert_attn_close(out[i:i + 1], want, what=f"fp8 128k: request {i} vs dequantised KV")
    # The same rows from a 2-request and a 1-request batch (other split points;
    # the 1-request batch is the bsz == 1 branch).
    for idx in ([1, 6], [3]):
        assert_attn_close(out[idx], run(subset(wl, idx)), what=f"fp8 128k: rows {idx}", **INV)
    # A small fixed grid splits every unit over far fewer workgroups.
    assert_attn_close(run(wl, decode_workgroups=17), out, what="fp8 128k: 17 workgroups", **INV)


@pytest.mark.parametrize("seed,kv_fp8", [(13, False), (22, False), (13, True)],
                         ids=["seed13", "seed22", "seed13-fp8"])
def test_full_size_extend_prefix_heavy_rows(gpu, seed, kv_fp8):
    """16 requests in 4 radix groups (prefix U[0, 4k] shared per group, 512..2k new
    tokens): the last 64 rows of the two requests with the most keys and the
    first 64 rows of the one with the longest prefix against the oracle; every
    row against each prefix group run as its own batch.  Seed 13 draws long
    prefixes (mean 3.5k), seed 22 typical ones (mean 2.0k); the fp8 case reads
    an e4m3 pool and is checked against the oracle over the dequantised pool."""
    wl = workloads.extend_prefix(device=gpu, seed=seed, kv_fp8=kv_fp8)
    out = run(wl)
    torch.cuda.synchronize()
    assert torch.isfinite(out.float()).all()
    heavy = sorted(range(len(wl.seq_lens)), key=lambda i: wl.seq_lens[i])[-2:]
    for i in heavy:
        _, b = rows_of(wl, i)
        assert_attn_close(out[b - 64:b], restatement(tail_rows(wl, i, 64)),
                          what=f"extend_prefix: last rows of request {i}, L={wl.seq_lens[i]}")
    deep = max(range(len(wl.seq_lens)), key=lambda i: wl.seq_lens[i] - wl.ext_lens[i])
    a, _ = rows_of(wl, deep)
    assert_attn_close(out[a:a + 64], restatement(head_rows(wl, deep, 64)),
                      what=f"extend_prefix: first rows of request {deep}")
    groups = wl.meta["prefix_groups"]
    for g in sorted(set(groups)):
        idx = [i for i, gg in enumerate(groups) if gg == g]
        rows = torch.cat([torch.arange(*rows_of(wl, i)) for i in idx]).to(gpu)
        assert_attn_close(out[rows], run(subset(wl, idx)), what=f"extend_prefix: group {g}",
                          **INV)
