"""Two tensor-parallel rank shares of ``FullAttention`` run from two Python
threads at the same time on one GPU.

The reference runs its ranks' forward passes from Python threads
(``tests/test_tensor_parallel.py:93-271``): heads are sharded per rank
(``full_attention.py:44-52``) and each rank's pool holds its own kv heads
(``hybrid_cache_pool.py:48``).  Here the two rank shares (12 q / 2 kv heads of
a 24 / 4 layer) share one GPU, each on its own stream and pool, and read the
same ``ForwardBatch`` (a mixed step: extends over prefixes and decodes).

Checks:
* reentrancy: each rank's attention output and o_proj partial are bit-identical
  whether the ranks run one after the other or concurrently, over repeated
  concurrent runs;
* the K / V rows each rank writes equal the TP = 1 pool's heads bit for bit,
  and the attention rows of the extend requests equal the matching heads of a
  TP = 1 call bit for bit: the same kernels see the same rows (inputs and
  weights on a 2^-4 grid make the projections exact in any summation order);
* decode rows within one bf16 ulp of TP = 1: the split-K decode kernel spreads
  a step's key tiles over its grid by the step's total work, which halves with
  the heads, so a request's tiles may be merged in a different order;
* the sum of the two ranks' o_proj partials equals the TP = 1 output within the
  module tolerance (the all-reduce itself is outside this path).
"""
import threading
from types import SimpleNamespace

import pytest
import torch

from tests.helpers import assert_attn_close
from tokenfactory_amd import full_attention as fa
from tokenfactory_amd import workloads
from tokenfactory_amd.full_attention import FullAttention

pytestmark = pytest.mark.gpu

HQ, HKV, D, HIDDEN, TP = 24, 4, 256, 256, 2
SEQ = [700, 40, 300, 1500, 90, 2]
EXT = [200, 1, 60, 1, 90, 1]


def config(tp):
    return SimpleNamespace(hidden_size=HIDDEN, num_attention_heads=HQ, num_key_value_heads=HKV,
                           head_dim=D, tp_size=tp, attn_output_gate=True, attention_bias=False,
                           rms_norm_eps=1e-6, partial_rotary_factor=0.25, rope_theta=1e7,
                           mrope_section=None, mrope_interleaved=True)


def grid(shape, lo, hi, gen, device):
    """bf16 values k / 16 for integer k in [lo, hi]."""
    k = torch.randint(lo, hi + 1, shape, generator=gen, device=device)
    return (k.float() / 16).to(torch.bfloat16)


class Pool:
    def __init__(self, k, v):
        self.k, self.v = k, v

    def get_full_kv_buffers(self, layer_idx):
        return self.k, self.v


def rank_module(full, r, device):
    """Rank r's share of ``full``: q heads [12 r, 12 r + 12) (with their gate
    rows), kv heads [2 r, 2 r + 2), and the matching o_proj input columns."""
    m = FullAttention(config(TP), layer_idx=0, dtype=torch.bfloat16).to(device)
    hq, hk = HQ // TP, HKV // TP
    with torch.no_grad():
        m.q_proj.weight.copy_(full.q_proj.weight[r * hq * 2 * D:(r + 1) * hq * 2 * D])
        m.k_proj.weight.copy_(full.k_proj.weight[r * hk * D:(r + 1) * hk * D])
        m.v_proj.weight.copy_(full.v_proj.weight[r * hk * D:(r + 1) * hk * D])
        m.o_proj.weight.copy_(full.o_proj.weight[:, r * hq * D:(r + 1) * hq * D])
        m.q_norm.weight.copy_(full.q_norm.weight)
        m.k_norm.weight.copy_(full.k_norm.weight)
    return m


def ulp_diff(a, b):
    """Largest distance in bf16 units in the last place (same-sign ordering)."""
    def key(x):
        i = x.contiguous().view(torch.int16).to(torch.int32)
        return torch.where(i < 0, -32768 - i, i)
    return int((key(a) - key(b)).abs().max())


def test_rank_shares_from_two_threads(gpu, monkeypatch):
    gen = torch.Generator(device=gpu)
    gen.manual_seed(31)
    wl = workloads.build("tp_threads", SEQ, EXT, num_q_heads=HQ, num_kv_heads=HKV, head_dim=D,
                         pool_slots=2 * sum(SEQ) + 64, device=gpu, seed=31)
    batch = wl.batch
    n_tok = sum(EXT)
    hidden = grid((n_tok, HIDDEN), -8, 8, gen, gpu)
    positions = torch.cat([torch.arange(s - e, s) for s, e in zip(SEQ, EXT)]).to(gpu)

    full = FullAttention(config(1), layer_idx=0, dtype=torch.bfloat16).to(gpu)
    with torch.no_grad():
        for lin in (full.q_proj, full.k_proj, full.v_proj, full.o_proj):
            lin.weight.copy_(grid(lin.weight.shape, -4, 4, gen, gpu))
        full.q_norm.weight.copy_(grid((D,), 8, 24, gen, gpu))
        full.k_norm.weight.copy_(grid((D,), 8, 24, gen, gpu))
    ranks = [rank_module(full, r, gpu) for r in range(TP)]

    captured = {}
    inner = fa.slot_based_attention

    def spy(q, kb, vb, fb, **kw):
        out = inner(q, kb, vb, fb, **kw)
        captured[threading.get_ident()] = out.clone()
        return out

    monkeypatch.setattr(fa, "slot_based_attention", spy)

    def rank_pool(r):
        hk = HKV // TP
        cut = slice(r * hk, (r + 1) * hk)
        return Pool(wl.k_pool[:, cut].clone(memory_format=torch.contiguous_format),
                    wl.v_pool[:, cut].clone(memory_format=torch.contiguous_format))

    print(f"[tp threads] TP=1 reference step, ext={EXT} L={SEQ}", flush=True)
    pool1 = Pool(wl.k_pool.clone(), wl.v_pool.clone())
    with torch.no_grad():
        out1 = full(hidden, positions, pool1, batch)
    attn1 = captured.pop(threading.get_ident())
    torch.cuda.synchronize()

    streams = [torch.cuda.Stream(device=gpu) for _ in range(TP)]

    errors = []

    def run_rank(r, pool, results):
        try:
            with torch.cuda.stream(streams[r]), torch.no_grad():
                out = ranks[r](hidden, positions, pool, batch)
                results[r] = (captured.pop(threading.get_ident()), out)
            streams[r].synchronize()
        except Exception as e:   # re-raised on the main thread
            errors.append(e)

    print("[tp threads] ranks one after the other", flush=True)
    alone, pools = {}, [rank_pool(r) for r in range(TP)]
    torch.cuda.synchronize()   # the pools' copies, made on this thread's stream
    for r in range(TP):
        t = threading.Thread(target=run_rank, args=(r, pools[r], alone))
        t.start()
        t.join()
    if errors:
        raise errors[0]
    assert set(alone) == {0, 1}

    loc = batch.out_cache_loc
    hq, hk = HQ // TP, HKV // TP
    ext_rows = torch.tensor([e > 1 for e in EXT for _ in range(e)], device=gpu)
    for r in range(TP):
        attn, _ = alone[r]
        assert torch.equal(pools[r].k[loc], pool1.k[loc][:, r * hk:(r + 1) * hk])
        assert torch.equal(pools[r].v[loc], pool1.v[loc][:, r * hk:(r + 1) * hk])
        want = attn1[:, r * hq:(r + 1) * hq]
        assert torch.equal(attn[ext_rows], want[ext_rows]), f"rank {r}: extend rows differ"
        assert ulp_diff(attn[~ext_rows], want[~ext_rows]) <= 1, f"rank {r}: decode rows"
    assert_attn_close(sum(alone[r][1].float() for r in range(TP)), out1.float(),
                      atol=4e-2, rtol=2e-2, norm_rel=1e-2, what="sum of o_proj partials")

    for it in range(3):
        print(f"[tp threads] concurrent run {it}", flush=True)
        together, pools = {}, [rank_pool(r) for r in range(TP)]
        torch.cuda.synchronize()
        threads = [threading.Thread(target=run_rank, args=(r, pools[r], together))
                   for r in range(TP)]
        for t in threads:
            t.start()
        for t in threads:
            t.join()
        if errors:
            raise errors[0]
        assert set(together) == {0, 1}, "a rank thread failed"
        for r in range(TP):
            assert torch.equal(together[r][0], alone[r][0]), f"run {it} rank {r}: attention"
            assert torch.equal(together[r][1], alone[r][1]), f"run {it} rank {r}: o_proj partial"
