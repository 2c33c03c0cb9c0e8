"""Device-side planning (tf_attn_plan_device) and a graph-captured step.

The device planner must produce exactly the host planners' lists
(tf_attn_plan_extend / tf_attn_plan_decode_items) followed by padding, and an
attention step planned on the device must equal the host-planned one bit for
bit (same work items, same kernels). A step captured once in a HIP graph is
replayed over batches with a different split of the same token count, with
eager work and synchronisation between replays; every replay must equal the
eager host-planned step on that batch.
"""
import numpy as np
import pytest
import torch

from tests.helpers import small_case
from tokenfactory_amd import _native, workloads
from tokenfactory_amd.attention import SlotAttentionCall
from tokenfactory_amd.planning import plan_decode_items, plan_extend

pytestmark = pytest.mark.gpu


def device_lists(call):
    torch.cuda.synchronize()
    m = call._meta.cpu().numpy()
    nw, nd = call.n_work, call.n_dec
    work = m[: nw * 8].reshape(nw, 8)
    items = m[nw * 8: nw * 8 + nd]
    rows = m[nw * 8 + nd: nw * 8 + 2 * nd]
    return work, items, rows, tuple(int(x) for x in m[nw * 8 + 2 * nd: nw * 8 + 2 * nd + 3])


@pytest.mark.parametrize("lens", [[1], [7], [3, 1, 700, 1, 22, 1, 1, 300],
                                  [2048] * 3 + [1] * 40 + [17, 513],
                                  [1] * 64, [5, 5, 5, 9, 9, 1, 5]])
def test_device_plan_matches_host_planner(gpu, lens):
    hq, hkv, d = 24, 4, 256
    wl = small_case([e + 3 for e in lens], lens, hq=hq, hkv=hkv, d=d, seed=len(lens),
                    device=gpu, dtype=torch.bfloat16)
    call = SlotAttentionCall(wl.q, wl.k_pool, wl.v_pool, wl.batch, scaling=wl.scale,
                             device_plan=True)
    call.run_plan()
    work, items, rows, (n_work, n_dec, flags) = device_lists(call)
    want = plan_extend(lens, hq, hkv, decode_to_decode_kernel=True)
    want_items, want_rows = plan_decode_items(lens)
    print(f"[plan] B={len(lens)} T={sum(lens)} work {n_work}/{call.n_work} decode {n_dec}",
          flush=True)
    assert flags == 0 and n_work == len(want) and n_dec == len(want_items)
    np.testing.assert_array_equal(work[:n_work], want)
    assert (work[n_work:] == 0).all()
    np.testing.assert_array_equal(items[:n_dec], want_items)
    np.testing.assert_array_equal(rows[:n_dec], want_rows)
    assert (items[n_dec:] == -1).all() and (rows[n_dec:] == 0).all()


def test_device_plan_flags_bad_lengths(gpu):
    wl = small_case([10, 20], [4, 6], hq=8, hkv=2, d=256, seed=1, device=gpu,
                    dtype=torch.bfloat16)
    call = SlotAttentionCall(wl.q, wl.k_pool, wl.v_pool, wl.batch, device_plan=True)
    wl.batch.extend_lens_tensor[1] = 0
    call.run_plan()
    assert device_lists(call)[3][2] & 2


@pytest.mark.parametrize("kind", ["mixed", "extend", "decode", "fp8"])
def test_device_planned_step_equals_host_planned(gpu, kind):
    if kind == "mixed":
        wl = workloads.mixed(device=gpu, n_extend=3, extend_new=140, prefix_hi=600, n_decode=9,
                             dec_lo=1, dec_hi=2200, pool_slots=1 << 15)
    elif kind == "extend":
        wl = small_case([400, 260, 90], [300, 60, 90], hq=24, hkv=4, d=256, seed=9,
                        device=gpu, dtype=torch.bfloat16)
    elif kind == "decode":
        wl = small_case([300, 2000, 47, 9], [1] * 4, hq=24, hkv=4, d=256, seed=10,
                        device=gpu, dtype=torch.bfloat16)
    else:
        wl = workloads.build("fp8p", [40, 300, 900], [40, 100, 1], num_q_heads=24,
                             num_kv_heads=4, head_dim=256, pool_slots=2048, device=gpu,
                             seed=44, kv_fp8=True)
    print(f"[plan] step {kind} ext={wl.ext_lens[:8]}", flush=True)
    kw = dict(scaling=wl.scale, k_scale=wl.k_scale, v_scale=wl.v_scale)
    host = SlotAttentionCall(wl.q, wl.k_pool, wl.v_pool, wl.batch, **kw).run().clone()
    dev = SlotAttentionCall(wl.q, wl.k_pool, wl.v_pool, wl.batch, device_plan=True, **kw).run()
    torch.cuda.synchronize()
    assert torch.equal(dev, host)


def _pair():
    """Two batches with the same request count, token count and tensor shapes
    but different extend / decode splits."""
    common = dict(hq=24, hkv=4, d=256, dtype=torch.bfloat16, pool=4096)
    a = dict(seq=[500, 300, 120, 41], ext=[200, 1, 60, 1], seed=21)
    b = dict(seq=[500, 90, 310, 7], ext=[1, 90, 170, 1], seed=22)
    return common, a, b


def _copy_into(dst, src):
    for x, y in ((dst.q, src.q), (dst.k_pool, src.k_pool), (dst.v_pool, src.v_pool),
                 (dst.batch.req_to_token, src.batch.req_to_token),
                 (dst.batch.seq_lens, src.batch.seq_lens),
                 (dst.batch.req_pool_indices, src.batch.req_pool_indices),
                 (dst.batch.extend_lens_tensor, src.batch.extend_lens_tensor)):
        assert x.shape == y.shape and x.dtype == y.dtype
        x.copy_(y)


def test_graph_captured_step_replays_over_changing_batches(gpu):
    common, a, b = _pair()
    mk = lambda c, dev: small_case(c["seq"], c["ext"], seed=c["seed"], device=dev, **common)
    live = mk(a, gpu)                      # the tensors the graph reads
    batches = [mk(a, gpu), mk(b, gpu), mk(a, gpu), mk(b, gpu)]
    call = SlotAttentionCall(live.q, live.k_pool, live.v_pool, live.batch, scaling=live.scale,
                             device_plan=True)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        call.run()                         # warm-up outside the capture
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        call.run()
    torch.cuda.synchronize()
    for r, wl in enumerate(batches):
        _copy_into(live, wl)
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        got = call.out.clone()
        # eager, host-planned, on the same batch, between replays
        want = SlotAttentionCall(wl.q, wl.k_pool, wl.v_pool, wl.batch, scaling=wl.scale).run()
        torch.cuda.synchronize()
        print(f"[plan] replay {r}: ext={wl.ext_lens}", flush=True)
        assert torch.equal(got, want), f"replay {r} differs from the eager step"
