"""Device req_to_token sync (tf_req_to_token_sync / DeviceReqToTokenTable).

Every check is bit-exact: after each step of a random serving schedule the
whole device table equals the CPU table kept by the reference's host loop
(engine/model_runner.py:147-167, restated in oracle/req_to_token.py); a sync
captured in a HIP graph and replayed over refilled arrays equals the kernel
contract on each replay; malformed entries write only what the contract
allows.
"""
import numpy as np
import pytest
import torch

from oracle.req_to_token import apply_sync_arrays, host_loop_sync
from tests.rtt_schedule import Schedule
from tokenfactory_amd.req_to_token import DeviceReqToTokenTable

pytestmark = pytest.mark.gpu


def _i64(x, dev):
    return torch.tensor(np.asarray(x, dtype=np.int64), dtype=torch.long, device=dev)


@pytest.mark.parametrize("seed", [0, 1, 2])
def test_schedule_matches_the_host_loop(gpu, seed):
    max_reqs, max_ctx = 16, 700
    sched = Schedule(seed, max_reqs, max_ctx, max_batch=12)
    ref = torch.full((max_reqs, max_ctx), -1, dtype=torch.long)
    ref_synced = [0] * max_reqs
    table = DeviceReqToTokenTable(max_reqs, max_ctx, device=gpu)

    def reset(r):
        ref_synced[r] = 0
        table.reset_req(r)

    def invalidate(r, pos):
        if pos < ref_synced[r]:
            ref_synced[r] = pos
        table.invalidate(r, pos)

    for step in range(40):
        sched.admit(reset)
        rows, prefix, seq, loc = sched.step()
        df = list(sched.pool.dirty_from)
        got_rows, got_prefix, got_seq = table.sync(rows, prefix, seq, _i64(loc, gpu),
                                                   sched.pool.req_to_token, df)
        host_loop_sync(ref, ref_synced, rows, prefix, seq, loc, sched.pool.req_to_token,
                       sched.pool.dirty_from)
        torch.cuda.synchronize()
        print(f"[rtt] seed {seed} step {step}: batch {len(rows)}", flush=True)
        assert torch.equal(table.tensor.cpu(), ref), f"step {step}: tables differ"
        assert got_rows.cpu().tolist() == rows and got_prefix.cpu().tolist() == prefix
        assert got_seq.cpu().tolist() == seq
        assert df == sched.pool.dirty_from and table.synced_lens == ref_synced
        sched.between_steps(invalidate)


def test_sync_from_device_replays_in_a_graph(gpu):
    """Decode steps of 8 requests: the arrays the graph reads are refilled
    between replays (eager work and synchronisation in between)."""
    max_reqs, max_ctx, b = 12, 64, 8
    table = DeviceReqToTokenTable(max_reqs, max_ctx, device=gpu)
    want = np.full((max_reqs, max_ctx), -1, dtype=np.int64)
    rng = np.random.default_rng(5)

    def batch():
        rows = rng.permutation(max_reqs)[:b]
        seq = rng.integers(1, max_ctx + 1, size=b)
        prefix = seq - 1
        loc = rng.integers(0, 1 << 40, size=b)
        return rows, prefix, seq, loc

    live = [torch.zeros(b, dtype=torch.long, device=gpu) for _ in range(4)]

    def fill(arrs):
        for t, x in zip(live, arrs):
            t.copy_(_i64(x, gpu))

    fill(batch())
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        table.sync_from_device(*live)       # warm-up outside the capture
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    table.tensor.fill_(-1)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        table.sync_from_device(*live)
    torch.cuda.synchronize()
    table.tensor.fill_(-1)
    for r in range(5):
        arrs = batch()
        fill(arrs)
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        apply_sync_arrays(want, *arrs)
        scratch = torch.randn(1024, device=gpu).sum()    # eager work between replays
        torch.cuda.synchronize()
        assert torch.isfinite(scratch)
        print(f"[rtt] replay {r}", flush=True)
        assert np.array_equal(table.tensor.cpu().numpy(), want), f"replay {r} differs"


@pytest.mark.parametrize("with_patches", [False, True])
def test_malformed_entries_follow_the_contract(gpu, with_patches):
    rows_n, cols = 6, 40
    rng = np.random.default_rng(17 + with_patches)
    for trial in range(6):
        b = int(rng.integers(1, 9))
        rows = rng.integers(-2, rows_n + 2, size=b)
        seq = rng.integers(-3, cols + 6, size=b)
        prefix = seq - rng.integers(-4, 12, size=b)
        n_loc = int(rng.integers(0, 30))
        loc = rng.integers(0, 1000, size=n_loc)
        args = [rows, prefix, seq, loc]
        if with_patches:
            pfrom = prefix - rng.integers(-3, 10, size=b)
            n_p = int(rng.integers(0, 25))
            poff = rng.integers(-2, n_p + 3, size=b)
            pvals = rng.integers(2000, 3000, size=n_p)
            args += [pfrom, poff, pvals]
        table = DeviceReqToTokenTable(rows_n, cols, device=gpu)
        want = np.full((rows_n, cols), -1, dtype=np.int64)
        apply_sync_arrays(want, *args)
        dev = [_i64(x, gpu) for x in args]
        if with_patches:
            table._launch(dev[0], dev[1], dev[2], dev[3], dev[4], dev[5], dev[6], len(pvals))
        else:
            table._launch(dev[0], dev[1], dev[2], dev[3], None, None, None, 0)
        torch.cuda.synchronize()
        print(f"[rtt] malformed trial {trial} (patches={with_patches}, b={b})", flush=True)
        assert np.array_equal(table.tensor.cpu().numpy(), want), f"trial {trial}"


@pytest.mark.parametrize("num_workgroups", [0, 1, 300])
def test_full_batch_and_long_rows(gpu, num_workgroups):
    """4096 requests in one call, and one request that writes 250k new positions
    after a 40k-position rewritten prefix, over several workgroup counts."""
    rng = np.random.default_rng(3)
    b, cols = 4096, 48
    table = DeviceReqToTokenTable(b, cols, device=gpu)
    rows = rng.permutation(b)
    seq = rng.integers(0, cols + 1, size=b)
    prefix = np.minimum(seq, rng.integers(0, cols + 1, size=b))
    loc = rng.integers(0, 1 << 50, size=int((seq - prefix).sum()))
    want = np.full((b, cols), -1, dtype=np.int64)
    apply_sync_arrays(want, rows, prefix, seq, loc)
    table.sync_from_device(*[_i64(x, gpu) for x in (rows, prefix, seq, loc)],
                           num_workgroups=num_workgroups)
    torch.cuda.synchronize()
    print(f"[rtt] 4096 requests, {num_workgroups} workgroups", flush=True)
    assert np.array_equal(table.tensor.cpu().numpy(), want)

    long_ctx = 300_000
    table = DeviceReqToTokenTable(3, long_ctx, device=gpu)
    host = [[-1] * long_ctx for _ in range(3)]
    host[1][:40_000] = rng.integers(0, 1 << 40, size=40_000).tolist()
    table.synced_lens[1] = 40_000
    df = [0, 0, 0]                          # the whole head of row 1 was rewritten
    new = rng.integers(0, 1 << 40, size=250_000)
    staged = table.plan([1], [40_000], [290_000], host, df)
    want = np.full((3, long_ctx), -1, dtype=np.int64)
    apply_sync_arrays(want, staged[:1], staged[1:2], staged[2:3], new, staged[3:4],
                      staged[4:5], staged[5:])
    table.synced_lens[1] = 40_000
    table.sync([1], [40_000], [290_000], _i64(new, gpu), host, [0, 0, 0])
    torch.cuda.synchronize()
    got = table.tensor.cpu().numpy()
    assert np.array_equal(got, want)
    assert got[1, :40_000].tolist() == host[1][:40_000]


def test_rejects_more_than_4096_requests(gpu):
    table = DeviceReqToTokenTable(2, 8, device=gpu)
    z = torch.zeros(4097, dtype=torch.long, device=gpu)
    with pytest.raises(NotImplementedError):
        table.sync_from_device(z, z, z, z)
