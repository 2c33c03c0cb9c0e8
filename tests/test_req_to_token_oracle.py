"""Pins of the req_to_token oracle and the host half of DeviceReqToTokenTable (CPU)."""
import numpy as np
import pytest
import torch

from oracle.req_to_token import HostReqToTokenPool, apply_sync_arrays, host_loop_sync
from tests.rtt_schedule import Schedule
from tokenfactory_amd.req_to_token import DeviceReqToTokenTable


def test_dirty_from_follows_rewrites():
    """tests/test_hybrid_radix_cache.py:636-643 of the reference."""
    pool = HostReqToTokenPool(max_reqs=4, max_context_len=8)
    r0 = pool.alloc_req()
    assert r0 is not None and pool.dirty_from[r0] == 0
    pool.write(r0, 0, [1, 2, 3])
    assert pool.dirty_from[r0] == 0
    pool.dirty_from[r0] = 3
    pool.write(r0, 0, [10, 11])
    assert pool.dirty_from[r0] == 0
    assert pool.get_req_slots(r0, 4) == [10, 11, 3, -1]
    pool.dirty_from[r0] = 3
    pool.write(r0, 5, [])          # an empty write moves nothing
    assert pool.dirty_from[r0] == 3
    pool.free_req(r0)
    assert pool.get_req_slots(r0, 8) == [-1] * 8 and pool.alloc_req() == r0


def _dedupe_scenario(sync):
    """tests/test_hybrid_radix_cache.py:696-711 reduced to its table operations:
    r2 computes its first chunk [0:3] into its own slots, the dedupe then points
    [0:3] at r1's slots, and the sync of r2's second chunk must carry the
    rewritten head to the device."""
    pool = HostReqToTokenPool(max_reqs=4, max_context_len=16)
    table = torch.full((4, 16), -1, dtype=torch.long)
    synced = [0] * 4
    r1, r2 = pool.alloc_req(), pool.alloc_req()
    pool.write(r1, 0, [1, 2, 3])
    sync(table, synced, [r1], [0], [3], [1, 2, 3], pool.req_to_token, pool.dirty_from)
    pool.write(r1, 3, [4, 5, 6])
    sync(table, synced, [r1], [3], [6], [4, 5, 6], pool.req_to_token, pool.dirty_from)
    pool.write(r2, 0, [7, 8, 9])
    sync(table, synced, [r2], [0], [3], [7, 8, 9], pool.req_to_token, pool.dirty_from)
    pool.write(r2, 0, [1, 2, 3])                     # dedupe onto r1's slots
    assert pool.dirty_from[r2] == 0
    pool.write(r2, 3, [10, 11, 12])
    sync(table, synced, [r2], [3], [6], [10, 11, 12], pool.req_to_token, pool.dirty_from)
    return table[r2, :3].tolist() == pool.req_to_token[r2][:3], table, pool, r2


def test_dedupe_resync_reaches_the_device():
    ok, table, pool, r2 = _dedupe_scenario(host_loop_sync)
    assert ok
    assert table[r2, :6].tolist() == [1, 2, 3, 10, 11, 12]


def test_dedupe_scenario_rejects_a_sync_that_ignores_dirty_from():
    def mutant(table, synced, rows, prefix, seq, loc, host, dirty_from):
        host_loop_sync(table, synced, rows, prefix, seq, loc, host, None)
    ok, _, _, _ = _dedupe_scenario(mutant)
    assert not ok


def test_plan_applied_by_the_kernel_contract_matches_the_host_loop():
    """DeviceReqToTokenTable.plan + the tf_req_to_token_sync contract reproduce
    the reference loop step by step (table, cursors and dirty_from), and the
    loop keeps every batch row equal to the host row up to its length."""
    for seed in range(6):
        max_reqs, max_ctx = 9, 160
        sched = Schedule(seed, max_reqs, max_ctx, max_batch=6)
        ref = torch.full((max_reqs, max_ctx), -1, dtype=torch.long)
        ref_synced = [0] * max_reqs
        dev = DeviceReqToTokenTable(max_reqs, max_ctx, device="cpu")
        mine = np.full((max_reqs, max_ctx), -1, dtype=np.int64)

        def reset(r):
            ref_synced[r] = 0
            dev.reset_req(r)

        def invalidate(r, pos):
            if pos < ref_synced[r]:
                ref_synced[r] = pos
            dev.invalidate(r, pos)

        n_patched = 0
        for _ in range(40):
            sched.admit(reset)
            rows, prefix, seq, loc = sched.step()
            df = list(sched.pool.dirty_from)
            staged = dev.plan(rows, prefix, seq, sched.pool.req_to_token, df)
            b = len(rows)
            n_patched += staged.size - 5 * b
            apply_sync_arrays(mine, staged[:b], staged[b:2 * b], staged[2 * b:3 * b], loc,
                              staged[3 * b:4 * b], staged[4 * b:5 * b], staged[5 * b:])
            host_loop_sync(ref, ref_synced, rows, prefix, seq, loc, sched.pool.req_to_token,
                           sched.pool.dirty_from)
            assert np.array_equal(mine, ref.numpy())
            assert df == sched.pool.dirty_from and dev.synced_lens == ref_synced
            for r, s in zip(rows, seq):
                assert ref[r, :s].tolist() == sched.pool.req_to_token[r][:s]
            sched.between_steps(invalidate)
        assert n_patched > 0


def test_kernel_contract_rules_for_out_of_range_entries():
    t = np.full((3, 6), -1, dtype=np.int64)
    rows = [0, 5, 1, 2, 2]
    prefix = [1, 0, 4, 3, 0]
    seq = [3, 2, 2, 7, 0]
    apply_sync_arrays(t, rows, prefix, seq, [10, 11, 12, 13], [0, 0, 0, 0, 0],
                      [0, 0, 0, 0, 0], [99])
    # row 0: patch [0,1) from patch_vals, new [1,3) from loc[0:2]; row 5 is not a
    # row, prefix 4 > seq 2 and seq 7 > 6 write nothing and take no entries;
    # the empty last request takes none either.
    assert t[0].tolist() == [99, 10, 11, -1, -1, -1]
    assert (t[1:] == -1).all()
    t = np.full((2, 6), -1, dtype=np.int64)
    apply_sync_arrays(t, [0, 1], [2, 0], [4, 3], [5, 6, 7], [0, 0], [1, 0], [1, 2])
    # row 0's patch run [0,2) needs patch_vals[1:3], past the end: dropped;
    # row 1 gets the one remaining out_cache_loc entry.
    assert t[0].tolist() == [-1, -1, 5, 6, -1, -1]
    assert t[1].tolist() == [7, -1, -1, -1, -1, -1]


def test_plan_rejects_duplicate_rows_and_bad_ranges():
    dev = DeviceReqToTokenTable(4, 8, device="cpu")
    host = [[-1] * 8 for _ in range(4)]
    with pytest.raises(ValueError):
        dev.plan([1, 1], [0, 0], [1, 1], host)
    with pytest.raises(ValueError):
        dev.plan([0], [3], [9], host)
    with pytest.raises(NotImplementedError):
        dev.plan(list(range(4097)), [0] * 4097, [0] * 4097, host)


def test_rejected_batch_moves_no_cursor():
    """A batch rejected anywhere (a later request out of range, or an
    out_cache_loc that does not hold one slot per new position) leaves every
    request's sync cursor and dirty_from mark where they were, so the next
    sync still rewrites what the rejected one would have."""
    dev = DeviceReqToTokenTable(4, 8, device="cpu")
    host = [[10 * r + i for i in range(8)] for r in range(4)]
    dev.plan([2], [0], [3], host)
    before = list(dev.synced_lens)
    df = [1, 1, 1, 1]
    with pytest.raises(ValueError):
        dev.plan([0, 3], [2, 5], [4, 9], host, df)      # row 3's [5, 9) leaves the table
    assert dev.synced_lens == before and df == [1, 1, 1, 1]
    loc = torch.arange(4, dtype=torch.long)               # 2 + 3 new positions need 5
    with pytest.raises(ValueError, match="out_cache_loc"):
        dev.sync([0, 2], [2, 3], [4, 6], loc, host, df)
    assert dev.synced_lens == before and df == [1, 1, 1, 1]
