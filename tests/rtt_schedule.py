"""Random serving schedules over the host req_to_token table, for the sync tests.

A schedule admits requests (some reusing a cached prefix, as the radix cache
does), runs mixed steps of chunked prefill and decode, and between steps
rewrites prefix positions the way the scheduler's concurrent-prefix dedupe
does (ReqToTokenPool.write, which moves dirty_from back), rolls back a
rejected draft slot (write of -1 plus invalidate_req_synced_len,
engine/model_runner.py:309-315) and frees finished requests.  Each table
under test follows it through ``reset`` / ``invalidate`` callbacks and syncs
the batch ``step`` returns.
"""
from __future__ import annotations

import random
from typing import Callable, List, Tuple

from oracle.req_to_token import HostReqToTokenPool


class Schedule:
    def __init__(self, seed: int, max_reqs: int, max_context_len: int, max_batch: int = 12):
        self.rng = random.Random(seed)
        self.pool = HostReqToTokenPool(max_reqs, max_context_len)
        self.max_ctx = max_context_len
        self.max_batch = max_batch
        self.next_slot = 1
        self.active = {}          # row -> [computed length, target length]
        self.cached_prefix: List[int] = []

    def _slots(self, n: int) -> List[int]:
        out = list(range(self.next_slot, self.next_slot + n))
        self.next_slot += n
        return out

    def admit(self, reset: Callable[[int], None]) -> None:
        rng = self.rng
        while len(self.active) < self.max_batch and rng.random() < 0.6:
            r = self.pool.alloc_req()
            if r is None:
                return
            reset(r)
            target = rng.randint(2, self.max_ctx - 2)
            reuse = 0
            if self.cached_prefix and rng.random() < 0.5:
                reuse = min(rng.randint(1, len(self.cached_prefix)), target - 1)
                self.pool.write(r, 0, self.cached_prefix[:reuse])
            self.active[r] = [reuse, target]

    def step(self) -> Tuple[List[int], List[int], List[int], List[int]]:
        """Writes this step's new slots into the host table and returns the
        batch (rows, prefix_lens, seq_lens, flattened out_cache_loc)."""
        rows, prefix, seq, loc = [], [], [], []
        for r, (done, target) in self.active.items():
            if done < target:
                n = min(self.rng.randint(1, 48), target - done)
            elif done < self.max_ctx:
                n = 1
            else:
                continue
            slots = self._slots(n)
            self.pool.write(r, done, slots)
            rows.append(r)
            prefix.append(done)
            seq.append(done + n)
            loc.extend(slots)
            self.active[r][0] = done + n
        return rows, prefix, seq, loc

    def between_steps(self, invalidate: Callable[[int, int], None]) -> None:
        rng = self.rng
        for r in list(self.active):
            done, target = self.active[r]
            u = rng.random()
            if u < 0.15 and done > 1:
                # Concurrent-prefix dedupe: the head of the row now points at
                # slots another request computed.
                k = rng.randint(1, done)
                self.pool.write(r, 0, self._slots(k))
            elif u < 0.25 and done > 2:
                # Rejected draft: the last position goes back to -1.
                pos = done - 1
                self.pool.write(r, pos, [-1])
                invalidate(r, pos)
                self.active[r][0] = pos
            elif u < 0.35 and done >= target:
                self.cached_prefix = self.pool.get_req_slots(r, done)
                self.pool.free_req(r)
                del self.active[r]
