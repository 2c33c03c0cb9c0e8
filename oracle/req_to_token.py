"""CPU restatement of the reference's req_to_token bookkeeping (test infrastructure).

Only the tests, the smoke check and the benchmark's CPU baseline use this
module; the product path never imports it.

* ``HostReqToTokenPool`` restates the host table ``ReqToTokenPool``
  (req_to_token_pool.py:10-48): rows of ``max_context_len`` slot ids, -1 for
  empty positions, and ``dirty_from``, the lowest position rewritten since the
  device copy of a row was last brought up to date.
* ``host_loop_sync`` restates the per-step incremental sync of the resident
  device table in the reference's ``ModelRunner._prepare_forward_batch``
  (engine/model_runner.py:147-167), on a CPU int64 tensor.
* ``apply_sync_arrays`` restates the contract of the C entry point
  ``tf_req_to_token_sync`` (one batch of flat int64 arrays, with its rules for
  out-of-range entries) in numpy.

Pins (tests/test_req_to_token_oracle.py): the reference's own unit test of
``dirty_from`` (tests/test_hybrid_radix_cache.py:626-643); its concurrent
prefix-dedupe scenario (:696-711), reduced to the table operations the
scheduler performs, with the assertion it makes; the invariant the sync exists
for (after a step, each batch row of the device table equals the host row up
to the request's length) over random multi-step schedules; and a planted
mutant (``dirty_from`` ignored) that the dedupe scenario rejects.
"""
from __future__ import annotations

from typing import List, Optional, Sequence

import numpy as np
import torch


class HostReqToTokenPool:
    """req_to_token_pool.py:10-48, same fields and rules."""

    def __init__(self, max_reqs: int, max_context_len: int):
        self.max_reqs = max_reqs
        self.max_context_len = max_context_len
        self.req_to_token: List[List[int]] = [[-1] * max_context_len for _ in range(max_reqs)]
        self.free_req_slots: List[int] = list(range(max_reqs - 1, -1, -1))
        self.dirty_from: List[int] = [0] * max_reqs

    def alloc_req(self) -> Optional[int]:          # :23-29
        if not self.free_req_slots:
            return None
        r = self.free_req_slots.pop()
        self.dirty_from[r] = 0
        return r

    def write(self, r: int, start: int, slots: Sequence[int]) -> None:   # :31-36
        if len(slots) and start < self.dirty_from[r]:
            self.dirty_from[r] = start
        row = self.req_to_token[r]
        for i, s in enumerate(slots):
            row[start + i] = int(s)

    def get_req_slots(self, r: int, seq_len: int) -> List[int]:       # :38-40
        return self.req_to_token[r][:seq_len]

    def free_req(self, r: int) -> None:              # :42-48
        self.req_to_token[r] = [-1] * self.max_context_len
        self.dirty_from[r] = 0
        self.free_req_slots.append(r)


def host_loop_sync(table: torch.Tensor, synced_lens: List[int], req_pool_indices: Sequence[int],
                   prefix_lens: Sequence[int], seq_lens: Sequence[int],
                   out_cache_loc: Sequence[int], host_table: Sequence[Sequence[int]],
                   dirty_from: Optional[List[int]] = None) -> None:
    """engine/model_runner.py:147-167 on a CPU int64 ``table``; updates
    ``synced_lens`` and ``dirty_from`` in place as the reference does."""
    loc = torch.as_tensor(np.asarray(out_cache_loc, dtype=np.int64))
    off = 0
    for r, start, seq in zip(req_pool_indices, prefix_lens, seq_lens):
        ext = seq - start
        synced = synced_lens[r]
        if dirty_from is not None and dirty_from[r] < synced:
            synced = dirty_from[r]
        if synced < start:
            table[r, synced:start] = torch.tensor(list(host_table[r][synced:start]),
                                                  dtype=torch.long)
        table[r, start:seq] = loc[off:off + ext]
        synced_lens[r] = seq
        if dirty_from is not None:
            dirty_from[r] = seq
        off += ext


def apply_sync_arrays(table: np.ndarray, req_pool_indices, prefix_lens, seq_lens,
                      out_cache_loc, patch_from=None, patch_offsets=None,
                      patch_vals=None) -> None:
    """The contract of ``tf_req_to_token_sync`` on a numpy int64 table [rows, cols]:
    request b writes ``table[r, patch_from:prefix]`` from ``patch_vals`` and
    ``table[r, prefix:seq]`` from the next ``seq - prefix`` entries of
    ``out_cache_loc``; a request with its row outside the table or not
    ``0 <= prefix <= seq <= cols`` writes nothing and takes no entries; a patch
    run outside ``[0, prefix)`` or past the end of ``patch_vals`` is dropped;
    entries past the end of ``out_cache_loc`` are not written."""
    rows, cols = table.shape
    loc = np.asarray(out_cache_loc, dtype=np.int64)
    pvals = None if patch_vals is None else np.asarray(patch_vals, dtype=np.int64)
    o = 0
    for b in range(len(req_pool_indices)):
        r, p, s = int(req_pool_indices[b]), int(prefix_lens[b]), int(seq_lens[b])
        if not (0 <= r < rows and 0 <= p <= s <= cols):
            continue
        if patch_from is not None:
            f, po = int(patch_from[b]), int(patch_offsets[b])
            n = p - f
            if 0 <= f < p and po >= 0 and pvals is not None and po + n <= pvals.size:
                table[r, f:p] = pvals[po:po + n]
        n_new = s - p
        take = loc[o:o + n_new]
        table[r, p:p + take.size] = take
        o += n_new
