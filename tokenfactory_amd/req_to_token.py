"""Resident device ``req_to_token`` table kept in step with the host table.

The reference's ``ModelRunner`` keeps a ``[max_reqs, max_context_len]`` int64
device copy of the host ``ReqToTokenPool`` rows, filled with -1
(engine/model_runner.py:67-74), and brings it up to date each step with a loop
over the batch (:147-167): for each request it copies the prefix positions the
host rewrote since the last sync (one ``torch.tensor`` host-to-device copy per
request) and then its new ``out_cache_loc`` slice.  Its per-row sync cursor is
reset when a request's state is reset or restored (:86-95) and moved back by
``invalidate_req_synced_len`` (:97-100).

``DeviceReqToTokenTable`` keeps the same cursor rules on the host, but a step is
one host-to-device copy of a packed int64 staging array (the batch's row ids,
lengths and every rewritten prefix run) and one ``tf_req_to_token_sync`` kernel.
``sync_from_device`` launches the kernel alone from arrays that are already on
the device (a decode step whose ``ForwardBatch`` tensors hold them), which a
HIP graph can capture.
"""
from __future__ import annotations

from typing import List, Optional, Sequence, Tuple

import numpy as np
import torch

from . import _native

MAX_BATCH = 4096


class DeviceReqToTokenTable:
    def __init__(self, max_reqs: int, max_context_len: int, device="cuda"):
        if max_reqs < 1 or max_context_len < 1:
            raise ValueError(f"table {max_reqs} x {max_context_len}")
        self.max_reqs = max_reqs
        self.max_context_len = max_context_len
        self.tensor = torch.full((max_reqs, max_context_len), -1, dtype=torch.long,
                                 device=device)
        self.device = self.tensor.device
        self.synced_lens: List[int] = [0] * max_reqs

    # engine/model_runner.py:86-95 (reset_req_linear_state / restore_req_linear_state)
    def reset_req(self, req_idx: int) -> None:
        self.synced_lens[req_idx] = 0

    # engine/model_runner.py:97-100
    def invalidate(self, req_idx: int, pos: int = 0) -> None:
        if pos < self.synced_lens[req_idx]:
            self.synced_lens[req_idx] = pos

    def plan(self, req_pool_indices: Sequence[int], prefix_lens: Sequence[int],
             seq_lens: Sequence[int], host_table: Sequence[Sequence[int]],
             dirty_from: Optional[List[int]] = None) -> np.ndarray:
        """Host half of a sync step: the cursor rules of model_runner.py:150-166
        (rewritten positions start at min(synced_len, dirty_from); afterwards
        both cursors move to the request's length).  Returns the int64 staging
        array ``[rows | prefix | seq | patch_from | patch_offsets | patch_vals]``
        and updates ``synced_lens`` and ``dirty_from`` in place (only once the
        whole batch has been checked: a rejected batch moves no cursor)."""
        staged, rows, seqs = self._plan(req_pool_indices, prefix_lens, seq_lens, host_table,
                                        dirty_from)
        self.mark_synced(rows, seqs, dirty_from)
        return staged

    def _plan(self, req_pool_indices, prefix_lens, seq_lens, host_table, dirty_from):
        """``plan`` without the cursor updates: (staging array, rows, lengths)."""
        b = len(req_pool_indices)
        if not (len(prefix_lens) == len(seq_lens) == b):
            raise ValueError("req_pool_indices, prefix_lens and seq_lens differ in length")
        if b > MAX_BATCH:
            raise NotImplementedError(f"{b} requests in one sync (at most {MAX_BATCH})")
        if len(set(req_pool_indices)) != b:
            raise ValueError("a request row appears twice in one batch")
        head = np.empty(5 * b, dtype=np.int64)
        head[:b] = req_pool_indices
        head[b:2 * b] = prefix_lens
        head[2 * b:3 * b] = seq_lens
        runs = []
        n_patch = 0
        for i in range(b):
            r, start, seq = int(head[i]), int(head[b + i]), int(head[2 * b + i])
            if not (0 <= r < self.max_reqs and 0 <= start <= seq <= self.max_context_len):
                raise ValueError(f"request row {r}: positions [{start}, {seq}) outside the "
                                 f"{self.max_reqs} x {self.max_context_len} table")
            synced = self.synced_lens[r]
            if dirty_from is not None and dirty_from[r] < synced:
                synced = dirty_from[r]
            head[3 * b + i] = min(synced, start)
            head[4 * b + i] = n_patch
            if synced < start:
                run = np.asarray(host_table[r][synced:start], dtype=np.int64)
                if run.size != start - synced:
                    raise ValueError(f"host row {r} is shorter than position {start}")
                runs.append(run)
                n_patch += run.size
        staged = np.concatenate([head] + runs) if runs else head
        return staged, [int(r) for r in head[:b]], [int(v) for v in head[2 * b:3 * b]]

    def sync(self, req_pool_indices: Sequence[int], prefix_lens: Sequence[int],
             seq_lens: Sequence[int], out_cache_loc: torch.Tensor,
             host_table: Sequence[Sequence[int]], dirty_from: Optional[List[int]] = None,
             ) -> Tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
        """One step of model_runner.py:147-167 on the current stream.  Returns
        device int64 views of (req_pool_indices, prefix_lens, seq_lens), which
        the caller can hand to ``ForwardBatch`` instead of copying them again."""
        b = len(req_pool_indices)
        # Everything is checked before any cursor moves: the batch, then the
        # new tokens' slots (one per position in [prefix, seq) of each request,
        # in batch order, as model_runner.py:148-165 consumes them).
        staged, rows_h, seqs_h = self._plan(req_pool_indices, prefix_lens, seq_lens, host_table,
                                            dirty_from)
        self._check_tensor("out_cache_loc", out_cache_loc)
        n_new = int(sum(int(sq) - int(p) for p, sq in zip(prefix_lens, seq_lens)))
        if out_cache_loc.numel() != n_new:
            raise ValueError(f"out_cache_loc holds {out_cache_loc.numel()} slots for {n_new} "
                             f"new positions")
        if b == 0:
            empty = torch.empty(0, dtype=torch.long, device=self.device)
            return empty, empty, empty
        pinned = torch.empty(staged.size, dtype=torch.long, pin_memory=True)
        pinned.numpy()[:] = staged
        dev = pinned.to(self.device, non_blocking=True)
        rows, prefix, seq = dev[:b], dev[b:2 * b], dev[2 * b:3 * b]
        n_patch = staged.size - 5 * b
        self._launch(rows, prefix, seq, out_cache_loc,
                     dev[3 * b:4 * b], dev[4 * b:5 * b], dev[5 * b:], n_patch)
        self.mark_synced(rows_h, seqs_h, dirty_from)
        return rows, prefix, seq

    def sync_from_device(self, req_pool_indices: torch.Tensor, prefix_lens: torch.Tensor,
                         seq_lens: torch.Tensor, out_cache_loc: torch.Tensor,
                         num_workgroups: int = 0) -> None:
        """The kernel alone, from device int64 arrays, with no rewritten prefix
        runs (graph-capturable).  The caller keeps the cursors with
        ``mark_synced``."""
        self._launch(req_pool_indices, prefix_lens, seq_lens, out_cache_loc, None, None, None,
                     0, num_workgroups)

    def mark_synced(self, req_pool_indices: Sequence[int], seq_lens: Sequence[int],
                    dirty_from: Optional[List[int]] = None) -> None:
        for r, seq in zip(req_pool_indices, seq_lens):
            self.synced_lens[r] = seq
            if dirty_from is not None:
                dirty_from[r] = seq

    def _check_tensor(self, name: str, t: torch.Tensor) -> None:
        if t.dtype != torch.long or t.device != self.device or not t.is_contiguous():
            raise ValueError(f"{name} must be a contiguous int64 tensor on {self.device}")

    def _launch(self, rows, prefix, seq, loc, pfrom, poff, pvals, n_patch,
                num_workgroups: int = 0) -> None:
        b = rows.numel()
        for name, t in (("req_pool_indices", rows), ("prefix_lens", prefix),
                        ("seq_lens", seq), ("out_cache_loc", loc)):
            self._check_tensor(name, t)
        if prefix.numel() != b or seq.numel() != b:
            raise ValueError("req_pool_indices, prefix_lens and seq_lens differ in length")
        stream = torch.cuda.current_stream(self.device).cuda_stream
        _native.call("tf_req_to_token_sync", self.tensor.data_ptr(), self.max_reqs,
                     self.tensor.stride(0), self.max_context_len, rows.data_ptr(),
                     prefix.data_ptr(), seq.data_ptr(), loc.data_ptr() if loc.numel() else None,
                     loc.numel(), None if pfrom is None else pfrom.data_ptr(),
                     None if poff is None else poff.data_ptr(),
                     None if pvals is None or n_patch == 0 else pvals.data_ptr(), n_patch,
                     b, num_workgroups, stream)
