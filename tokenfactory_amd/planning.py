"""Host-side work planning for the extend and mixed branches.

Thin wrappers over the library's C planners (``tf_attn_plan_extend`` /
``tf_attn_plan_decode_items``) that take the host-side ``ForwardBatch.extend_lens``
list, so a step never needs a device->host copy to schedule its kernels.
"""
from __future__ import annotations

from typing import Sequence, Tuple

import numpy as np

from . import _native

EXTEND_TILE_ROWS = 256   # (token, q-head) rows per extend work item
WORK_FIELDS = 8          # int32 fields per extend work item


def _lens_array(extend_lens: Sequence[int]) -> np.ndarray:
    arr = np.ascontiguousarray(np.asarray(extend_lens, dtype=np.int64))
    if arr.ndim != 1:
        raise ValueError("extend_lens must be one-dimensional")
    return arr


def plan_extend(extend_lens: Sequence[int], num_q_heads: int, num_kv_heads: int,
                decode_to_decode_kernel: bool) -> np.ndarray:
    """Extend work items ``[n, 8]`` int32: ``{b, kv_head, row0, q_start, ext, 0, 0, 0}``."""
    lens = _lens_array(extend_lens)
    lib = _native.load()
    ptr = lens.ctypes.data if lens.size else None
    n = _native.call("tf_attn_plan_extend", ptr, len(lens), num_q_heads, num_kv_heads,
                     int(bool(decode_to_decode_kernel)), None, 0)
    work = np.zeros((max(n, 1), WORK_FIELDS), dtype=np.int32)
    if n:
        got = _native.call("tf_attn_plan_extend", ptr, len(lens), num_q_heads, num_kv_heads,
                           int(bool(decode_to_decode_kernel)), work.ctypes.data, n)
        assert got == n
    del lib
    return work[:n]


def plan_decode_items(extend_lens: Sequence[int]) -> Tuple[np.ndarray, np.ndarray]:
    """Batch indices of the ``ext == 1`` requests and their rows in the flattened q."""
    lens = _lens_array(extend_lens)
    ptr = lens.ctypes.data if lens.size else None
    n = _native.call("tf_attn_plan_decode_items", ptr, len(lens), None, None, 0)
    items = np.zeros(max(n, 1), dtype=np.int32)
    rows = np.zeros(max(n, 1), dtype=np.int32)
    if n:
        _native.call("tf_attn_plan_decode_items", ptr, len(lens), items.ctypes.data,
                     rows.ctypes.data, n)
    return items[:n], rows[:n]
