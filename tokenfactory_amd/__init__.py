"""MI355X (gfx950) full-attention hot path for tokenFactory's hybrid Qwen3.8 model.

Public surface (the reference's names and contracts, see each module):

* ``ForwardBatch``      - per-step batch metadata (``qwen3_8/forward_batch.py``)
* ``FullAttnKVPool``    - slot-indexed K/V pool, bf16 or fp8-e4m3 + scales
* ``FullAttention``     - module with the reference's ``forward`` /
  ``_slot_based_attention`` signatures
* ``slot_based_attention`` / ``write_kv`` / ``gather_kv`` /
  ``qk_norm_rope_kv_write`` - the kernels' Python entry points
"""
from .forward_batch import ForwardBatch
from .attention import gather_kv, qk_norm_rope_kv_write, slot_based_attention, write_kv
from .kv_pool import FullAttnKVPool
from .full_attention import FullAttention

__all__ = [
    "ForwardBatch",
    "FullAttnKVPool",
    "FullAttention",
    "gather_kv",
    "qk_norm_rope_kv_write",
    "slot_based_attention",
    "write_kv",
]
