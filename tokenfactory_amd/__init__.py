"""MI355X (gfx950) full-attention hot path for tokenFactory's hybrid Qwen3.8 model.

Public surface (the reference's names and contracts, see each module):

* ``ForwardBatch``      - per-step batch metadata (``qwen3_8/forward_batch.py``)
* ``FullAttnKVPool``    - slot-indexed K/V pool, bf16 or fp8-e4m3 + scales
* ``FullAttention``     - module with the reference's ``forward`` /
  ``_slot_based_attention`` signatures
* ``slot_based_attention`` / ``write_kv`` / ``gather_kv`` /
  ``qk_norm_rope_kv_write`` - the kernels' Python entry points
* ``LinearAttention`` / ``gdn_decode_step`` - Gated DeltaNet decode step
  (``qwen3_8/linear_attention.py``)
* ``Fp8Linear`` / ``block_fp8_linear`` - block-FP8 linear (``qwen3_8/fp8_linear.py``,
  ``qwen3_8/fp8_triton.py``) on the gfx950 FP8 GEMM
"""
from .forward_batch import ForwardBatch
from .attention import gather_kv, qk_norm_rope_kv_write, slot_based_attention, write_kv
from .kv_pool import FullAttnKVPool
from .fp8_linear import Fp8Linear, block_fp8_linear
from .full_attention import FullAttention
from .linear_attention import LinearAttention, gdn_decode_step

__all__ = [
    "Fp8Linear",
    "ForwardBatch",
    "FullAttnKVPool",
    "FullAttention",
    "LinearAttention",
    "block_fp8_linear",
    "gdn_decode_step",
    "gather_kv",
    "qk_norm_rope_kv_write",
    "slot_based_attention",
    "write_kv",
]
