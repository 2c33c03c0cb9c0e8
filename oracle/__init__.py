"""CPU oracle for the slot-indirected full-attention path.

TEST INFRASTRUCTURE ONLY. Nothing in ``tokenfactory_amd`` imports this package:
only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` use it, and only as the checker (or, for the CPU baseline, as the
timed restatement of the reference's CPU path), never as the product.

Modules
-------
``slot_attention``
    Op-for-op PyTorch restatement of ``Qwen3_8FullAttention._slot_based_attention``
    (reference ``qwen3_8/full_attention.py:163-283``) and of the KV scatter-write
    (``full_attention.py:146-149``). Runs in fp32 on the CPU.
``brute``
    Independent float64 NumPy loop oracle of the same attention semantics
    (explicit per request / per query / per head softmax over the visible keys).
``kv_quant``
    fp8-e4m3fn per-tensor quantisation of KV rows and its exact dequantisation.
``gdn``
    The Gated DeltaNet layer: decode step, chunked WY prefill, causal conv and
    gated RMSNorm of ``qwen3_8/linear_attention.py`` / ``rms_norm_gated.py``.
``fp8_linear``
    The block-FP8 linear (o_proj): dynamic activation quantisation and the
    block-scaled GEMM of ``qwen3_8/fp8_triton.py:17-98, 127-130``.

Pinning (what fixes each function independently of retyping it; see
``tests/test_oracle_pins.py``):

* slot gather: closed form ``pool[req_to_token[r, :L]]`` checked against
  explicit per-element loops and the ``-1 -> slot 0`` clamp convention;
* masks / GQA map / scale: closed-form special cases (single key returns V,
  equal keys return the mean of the visible V rows, a dominant key returns its V
  row), the MHA-expansion identity for GQA, permutation invariance over
  physical slot placement, cached-prefix extend equals rows of a full prefill,
  chunked extend equals one-shot extend, decode equals the last prefill row;
* the restatement and the brute-force oracle agree to fp32 rounding on random
  inputs for all three branches;
* planted mistakes (wrong GQA map, off-by-one causal mask, missing scale,
  unclamped padding) each fail at least one pin.
"""
