"""Loader for the module-level golden vectors (``tests/golden/module_golden.npz``,
written by ``tests/golden/make_module_golden.py`` from the reference's own
``Qwen3_8FullAttention`` in fp32)."""
from __future__ import annotations

import json
from pathlib import Path
from types import SimpleNamespace

import numpy as np
import torch

from tokenfactory_amd.forward_batch import ForwardBatch

PATH = Path(__file__).resolve().parent / "golden" / "module_golden.npz"
CASES = ("mixed", "decode", "single")


def load():
    d = np.load(PATH)          # allow_pickle stays False
    meta = json.loads(bytes(d["meta_json"]).decode())
    return d, meta


def bf16(a: np.ndarray) -> torch.Tensor:
    """uint16 bf16 bit patterns -> float32 tensor."""
    return torch.from_numpy(a.astype(np.int16)).view(torch.bfloat16).float()


def config(meta) -> SimpleNamespace:
    return SimpleNamespace(
        hidden_size=meta["hidden_size"], num_attention_heads=meta["num_attention_heads"],
        num_key_value_heads=meta["num_key_value_heads"], head_dim=meta["head_dim"],
        tp_size=1, attn_output_gate=meta["attn_output_gate"], attention_bias=False,
        rms_norm_eps=meta["rms_norm_eps"], partial_rotary_factor=meta["partial_rotary_factor"],
        rope_theta=meta["rope_theta"], mrope_section=meta["mrope_section"],
        mrope_interleaved=meta["mrope_interleaved"])


def load_weights(module, d) -> None:
    with torch.no_grad():
        for name in ("q_proj", "k_proj", "v_proj", "o_proj"):
            w = getattr(module, name).weight
            w.copy_(bf16(d[f"w_{name}"]).to(w.dtype))
        module.q_norm.weight.copy_(bf16(d["w_q_norm"]))
        module.k_norm.weight.copy_(bf16(d["w_k_norm"]))


def batch(d, meta, name, device) -> ForwardBatch:
    c = meta["cases"][name]
    return ForwardBatch(
        batch_size=len(c["req"]),
        req_pool_indices=torch.tensor(c["req"], dtype=torch.int64, device=device),
        seq_lens=torch.tensor(c["seq"], dtype=torch.int64, device=device),
        prefix_lens=torch.tensor([s - e for s, e in zip(c["seq"], c["ext"])], device=device),
        extend_lens=list(c["ext"]),
        out_cache_loc=torch.from_numpy(d[f"{name}_out_cache_loc"]).to(device),
        req_to_token=torch.from_numpy(d["req_to_token"]).to(device),
        is_prefill=max(c["ext"]) > 1)


def expected(d, name, what) -> torch.Tensor:
    return torch.from_numpy(d[f"{name}_{what}"].astype(np.float32))
