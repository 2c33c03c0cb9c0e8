"""Writes the module-level golden vectors (``module_golden.npz``).

Run in the build container, where the reference checkout is readable:

    python tests/golden/make_module_golden.py /root/reference

It imports the reference's ``Qwen3_8FullAttention`` (``qwen3_8/full_attention.py``)
on the CPU in fp32 with a mini configuration (hidden 32, 4 q / 2 kv heads,
head_dim 256, no fp8 quantisation), runs ``forward`` on three batches that
exercise its three attention branches, and stores inputs, weights and outputs.
Nothing else pins the module's composition (projections -> q/k RMSNorm ->
partial M-RoPE -> KV write -> attention -> silu gate -> o_proj), so these
vectors do. Weights, hidden states and the pre-filled pool are rounded to bf16
values first so that a bf16 implementation sees exactly the same inputs.
Only numbers are stored (``numpy.savez_compressed``, no pickles); outputs are
kept as float16.
"""
import json
import sys
from pathlib import Path

import numpy as np
import torch

OUT = Path(__file__).resolve().parent / "module_golden.npz"


def bf16_round(t):
    return t.to(torch.bfloat16).to(torch.float32)


def bits(t):
    return t.to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)


def main(ref_root: str) -> None:
    # The reference tree is read-only: importing it must not write bytecode there.
    sys.dont_write_bytecode = True
    sys.path.insert(0, ref_root)
    from qwen3_8.config import Qwen3_8Config
    from qwen3_8.forward_batch import ForwardBatch
    from qwen3_8.full_attention import Qwen3_8FullAttention

    torch.manual_seed(2026)
    cfg = Qwen3_8Config(hidden_size=32, num_hidden_layers=4,
                        layer_types=["linear_attention"] * 3 + ["full_attention"],
                        num_attention_heads=4, num_key_value_heads=2, head_dim=256,
                        quantization_config=None)
    layer = Qwen3_8FullAttention(cfg, layer_idx=3).float().eval()
    with torch.no_grad():
        for lin in (layer.q_proj, layer.k_proj, layer.v_proj, layer.o_proj):
            lin.weight.copy_(bf16_round(torch.randn_like(lin.weight) * lin.in_features ** -0.5))
        layer.q_norm.weight.copy_(bf16_round(1.0 + 0.3 * torch.randn(256)))
        layer.k_norm.weight.copy_(bf16_round(1.0 + 0.3 * torch.randn(256)))

    S, Hkv, D = 48, 2, 256
    k0 = bf16_round(torch.randn(S, Hkv, D))
    v0 = bf16_round(torch.randn(S, Hkv, D))
    k0[0] = 0
    v0[0] = 0

    class Pool:
        def __init__(self):
            self.k = k0.clone()
            self.v = v0.clone()

        def get_full_kv_buffers(self, layer_idx):
            return self.k, self.v

    captured = {}
    inner = layer._slot_based_attention

    def spy(q, kb, vb, batch):
        out = inner(q, kb, vb, batch)
        captured["q"] = q.detach().clone()
        captured["attn"] = out.detach().clone()
        return out

    layer._slot_based_attention = spy

    rtt = torch.full((4, 32), -1, dtype=torch.int64)
    # slots: request 0 owns 1..9, request 1 owns 10..15, request 2 shares
    # request 0's first 5 slots (a radix prefix) then 16..19; request 3 uses 20..
    rtt[0, :9] = torch.arange(1, 10)
    rtt[1, :6] = torch.arange(10, 16)
    rtt[2, :5] = torch.arange(1, 6)
    rtt[2, 5:9] = torch.arange(16, 20)
    rtt[3, :12] = torch.arange(20, 32)

    cases = {
        # mixed: r0 extends 4 tokens on a 5-token prefix, r1 prefills 6, r2 decodes 1
        "mixed": dict(req=[0, 1, 2], seq=[9, 6, 9], ext=[4, 6, 1], mrope=False),
        # pure decode with 3-D (M-RoPE) positions
        "decode": dict(req=[0, 2, 3], seq=[9, 9, 12], ext=[1, 1, 1], mrope=True),
        # bsz == 1 extend over a cached prefix
        "single": dict(req=[3], seq=[12], ext=[7], mrope=False),
    }
    data = {"k_pool0": bits(k0), "v_pool0": bits(v0), "req_to_token": rtt.numpy()}
    for name in ("q_proj", "k_proj", "v_proj", "o_proj"):
        data[f"w_{name}"] = bits(getattr(layer, name).weight.detach())
    data["w_q_norm"] = bits(layer.q_norm.weight.detach())
    data["w_k_norm"] = bits(layer.k_norm.weight.detach())
    meta = {"hidden_size": 32, "num_attention_heads": 4, "num_key_value_heads": 2,
            "head_dim": 256, "rms_norm_eps": cfg.rms_norm_eps,
            "partial_rotary_factor": cfg.partial_rotary_factor, "rope_theta": cfg.rope_theta,
            "mrope_section": cfg.mrope_section, "mrope_interleaved": cfg.mrope_interleaved,
            "attn_output_gate": cfg.attn_output_gate, "pool_slots": S, "cases": {}}
    for name, c in cases.items():
        pool = Pool()
        T = sum(c["ext"])
        hidden = bf16_round(torch.randn(T, 32))
        loc, pos = [], []
        for r, L, e in zip(c["req"], c["seq"], c["ext"]):
            loc += rtt[r, L - e:L].tolist()
            pos += list(range(L - e, L))
        pos = torch.tensor(pos, dtype=torch.int64)
        if c["mrope"]:
            pos = torch.stack([pos, pos + 3, pos * 2])
        batch = ForwardBatch(
            batch_size=len(c["req"]),
            req_pool_indices=torch.tensor(c["req"], dtype=torch.int64),
            seq_lens=torch.tensor(c["seq"], dtype=torch.int64),
            prefix_lens=torch.tensor([L - e for L, e in zip(c["seq"], c["ext"])]),
            extend_lens=list(c["ext"]),
            out_cache_loc=torch.tensor(loc, dtype=torch.int64),
            req_to_token=rtt,
            is_prefill=max(c["ext"]) > 1)
        with torch.no_grad():
            out = layer(hidden, pos, pool, batch)
        meta["cases"][name] = {k: c[k] for k in ("req", "seq", "ext")}
        data[f"{name}_hidden"] = bits(hidden)
        data[f"{name}_positions"] = pos.numpy()
        data[f"{name}_out_cache_loc"] = np.array(loc, dtype=np.int64)
        # outputs as float16: their relative rounding (5e-4) is far below any
        # tolerance they are compared at
        data[f"{name}_q"] = captured["q"].numpy().astype(np.float16)
        data[f"{name}_k_written"] = pool.k[loc].numpy().astype(np.float16)
        data[f"{name}_v_written"] = pool.v[loc].numpy().astype(np.float16)
        data[f"{name}_attn"] = captured["attn"].numpy().astype(np.float16)
        data[f"{name}_out"] = out.numpy().astype(np.float16)
    data["meta_json"] = np.frombuffer(json.dumps(meta).encode(), dtype=np.uint8)
    np.savez_compressed(OUT, **data)
    print(f"wrote {OUT} ({OUT.stat().st_size} bytes)")


if __name__ == "__main__":
    main(sys.argv[1] if len(sys.argv) > 1 else "/root/reference")
