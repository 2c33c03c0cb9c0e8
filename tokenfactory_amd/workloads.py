"""Seeded synthetic attention workloads shaped like a serving step of the model.

Each workload is one full-attention layer's step: a slot pool with K/V rows
~ N(0, 1), a ``req_to_token`` table whose rows hold randomly scattered slot ids
(slot 0 reserved, ``-1`` past each request's length, as
``req_to_token_pool.py:13-16`` / ``token_to_kv_pool.py:20-23``), a
``ForwardBatch`` built the way ``engine/model_runner.py:108-188`` builds it,
and queries ~ N(0, 1).

Named workloads (sizes are the serving shapes they stand for):

* ``decode_cpu_small``  B=4, L=128/256/384/512, 16 q / 2 kv heads, D=256, fp32,
  4096-slot pool (the reference's CPU decode case);
* ``decode_b64``        B=64, L~U[1k,8k], 24/4 heads, D=256, bf16, 1M-slot pool;
* ``extend_prefix``     16 requests in 4 groups of 4 sharing a radix prefix
  P~U[0,4k], new N~U[512,2k] each, bf16;
* ``mixed``             4 extends of 2048 tokens on P~U[0,8k] + 128 decodes with
  L~U[512,16k], bf16;
* ``decode_fp8_128k``   B=8, L=131072, fp8-e4m3 KV with per-tensor scales
  amax/448, bf16 queries.

``scaled`` variants shrink lengths/batch for tests while keeping the structure.
"""
from __future__ import annotations

from dataclasses import dataclass, field
from typing import List, Optional

import numpy as np
import torch

from .forward_batch import ForwardBatch

E4M3_MAX = 448.0


@dataclass
class Workload:
    name: str
    q: torch.Tensor                  # [T, Hq, D]
    k_pool: torch.Tensor             # [S, Hkv, D]
    v_pool: torch.Tensor
    batch: ForwardBatch
    seq_lens: List[int]
    ext_lens: List[int]
    rows: List[int]
    num_q_heads: int
    num_kv_heads: int
    head_dim: int
    scale: float
    k_scale: Optional[torch.Tensor] = None   # fp32 [1] for fp8 pools
    v_scale: Optional[torch.Tensor] = None
    meta: dict = field(default_factory=dict)

    @property
    def kv_elem_bytes(self) -> int:
        return self.k_pool.element_size()

    def decode_bytes(self, only_decode_rows: bool = True) -> int:
        """Algorithmic HBM bytes of the decode requests: K+V rows, int64 slot ids,
        q read and out written (bf16)."""
        row = 2 * self.num_kv_heads * self.head_dim * self.kv_elem_bytes + 8
        total = 0
        n_req = 0
        for L, e in zip(self.seq_lens, self.ext_lens):
            if only_decode_rows and e != 1:
                continue
            total += L * row
            n_req += 1
        return total + n_req * self.num_q_heads * self.head_dim * 2 * 2

    def extend_flops(self) -> int:
        """Causal (unmasked pairs only) FLOPs of the extend requests: QK^T + PV."""
        pairs = 0
        for L, e in zip(self.seq_lens, self.ext_lens):
            if e == 1:
                continue
            p = L - e
            pairs += e * p + e * (e + 1) // 2
        return 4 * self.num_q_heads * self.head_dim * pairs

    def decode_flops(self) -> int:
        return 4 * self.num_q_heads * self.head_dim * sum(
            L for L, e in zip(self.seq_lens, self.ext_lens) if e == 1)


def _fill_pool(n_slots, n_kv, dim, dtype, device, gen):
    pool = torch.randn((n_slots, n_kv, dim), generator=gen, device=device, dtype=torch.float32)
    return pool.to(dtype)


def _quantize(pool_f32):
    amax = pool_f32.abs().max().item()
    scale = amax / E4M3_MAX
    q = (pool_f32 / scale).clamp(-E4M3_MAX, E4M3_MAX).to(torch.float8_e4m3fn)
    return q, scale


def build(name: str, seq_lens: List[int], ext_lens: List[int], *, num_q_heads: int,
          num_kv_heads: int, head_dim: int, pool_slots: int, device="cuda",
          dtype=torch.bfloat16, kv_fp8: bool = False, seed: int = 0,
          prefix_groups: Optional[List[int]] = None, shared_prefix_lens: Optional[List[int]] = None,
          scale: Optional[float] = None, max_reqs: Optional[int] = None,
          q_std: float = 1.0) -> Workload:
    """Builds a workload from explicit per-request lengths.

    ``prefix_groups[b]`` (optional) names the radix-prefix group of request b;
    requests of a group share the slot ids of their first
    ``shared_prefix_lens[group]`` positions (read-only aliasing, as radix prefix
    hits produce, ``scheduler.py:187-224``).
    """
    device = torch.device(device)
    rng = np.random.default_rng(seed)
    gen = torch.Generator(device=device)
    gen.manual_seed(seed)
    bsz = len(seq_lens)
    assert len(ext_lens) == bsz
    for L, e in zip(seq_lens, ext_lens):
        if not (1 <= e <= L):
            raise ValueError(f"need 1 <= ext <= seq_len, got ext={e}, L={L}")

    # ---- slot assignment (slot 0 reserved): shared prefixes first.
    shared = {}
    need = 0
    if prefix_groups is not None:
        for grp in sorted(set(prefix_groups)):
            need += shared_prefix_lens[grp]
    for b in range(bsz):
        own_start = shared_prefix_lens[prefix_groups[b]] if prefix_groups is not None else 0
        need += seq_lens[b] - own_start
    if need >= pool_slots:
        raise ValueError(f"pool of {pool_slots} slots too small for {need} tokens")
    perm = rng.permutation(pool_slots - 1)[:need] + 1
    cursor = 0
    if prefix_groups is not None:
        for grp in sorted(set(prefix_groups)):
            n = shared_prefix_lens[grp]
            shared[grp] = perm[cursor:cursor + n]
            cursor += n
    max_ctx = max(seq_lens)
    max_reqs = max_reqs or max(2 * bsz, 8)
    rtt = np.full((max_reqs, max_ctx + 16), -1, dtype=np.int64)
    rows = rng.permutation(max_reqs)[:bsz].tolist()
    for b in range(bsz):
        L = seq_lens[b]
        if prefix_groups is not None:
            pre = shared[prefix_groups[b]]
            assert len(pre) <= L
            rtt[rows[b], :len(pre)] = pre
            own = L - len(pre)
            rtt[rows[b], len(pre):L] = perm[cursor:cursor + own]
            cursor += own
        else:
            rtt[rows[b], :L] = perm[cursor:cursor + L]
            cursor += L

    # ---- tensors
    if kv_fp8:
        kf = torch.randn((pool_slots, num_kv_heads, head_dim), generator=gen, device=device)
        vf = torch.randn((pool_slots, num_kv_heads, head_dim), generator=gen, device=device)
        k_pool, ks = _quantize(kf)
        v_pool, vs = _quantize(vf)
        del kf, vf
        k_scale = torch.tensor([ks], dtype=torch.float32, device=device)
        v_scale = torch.tensor([vs], dtype=torch.float32, device=device)
    else:
        k_pool = _fill_pool(pool_slots, num_kv_heads, head_dim, dtype, device, gen)
        v_pool = _fill_pool(pool_slots, num_kv_heads, head_dim, dtype, device, gen)
        k_scale = v_scale = None
    n_tok = int(sum(ext_lens))
    q_dtype = dtype if not kv_fp8 else torch.bfloat16
    q = (torch.randn((n_tok, num_q_heads, head_dim), generator=gen, device=device)
         * q_std).to(q_dtype)

    out_cache_loc = []
    for b in range(bsz):
        L, e = seq_lens[b], ext_lens[b]
        out_cache_loc.extend(rtt[rows[b], L - e:L].tolist())
    to_dev = lambda x: torch.tensor(x, dtype=torch.long, device=device)
    batch = ForwardBatch(
        batch_size=bsz,
        req_pool_indices=to_dev(rows),
        seq_lens=to_dev(seq_lens),
        prefix_lens=to_dev([L - e for L, e in zip(seq_lens, ext_lens)]),
        extend_lens=list(ext_lens),
        out_cache_loc=to_dev(out_cache_loc),
        req_to_token=torch.from_numpy(rtt).to(device),
        is_prefill=any(e > 1 for e in ext_lens),
        max_seq_len=max(seq_lens),
        max_extend_len=max(ext_lens),
        extend_lens_tensor=to_dev(ext_lens),
        req_pool_indices_list=list(rows),
    )
    return Workload(name=name, q=q, k_pool=k_pool, v_pool=v_pool, batch=batch,
                    seq_lens=list(seq_lens), ext_lens=list(ext_lens), rows=rows,
                    num_q_heads=num_q_heads, num_kv_heads=num_kv_heads, head_dim=head_dim,
                    scale=scale if scale is not None else head_dim ** -0.5,
                    k_scale=k_scale, v_scale=v_scale,
                    meta={"pool_slots": pool_slots, "seed": seed,
                          "prefix_groups": prefix_groups,
                          "shared_prefix_lens": shared_prefix_lens})


def rebatch(wl: Workload, seq_lens, ext_lens, q, rows=None) -> Workload:
    """A workload sharing ``wl``'s pools and req_to_token table, with new
    per-request lengths and queries (rows default to the first len(seq_lens)
    rows of ``wl``)."""
    import copy
    rows = list(rows if rows is not None else wl.rows[:len(seq_lens)])
    dev = wl.q.device
    t = lambda x: torch.tensor(list(x), dtype=torch.long, device=dev)
    batch = ForwardBatch(
        batch_size=len(seq_lens), req_pool_indices=t(rows), seq_lens=t(seq_lens),
        prefix_lens=t([L - e for L, e in zip(seq_lens, ext_lens)]),
        extend_lens=list(ext_lens), out_cache_loc=t([0] * sum(ext_lens)),
        req_to_token=wl.batch.req_to_token, is_prefill=max(ext_lens) > 1,
        max_seq_len=max(seq_lens), max_extend_len=max(ext_lens),
        extend_lens_tensor=t(ext_lens), req_pool_indices_list=rows)
    new = copy.copy(wl)
    new.q = q
    new.batch = batch
    new.seq_lens = list(seq_lens)
    new.ext_lens = list(ext_lens)
    new.rows = rows
    return new


def subset(wl: Workload, indices) -> Workload:
    """The requests ``indices`` of ``wl`` as their own batch (same pools)."""
    starts = np.cumsum([0] + list(wl.ext_lens))
    q = torch.cat([wl.q[starts[i]:starts[i + 1]] for i in indices])
    return rebatch(wl, [wl.seq_lens[i] for i in indices], [wl.ext_lens[i] for i in indices],
                   q, rows=[wl.rows[i] for i in indices])


# ---------------------------------------------------------------- named configs

def decode_cpu_small(device="cpu", seed=7) -> Workload:
    return build("decode_cpu_small", [128, 256, 384, 512], [1, 1, 1, 1], num_q_heads=16,
                 num_kv_heads=2, head_dim=256, pool_slots=4096, device=device,
                 dtype=torch.float32, seed=seed)


def decode_b64(device="cuda", seed=11, batch=64, lo=1024, hi=8192, pool_slots=(1 << 20) + 1,
               num_q_heads=24, num_kv_heads=4) -> Workload:
    rng = np.random.default_rng(seed)
    lens = rng.integers(lo, hi + 1, size=batch).tolist()
    return build("decode_b64", lens, [1] * batch, num_q_heads=num_q_heads,
                 num_kv_heads=num_kv_heads, head_dim=256, pool_slots=pool_slots,
                 device=device, seed=seed, scale=1.0 / 16)


def extend_prefix(device="cuda", seed=13, n_groups=4, per_group=4, prefix_hi=4096,
                  new_lo=512, new_hi=2048, pool_slots=1 << 18, kv_fp8=False) -> Workload:
    rng = np.random.default_rng(seed)
    prefixes = rng.integers(0, prefix_hi + 1, size=n_groups).tolist()
    groups, seq, ext = [], [], []
    for g in range(n_groups):
        for _ in range(per_group):
            n = int(rng.integers(new_lo, new_hi + 1))
            groups.append(g)
            seq.append(prefixes[g] + n)
            ext.append(n)
    return build("extend_prefix", seq, ext, num_q_heads=24, num_kv_heads=4, head_dim=256,
                 pool_slots=pool_slots, device=device, seed=seed, prefix_groups=groups,
                 shared_prefix_lens=prefixes, kv_fp8=kv_fp8)


def mixed(device="cuda", seed=17, n_extend=4, extend_new=2048, prefix_hi=8192, n_decode=128,
          dec_lo=512, dec_hi=16384, pool_slots=(1 << 21) + 1) -> Workload:
    rng = np.random.default_rng(seed)
    seq, ext = [], []
    for _ in range(n_extend):
        p = int(rng.integers(0, prefix_hi + 1))
        seq.append(p + extend_new)
        ext.append(extend_new)
    for _ in range(n_decode):
        seq.append(int(rng.integers(dec_lo, dec_hi + 1)))
        ext.append(1)
    return build("mixed", seq, ext, num_q_heads=24, num_kv_heads=4, head_dim=256,
                 pool_slots=pool_slots, device=device, seed=seed)


def decode_fp8_128k(device="cuda", seed=19, batch=8, length=131072, pool_slots=None) -> Workload:
    pool_slots = pool_slots or batch * length + 1024
    return build("decode_fp8_128k", [length] * batch, [1] * batch, num_q_heads=24,
                 num_kv_heads=4, head_dim=256, pool_slots=pool_slots, device=device,
                 seed=seed, kv_fp8=True)
