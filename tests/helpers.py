"""Shared test helpers: small workload builders, oracle runners, tolerance checks."""
from __future__ import annotations

import numpy as np
import torch

from oracle.brute import attention_brute, attention_dense
from oracle.kv_quant import dequantize_e4m3
from oracle.slot_attention import slot_based_attention_ref
from tokenfactory_amd import workloads

# bf16 attention tolerance: |out - ref| <= ATOL + RTOL * |ref| elementwise against
# an fp32 reference, plus a relative Frobenius bound that stays meaningful when
# a flat softmax makes the outputs small.
ATOL = 2e-2
RTOL = 1e-2
NORM_REL = 1e-2


def small_case(seq_lens, ext_lens, hq=4, hkv=1, d=32, seed=0, pool=None, groups=None,
               prefixes=None, dtype=torch.float32, device="cpu", q_std=1.0, scale=None):
    pool = pool or (sum(seq_lens) + 64) * 2
    return workloads.build("case", list(seq_lens), list(ext_lens), num_q_heads=hq,
                           num_kv_heads=hkv, head_dim=d, pool_slots=pool, device=device,
                           dtype=dtype, seed=seed, prefix_groups=groups,
                           shared_prefix_lens=prefixes, q_std=q_std, scale=scale)


def rebatch(wl, seq_lens, ext_lens, q, rows=None):
    """A workload sharing ``wl``'s pools and req_to_token table with new per-request
    lengths / queries (rows default to the first len(seq_lens) rows of ``wl``)."""
    import copy
    from tokenfactory_amd import ForwardBatch
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


def float_pools(wl):
    """K/V pools as fp32 (dequantised for an fp8 pool)."""
    if wl.k_pool.dtype == torch.float8_e4m3fn:
        return (dequantize_e4m3(wl.k_pool, wl.k_scale.float().cpu().item()),
                dequantize_e4m3(wl.v_pool, wl.v_scale.float().cpu().item()))
    return wl.k_pool.float(), wl.v_pool.float()


class _HostBatch:
    """ForwardBatch fields moved to the CPU for the restatement."""

    def __init__(self, batch):
        for name in ("batch_size", "extend_lens", "is_prefill", "max_seq_len",
                     "max_extend_len", "req_pool_indices_list"):
            setattr(self, name, getattr(batch, name))
        for name in ("req_pool_indices", "seq_lens", "prefix_lens", "out_cache_loc",
                     "req_to_token", "extend_lens_tensor"):
            t = getattr(batch, name)
            setattr(self, name, None if t is None else t.cpu())


def _compact(wl):
    """Only the pool rows the batch references, with req_to_token renumbered to them
    (rows 0..B-1); -1 entries stay -1. Keeps the oracle's host copies small."""
    b = wl.batch
    width = b.max_seq_len
    sub = b.req_to_token[b.req_pool_indices, :width]
    used, inv = torch.unique(sub.clamp(min=0), return_inverse=True)
    kp = wl.k_pool[used].cpu()
    vp = wl.v_pool[used].cpu()
    rtt = torch.full((b.batch_size, width + 1), -1, dtype=torch.long)
    rtt[:, :width] = torch.where(sub >= 0, inv, torch.full_like(inv, -1)).cpu()
    return kp, vp, rtt


def restatement(wl):
    """The op-for-op restatement of the reference, in fp32 on the CPU."""
    kp, vp, rtt = _compact(wl)
    if kp.dtype == torch.float8_e4m3fn:
        kf = dequantize_e4m3(kp, wl.k_scale.float().cpu().item())
        vf = dequantize_e4m3(vp, wl.v_scale.float().cpu().item())
    else:
        kf, vf = kp.float(), vp.float()
    batch = _HostBatch(wl.batch)
    batch.req_to_token = rtt
    batch.req_pool_indices = torch.arange(wl.batch.batch_size)
    batch.req_pool_indices_list = list(range(wl.batch.batch_size))
    return slot_based_attention_ref(wl.q.float().cpu(), kf, vf, batch,
                                    wl.num_q_heads // wl.num_kv_heads, wl.scale)


def brute(wl, dense=False):
    kf, vf = float_pools(wl)
    seq = [wl.batch.max_seq_len] if wl.batch.batch_size == 1 else wl.seq_lens
    fn = attention_dense if dense else attention_brute
    return fn(wl.q.float().cpu().numpy(), kf.cpu().numpy(), vf.cpu().numpy(),
              wl.batch.req_to_token.cpu().numpy(), wl.rows, seq, wl.ext_lens, wl.scale)


def assert_attn_close(out, ref, atol=ATOL, rtol=RTOL, norm_rel=NORM_REL, what=""):
    out = torch.as_tensor(out).float().cpu()
    ref = torch.as_tensor(ref).float().cpu()
    assert out.shape == ref.shape, (out.shape, ref.shape)
    assert torch.isfinite(out).all(), f"{what}: non-finite output"
    err = (out - ref).abs()
    bound = atol + rtol * ref.abs()
    bad = err > bound
    rel = (err.norm() / ref.norm().clamp_min(1e-30)).item()
    assert not bad.any(), (f"{what}: {int(bad.sum())} elements outside atol={atol}, rtol={rtol};"
                           f" max abs err {err.max().item():.3e}, rel-norm {rel:.3e}")
    assert rel <= norm_rel, f"{what}: relative norm error {rel:.3e} > {norm_rel}"
    return err.max().item(), rel


def as_numpy(x):
    return np.asarray(torch.as_tensor(x).float().cpu().numpy(), dtype=np.float64)
