"""Benchmark of the MI355X full-attention hot path (one GPU).

Headline (``value``): decode attention over the slot-indirected KV pool for a
64-request step of the 27B hybrid model's full-attention layer at TP=1 -
batch 64, context lengths uniform in [1k, 8k], 24 q / 4 kv heads, head_dim 256,
bf16 KV in a 1M-slot pool with randomly scattered slots - as whole-job HBM
throughput: algorithmic bytes (K/V rows + int64 slot ids + q in + out) divided
by the time of the step's launches (streaming kernel + split merge), inputs
resident in HBM. Two independent step instances alternate so the 256 MB
Infinity Cache cannot serve one step's KV from the previous step.

``roofline`` covers the dominant kernel (the streaming decode kernel), timed
with HIP events recorded on the stream it is launched on. ``secondary`` holds
the other serving shapes (prefill/extend with radix prefixes on MFMA, the mixed
chunked-prefill + decode step, fp8-KV decode at 128k context) with their own
roofline fractions. ``cpu_baseline`` times the oracle's op-for-op restatement of
the reference's CPU decode path on a bounded sample of the same step.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--only ...] [--no-cpu]
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

REPO = Path(__file__).resolve().parent
sys.path.insert(0, str(REPO))

HBM_PEAK = 8.0e12          # MI355X HBM3E bytes/s
MFMA_BF16_PEAK = 2.5e15    # MI355X dense bf16 FLOP/s
FP8_PEAK_TFLOPS = 5000.0   # MI355X dense fp8 TFLOP/s
METRIC = ("decode attn HBM GB/s (% peak) + prefill attn TFLOP/s (% MFMA peak), 1 MI355X")


def log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--only", default="decode,extend,mixed,fp8,prep,gate,plan,rtt,oproj,gdn",
                    help="comma list of decode,extend,mixed,fp8,prep,gate,plan,rtt,oproj,gdn,copy")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--workgroups", type=int, default=0,
                    help="decode persistent grid size (0 = one per CU)")
    return ap.parse_args()


def _event(torch, stream):
    ev = torch.cuda.Event(enable_timing=True)
    ev.record(stream)
    return ev


def time_steps(torch, calls, steps, warmup, step_fns):
    """Whole-step time: ``warmup`` untimed steps, then ``steps`` steps cycling over
    ``calls`` between one pair of HIP events on the launch stream (no event in
    between, so nothing idles the GPU inside the timed region). Returns ms/step."""
    stream = torch.cuda.current_stream()
    for i in range(warmup):
        for fn in step_fns(calls[i % len(calls)]):
            fn()
    torch.cuda.synchronize()
    start = _event(torch, stream)
    for i in range(steps):
        for fn in step_fns(calls[i % len(calls)]):
            fn()
    end = _event(torch, stream)
    torch.cuda.synchronize()
    return start.elapsed_time(end) / steps


def time_kernel(torch, calls, steps, launch):
    """Average duration of one kernel: every launch bracketed by HIP events
    recorded on the stream the kernel is launched on. Returns ms/launch."""
    stream = torch.cuda.current_stream()
    pairs = []
    for i in range(steps):
        a = _event(torch, stream)
        launch(calls[i % len(calls)])
        pairs.append((a, _event(torch, stream)))
    torch.cuda.synchronize()
    times = sorted(a.elapsed_time(b) for a, b in pairs)
    _LAST_SPREAD.update(p10=_pct(times, 0.1), p50=_pct(times, 0.5), p90=_pct(times, 0.9))
    return sum(times) / steps


_LAST_SPREAD = {}


def _pct(sorted_times, f):
    return sorted_times[min(len(sorted_times) - 1, int(f * len(sorted_times)))]


def last_spread():
    """p10 / median / p90 (ms) of the launches timed by the last time_kernel call."""
    return dict(_LAST_SPREAD)


def bench_decode(torch, workloads, SlotAttentionCall, args):
    log("building decode_b64 (2 independent instances, 1M-slot pools)")
    wls = [workloads.decode_b64(device="cuda", seed=11), workloads.decode_b64(device="cuda",
                                                                              seed=12)]
    calls = [SlotAttentionCall(w.q, w.k_pool, w.v_pool, w.batch, scaling=w.scale,
                               decode_workgroups=args.workgroups) for w in wls]
    nbytes = sum(w.decode_bytes() for w in wls) / len(wls)
    ms = time_steps(torch, calls, args.steps, args.warmup, lambda c: [c.run])
    k_ms = time_kernel(torch, calls, args.steps, lambda c: c.run_decode_partial())
    k_spread = last_spread()
    m_ms = time_kernel(torch, calls, args.steps, lambda c: c.run_decode_merge())
    value = nbytes / (ms * 1e-3)
    ach = nbytes / (k_ms * 1e-3)
    res = {
        "value": value, "ms_per_step": ms, "bytes_per_step": nbytes,
        "roofline": {"bound": "hbm", "achieved": ach / 1e9, "peak": HBM_PEAK / 1e9,
                     "unit": "GB/s", "frac": ach / HBM_PEAK, "traffic": None,
                     "kernel": "decode_kernel<bf16> (tf_attn_decode_partial)",
                     "kernel_ms": k_ms, "kernel_ms_p10_p50_p90": k_spread,
                     "merge_kernel_ms": m_ms},
        "workloads": wls,
    }
    log(f"decode_b64: {ms*1e3:.1f} us/step, {value/1e9:.0f} GB/s ({value/HBM_PEAK*100:.1f}% "
        f"of HBM peak); streaming kernel {k_ms*1e3:.1f} us ({ach/HBM_PEAK*100:.1f}%), "
        f"merge kernel {m_ms*1e3:.1f} us")
    return res


def bench_extend(torch, workloads, SlotAttentionCall, args, seed=13, kv_fp8=False):
    log(f"building extend_prefix (16 requests, 4 radix groups, seed {seed}"
        f"{', fp8-e4m3 KV' if kv_fp8 else ''})")
    wl = workloads.extend_prefix(device="cuda", seed=seed, kv_fp8=kv_fp8)
    call = SlotAttentionCall(wl.q, wl.k_pool, wl.v_pool, wl.batch, scaling=wl.scale,
                             k_scale=wl.k_scale, v_scale=wl.v_scale)
    # About 2 ms per step: half the step count, and the full warm-up so that
    # the clocks have settled (MFMA-heavy launches ramp over the first ~20 ms).
    steps = max(3, args.steps // 2)
    ms = time_steps(torch, [call], steps, max(1, args.warmup), lambda c: [c.run])
    k_ms = time_kernel(torch, [call], steps, lambda c: c.run_extend())
    k_spread = last_spread()
    flops = wl.extend_flops()
    tf = flops / (k_ms * 1e-3)
    prefixes = sorted(set(L - e for L, e in zip(wl.seq_lens, wl.ext_lens)))
    log(f"extend_prefix seed {seed}{' fp8' if kv_fp8 else ''}: {ms*1e3:.1f} us/step, "
        f"{tf/1e12:.1f} TFLOP/s ({tf/MFMA_BF16_PEAK*100:.1f}% of bf16 MFMA peak)")
    return {"workload": f"extend_prefix seed {seed}: 16 requests in 4 radix-prefix groups of 4, "
                        f"prefix U[0,4k] shared per group (drawn: {prefixes}), new tokens "
                        f"U[512,2k], causal, 24q/4kv, head_dim 256, "
                        + ("fp8-e4m3 KV (per-tensor scales amax/448) read as bf16, bf16 "
                           "queries" if kv_fp8 else "bf16"),
            "value": flops / (ms * 1e-3) / 1e12, "unit": "TFLOP/s", "ms_per_step": ms,
            "steps": steps, "flops_per_step": flops, "kernel_ms": k_ms,
            "kernel_ms_p10_p50_p90": k_spread,
            "roofline": {"bound": "mfma", "achieved": tf / 1e12, "peak": MFMA_BF16_PEAK / 1e12,
                         "unit": "TFLOP/s", "frac": tf / MFMA_BF16_PEAK,
                         "kernel": "extend_mfma_kernel<true>" if kv_fp8 else "extend_mfma_kernel<false>"}}


def bench_mixed(torch, workloads, SlotAttentionCall, args):
    """The mixed step as the module sees it: ``slot_based_attention`` per layer,
    16 full-attention layers per model step, each step a new ``ForwardBatch``
    (as the model runner builds one per step): the step's first call plans on
    the device, the other 15 reuse the plan, and the decode launches run on a
    second stream beside the extend kernel."""
    from tokenfactory_amd import slot_based_attention
    from tokenfactory_amd.forward_batch import ForwardBatch
    log("building mixed (4 x 2k extend + 128 decode, 2M-slot pool)")
    wl = workloads.mixed(device="cuda")
    b0 = wl.batch
    layers = 16

    def new_step():
        return ForwardBatch(batch_size=b0.batch_size, req_pool_indices=b0.req_pool_indices,
                            seq_lens=b0.seq_lens, prefix_lens=b0.prefix_lens,
                            extend_lens=list(b0.extend_lens), out_cache_loc=b0.out_cache_loc,
                            req_to_token=b0.req_to_token, is_prefill=b0.is_prefill,
                            max_seq_len=b0.max_seq_len, max_extend_len=b0.max_extend_len,
                            req_pool_indices_list=b0.req_pool_indices_list)

    def model_step(batch):
        for _ in range(layers):
            slot_based_attention(wl.q, wl.k_pool, wl.v_pool, batch, scaling=wl.scale)

    # About 23 ms per model step; the warm-up lets the clocks settle.
    steps = max(2, args.steps // 8)
    warm = [new_step() for _ in range(max(1, args.warmup // 4))]
    timed = [new_step() for _ in range(steps)]
    torch.cuda.synchronize()
    for b in warm:
        model_step(b)
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream()
    start = _event(torch, stream)
    for b in timed:
        model_step(b)
    end = _event(torch, stream)
    torch.cuda.synchronize()
    ms = start.elapsed_time(end) / (steps * layers)
    # The same launches from one prebuilt call, and each kernel on its own.
    call = SlotAttentionCall(wl.q, wl.k_pool, wl.v_pool, wl.batch, scaling=wl.scale,
                             overlap_decode=True)
    ms_call = time_steps(torch, [call], max(3, args.steps // 2), max(1, args.warmup // 2),
                         lambda c: [c.run])
    ph = {"extend": time_kernel(torch, [call], max(3, args.steps // 2),
                                lambda c: c.run_extend()),
          "decode": time_kernel(torch, [call], max(3, args.steps // 2),
                                lambda c: c.run_decode_partial())}
    flops, nbytes = wl.extend_flops(), wl.decode_bytes()
    bound_ms = (flops / MFMA_BF16_PEAK + nbytes / HBM_PEAK) * 1e3
    log(f"mixed: {ms*1e3:.1f} us per layer through slot_based_attention ({layers} layers per "
        f"step, one plan per step; prebuilt call {ms_call*1e3:.1f} us; extend kernel "
        f"{ph['extend']*1e3:.1f}, decode streaming kernel {ph['decode']*1e3:.1f}); serial "
        f"roofline {bound_ms*1e3:.0f} us ({bound_ms/ms*100:.1f}%)")
    return {"workload": "mixed: 4 extend requests of 2048 new tokens on U[0,8k] prefixes + "
                        "128 decode requests with contexts U[512,16k], 24q/4kv, head_dim 256, "
                        "bf16; slot_based_attention per layer, 16 layers per model step, a new "
                        "ForwardBatch per step (planned once on the device, decode launches "
                        "on a second stream beside the extend kernel)",
            "value": bound_ms / ms, "unit": "fraction of serial roofline",
            "ms_per_layer": ms, "model_steps": steps, "layers_per_step": layers,
            "prebuilt_call_ms": ms_call,
            "extend_kernel_ms": ph["extend"], "decode_kernel_ms": ph["decode"],
            "extend_tflops": flops / (ph["extend"] * 1e-3) / 1e12,
            "decode_gbps": nbytes / (ph["decode"] * 1e-3) / 1e9,
            "roofline": {"bound": "mfma+hbm (serial)", "achieved": bound_ms / ms, "peak": 1.0,
                         "unit": "fraction", "frac": bound_ms / ms}}


def bench_fp8(torch, workloads, SlotAttentionCall, args):
    log("building decode_fp8_128k (8 x 128k tokens, fp8-e4m3 KV)")
    wl = workloads.decode_fp8_128k(device="cuda")
    call = SlotAttentionCall(wl.q, wl.k_pool, wl.v_pool, wl.batch, scaling=wl.scale,
                             k_scale=wl.k_scale, v_scale=wl.v_scale)
    ms = time_steps(torch, [call], args.steps, args.warmup, lambda c: [c.run])
    k_ms = time_kernel(torch, [call], args.steps, lambda c: c.run_decode_partial())
    nbytes = wl.decode_bytes()
    value = nbytes / (ms * 1e-3)
    ach = nbytes / (k_ms * 1e-3)
    log(f"decode_fp8_128k: {ms*1e3:.1f} us/step, {value/1e9:.0f} GB/s "
        f"({value/HBM_PEAK*100:.1f}%); streaming kernel {ach/HBM_PEAK*100:.1f}%")
    return {"workload": "decode_fp8_128k: batch 8, 131072-token contexts, 24q/4kv, head_dim "
                        "256, fp8-e4m3 KV with per-tensor scales amax/448, bf16 queries",
            "value": value / 1e9, "unit": "GB/s", "ms_per_step": ms, "steps": args.steps,
            "bytes_per_step": nbytes, "kernel_ms": k_ms,
            "roofline": {"bound": "hbm", "achieved": ach / 1e9, "peak": HBM_PEAK / 1e9,
                         "unit": "GB/s", "frac": ach / HBM_PEAK,
                         "kernel": "decode_kernel<fp8>"}}


def bench_prep(torch, args):
    """Fused q/k RMSNorm + partial RoPE + KV write over one 20k-token prefill
    step (24 q / 4 kv heads, head_dim 256, bf16): HBM-bound elementwise work."""
    from oracle.qk_prep import inv_freq_ref
    from tokenfactory_amd import qk_norm_rope_kv_write
    T, hq, hkv, d, pool = 20480, 24, 4, 256, 1 << 18
    g = torch.Generator(device="cuda").manual_seed(23)
    qg = torch.randn(T, hq, 2 * d, device="cuda", generator=g).to(torch.bfloat16)
    k = torch.randn(T, hkv, d, device="cuda", generator=g).to(torch.bfloat16)
    v = torch.randn(T, hkv, d, device="cuda", generator=g).to(torch.bfloat16)
    qw = torch.ones(d, device="cuda")
    kw = torch.ones(d, device="cuda")
    pos = torch.arange(T, device="cuda")
    loc = torch.randperm(pool - 1, device="cuda", generator=g)[:T] + 1
    kp = torch.zeros(pool, hkv, d, dtype=torch.bfloat16, device="cuda")
    vp = torch.zeros_like(kp)
    out = torch.empty(T, hq, d, dtype=torch.bfloat16, device="cuda")
    invf = inv_freq_ref(64, 1e7).cuda()
    q = qg[:, :, :d]
    fn = lambda: qk_norm_rope_kv_write(q, k, v, qw, kw, 1e-6, pos, invf, 64, [11, 11, 10],
                                       True, kp, vp, loc, out=out)
    for _ in range(max(1, args.warmup)):
        fn()
    torch.cuda.synchronize()
    k_ms = time_kernel(torch, [None], args.steps, lambda c: fn())
    # read q, k, v and positions / slots; write q_out, K, V rows
    nbytes = T * ((hq + 2 * hkv) * d * 2 * 2 + 16)
    log(f"qk_prep (20k tokens): {k_ms*1e3:.1f} us, {nbytes/(k_ms*1e-3)/1e9:.0f} GB/s "
        f"({nbytes/(k_ms*1e-3)/HBM_PEAK*100:.1f}% of HBM peak)")
    return {"workload": "fused q/k RMSNorm + partial RoPE + KV write: 20480 tokens, 24q/4kv, "
                        "head_dim 256, bf16, scattered slots",
            "value": nbytes / (k_ms * 1e-3) / 1e9, "unit": "GB/s", "kernel_ms": k_ms,
            "bytes_per_launch": nbytes,
            "roofline": {"bound": "hbm", "achieved": nbytes / (k_ms * 1e-3) / 1e9,
                         "peak": HBM_PEAK / 1e9, "unit": "GB/s",
                         "frac": nbytes / (k_ms * 1e-3) / HBM_PEAK,
                         "kernel": "qk_prep_kernel"}}


def bench_gate(torch, workloads, SlotAttentionCall, args):
    """The module's output gate ``attn * F.silu(gate)`` (full_attention.py:157-159)
    over the extend_prefix step: fused into the extend kernel's output write
    against the reference's two PyTorch ops after an ungated kernel."""
    import torch.nn.functional as F
    wl = workloads.extend_prefix(device="cuda")
    T, H, D = wl.q.shape
    g = torch.Generator(device="cuda").manual_seed(29)
    qg = torch.randn((T, H, 2 * D), device="cuda", generator=g).to(torch.bfloat16)
    gate = qg[..., D:]
    plain = SlotAttentionCall(wl.q, wl.k_pool, wl.v_pool, wl.batch, scaling=wl.scale)
    gated = SlotAttentionCall(wl.q, wl.k_pool, wl.v_pool, wl.batch, scaling=wl.scale, gate=gate)
    steps = max(3, args.steps // 2)
    for c in (plain, gated):
        time_steps(torch, [c], 2, max(1, args.warmup), lambda x: [x.run_extend])
    k_plain = time_kernel(torch, [plain], steps, lambda c: c.run_extend())
    k_gated = time_kernel(torch, [gated], steps, lambda c: c.run_extend())
    attn = plain.out
    ops = lambda: attn.reshape(T, H * D) * F.silu(gate.reshape(T, H * D))
    ops_ms = time_steps(torch, [None], steps, max(1, args.warmup), lambda c: [ops])
    log(f"output gate over extend_prefix: fused +{(k_gated-k_plain)*1e3:.1f} us in the extend "
        f"kernel ({k_plain*1e3:.1f} -> {k_gated*1e3:.1f} us); reference ops {ops_ms*1e3:.1f} us")
    return {"workload": "attn * silu(gate) on the extend_prefix step (20k tokens x 24 heads x "
                        "256, bf16; gate = strided view of the q projection)",
            "extend_kernel_ms": k_plain, "extend_kernel_gated_ms": k_gated,
            "fused_cost_ms": k_gated - k_plain, "reference_ops_ms": ops_ms}


def bench_oproj(torch, args):
    """The block-FP8 o_proj after the gated attention (fp8_linear.py:181-201 ->
    triton_block_fp8_linear): 24 x 256 -> 5120, 128 x 128 weight-scale blocks,
    at the token counts of the decode_b64, mixed and extend_prefix steps."""
    from tokenfactory_amd import fp8_linear as fl
    from oracle.fp8_linear import quantize_weight_blocks
    n_out, k_in = 5120, 24 * 256
    g = torch.Generator().manual_seed(31)
    wq, ws = quantize_weight_blocks(torch.randn((n_out, k_in), generator=g) * 0.02)
    wq, ws = wq.cuda(), ws.cuda()
    steps = max(5, args.steps)
    res = {}
    for m in (64, 8320, 21938):
        x = (torch.randn((m, k_in), device="cuda") * 2).to(torch.bfloat16)
        xq, sx = fl.quantize_activations(x)
        out = torch.empty((m, n_out), dtype=torch.bfloat16, device="cuda")
        gemm = lambda _: fl.block_fp8_gemm(xq, sx, wq, ws, None, out=out)
        quant = lambda _: fl.quantize_activations(x)
        # the module's path: the attention output write leaves amax|x| (out_amax)
        amax = (x.view(torch.int16).to(torch.int32) & 0x7fff).max().reshape(1)
        quant_amax = lambda _: fl.quantize_activations(x, amax=amax)
        for fn in (gemm, quant, quant_amax):
            time_kernel(torch, [None], max(2, args.warmup), fn)
        t_gemm = time_kernel(torch, [None], steps, gemm)
        t_quant = time_kernel(torch, [None], steps, quant)
        t_quant_amax = time_kernel(torch, [None], steps, quant_amax)
        flops = 2.0 * m * n_out * k_in
        tf = flops / (t_gemm * 1e-3) / 1e12
        wbytes = n_out * k_in + ws.numel() * 4 + m * k_in + m * n_out * 2
        res[f"m{m}"] = {"gemm_ms": t_gemm, "quant_ms": t_quant,
                        "quant_from_attention_amax_ms": t_quant_amax, "gemm_tflops": tf,
                        "gemm_frac_of_fp8_peak": tf / FP8_PEAK_TFLOPS,
                        "gemm_gbps": wbytes / (t_gemm * 1e-3) / 1e9}
        if m <= 512:
            # Decode-sized calls are short enough that per-launch events add
            # host latency: the device time per call from a graph of 20 calls
            # (GEMM and split-K reduction kernels back to back).
            side = torch.cuda.Stream()
            side.wait_stream(torch.cuda.current_stream())
            with torch.cuda.stream(side):
                gemm(None)
            torch.cuda.current_stream().wait_stream(side)
            graph = torch.cuda.CUDAGraph()
            with torch.cuda.graph(graph, stream=side):
                for _ in range(20):
                    gemm(None)
            t_graph = time_steps(torch, [None], 5, 2, lambda c: [graph.replay]) / 20
            res[f"m{m}"].update({"gemm_graph_ms": t_graph,
                                 "gemm_graph_gbps": wbytes / (t_graph * 1e-3) / 1e9,
                                 "gemm_graph_frac_of_hbm": wbytes / (t_graph * 1e-3) / HBM_PEAK})
            log(f"o_proj fp8 m={m}: gemm device time {t_graph*1e3:.1f} us per call in a graph "
                f"({wbytes / t_graph / 1e6:.0f} GB/s, {wbytes / (t_graph * 1e-3) / HBM_PEAK * 100:.1f}% "
                f"of HBM)")
        log(f"o_proj fp8 m={m}: gemm {t_gemm*1e3:.1f} us = {tf:.0f} TFLOP/s "
            f"({tf / FP8_PEAK_TFLOPS * 100:.1f}% of fp8 peak, {wbytes / t_gemm / 1e6:.0f} GB/s), "
            f"activation quant {t_quant*1e3:.1f} us ({t_quant_amax*1e3:.1f} us from the "
            f"attention's amax)")
        del x, xq, out
    res["workload"] = ("block-FP8 o_proj: bf16 [m, 6144] -> dynamic e4m3 -> x e4m3 [5120, 6144] "
                       "with 128x128 fp32 block scales -> bf16 [m, 5120]; m = tokens of the "
                       "decode_b64, mixed and extend_prefix steps")
    return res


def bench_gdn(torch, args):
    """Gated DeltaNet decode step (linear_attention.py:244-298 + the gated norm,
    :325) for 64 requests at one GPU's shape (16 key / 48 value heads of 128),
    states scattered over a 256-slot pool: the fused kernel against the
    reference's PyTorch op sequence on the same device.  Successive steps cycle
    over four disjoint 64-request sets that cover the pool, so the 604 MB of
    other states touched between two steps of one set keep the 256 MB Infinity
    Cache from serving a set's 201 MB of states to its next step."""
    import torch.nn.functional as F
    from tokenfactory_amd.linear_attention import gdn_decode_step
    bsz, hk, hv, slots = 64, 16, 48, 256
    conv_dim = 2 * hk * 128 + hv * 128
    g = torch.Generator(device="cuda").manual_seed(37)
    rnd = lambda *s: torch.randn(s, device="cuda", generator=g)
    cs = rnd(slots, conv_dim, 3).to(torch.bfloat16)
    ss = rnd(slots, hv, 128, 128) * 0.2
    req_sets = list(torch.randperm(slots, device="cuda", generator=g).view(4, bsz))
    qkv = rnd(bsz, conv_dim).to(torch.bfloat16)
    a, b = rnd(bsz, hv).to(torch.bfloat16), rnd(bsz, hv).to(torch.bfloat16)
    z = rnd(bsz, hv * 128).to(torch.bfloat16)
    conv_w = (rnd(conv_dim, 4) * 0.5).to(torch.bfloat16).float()
    a_log, dt_bias = rnd(hv) - 2, rnd(hv)
    norm_w = torch.ones(hv * 128, device="cuda")
    step = lambda rq: gdn_decode_step(qkv, b, a, z, conv_w, a_log, dt_bias, norm_w, 1e-6, cs, ss,
                                      rq, hk, hv)
    steps = max(8, args.steps)
    time_kernel(torch, req_sets, max(4, args.warmup), step)
    t = time_kernel(torch, req_sets, steps, step)
    state_bytes = bsz * hv * 128 * 128 * 4 * 2
    other = bsz * (conv_dim * 2 * 7 + hv * 4 + hv * 128 * 2 * 2) + conv_dim * 16
    gbps = (state_bytes + other) / (t * 1e-3) / 1e9

    def ref_ops(rq):
        # the reference's _batched_decode_step and norm as PyTorch ops
        padded = torch.cat([cs[rq], qkv.unsqueeze(-1)], dim=-1)
        cs[rq] = padded[:, :, 1:]
        y = F.silu(F.conv1d(padded, conv_w.to(torch.bfloat16).unsqueeze(1),
                            groups=conv_dim).squeeze(-1))
        q, k, v = y.split([hk * 128, hk * 128, hv * 128], dim=-1)
        qn = F.normalize(q.view(bsz, hk, 128).float(), dim=-1) * 128 ** -0.5
        kn = F.normalize(k.view(bsz, hk, 128).float(), dim=-1)
        qn, kn = qn.repeat_interleave(3, 1), kn.repeat_interleave(3, 1)
        decay = -torch.exp(a_log) * F.softplus(a.float() + dt_bias)
        st = ss[rq] * torch.exp(decay)[..., None, None]
        vp = torch.einsum("bhkd,bhk->bhd", st, kn)
        delta = torch.sigmoid(b.float())[..., None] * (v.view(bsz, hv, 128).float() - vp)
        st = st + torch.einsum("bhk,bhd->bhkd", kn, delta)
        ss[rq] = st
        o = torch.einsum("bhkd,bhk->bhd", st, qn).reshape(bsz, -1).to(torch.bfloat16)
        x = o.float().view(bsz, hv, 128)
        xn = (x * torch.rsqrt(x.pow(2).mean(-1, keepdim=True) + 1e-6)).view(bsz, -1)
        return (norm_w * xn * F.silu(z.float())).to(torch.bfloat16)

    ref_ms = time_steps(torch, req_sets, steps, max(1, args.warmup),
                        lambda rq: [lambda: ref_ops(rq)])
    log(f"gdn decode B={bsz}: fused kernel {t*1e3:.1f} us = {gbps:.0f} GB/s "
        f"({gbps * 1e9 / HBM_PEAK * 100:.1f}% of HBM peak); reference ops {ref_ms*1e3:.1f} us")
    res = {"workload": "Gated DeltaNet decode step: 64 requests, 16 key / 48 value heads of "
                       "128, fp32 128x128 states scattered in a 256-slot pool, bf16 conv state; "
                       "steps cycle over 4 disjoint request sets covering the pool",
           "kernel_ms": t, "bytes_per_launch": state_bytes + other, "gbps": gbps,
           "frac_of_hbm_peak": gbps * 1e9 / HBM_PEAK, "reference_ops_ms": ref_ms}

    # the mixed step's shape: 4 requests extending by 2048 tokens + 128 decodes
    from tokenfactory_amd.linear_attention import gdn_extend_step
    lens = [2048] * 4 + [1] * 128
    n_tok = sum(lens)
    req = torch.randperm(slots, device="cuda", generator=g)[:len(lens)]
    qkv = rnd(n_tok, conv_dim).to(torch.bfloat16)
    a, b = rnd(n_tok, hv).to(torch.bfloat16), rnd(n_tok, hv).to(torch.bfloat16)
    z = rnd(n_tok, hv * 128).to(torch.bfloat16)
    ext = lambda _: gdn_extend_step(qkv, b, a, z, conv_w, a_log, dt_bias, norm_w, 1e-6, cs, ss,
                                    req, lens, hk, hv)
    time_kernel(torch, [None], 2, ext)
    te = time_kernel(torch, [None], max(3, steps // 4), ext)
    log(f"gdn extend (4 x 2048 + 128 x 1 tokens): {te*1e3:.1f} us, "
        f"{n_tok / (te * 1e-3) / 1e6:.2f} M tokens/s, {te * 1e6 / 2048:.0f} ns per token of "
        f"the longest request")
    res["extend_mixed"] = {"workload": "4 requests x 2048 new tokens + 128 decodes, same heads",
                           "ms": te, "tokens_per_s": n_tok / (te * 1e-3)}
    return res


def bench_plan(torch, workloads, SlotAttentionCall, args):
    """Whole mixed step as a caller sees it, wall clock per step: host-planned
    (plan + pinned upload + launches), device-planned (planner kernel +
    launches) and the device-planned step replayed from a HIP graph."""
    import time
    n = max(5, args.steps // 2)
    res = {}
    for tag, wl in (("mixed", workloads.mixed(device="cuda")),
                    ("small_mixed", workloads.mixed(device="cuda", n_extend=2, extend_new=64,
                                                    prefix_hi=512, n_decode=16, dec_lo=256,
                                                    dec_hi=2048, pool_slots=1 << 16))):
        res[tag] = _plan_step(torch, wl, SlotAttentionCall, args, n, time)
        r = res[tag]
        log(f"{tag} step (wall / host enqueue per step): host-planned "
            f"{r['host_planned_ms']*1e3:.0f} / {r['host_planned_cpu_ms']*1e3:.0f} us, "
            f"device-planned {r['device_planned_ms']*1e3:.0f} / "
            f"{r['device_planned_cpu_ms']*1e3:.0f} us, graph replay "
            f"{r['graph_replay_ms']*1e3:.0f} / {r['graph_replay_cpu_ms']*1e3:.0f} us")
    res["workload"] = ("one attention step incl. planning and launch: mixed (4 x 2k extend + "
                       "128 decode) and small_mixed (2 x 64 extend + 16 decode, contexts "
                       "U[256, 2k])")
    return res


def _plan_step(torch, wl, SlotAttentionCall, args, n, time):
    kw = dict(scaling=wl.scale)

    def wall(fn):
        """(wall ms per step, host ms per step spent enqueuing)."""
        for _ in range(max(2, args.warmup // 2)):
            fn()
        torch.cuda.synchronize()
        host = 0.0
        t0 = time.perf_counter()
        for _ in range(n):
            h = time.perf_counter()
            fn()
            host += time.perf_counter() - h
        torch.cuda.synchronize()
        return (time.perf_counter() - t0) / n * 1e3, host / n * 1e3

    host_ms = wall(lambda: SlotAttentionCall(wl.q, wl.k_pool, wl.v_pool, wl.batch, **kw).run())
    dev_ms = wall(lambda: SlotAttentionCall(wl.q, wl.k_pool, wl.v_pool, wl.batch,
                                            device_plan=True, **kw).run())
    call = SlotAttentionCall(wl.q, wl.k_pool, wl.v_pool, wl.batch, device_plan=True, **kw)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        call.run()
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        call.run()
    graph_ms = wall(graph.replay)
    return {"host_planned_ms": host_ms[0], "device_planned_ms": dev_ms[0],
            "graph_replay_ms": graph_ms[0], "host_planned_cpu_ms": host_ms[1],
            "device_planned_cpu_ms": dev_ms[1], "graph_replay_cpu_ms": graph_ms[1]}


def bench_rtt_sync(torch, args):
    """Per-step sync of the resident device req_to_token table, wall clock per
    step: the reference's per-request loop (engine/model_runner.py:147-167: a
    host-to-device copy of each rewritten prefix run, a slice copy of each
    request's out_cache_loc) against DeviceReqToTokenTable.sync (one pinned
    copy + one kernel), and the kernel alone replayed from a HIP graph for the
    decode-only step."""
    import time
    import numpy as np
    from tokenfactory_amd.req_to_token import DeviceReqToTokenTable
    rng = np.random.default_rng(7)
    max_reqs, max_ctx = 512, 32768
    n = max(20, args.steps * 2)
    rows = rng.permutation(max_reqs)[:132].tolist()
    ext_rows, dec_rows = rows[:4], rows[4:]
    dec_seq = rng.integers(512, 16384, size=128).tolist()
    ext_prefix = rng.integers(0, 8192, size=4).tolist()
    host = [[] for _ in range(max_reqs)]
    for r, s in zip(dec_rows, dec_seq):
        host[r] = rng.integers(1, 1 << 21, size=s).tolist()
    for r, p in zip(ext_rows, ext_prefix):
        host[r] = rng.integers(1, 1 << 21, size=p + 2048).tolist()
    cases = {
        "decode_128": (dec_rows, [s - 1 for s in dec_seq], dec_seq, {}),
        "mixed_restore": (ext_rows + dec_rows, ext_prefix + [s - 1 for s in dec_seq],
                          [p + 2048 for p in ext_prefix] + dec_seq,
                          {r: 0 for r in ext_rows}),
    }
    ref_tensor = torch.full((max_reqs, max_ctx), -1, dtype=torch.long, device="cuda")
    table = DeviceReqToTokenTable(max_reqs, max_ctx, device="cuda")
    res = {}
    for tag, (rr, pp, ss, synced_at) in cases.items():
        loc_list = [x for r, p, s in zip(rr, pp, ss) for x in host[r][p:s]]
        loc = torch.tensor(loc_list, dtype=torch.long, device="cuda")
        cursors = [synced_at.get(r, p) for r, p in zip(rr, pp)]

        def ref_step():
            off = 0
            for r, p, s, c in zip(rr, pp, ss, cursors):
                if c < p:
                    ref_tensor[r, c:p] = torch.tensor(host[r][c:p], dtype=torch.long,
                                                      device="cuda")
                ref_tensor[r, p:s] = loc[off:off + s - p]
                off += s - p

        def our_step():
            for r, c in zip(rr, cursors):
                table.synced_lens[r] = c
            table.sync(rr, pp, ss, loc, host)

        def wall(fn):
            for _ in range(3):
                fn()
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            for _ in range(n):
                fn()
            torch.cuda.synchronize()
            return (time.perf_counter() - t0) / n * 1e3

        r = {"reference_loop_ms": wall(ref_step), "sync_ms": wall(our_step)}
        torch.cuda.synchronize()
        if not torch.equal(table.tensor, ref_tensor):
            raise RuntimeError(f"req_to_token sync differs from the reference loop ({tag})")
        if not synced_at:
            dev = [torch.tensor(x, dtype=torch.long, device="cuda") for x in (rr, pp, ss)]
            side = torch.cuda.Stream()
            side.wait_stream(torch.cuda.current_stream())
            with torch.cuda.stream(side):
                table.sync_from_device(dev[0], dev[1], dev[2], loc)
            torch.cuda.current_stream().wait_stream(side)
            graph = torch.cuda.CUDAGraph()
            with torch.cuda.graph(graph):
                table.sync_from_device(dev[0], dev[1], dev[2], loc)
            r["graph_replay_ms"] = wall(graph.replay)
        r["patched_positions"] = sum(p - c for p, c in zip(pp, cursors))
        r["new_positions"] = len(loc_list)
        res[tag] = r
        log(f"req_to_token sync {tag}: reference loop {r['reference_loop_ms']*1e3:.0f} us, "
            f"one kernel {r['sync_ms']*1e3:.0f} us"
            + (f", graph replay {r['graph_replay_ms']*1e3:.0f} us" if "graph_replay_ms" in r
               else ""))
    res["workload"] = ("512 x 32768 table; decode_128: 128 decode rows (contexts U[512, 16k]); "
                       "mixed_restore: those plus 4 requests extending 2048 tokens after a "
                       "prefix of U[0, 8k) rewritten since the last sync")
    return res


def bench_copy(torch, args):
    """A plain device copy of known size, the reference point for HBM counters."""
    n = 1 << 30
    src = torch.empty(n, dtype=torch.uint8, device="cuda")
    dst = torch.empty_like(src)
    ms = time_steps(torch, [None], args.steps, args.warmup,
                    lambda c: [lambda: dst.copy_(src)])
    log(f"copy 1 GiB: {ms*1e3:.1f} us, {2*n/(ms*1e-3)/1e9:.0f} GB/s (read+write)")
    return {"bytes_read": n, "bytes_written": n, "ms": ms}


def _time_host(fn, seconds, min_runs):
    """Median, p10 and p90 (s) of ``fn`` over at least ``min_runs`` runs and
    ``seconds`` of wall time, after 10 warm-up runs."""
    for _ in range(10):
        fn()
    times = []
    t_end = time.perf_counter() + seconds
    while time.perf_counter() < t_end or len(times) < min_runs:
        t0 = time.perf_counter_ns()
        fn()
        times.append((time.perf_counter_ns() - t0) * 1e-9)
    times.sort()
    return _pct(times, 0.5), _pct(times, 0.1), _pct(times, 0.9), len(times)


def cpu_baseline(torch, dec_res):
    """The oracle's op-for-op restatement of the reference decode branch
    (full_attention.py:215-242), fp32, on every host core this process may use.

    Headline: the reference's own CPU decode case (batch 4, contexts
    128/256/384/512, 16 q / 2 kv heads, head_dim 256, fp32 4096-slot pool).
    Also reported: 4 requests of the GPU headline step (decode_b64), in the same
    bf16 algorithmic bytes as the GPU line."""
    from oracle.harness import prepare_host_inputs
    from oracle.slot_attention import slot_based_attention_ref
    from tokenfactory_amd import workloads
    from tokenfactory_amd.workloads import subset
    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
    cpu = None
    try:
        with open("/proc/cpuinfo") as fh:
            cpu = next((ln.split(":", 1)[1].strip() for ln in fh if "model name" in ln), None)
    except OSError:
        pass

    small = workloads.decode_cpu_small(device="cpu")
    args = (small.q, small.k_pool, small.v_pool, small.batch,
            small.num_q_heads // small.num_kv_heads, small.scale)
    med, p10, p90, n = _time_host(lambda: slot_based_attention_ref(*args), 12.0, 50)
    # fp32 everywhere: K/V rows, int64 slot ids, q read and out written.
    sum_l = sum(small.seq_lens)
    nbytes = (sum_l * (2 * small.num_kv_heads * small.head_dim * 4 + 8)
              + 2 * len(small.seq_lens) * small.num_q_heads * small.head_dim * 4)
    flops = 4 * small.num_q_heads * small.head_dim * sum_l
    log(f"cpu baseline (reference CPU decode case): {med*1e3:.3f} ms on {cores} threads "
        f"({nbytes/med/1e9:.2f} GB/s)")

    wl = dec_res["workloads"][0]
    sub = subset(wl, [0, 17, 40, 63])
    host_args = prepare_host_inputs(sub)
    med2, _, _, n2 = _time_host(lambda: slot_based_attention_ref(*host_args), 8.0, 3)
    b2 = sub.decode_bytes()
    log(f"cpu baseline (4 decode_b64 requests): {med2*1e3:.1f} ms ({b2/med2/1e9:.2f} GB/s)")
    return {"value": nbytes / med / 1e9, "unit": "GB/s", "cores": cores, "kind": "port",
            "sample": "the reference's CPU decode case: batch 4, contexts 128/256/384/512, "
                      "16 q / 2 kv heads, head_dim 256, fp32 KV in a 4096-slot pool, slots a "
                      "seeded random subset; fp32 op-for-op restatement of "
                      "full_attention.py:215-242 (padded gather, clamp, repeat_interleave, "
                      f"-inf mask, SDPA); median of {n} runs after 10 warm-up runs; "
                      "algorithmic fp32 bytes (K/V rows, int64 slot ids, q, out)",
            "ms_per_call": med * 1e3, "ms_p10_p90": [p10 * 1e3, p90 * 1e3],
            "bytes_per_call": nbytes, "gflops": flops / med / 1e9, "cpu_model": cpu,
            "decode_b64_sample": {
                "value": b2 / med2 / 1e9, "unit": "GB/s", "ms_per_sample": med2 * 1e3,
                "runs": n2,
                "sample": f"4 of the 64 decode_b64 requests (contexts {sub.seq_lens}), "
                          "same restatement in fp32, bf16 algorithmic bytes as the GPU line"}}


def measured_traffic():
    """HBM bytes per launch of the decode kernel from the committed FETCH_SIZE /
    WRITE_SIZE measurement, or None when that measurement was taken on other
    kernel sources than the ones built now (the file records their hash)."""
    import hashlib
    f = REPO / "profiles" / "decode_b64_hbm_traffic.json"
    try:
        rec = json.loads(f.read_text())
    except (ValueError, OSError):
        return None
    srcs = rec.get("sources", {})
    for name, digest in srcs.items():
        path = REPO / "tokenfactory_amd" / "csrc" / name
        if not path.exists() or hashlib.sha256(path.read_bytes()).hexdigest() != digest:
            log(f"traffic: {f.name} was measured on another {name}; reporting null")
            return None
    return rec.get("bytes_per_launch") if srcs else None


def main():
    args = parse()
    if args.gpus != 1:
        print(json.dumps({"error": "one GPU only: the full-attention path at TP=1 runs on "
                                   "one GPU and needs no collective, and no multi-GPU "
                                   "sharding is implemented; run with --gpus 1"}))
        sys.exit(2)
    import torch
    if not torch.cuda.is_available():
        print(json.dumps({"error": "no ROCm GPU visible"}))
        sys.exit(1)
    from tokenfactory_amd import _native, workloads
    from tokenfactory_amd.attention import SlotAttentionCall
    _native.load()
    only = set(args.only.split(","))
    secondary = {}
    dec = None
    if "copy" in only:
        secondary["copy_1gib"] = bench_copy(torch, args)
    if "decode" in only:
        dec = bench_decode(torch, workloads, SlotAttentionCall, args)
    if "extend" in only:
        secondary["extend_prefix"] = bench_extend(torch, workloads, SlotAttentionCall, args)
        torch.cuda.empty_cache()
        secondary["extend_prefix_seed22"] = bench_extend(torch, workloads, SlotAttentionCall,
                                                         args, seed=22)
        torch.cuda.empty_cache()
        secondary["extend_prefix_fp8"] = bench_extend(torch, workloads, SlotAttentionCall,
                                                      args, kv_fp8=True)
        torch.cuda.empty_cache()
    if "mixed" in only:
        secondary["mixed"] = bench_mixed(torch, workloads, SlotAttentionCall, args)
        torch.cuda.empty_cache()
    if "fp8" in only:
        secondary["decode_fp8_128k"] = bench_fp8(torch, workloads, SlotAttentionCall, args)
        torch.cuda.empty_cache()
    if "prep" in only:
        secondary["qk_prep_20k"] = bench_prep(torch, args)
    if "plan" in only:
        secondary["step_planning"] = bench_plan(torch, workloads, SlotAttentionCall, args)
    if "rtt" in only:
        secondary["req_to_token_sync"] = bench_rtt_sync(torch, args)
    if "gate" in only:
        secondary["output_gate"] = bench_gate(torch, workloads, SlotAttentionCall, args)
        torch.cuda.empty_cache()
    if "gdn" in only:
        secondary["gdn_decode_b64"] = bench_gdn(torch, args)
        torch.cuda.empty_cache()
    if "oproj" in only:
        secondary["oproj_fp8"] = bench_oproj(torch, args)
        torch.cuda.empty_cache()
    if dec is None:
        print(json.dumps({"metric": METRIC, "value": None, "secondary": secondary},
                         default=float))
        return
    dec["roofline"]["traffic"] = measured_traffic()
    cpu = None if args.no_cpu else cpu_baseline(torch, dec)
    line = {
        "metric": METRIC,
        "value": dec["value"] / 1e9,
        "unit": "GB/s",
        "pct_of_peak": dec["value"] / HBM_PEAK * 100,
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": dec["ms_per_step"],
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded N(0,1) q/K/V, random scattered slots)",
        "config": {"workload": "decode_b64: batch 64, contexts U[1k,8k], 24 q / 4 kv heads, "
                               "head_dim 256, softmax scale 1/16, bf16 KV in a 1M-slot pool "
                               "with randomly scattered slots (two alternating instances)",
                   "bytes_per_step": dec["bytes_per_step"],
                   "decode_workgroups": args.workgroups or "1 per CU"},
        "roofline": dec["roofline"],
        "cpu_baseline": cpu,
        "secondary": secondary,
    }
    print(json.dumps(line, default=float))


if __name__ == "__main__":
    main()
