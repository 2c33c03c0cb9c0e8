"""Gated DeltaNet decode step on the GPU against the oracle.

Each case runs three consecutive decode steps on the GPU (``tf_gdn_decode``)
and in the oracle from the same random conv / SSM states, slots scattered over
a larger pool, and checks after every step:

* conv state: bit-exact (it is a shift of bf16 values);
* slots no request uses: bit-identical to before;
* SSM state (fp32): the kernel sums S^T k and S^T q in another order and fuses
  multiply-adds, and a conv output can round to the neighbouring bf16 value
  (exp and division are 1-ulp accurate on both sides), which then feeds the
  update; allowed: |diff| <= 1e-5 max|S| on all but 1e-3 of the elements and
  <= 1e-2 max|S| everywhere;
* outputs (bf16, pre-norm and normed): the bf16 bar of 2e-2 absolute /
  1e-2 relative, with at most 1e-3 of the elements off by more than one
  bf16 ulp.
"""
import pytest
import torch

from oracle import gdn as og
from tokenfactory_amd.linear_attention import gdn_decode_step, gdn_extend_step

pytestmark = pytest.mark.gpu


def make_params(hk, hv, seed):
    g = torch.Generator().manual_seed(seed)
    conv_dim = 2 * hk * 128 + hv * 128
    # bf16-valued conv taps (the model's dtype): the four-tap sums are exact in fp32
    conv_w = (torch.randn((conv_dim, 4), generator=g) * 0.5).to(torch.bfloat16).float()
    a_log = (torch.rand((hv,), generator=g) * 2 - 2.5).to(torch.bfloat16).float()
    dt_bias = torch.rand((hv,), generator=g).to(torch.bfloat16).float()
    norm_w = (1 + 0.1 * torch.randn((hv * 128,), generator=g)).to(torch.bfloat16).float()
    return conv_w, a_log, dt_bias, norm_w


def make_step(bsz, hk, hv, seed):
    g = torch.Generator().manual_seed(seed)
    conv_dim = 2 * hk * 128 + hv * 128
    qkv = torch.randn((bsz, conv_dim), generator=g).to(torch.bfloat16)
    a = torch.randn((bsz, hv), generator=g).to(torch.bfloat16)
    b = torch.randn((bsz, hv), generator=g).to(torch.bfloat16)
    z = torch.randn((bsz, hv * 128), generator=g).to(torch.bfloat16)
    return qkv, a, b, z


def close_fraction(got, want, tight, loose, frac, what):
    d = (got - want).abs()
    bad = int((d > tight).sum())
    assert float(d.max()) <= loose, f"{what}: max diff {float(d.max()):.3e} > {loose:.3e}"
    assert bad <= max(1, int(frac * d.numel())), f"{what}: {bad} of {d.numel()} above {tight:.3e}"


def check_outputs(got, want, what):
    g, w = got.float(), want.float()
    assert torch.allclose(g, w, atol=2e-2, rtol=1e-2), what
    ulp = w.abs().clamp_min(2.0 ** -126) * 2.0 ** -7
    bad = int(((g - w).abs() > ulp).sum())
    assert bad <= max(1, g.numel() // 1000), f"{what}: {bad} elements off by more than 1 ulp"


def check_chunked_outputs(got, want, what, normed):
    """Outputs of the chunked extend form against the oracle's sequence.  Their
    fp32 sums differ by about 1e-6 of the largest output, which for outputs
    below 1/256 of the largest exceeds their own bf16 ulp, so the ulp is taken
    of max(|w|, max|w| / 256).  The pre-norm output (bf16(o)) must be within one
    such ulp everywhere (up to 1e-4 of the elements beyond it); the normed
    output within two, as a one-ulp flip of bf16(o) carries through the norm,
    and at most 0.1 % beyond one."""
    g, w = got.float(), want.float()
    amax = float(w.abs().max())
    ulp = torch.clamp(w.abs(), min=max(amax / 256, 2.0 ** -126)) * 2.0 ** -7
    d = (g - w).abs()
    worst = float((d / ulp).max())
    one = int((d > ulp).sum())
    if normed:
        assert worst <= 2.0, f"{what}: an element off by {worst:.2f} floored ulps"
        assert one <= max(1, g.numel() // 1000), f"{what}: {one} elements beyond 1 floored ulp"
    else:
        assert one <= max(1, g.numel() // 10000), f"{what}: {one} elements beyond 1 floored ulp"


@pytest.mark.parametrize("bsz,hk,hv", [(1, 16, 48), (7, 16, 48), (64, 16, 48), (9, 4, 12),
                                        # one, two and four value heads per key head
                                        (5, 8, 8), (6, 4, 8), (3, 2, 8)])
def test_decode_steps_match_oracle(gpu, bsz, hk, hv):
    print(f"[gdn] B={bsz} Hk={hk} Hv={hv}", flush=True)
    n_slots = bsz + 5
    conv_dim = 2 * hk * 128 + hv * 128
    g = torch.Generator().manual_seed(bsz * 100 + hk)
    conv_state = torch.randn((n_slots, conv_dim, 3), generator=g).to(torch.bfloat16)
    ssm_state = torch.randn((n_slots, hv, 128, 128), generator=g) * 0.2
    req = torch.randperm(n_slots, generator=g)[:bsz].to(torch.int64)
    params = make_params(hk, hv, bsz + hv)
    cs_gpu, ss_gpu = conv_state.to(gpu), ssm_state.to(gpu)
    gp = [p.to(gpu) for p in params]
    untouched = torch.ones(n_slots, dtype=torch.bool)
    untouched[req] = False
    for step in range(3):
        qkv, a, b, z = make_step(bsz, hk, hv, 1000 * step + bsz)
        out, core = gdn_decode_step(qkv.to(gpu), b.to(gpu), a.to(gpu), z.to(gpu), *gp, 1e-6,
                                    cs_gpu, ss_gpu, req.to(gpu), hk, hv, return_core=True)
        want_out, want_core = og.gdn_decode(qkv, a, b, z, *params, 1e-6, conv_state, ssm_state,
                                            req, hk, hv)
        torch.cuda.synchronize()
        what = f"B={bsz} Hk={hk} Hv={hv} step {step}"
        assert torch.equal(cs_gpu.cpu(), conv_state), f"{what}: conv state"
        ss = ss_gpu.cpu()
        assert torch.equal(ss[untouched], ssm_state[untouched]), f"{what}: untouched slots"
        scale = float(ssm_state.abs().max())
        close_fraction(ss[~untouched], ssm_state[~untouched], 1e-5 * scale, 1e-2 * scale, 1e-3,
                       f"{what}: ssm state")
        check_outputs(core.cpu(), want_core, f"{what}: pre-norm output")
        check_outputs(out.cpu(), want_out, f"{what}: normed output")
        print(f"[gdn] {what}: max |dS| {float((ss - ssm_state).abs().max()):.2e}", flush=True)


def test_decode_misaligned_rows_match_oracle(gpu):
    """qkv rows and conv-state slots at odd element offsets: the conv runs per
    channel where a row or slot is not 8-byte aligned, four channels at a time
    where it is; both agree with the oracle bit for bit on the conv state."""
    bsz, hk, hv, n_slots = 6, 4, 12, 9
    conv_dim = 2 * hk * 128 + hv * 128
    g = torch.Generator().manual_seed(29)
    conv_state = torch.randn((n_slots, conv_dim, 3), generator=g).to(torch.bfloat16)
    ssm_state = torch.randn((n_slots, hv, 128, 128), generator=g) * 0.2
    req = torch.tensor([0, 3, 8, 1, 6, 5], dtype=torch.int64)
    params = make_params(hk, hv, 31)
    gp = [p.to(gpu) for p in params]
    # slot r starts at element 1 + r * (3 conv_dim + 1): the alignment varies by slot
    cs_big = torch.zeros(1 + n_slots * (3 * conv_dim + 1), dtype=torch.bfloat16, device=gpu)
    cs_gpu = cs_big.as_strided((n_slots, conv_dim, 3), (3 * conv_dim + 1, 3, 1), 1)
    cs_gpu.copy_(conv_state.to(gpu))
    ss_gpu = ssm_state.to(gpu)
    for step in range(2):
        qkv, a, b, z = make_step(bsz, hk, hv, 77 + step)
        qkv_big = torch.zeros((bsz, conv_dim + 3), dtype=torch.bfloat16)
        qkv_big[:, 1:1 + conv_dim] = qkv
        qkv_view = qkv_big.to(gpu)[:, 1:1 + conv_dim]     # row bi at element 1 + bi (conv_dim + 3)
        out, core = gdn_decode_step(qkv_view, b.to(gpu), a.to(gpu), z.to(gpu), *gp, 1e-6,
                                    cs_gpu, ss_gpu, req.to(gpu), hk, hv, return_core=True)
        want_out, want_core = og.gdn_decode(qkv, a, b, z, *params, 1e-6, conv_state, ssm_state,
                                            req, hk, hv)
        torch.cuda.synchronize()
        what = f"misaligned step {step}"
        assert torch.equal(cs_gpu.cpu(), conv_state), f"{what}: conv state"
        pads = cs_big[0::3 * conv_dim + 1].float()   # before slot 0 and after every slot
        assert pads.numel() == n_slots + 1 and (pads == 0).all(), f"{what}: padding written"
        scale = float(ssm_state.abs().max())
        close_fraction(ss_gpu.cpu(), ssm_state, 1e-5 * scale, 1e-2 * scale, 1e-3,
                       f"{what}: ssm state")
        check_outputs(core.cpu(), want_core, f"{what}: pre-norm output")
        check_outputs(out.cpu(), want_out, f"{what}: normed output")


@pytest.mark.parametrize("lens,hk,hv", [([5], 16, 48), ([1, 70, 3, 130], 16, 48),
                                         ([200, 1, 1, 64, 2], 4, 12),
                                         # 32-token chunk edges: exact, one over, one short
                                         ([32, 64, 33, 31, 1, 2], 4, 12),
                                         # one, two and four value heads per key head
                                         ([40, 1, 7], 8, 8), ([3, 66, 1], 4, 8),
                                         ([1, 35], 2, 8),
                                         # eight: two passes of the prep's head loop
                                         ([5, 40], 1, 8)])
def test_extend_matches_oracle(gpu, lens, hk, hv):
    """Mixed extend lengths against the oracle's per-request loop (chunked WY
    update for ext > 1): two consecutive calls, the second with other lengths.
    The kernel runs the chunked form with 32-token chunks on MFMAs (bf16
    high/low operand splits, fp32 accumulation); against the oracle's 64-token
    chunks the fp32 state agrees to ~1e-4 relative (allowed: 2e-4 max|S| on all
    but 1e-3 of the elements)."""
    print(f"[gdn extend] lens={lens} Hk={hk} Hv={hv}", flush=True)
    n_slots = len(lens) + 3
    conv_dim = 2 * hk * 128 + hv * 128
    g = torch.Generator().manual_seed(sum(lens) + hk)
    conv_state = torch.randn((n_slots, conv_dim, 3), generator=g).to(torch.bfloat16)
    ssm_state = torch.randn((n_slots, hv, 128, 128), generator=g) * 0.2
    req = torch.randperm(n_slots, generator=g)[:len(lens)].to(torch.int64)
    params = make_params(hk, hv, len(lens) + hv)
    cs_gpu, ss_gpu = conv_state.to(gpu), ssm_state.to(gpu)
    gp = [p.to(gpu) for p in params]
    for call, ls in enumerate((lens, [max(1, e // 2) for e in reversed(lens)])):
        qkv, a, b, z = make_step(sum(ls), hk, hv, 77 + call)
        out, core = gdn_extend_step(qkv.to(gpu), b.to(gpu), a.to(gpu), z.to(gpu), *gp, 1e-6,
                                    cs_gpu, ss_gpu, req.to(gpu), ls, hk, hv, return_core=True)
        want_out, want_core = og.gdn_extend(qkv, a, b, z, *params, 1e-6, conv_state, ssm_state,
                                            req, ls, hk, hv)
        torch.cuda.synchronize()
        what = f"lens={ls} call {call}"
        assert torch.equal(cs_gpu.cpu(), conv_state), f"{what}: conv state"
        scale = float(ssm_state.abs().max())
        close_fraction(ss_gpu.cpu(), ssm_state, 2e-4 * scale, 1e-2 * scale, 1e-3,
                       f"{what}: ssm state")
        check_chunked_outputs(core.cpu(), want_core, f"{what}: pre-norm output", False)
        check_chunked_outputs(out.cpu(), want_out, f"{what}: normed output", True)


def test_extend_of_single_tokens_equals_decode(gpu):
    hk, hv, bsz = 16, 48, 6
    conv_dim = 2 * hk * 128 + hv * 128
    g = torch.Generator().manual_seed(11)
    cs = torch.randn((bsz + 2, conv_dim, 3), generator=g).to(torch.bfloat16).to(gpu)
    ss = (torch.randn((bsz + 2, hv, 128, 128), generator=g) * 0.2).to(gpu)
    cs2, ss2 = cs.clone(), ss.clone()
    req = torch.tensor([3, 0, 7, 1, 5, 2], device=gpu)
    gp = [p.to(gpu) for p in make_params(hk, hv, 4)]
    qkv, a, b, z = (x.to(gpu) for x in make_step(bsz, hk, hv, 12))
    o1 = gdn_decode_step(qkv, b, a, z, *gp, 1e-6, cs, ss, req, hk, hv)
    o2 = gdn_extend_step(qkv, b, a, z, *gp, 1e-6, cs2, ss2, req, [1] * bsz, hk, hv)
    torch.cuda.synchronize()
    # same math; the two recurrence kernels split the row reductions differently
    assert torch.equal(cs, cs2)
    scale = float(ss.abs().max())
    close_fraction(ss2.cpu(), ss.cpu(), 1e-6 * scale, 1e-5 * scale, 1e-3, "ssm state")
    check_outputs(o2.cpu(), o1.cpu(), "output")


def test_out_of_pool_slots_are_skipped(gpu):
    hk, hv, n_slots = 4, 12, 6
    conv_dim = 2 * hk * 128 + hv * 128
    cs = torch.randn((n_slots, conv_dim, 3)).to(torch.bfloat16).to(gpu)
    ss = torch.randn((n_slots, hv, 128, 128), device=gpu)
    cs0, ss0 = cs.clone(), ss.clone()
    qkv, a, b, z = make_step(3, hk, hv, 7)
    req = torch.tensor([-1, n_slots, 2], dtype=torch.int64, device=gpu)
    params = [p.to(gpu) for p in make_params(hk, hv, 3)]
    gdn_decode_step(qkv.to(gpu), b.to(gpu), a.to(gpu), z.to(gpu), *params, 1e-6, cs, ss, req,
                    hk, hv)
    torch.cuda.synchronize()
    keep = torch.tensor([True, True, False, True, True, True])
    assert torch.equal(cs[keep.to(gpu)], cs0[keep.to(gpu)])
    assert torch.equal(ss[keep.to(gpu)], ss0[keep.to(gpu)])
    assert not torch.equal(ss[2], ss0[2])


@pytest.mark.parametrize("lens", [[40, 1, 70], [1, 40, 70]])
def test_extend_out_of_pool_slots_are_skipped(gpu, lens):
    """Extend batch with requests on slot -1 and on slot n_slots beside a valid
    one: the skipped requests touch no conv or SSM slot and their output rows
    are zeros; the valid request matches the oracle run on it alone."""
    hk, hv, n_slots = 4, 12, 6
    conv_dim = 2 * hk * 128 + hv * 128
    g = torch.Generator().manual_seed(sum(lens))
    conv_state = torch.randn((n_slots, conv_dim, 3), generator=g).to(torch.bfloat16)
    ssm_state = torch.randn((n_slots, hv, 128, 128), generator=g) * 0.2
    params = make_params(hk, hv, 5)
    cs, ss = conv_state.to(gpu), ssm_state.to(gpu)
    req = torch.tensor([-1, n_slots, 2], dtype=torch.int64)
    qkv, a, b, z = make_step(sum(lens), hk, hv, 91)
    gp = [p.to(gpu) for p in params]
    # Leave NaNs in the memory the caching allocator hands out next, so rows the
    # kernels did not write would not read as zeros by chance.
    poison = torch.full((2, sum(lens), hv * 128), float("nan"), dtype=torch.bfloat16,
                        device=gpu)
    del poison
    got, core = gdn_extend_step(qkv.to(gpu), b.to(gpu), a.to(gpu), z.to(gpu), *gp, 1e-6, cs,
                                ss, req.to(gpu), lens, hk, hv, return_core=True)
    torch.cuda.synchronize()
    keep = torch.ones(n_slots, dtype=torch.bool)
    keep[2] = False
    assert torch.equal(cs.cpu()[keep], conv_state[keep]), "skipped: conv slots touched"
    assert torch.equal(ss.cpu()[keep], ssm_state[keep]), "skipped: ssm slots touched"
    t0, t1 = lens[0] + lens[1], sum(lens)
    assert torch.equal(got[:t0].cpu(), torch.zeros((t0, hv * 128), dtype=torch.bfloat16))
    assert torch.equal(core[:t0].cpu(), torch.zeros((t0, hv * 128), dtype=torch.bfloat16))
    want_out, want_core = og.gdn_extend(qkv[t0:t1], a[t0:t1], b[t0:t1], z[t0:t1], *params,
                                        1e-6, conv_state, ssm_state, req[2:], lens[2:], hk, hv)
    scale = float(ssm_state.abs().max())
    close_fraction(ss.cpu()[2], ssm_state[2], 2e-4 * scale, 1e-2 * scale, 1e-3,
                   "valid request: ssm state")
    assert torch.equal(cs.cpu()[2], conv_state[2]), "valid request: conv state"
    check_outputs(core[t0:t1].cpu(), want_core, "valid request: pre-norm output")
    check_outputs(got[t0:t1].cpu(), want_out, "valid request: normed output")


def _extend_native(qkv, b, a, z, params, cs, ss, req, lens, hk, hv, out, core, tok, ws, stream):
    """tf_gdn_extend on caller-made tensors (views, preallocated workspace)."""
    from tokenfactory_amd import _native
    from tokenfactory_amd.linear_attention import CONV_KERNEL, HEAD_DIM
    conv_w, a_log, dt_bias, norm_w = params
    p = lambda t: 0 if t is None else t.data_ptr()
    _native.call("tf_gdn_extend", p(qkv), qkv.stride(0), p(a), p(b), a.stride(0), p(z),
                 z.stride(0), p(conv_w), p(a_log), p(dt_bias), p(norm_w), 1e-6, p(cs),
                 cs.stride(0), p(ss), ss.stride(0), p(req), p(tok), len(lens), qkv.shape[0],
                 max(lens), cs.shape[0], hk, hv, HEAD_DIM, HEAD_DIM, CONV_KERNEL, p(out),
                 out.stride(0), p(core), core.stride(0), p(ws), ws.numel(), stream)


def test_extend_strided_views_and_graph_replay(gpu):
    """z, out and core_out as column views of wider tensors at an 8-byte (not
    16-byte) offset, on a batch that mixes one-token and multi-token requests
    (the one-token recurrence then runs on the library's second stream beside
    the chunked pass): the outputs equal gdn_extend_step's on contiguous
    tensors bit for bit, the columns around the views keep their contents,
    and the call captured in a HIP graph replays to the same bits three times,
    with eager work between the replays."""
    from tokenfactory_amd import _native
    hk, hv, lens = 4, 12, [1, 70, 1, 33, 1, 2]
    n_tok, vd = sum(lens), hv * 128
    n_slots = len(lens) + 2
    g = torch.Generator().manual_seed(123)
    conv_state = torch.randn((n_slots, 2 * hk * 128 + vd, 3), generator=g).to(torch.bfloat16)
    ssm_state = torch.randn((n_slots, hv, 128, 128), generator=g) * 0.2
    req = torch.randperm(n_slots, generator=g)[:len(lens)].to(gpu)
    params = [p.to(gpu) for p in make_params(hk, hv, 9)]
    qkv, a, b, z = (x.to(gpu) for x in make_step(n_tok, hk, hv, 55))
    cs, ss = conv_state.to(gpu), ssm_state.to(gpu)
    want_out, want_core = gdn_extend_step(qkv, b, a, z, *params, 1e-6, cs, ss, req, lens, hk, hv,
                                          return_core=True)
    want_cs, want_ss = cs.clone(), ss.clone()

    zbig = torch.full((n_tok, vd + 8), 7.0, dtype=torch.bfloat16, device=gpu)
    zbig[:, 4:4 + vd] = z
    zv = zbig[:, 4:4 + vd]
    outbig = torch.full((n_tok, vd + 8), -3.0, dtype=torch.bfloat16, device=gpu)
    corebig = torch.full((n_tok, vd + 12), 5.0, dtype=torch.bfloat16, device=gpu)
    out, core = outbig[:, 4:4 + vd], corebig[:, 8:8 + vd]
    assert out.data_ptr() % 16 == 8 and zv.data_ptr() % 16 == 8
    offs = [0]
    for e in lens:
        offs.append(offs[-1] + e)
    tok = torch.tensor(offs, dtype=torch.int32, device=gpu)
    nbytes = _native.load().tf_gdn_extend_workspace_bytes(n_tok, len(lens), hk, hv)
    ws = torch.empty((nbytes,), dtype=torch.uint8, device=gpu)

    def run(stream):
        cs.copy_(conv_state.to(gpu))
        ss.copy_(ssm_state.to(gpu))
        _extend_native(qkv, b, a, zv, params, cs, ss, req, lens, hk, hv, out, core, tok, ws,
                       stream)

    def check(what):
        assert torch.equal(out, want_out), f"{what}: out"
        assert torch.equal(core, want_core), f"{what}: core_out"
        assert torch.equal(ss, want_ss) and torch.equal(cs, want_cs), f"{what}: states"
        assert (outbig[:, :4] == -3).all() and (outbig[:, 4 + vd:] == -3).all(), what
        assert (corebig[:, :8] == 5).all() and (corebig[:, 8 + vd:] == 5).all(), what

    run(torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    check("eager")
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=side):
        _extend_native(qkv, b, a, zv, params, cs, ss, req, lens, hk, hv, out, core, tok, ws,
                       side.cuda_stream)
    torch.cuda.synchronize()
    for r in range(3):
        cs.copy_(conv_state.to(gpu))
        ss.copy_(ssm_state.to(gpu))
        out.fill_(0)
        core.fill_(0)
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        check(f"replay {r}")
        float(torch.randn(1 << 16, device=gpu).sum())   # eager work between replays


def test_decode_graph_replay(gpu):
    """A decode step captured in a HIP graph (its output and workspace from the
    graph's pool) and replayed over new inputs three times, with eager work
    between the replays: every replay equals an eager step over the same
    inputs and states bit for bit (outputs, conv and ssm states)."""
    hk, hv, bsz, n_slots = 16, 48, 8, 12
    conv_dim = 2 * hk * 128 + hv * 128
    g = torch.Generator().manual_seed(321)
    cs = torch.randn((n_slots, conv_dim, 3), generator=g).to(torch.bfloat16).to(gpu)
    ss = (torch.randn((n_slots, hv, 128, 128), generator=g) * 0.2).to(gpu)
    cs_e, ss_e = cs.clone(), ss.clone()
    req = torch.randperm(n_slots, generator=g)[:bsz].to(gpu)
    gp = [p.to(gpu) for p in make_params(hk, hv, 17)]
    qkv, a, b, z = (x.to(gpu) for x in make_step(bsz, hk, hv, 40))
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):           # warm-up outside the capture
        gdn_decode_step(qkv, b, a, z, *gp, 1e-6, cs.clone(), ss.clone(), req, hk, hv)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out_g, core_g = gdn_decode_step(qkv, b, a, z, *gp, 1e-6, cs, ss, req, hk, hv,
                                        return_core=True)
    torch.cuda.synchronize()
    for r in range(3):
        nq, na, nb, nz = (x.to(gpu) for x in make_step(bsz, hk, hv, 50 + r))
        for dst, src in ((qkv, nq), (a, na), (b, nb), (z, nz)):
            dst.copy_(src)
        graph.replay()
        want_out, want_core = gdn_decode_step(nq, nb, na, nz, *gp, 1e-6, cs_e, ss_e, req, hk,
                                              hv, return_core=True)
        torch.cuda.synchronize()
        what = f"replay {r}"
        assert torch.equal(out_g, want_out) and torch.equal(core_g, want_core), what
        assert torch.equal(cs, cs_e) and torch.equal(ss, ss_e), f"{what}: states"
        float(torch.randn(1 << 16, device=gpu).sum())   # eager work between replays


def test_decode_out_of_pool_rows_are_zero(gpu):
    hk, hv, n_slots = 4, 12, 6
    conv_dim = 2 * hk * 128 + hv * 128
    cs = torch.randn((n_slots, conv_dim, 3)).to(torch.bfloat16).to(gpu)
    ss = torch.randn((n_slots, hv, 128, 128), device=gpu)
    qkv, a, b, z = make_step(3, hk, hv, 8)
    req = torch.tensor([4, -1, n_slots], dtype=torch.int64, device=gpu)
    params = [p.to(gpu) for p in make_params(hk, hv, 3)]
    out, core = gdn_decode_step(qkv.to(gpu), b.to(gpu), a.to(gpu), z.to(gpu), *params, 1e-6,
                                cs, ss, req, hk, hv, return_core=True)
    torch.cuda.synchronize()
    assert torch.equal(out[1:].cpu(), torch.zeros((2, hv * 128), dtype=torch.bfloat16))
    assert torch.equal(core[1:].cpu(), torch.zeros((2, hv * 128), dtype=torch.bfloat16))
    assert torch.isfinite(out[0].float()).all()


def test_layout_checks(gpu):
    hk, hv = 4, 12
    params = [p.to(gpu) for p in make_params(hk, hv, 3)]
    qkv, a, b, z = (x.to(gpu) for x in make_step(2, hk, hv, 7))
    cs = torch.zeros((4, 2 * hk * 128 + hv * 128, 3), dtype=torch.bfloat16, device=gpu)
    ss = torch.zeros((4, hv, 128, 128), device=gpu)
    req = torch.tensor([0, 1], device=gpu)
    with pytest.raises(ValueError):
        gdn_decode_step(qkv, b, a, z, *params, 1e-6, cs, ss.half(), req, hk, hv)
    ss10 = torch.zeros((4, 10, 128, 128), device=gpu)
    with pytest.raises(ValueError):            # value heads not a multiple of key heads
        gdn_decode_step(qkv, b, a, z, *params, 1e-6, cs, ss10, req, 3, 10)


class _StatePool:
    def __init__(self, cs, ss):
        self.cs, self.ss = cs, ss

    def get_linear_states(self, layer_idx):
        return self.cs, self.ss


def test_linear_attention_module_decode(gpu):
    """``LinearAttention.forward`` equals its own projections -> the oracle's
    step -> its out_proj, on an all-decode batch and then on a mixed batch."""
    from types import SimpleNamespace
    from tokenfactory_amd.forward_batch import ForwardBatch
    from tokenfactory_amd.linear_attention import LinearAttention

    cfg = SimpleNamespace(hidden_size=256, linear_num_key_heads=2, linear_num_value_heads=6,
                          linear_key_head_dim=128, linear_value_head_dim=128,
                          linear_conv_kernel_dim=4, rms_norm_eps=1e-6, tp_size=1)
    torch.manual_seed(0)
    mod = LinearAttention(cfg, layer_idx=0).to(gpu)
    with torch.no_grad():
        for p in mod.parameters():
            p.copy_((torch.randn_like(p.float()) * 0.1).to(p.dtype))
        mod.A_log.fill_(-1.0)
    bsz, n_slots = 5, 9
    cs = torch.randn((n_slots, mod.conv_dim, 3)).to(torch.bfloat16)
    ss = torch.randn((n_slots, 6, 128, 128)) * 0.2
    pool = _StatePool(cs.to(gpu), ss.to(gpu))
    req = torch.tensor([7, 0, 3, 8, 2], dtype=torch.int64)
    batch = ForwardBatch(batch_size=bsz, req_pool_indices=req.to(gpu),
                         seq_lens=torch.full((bsz,), 10, device=gpu),
                         prefix_lens=torch.full((bsz,), 9, device=gpu), extend_lens=[1] * bsz,
                         out_cache_loc=torch.zeros((bsz,), dtype=torch.int64, device=gpu),
                         req_to_token=torch.zeros((n_slots, 16), dtype=torch.int64, device=gpu),
                         is_prefill=False)
    hidden = (torch.randn((bsz, 256)) * 0.5).to(torch.bfloat16).to(gpu)
    with torch.no_grad():
        got = mod(hidden, pool, batch)
        qkv, z = mod.in_proj_qkv(hidden), mod.in_proj_z(hidden)
        b, a = mod.in_proj_b(hidden), mod.in_proj_a(hidden)
        conv_w, a_log, dt_bias, norm_w = (t.cpu() for t in mod._kernel_params())
        core_out, _ = og.gdn_decode(qkv.cpu(), a.cpu(), b.cpu(), z.cpu(), conv_w, a_log, dt_bias,
                                    norm_w, 1e-6, cs, ss, req, 2, 6)
        want = mod.out_proj(core_out.to(gpu))
    torch.cuda.synchronize()
    assert torch.allclose(got.float(), want.float(), atol=2e-2, rtol=1e-2)
    assert torch.equal(pool.cs.cpu(), cs)
    # a mixed batch: the extend path, against the oracle's per-request loop
    lens = [1, 4, 1, 9, 2]
    hidden = (torch.randn((sum(lens), 256)) * 0.5).to(torch.bfloat16).to(gpu)
    batch.extend_lens = lens
    with torch.no_grad():
        got = mod(hidden, pool, batch)
        qkv, z = mod.in_proj_qkv(hidden), mod.in_proj_z(hidden)
        b, a = mod.in_proj_b(hidden), mod.in_proj_a(hidden)
        core_out, _ = og.gdn_extend(qkv.cpu(), a.cpu(), b.cpu(), z.cpu(), conv_w, a_log,
                                    dt_bias, norm_w, 1e-6, cs, ss, req, lens, 2, 6)
        want = mod.out_proj(core_out.to(gpu))
    torch.cuda.synchronize()
    assert torch.allclose(got.float(), want.float(), atol=2e-2, rtol=1e-2)
    assert torch.equal(pool.cs.cpu(), cs)
