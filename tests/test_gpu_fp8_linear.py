"""Block-FP8 linear on the GPU against the oracle.

* Activation quantisation (``tf_fp8_act_quant``): bit-exact -- the same
  ``x_scale`` and the same e4m3 byte for every element (NaN positions equal).
* GEMM (``tf_fp8_block_gemm``): the kernel forms the same fp8 x fp8 products
  exactly, accumulates them in fp32 in its own order and rounds to bf16; the
  oracle accumulates exactly. Allowed: one bf16 rounding (2^-8 relative) plus
  2^-16 of the absolute sum of the terms (fp32 accumulation), and in any case
  the bf16 bar of 2e-2 absolute / 1e-2 relative against the fp32 reference,
  the absolute part taken in units of the output's RMS (without block scales
  the raw e4m3 weights reach 448 and outputs run into the thousands).
"""
import math

import pytest
import torch

from oracle import fp8_linear as ofl
from tokenfactory_amd import fp8_linear as fl

pytestmark = pytest.mark.gpu


def make_weight(n, k, bh, bw, seed, device):
    g = torch.Generator().manual_seed(seed)
    w = torch.randn((n, k), generator=g) * (torch.rand((n, 1), generator=g) + 0.05) * 0.05
    wq, ws = ofl.quantize_weight_blocks(w, bh, bw)
    return wq.to(device), ws.to(device)


def make_x(m, k, seed, device, scale=2.0, row_stride=None):
    g = torch.Generator().manual_seed(seed + 1000)
    x = (torch.randn((m, k), generator=g) * scale).to(torch.bfloat16)
    if row_stride is None:
        return x.to(device)
    buf = torch.zeros((m, row_stride), dtype=torch.bfloat16)
    buf[:, :k] = x
    return buf.to(device)[:, :k]


def check_quant(x):
    xq, sx = fl.quantize_activations(x)
    ref_q, ref_s = ofl.quantize_activations(x.cpu())
    torch.cuda.synchronize()
    got_s, want_s = float(sx.cpu()), float(ref_s)
    assert (math.isnan(got_s) and math.isnan(want_s)) or got_s == want_s, (got_s, want_s)
    gq, wq = xq.cpu().float(), ref_q.float()
    assert torch.equal(torch.isnan(gq), torch.isnan(wq))
    ok = ~torch.isnan(wq)
    same = xq.cpu().view(torch.uint8)[ok] == ref_q.view(torch.uint8)[ok]
    assert bool(same.all()), f"{int((~same).sum())} of {int(ok.sum())} e4m3 bytes differ"
    return xq, sx


@pytest.mark.parametrize("m,k,row_stride", [(1, 6144, None), (7, 6144, None), (300, 1536, None),
                                            (64, 16, None), (33, 512, 528)])
def test_quant_bit_exact(gpu, m, k, row_stride):
    print(f"[fp8 quant] m={m} k={k} stride={row_stride}", flush=True)
    check_quant(make_x(m, k, m + k, gpu, row_stride=row_stride))


def test_quant_special_values(gpu):
    print("[fp8 quant] special values", flush=True)
    x = make_x(40, 256, 5, gpu, scale=1e-3)
    x[3, :8] = torch.tensor([0.0, -0.0, 1e-30, -1e-30, 65504.0, -3.0e38, 2.0 ** -133, 1.0],
                            dtype=torch.bfloat16)
    check_quant(x)                       # a huge amax drives most entries to zero
    check_quant(torch.zeros((5, 64), dtype=torch.bfloat16, device=gpu))
    y = make_x(9, 128, 6, gpu)
    y[2, 7] = float("inf")
    check_quant(y)                       # x_scale = inf: finite / inf = 0, inf / inf = NaN
    z = make_x(9, 128, 7, gpu)
    z[4, 100] = float("nan")
    check_quant(z)                       # NaN amax: everything NaN


def gemm_case(gpu, m, n, k, bh=128, bw=128, bias=False, no_scales=False, out_stride=None,
              seed=0):
    print(f"[fp8 gemm] m={m} n={n} k={k} bh={bh} bw={bw} bias={bias} "
          f"no_scales={no_scales} out_stride={out_stride}", flush=True)
    wq, ws = make_weight(n, k, bh, bw, seed, gpu)
    if no_scales:
        ws = None
    x = make_x(m, k, seed, gpu)
    b = None
    if bias:
        g = torch.Generator().manual_seed(seed + 7)
        b = torch.randn((n,), generator=g).to(torch.bfloat16).to(gpu)
    xq, sx = check_quant(x)
    out = None
    if out_stride is not None:
        out = torch.full((m, out_stride), float("nan"), dtype=torch.bfloat16, device=gpu)[:, :n]
    got = fl.block_fp8_gemm(xq, sx, wq, ws, b, bh, bw, out=out)
    torch.cuda.synchronize()
    ref = ofl.block_gemm(xq.cpu(), sx.cpu(), wq.cpu(), None if ws is None else ws.cpu(), bh, bw,
                         None if b is None else b.cpu())
    mag = ofl.block_gemm(xq.cpu().float().abs().to(torch.float8_e4m3fn), sx.cpu(),
                         wq.cpu().float().abs().to(torch.float8_e4m3fn),
                         None if ws is None else ws.cpu(), bh, bw)
    if b is not None:
        mag += b.cpu().float().abs()[None, :]
    g32 = got.cpu().float()
    assert torch.isfinite(g32).all()
    err = (g32 - ref).abs()
    bound = ref.abs() * 2.0 ** -8 + mag * 2.0 ** -16 + 1e-30
    worst = float((err / bound).max())
    assert worst <= 1.0, f"error {worst:.3f} x the bound"
    rms = float(ref.pow(2).mean().sqrt())
    assert torch.allclose(g32, ref, atol=2e-2 * rms, rtol=1e-2)
    if out_stride is not None:          # the padding columns stay untouched
        full = out.as_strided((m, out_stride), (out_stride, 1)).cpu()
        assert torch.isnan(full[:, n:].float()).all()
    print(f"[fp8 gemm] max |err| {float(err.max()):.3e}, worst/bound {worst:.3f}", flush=True)


@pytest.mark.parametrize("m,bh", [(8, 128), (64, 128), (300, 128), (1100, 128), (64, 96),
                                  (1100, 96)])
def test_gemm_scale_indexing_closed_form(gpu, m, bh):
    """Row r of xq holds 1.0 at one column of K block kb0[r] and 2.0 at one of
    another block kb1[r]; the weights are all 1.0, x_scale is 0.25 and the block
    scales are distinct powers of two.  Then out[r, n] = 0.25 (ws[n / bh, kb0] +
    2 ws[n / bh, kb1]) is exact in fp32 and the kernel must return its bf16
    rounding bit for bit; a transposed or shifted scale index, or a K slice
    taken from the wrong place, changes the powers."""
    print(f"[fp8 gemm] closed form m={m} bh={bh}", flush=True)
    n, k = 640, 1024
    nb, kb = -(-n // bh), k // 128
    e = (torch.arange(nb)[:, None] * 3 + torch.arange(kb)[None, :] * 5) % 11 - 5
    ws = torch.pow(2.0, e.double())
    g = torch.Generator().manual_seed(m + bh)
    kb0 = torch.randint(0, kb, (m,), generator=g)
    kb1 = (kb0 + torch.randint(1, kb, (m,), generator=g)) % kb
    x = torch.zeros((m, k))
    rows = torch.arange(m)
    x[rows, kb0 * 128 + torch.randint(0, 128, (m,), generator=g)] = 1.0
    x[rows, kb1 * 128 + torch.randint(0, 128, (m,), generator=g)] = 2.0
    xq = x.to(torch.float8_e4m3fn).to(gpu)
    wq = torch.ones((n, k)).to(torch.float8_e4m3fn).to(gpu)
    sx = torch.tensor([0.25], device=gpu)
    got = fl.block_fp8_gemm(xq, sx, wq, ws.float().to(gpu), None, bh, 128)
    torch.cuda.synchronize()
    nblk = torch.arange(n) // bh
    want = 0.25 * (ws[nblk[None, :], kb0[:, None]] + 2.0 * ws[nblk[None, :], kb1[:, None]])
    assert torch.equal(got.cpu(), want.to(torch.bfloat16)), "outputs differ from the closed form"


@pytest.mark.parametrize("m", [1, 8, 32, 33, 64, 100, 128, 129, 300])
def test_gemm_oproj_shape(gpu, m):
    # o_proj of one GPU: in = 24 heads x 256, out = hidden 5120
    gemm_case(gpu, m, 5120, 6144, seed=m)


@pytest.mark.parametrize("m,n", [(1025, 640), (1500, 320), (2048, 5120)])
def test_gemm_large_m(gpu, m, n):
    # the 8-wave tiles for large M (one round of 192-row tiles at these
    # sizes), ragged in M and in N tiles
    gemm_case(gpu, m, n, 6144 if n < 5120 else 1536, bias=n == 320, seed=m)


@pytest.mark.parametrize("bh", [128, 48])
def test_gemm_256_row_tiles(gpu, bh):
    # m = 8320 runs the 256 x 256 tiles (33 x 20 tiles, the last m-tile half
    # full: three rounds of 256-row tiles end before four of 192-row ones),
    # dealt to the XCDs in groups; bh = 48 gives each column its own scale
    gemm_case(gpu, 8320, 5120, 256, bh=bh, bias=bh == 48, seed=15 + bh)


@pytest.mark.parametrize("m,n", [(1100, 256), (2000, 768), (1030, 2304)])
def test_gemm_tile_order_edges(gpu, m, n):
    # the XCD-grouped tile order (192-row tiles here) with fewer tiles than
    # XCDs (6 x 1), with a tile count that is not a multiple of 8 and a last
    # group of m-tiles shorter than the first (11 x 3 = 33: groups of 8 and 3
    # m-tiles), and with fewer m-tiles than a group holds (6 x 9)
    gemm_case(gpu, m, n, 256, bias=True, seed=m + n)


@pytest.mark.parametrize("k", [128, 256, 384])
def test_gemm_short_k(gpu, k):
    # one, two and three 128-wide K slices: the staging pipeline's edge cases
    gemm_case(gpu, 70, 256, k, seed=k)


def test_gemm_ragged_n_bias_and_strides(gpu):
    gemm_case(gpu, 45, 130, 512, bias=True, out_stride=136, seed=11)


def test_gemm_odd_blocks(gpu):
    gemm_case(gpu, 200, 320, 768, bh=48, bw=256, bias=True, seed=12)


def test_gemm_without_block_scales(gpu):
    gemm_case(gpu, 90, 384, 1024, no_scales=True, seed=13)


def test_gemm_tp4_row_parallel_shape(gpu):
    # a TP=4 rank's o_proj shard: in = 6144 / 4
    gemm_case(gpu, 513, 5120, 1536, seed=14)


def test_linear_end_to_end(gpu):
    print("[fp8 linear] 3-D input", flush=True)
    wq, ws = make_weight(640, 768, 128, 128, 21, gpu)
    x = make_x(2 * 37, 768, 21, gpu).view(2, 37, 768)
    got = fl.block_fp8_linear(x, wq, ws, None)
    torch.cuda.synchronize()
    ref, _, _ = ofl.block_fp8_linear(x.reshape(-1, 768).cpu(), wq.cpu(), ws.cpu())
    assert got.shape == (2, 37, 640) and got.dtype == torch.bfloat16
    assert torch.allclose(got.reshape(-1, 640).cpu().float(), ref, atol=2e-2, rtol=1e-2)


def test_module_forward(gpu):
    print("[fp8 linear] Fp8Linear module", flush=True)
    lin = fl.Fp8Linear(512, 256, bias=True, device=gpu)
    g = torch.Generator().manual_seed(3)
    lin.quantize_from(torch.randn((256, 512), generator=g).to(gpu) * 0.02)
    lin.bias.copy_(torch.randn((256,), generator=g).to(torch.bfloat16).to(gpu))
    x = make_x(19, 512, 3, gpu)
    got = lin(x)
    torch.cuda.synchronize()
    ref, _, _ = ofl.block_fp8_linear(x.cpu(), lin.weight.cpu(), lin.weight_scale_inv.cpu(),
                                     lin.bias.cpu())
    assert torch.allclose(got.cpu().float(), ref, atol=2e-2, rtol=1e-2)


@pytest.mark.parametrize("k", [32, 192])
def test_gemm_ragged_k(gpu, k):
    # K not a multiple of 128: the operands are zero-padded to the next slice
    gemm_case(gpu, 11, 256, k, bias=True, seed=k + 1)


def test_gemm_rejects_bad_layouts(gpu):
    sx = torch.ones((1,), dtype=torch.float32, device=gpu)
    wq, ws = make_weight(128, 256, 128, 128, 0, gpu)
    xq = torch.zeros((4, 256), dtype=torch.float8_e4m3fn, device=gpu)
    with pytest.raises(NotImplementedError):  # block_w not a multiple of 128
        fl.block_fp8_gemm(xq, sx, wq, torch.ones((1, 4), device=gpu), None, 128, 64)


def test_gemm_split_k_graph_replays(gpu):
    """A split-K call (partials, then the reduce launch) captured in a graph
    replays bit-identically to the eager call, with eager calls of another
    shape between the replays."""
    print("[fp8 gemm] split-K graph replays", flush=True)
    wq, ws = make_weight(5120, 6144, 128, 128, 43, gpu)
    x = make_x(64, 6144, 5, gpu)
    xq, sx = fl.quantize_activations(x)
    want = fl.block_fp8_gemm(xq, sx, wq, ws, None).clone()
    other = make_x(100, 6144, 6, gpu)
    oq, osx = fl.quantize_activations(other)
    other_want = fl.block_fp8_gemm(oq, osx, wq, ws, None).clone()
    out = torch.empty_like(want)
    stream = torch.cuda.Stream(device=gpu)
    stream.wait_stream(torch.cuda.current_stream(gpu))
    with torch.cuda.stream(stream):
        fl.block_fp8_gemm(xq, sx, wq, ws, None, out=out)    # warm-up on the capture stream
        stream.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=stream):
            fl.block_fp8_gemm(xq, sx, wq, ws, None, out=out)
    torch.cuda.current_stream(gpu).wait_stream(stream)
    for r in range(4):
        out.zero_()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, want), f"replay {r} differs from the eager call"
        got = fl.block_fp8_gemm(oq, osx, wq, ws, None)
        torch.cuda.synchronize()
        assert torch.equal(got, other_want), f"eager call after replay {r} differs"


def test_gemm_split_k_repeats_bit_identically(gpu):
    """Split-K sums its partials in a fixed order: repeated calls (with other
    shapes, and other split counts, in between) give identical bits."""
    print("[fp8 gemm] split-K repeats", flush=True)
    wq, ws = make_weight(5120, 6144, 128, 128, 41, gpu)
    outs = {}
    for m in (64, 100, 64, 8, 64, 100):
        x = make_x(m, 6144, m, gpu)
        xq, sx = fl.quantize_activations(x)
        got = fl.block_fp8_gemm(xq, sx, wq, ws, None)
        torch.cuda.synchronize()
        if m in outs:
            assert torch.equal(got, outs[m]), f"m={m}: a repeated call differs"
        else:
            outs[m] = got.clone()
    gemm_case(gpu, 64, 5120, 6144, seed=64)
