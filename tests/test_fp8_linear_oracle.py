"""Pins of the block-FP8 linear oracle (CPU only).

Each check fixes the oracle by something other than its own formula: the e4m3
bit layout, tie cases of the rounding, closed forms of the GEMM, explicit
loops on tiny inputs, and the parameter shapes the reference's own tests state.
"""
import math

import numpy as np
import pytest
import torch

from oracle import fp8_linear as ofl
from tokenfactory_amd.fp8_linear import Fp8Linear


def e4m3_from_bits(code: int) -> float:
    """OCP E4M3FN: 1 sign, 4 exponent (bias 7), 3 mantissa bits; no inf,
    S.1111.111 is NaN; exponent 0 is subnormal (m / 8 * 2^-6)."""
    s = -1.0 if code & 0x80 else 1.0
    e, m = (code >> 3) & 0xF, code & 7
    if e == 15 and m == 7:
        return math.nan
    if e == 0:
        return s * (m / 8.0) * 2.0 ** -6
    return s * (1 + m / 8.0) * 2.0 ** (e - 7)


def test_e4m3_decode_table():
    codes = torch.arange(256, dtype=torch.uint8).view(torch.float8_e4m3fn).float()
    for c in range(256):
        want = e4m3_from_bits(c)
        got = float(codes[c])
        assert (math.isnan(want) and math.isnan(got)) or got == want, (c, got, want)
    assert float(codes[0x7E]) == 448.0 and float(codes[0x01]) == 2.0 ** -9


def test_e4m3_encode_ties_to_even():
    pos = sorted(e4m3_from_bits(c) for c in range(0x7F))
    mids = [(a + b) / 2 for a, b in zip(pos[:-1], pos[1:])]
    x = torch.tensor(mids, dtype=torch.float32)
    q = x.to(torch.float8_e4m3fn).view(torch.uint8).numpy().astype(int)
    for i, code in enumerate(q):
        # the midpoint of codes i and i + 1 goes to the even one
        assert code in (i, i + 1) and code % 2 == 0, (mids[i], code)


def test_activation_scale_is_bf16_rounded():
    # amax = 1.0: x_scale = bf16(1 / 448); all-zero x: the 1e-12 floor
    x = torch.zeros((3, 32), dtype=torch.bfloat16)
    x[1, 5] = -1.0
    xq, sx = ofl.quantize_activations(x)
    want = float(torch.tensor(1.0 / 448.0, dtype=torch.float32).to(torch.bfloat16))
    assert float(sx) == want and float(sx) != np.float32(1.0) / np.float32(448.0)
    assert float(xq.float()[1, 5]) == pytest.approx(-1.0 / want, rel=2 ** -3)
    _, s0 = ofl.quantize_activations(torch.zeros((2, 16), dtype=torch.bfloat16))
    assert float(s0) == float(torch.tensor(1e-12 / 448.0).to(torch.bfloat16)) > 0
    # the largest |x| maps to +-448 exactly when x_scale is exact
    x = torch.tensor([[448.0 * 2.0 ** -4, -1.0, 0.5, 0.0] * 4], dtype=torch.bfloat16)
    xq, sx = ofl.quantize_activations(x)
    assert float(sx) == 2.0 ** -4 and float(xq.float()[0, 0]) == 448.0


def test_nan_in_activations_poisons_scale():
    x = torch.ones((2, 16), dtype=torch.bfloat16)
    x[0, 3] = float("nan")
    xq, sx = ofl.quantize_activations(x)
    assert math.isnan(float(sx)) and torch.isnan(xq.float()).all()


def rand_case(m, n, k, bh=128, bw=128, seed=0, bias=True):
    g = torch.Generator().manual_seed(seed)
    x = (torch.randn((m, k), generator=g) * 3).to(torch.bfloat16)
    w = torch.randn((n, k), generator=g) * torch.rand((n, 1), generator=g) * 0.1
    wq, ws = ofl.quantize_weight_blocks(w, bh, bw)
    b = (torch.randn((n,), generator=g)).to(torch.bfloat16) if bias else None
    return x, wq, ws, b


@pytest.mark.parametrize("m,n,k,bh,bw", [(5, 200, 384, 128, 128), (3, 130, 256, 64, 256),
                                         (1, 16, 128, 128, 128)])
def test_gemm_equals_dequantized_matmul(m, n, k, bh, bw):
    x, wq, ws, b = rand_case(m, n, k, bh, bw)
    out, xq, sx = ofl.block_fp8_linear(x, wq, ws, b, bh, bw)
    closed = (xq.to(torch.float64) * float(sx)) @ ofl.dequantize_weight(wq, ws, bh, bw).T
    closed += b.to(torch.float64)[None, :]
    assert torch.allclose(out.double(), closed, rtol=1e-6, atol=1e-6)


def test_gemm_explicit_loops_tiny():
    x, wq, ws, b = rand_case(2, 3, 256, 2, 128, seed=3)
    xq, sx = ofl.quantize_activations(x)
    got = ofl.block_gemm(xq, sx, wq, ws, 2, 128, b)
    a, w = xq.float().tolist(), wq.float().tolist()
    for i in range(2):
        for j in range(3):
            acc = 0.0
            for k in range(256):
                acc += a[i][k] * w[j][k] * float(sx) * float(ws[j // 2, k // 128])
            acc += float(b[j])
            assert got[i, j].item() == pytest.approx(acc, rel=1e-6, abs=1e-6)


def test_gemm_all_ones_exposes_scale_index():
    m, n, k, bh, bw = 4, 384, 512, 128, 128
    ws = torch.arange(1, 3 * 4 + 1, dtype=torch.float32).reshape(3, 4) / 7.0
    xq = torch.ones((m, k)).to(torch.float8_e4m3fn)
    wq = torch.ones((n, k)).to(torch.float8_e4m3fn)
    sx = torch.tensor([0.5])
    out = ofl.block_gemm(xq, sx, wq, ws, bh, bw)
    want = 0.5 * 128 * ws.double().sum(dim=1)        # per n-block
    for j in range(n):
        assert out[0, j].item() == pytest.approx(float(want[j // bh]), rel=1e-6)
    # no block scales: every scale is 1
    out1 = ofl.block_gemm(xq, sx, wq, None)
    assert torch.all(out1 == 0.5 * k)


def test_fp8_linear_parameter_shapes_match_reference_checkpoints():
    # tests/test_qwen3_8_model.py:66-71 (q_proj with gate) and
    # tests/test_tensor_parallel.py:47-60 (TP=4 row-parallel out_proj)
    q = Fp8Linear(5120, 24 * 256 * 2, device="meta")
    assert q.weight.shape == (12288, 5120) and q.weight_scale_inv.shape == (96, 40)
    o = Fp8Linear(6144 // 4, 5120, device="meta")
    assert o.weight.shape == (5120, 1536) and o.weight_scale_inv.shape == (40, 12)
    assert q.weight.dtype == torch.float8_e4m3fn and q.weight_scale_inv.dtype == torch.float32


def test_fp8_linear_quantize_from_round_trip():
    g = torch.Generator().manual_seed(1)
    w = torch.randn((200, 384), generator=g)
    lin = Fp8Linear(384, 200, block_size=(128, 128))
    lin.quantize_from(w)
    wq, ws = ofl.quantize_weight_blocks(w)
    assert torch.equal(lin.weight.view(torch.uint8), wq.view(torch.uint8))
    assert torch.equal(lin.weight_scale_inv, ws)
    deq = lin.dequantize_weight(torch.float32)
    assert torch.allclose(deq.double(), ofl.dequantize_weight(wq, ws), rtol=1e-6, atol=0)
    # e4m3 keeps 3 mantissa bits: |w - deq| <= 2^-4 |w| (+ the subnormal floor)
    assert ((w - deq).abs() <= w.abs() * 2 ** -4 + ws.max() * 2 ** -9).all()
