"""KV write and slot gather kernels vs PyTorch indexing / the oracle (bit-exact)."""
import pytest
import torch

from oracle.kv_quant import quantize_e4m3
from oracle.slot_attention import gather_kv_ref
from tests.helpers import small_case
from tokenfactory_amd import gather_kv, slot_based_attention, write_kv

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32, torch.float8_e4m3fn])
def test_gather_is_bit_exact(gpu, dtype):
    wl = small_case([37, 1, 130, 64, 5], [1] * 5, hq=8, hkv=2, d=256, seed=21, device=gpu)
    pool = wl.k_pool.float()
    pool = pool.to(dtype) if dtype != torch.float8_e4m3fn else quantize_e4m3(pool, 0.01)
    # Two extra rows of the table are entirely -1 (padding clamps to slot 0).
    rpi = torch.cat([wl.batch.req_pool_indices,
                     torch.tensor([w for w in range(wl.batch.req_to_token.shape[0])
                                   if w not in wl.rows][:2], device=gpu)])
    got = gather_kv(pool, wl.batch.req_to_token, rpi, wl.batch.max_seq_len)
    ref = gather_kv_ref(pool.cpu(), wl.batch.req_to_token.cpu(), rpi.cpu(),
                        wl.batch.max_seq_len)
    assert torch.equal(got.cpu().view(torch.uint8), ref.view(torch.uint8))


def test_kv_write_bf16_is_bit_exact(gpu):
    g = torch.Generator(device=gpu).manual_seed(1)
    S, T, H, D = 512, 77, 4, 256
    kb = torch.zeros((S, H, D), dtype=torch.bfloat16, device=gpu)
    vb = torch.zeros_like(kb)
    loc = torch.randperm(S - 1, generator=g, device=gpu)[:T] + 1
    k = torch.randn((T, H, D), generator=g, device=gpu).to(torch.bfloat16)
    v = torch.randn((T, H, D), generator=g, device=gpu).to(torch.bfloat16)
    write_kv(kb, vb, loc, k, v)
    rk, rv = torch.zeros_like(kb), torch.zeros_like(vb)
    rk[loc], rv[loc] = k, v
    assert torch.equal(kb, rk) and torch.equal(vb, rv)


def test_kv_write_fp32_source_rounds_like_torch(gpu):
    g = torch.Generator(device=gpu).manual_seed(2)
    S, T, H, D = 300, 33, 2, 256
    kb = torch.zeros((S, H, D), dtype=torch.bfloat16, device=gpu)
    vb = torch.zeros_like(kb)
    loc = torch.randperm(S - 1, generator=g, device=gpu)[:T] + 1
    k = torch.randn((T, H, D), generator=g, device=gpu) * 3
    v = torch.randn((T, H, D), generator=g, device=gpu) * 1e-3
    write_kv(kb, vb, loc, k, v)
    rk, rv = torch.zeros_like(kb), torch.zeros_like(vb)
    rk[loc], rv[loc] = k.to(torch.bfloat16), v.to(torch.bfloat16)
    assert torch.equal(kb, rk) and torch.equal(vb, rv)


def _special_values(n, device):
    """Values that exercise e4m3 rounding: ties, subnormals, saturation, signs."""
    codes = torch.arange(256, dtype=torch.uint8).view(torch.float8_e4m3fn).float()
    codes = codes[torch.isfinite(codes)]
    mids = (codes.sort().values[1:] + codes.sort().values[:-1]) / 2     # exact ties
    extra = torch.tensor([0.0, -0.0, 448.0, 449.0, 464.0, 500.0, 1e6, -1e6, 2.0 ** -10,
                          2.0 ** -9, 1.5 * 2.0 ** -9, 3 * 2.0 ** -10, 2.0 ** -6 * 0.9999])
    vals = torch.cat([codes, mids, extra])
    reps = (n + vals.numel() - 1) // vals.numel()
    return vals.repeat(reps)[:n].to(device)


@pytest.mark.parametrize("src_dtype", [torch.float32, torch.bfloat16])
def test_kv_write_fp8_matches_oracle_quantisation(gpu, src_dtype):
    S, T, H, D = 128, 40, 2, 256
    kb = torch.zeros((S, H, D), dtype=torch.float8_e4m3fn, device=gpu)
    vb = torch.zeros_like(kb)
    loc = torch.arange(1, T + 1, device=gpu)
    k = _special_values(T * H * D, gpu).view(T, H, D)
    g = torch.Generator(device=gpu).manual_seed(3)
    v = torch.randn((T, H, D), generator=g, device=gpu) * 5
    k, v = k.to(src_dtype), v.to(src_dtype)
    ks = torch.tensor([1.0], device=gpu)
    vs = torch.tensor([0.37], device=gpu)
    write_kv(kb, vb, loc, k, v, ks, vs)
    want_k = quantize_e4m3(k.cpu(), 1.0)
    want_v = quantize_e4m3(v.cpu(), 0.37)
    assert torch.equal(kb[1:T + 1].cpu().view(torch.uint8), want_k.view(torch.uint8))
    assert torch.equal(vb[1:T + 1].cpu().view(torch.uint8), want_v.view(torch.uint8))


def test_fp8_decode_of_single_key_returns_exact_dequantised_row(gpu):
    """L = 1: softmax weight is exactly 1, so the output is v_scale * e4m3(V) rounded
    to bf16 - this checks the in-kernel e4m3 -> bf16 conversion on every code."""
    codes = torch.arange(256, dtype=torch.uint8)
    finite = torch.isfinite(codes.view(torch.float8_e4m3fn).float())
    codes = codes[finite]                                          # 254 codes
    n_req = 4
    wl = small_case([1] * n_req, [1] * n_req, hq=6, hkv=1, d=256, seed=5, device=gpu,
                    dtype=torch.bfloat16)
    kq = torch.zeros(wl.k_pool.shape, dtype=torch.uint8)
    vq = torch.zeros(wl.v_pool.shape, dtype=torch.uint8)
    flat = codes.repeat(8)[: n_req * 256]
    rtt = wl.batch.req_to_token.cpu()
    for b in range(n_req):
        slot = int(rtt[wl.rows[b], 0])
        vq[slot, 0] = flat[b * 256:(b + 1) * 256]
    k_pool = kq.view(torch.float8_e4m3fn).to(gpu)
    v_pool = vq.view(torch.float8_e4m3fn).to(gpu)
    vs = 0.5
    out = slot_based_attention(wl.q, k_pool, v_pool, wl.batch, scaling=wl.scale,
                               k_scale=torch.tensor([1.0], device=gpu),
                               v_scale=torch.tensor([vs], device=gpu))
    for b in range(n_req):
        want = (flat[b * 256:(b + 1) * 256].view(torch.float8_e4m3fn).float() * vs)
        want = want.to(torch.bfloat16)
        for h in range(6):
            assert torch.equal(out[b, h].cpu(), want), (b, h)
