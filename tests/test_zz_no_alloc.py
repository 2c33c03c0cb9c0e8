"""tf_attn_decode_noalloc (split scratch in a library-owned static device array)
against tf_attn_decode (caller workspace), through the C ABI.

The two entry points run the same kernels with the same split plan, so their
outputs must be bit-identical.  Two calls in a row, the second with a smaller
input (the static array still holds the first call's partials), then a call
whose scratch need exceeds the array, which must be rejected before launching.
"""
import pytest
import torch

from tests.helpers import assert_attn_close, restatement, small_case
from tokenfactory_amd import _native, workloads
from tokenfactory_amd.attention import SlotAttentionCall

pytestmark = pytest.mark.gpu


def _ptr(t):
    return None if t is None else t.data_ptr()


def noalloc(call, out, num_workgroups=0):
    """tf_attn_decode_noalloc with the arguments ``call`` passes to tf_attn_decode."""
    return _native.call("tf_attn_decode_noalloc", call.q.data_ptr(), call.q.stride(0),
                        *call._pool_args, _ptr(call._items), _ptr(call._rows), call.n_dec,
                        call.n_q, call.n_kv, call.head_dim, call.scaling,
                        out.data_ptr(), out.stride(0), call.max_len, num_workgroups,
                        *call._epilogue_args, call.stream.cuda_stream)


def check_pair(wl, what, gate=None, workgroups=0):
    print(f"[noalloc] {what}: B={wl.batch.batch_size} L<={wl.batch.max_seq_len}", flush=True)
    call = SlotAttentionCall(wl.q, wl.k_pool, wl.v_pool, wl.batch, scaling=wl.scale,
                             k_scale=wl.k_scale, v_scale=wl.v_scale, gate=gate,
                             decode_workgroups=workgroups)
    assert call.n_dec and not call.n_work
    want = call.run().clone()
    got = torch.full_like(want, float("nan"))
    noalloc(call, got, workgroups)
    torch.cuda.synchronize()
    assert torch.equal(got, want), f"{what}: no-alloc decode differs from tf_attn_decode"
    return got


def test_noalloc_decode_matches_workspace_decode_twice(gpu):
    big = workloads.decode_b64(device=gpu, pool_slots=(1 << 19) + 1)
    out = check_pair(big, "decode_b64 shape")
    sub = [0, 17, 40, 63]
    small = workloads.subset(big, sub)
    assert_attn_close(out[sub], restatement(small), what="noalloc vs oracle (4 rows)")
    # Second call, smaller: 9 requests, an fp8 pool, a fixed grid of 37 workgroups.
    fp8 = workloads.build("fp8", [5, 700, 64, 3000, 1, 17, 900, 2048, 33], [1] * 9,
                          num_q_heads=24, num_kv_heads=4, head_dim=256, pool_slots=8192,
                          device=gpu, seed=3, kv_fp8=True)
    got = check_pair(fp8, "fp8, 37 workgroups", workgroups=37)
    assert_attn_close(got, restatement(fp8), what="noalloc fp8 vs oracle")


def test_noalloc_decode_with_gate_and_bsz1(gpu):
    wl = small_case([4097], [1], hq=24, hkv=4, d=256, seed=5, device=gpu,
                    dtype=torch.bfloat16)
    gate = torch.randn_like(wl.q)
    check_pair(wl, "bsz 1, gated", gate=gate)


def test_noalloc_rejects_calls_beyond_the_static_array(gpu):
    # 2048 requests x 4 kv heads = 8192 split units -> ~139 MB of partials > 32 MiB.
    wl = small_case([2] * 2048, [1] * 2048, hq=24, hkv=4, d=256, seed=1, device=gpu,
                    dtype=torch.bfloat16)
    call = SlotAttentionCall(wl.q, wl.k_pool, wl.v_pool, wl.batch, scaling=wl.scale)
    out = torch.zeros_like(wl.q)
    with pytest.raises(NotImplementedError, match="static buffer"):
        noalloc(call, out)
    torch.cuda.synchronize()
    assert not out.any(), "a rejected call must not launch"
