"""Pins the CPU oracle independently of its own formulas (CPU only).

Two independent statements of the reference's attention semantics - the op-for-op
PyTorch restatement (``oracle.slot_attention``) and the float64 loop oracle
(``oracle.brute``) - are checked against each other and against facts that do
not restate either: closed-form special cases, invariances of the slot
indirection, the reference's own cache-equivalence property
(``tests/test_hybrid_radix_cache.py:111-223`` of the reference), and planted
mistakes that must each break at least one pin.
"""
import numpy as np
import pytest
import torch

from oracle.brute import attention_brute, attention_dense
from oracle.slot_attention import gather_kv_ref, slot_based_attention_ref
from tests.helpers import as_numpy, brute, rebatch, restatement, small_case

CASES = [
    # (seq_lens, ext_lens, hq, hkv) covering the three reference branches
    ([7], [1], 4, 1),               # bsz == 1, decode
    ([9], [5], 4, 2),               # bsz == 1, extend with a prefix
    ([6], [6], 2, 2),               # bsz == 1, pure prefill
    ([5, 9, 3], [1, 1, 1], 4, 1),   # batched pure decode
    ([8, 4, 11], [4, 1, 2], 8, 2),  # batched extend / mixed
    ([12, 12], [12, 3], 4, 4),      # prefill + extend, MHA
]


@pytest.mark.parametrize("seq,ext,hq,hkv", CASES)
def test_dense_oracle_matches_loop_oracle(seq, ext, hq, hkv):
    wl = small_case(seq, ext, hq, hkv, d=16, seed=1)
    np.testing.assert_allclose(brute(wl, dense=True), brute(wl), rtol=1e-12, atol=1e-12)


@pytest.mark.parametrize("seq,ext,hq,hkv", CASES)
def test_restatement_matches_loop_oracle(seq, ext, hq, hkv):
    wl = small_case(seq, ext, hq, hkv, d=32, seed=2)
    got = as_numpy(restatement(wl))
    np.testing.assert_allclose(got, brute(wl), rtol=1e-5, atol=2e-6)


def test_restatement_matches_oracle_at_head_dim_256_with_shared_prefixes():
    wl = small_case([40, 37, 12, 30], [9, 1, 1, 6], hq=6, hkv=1, d=256, seed=3,
                    groups=[0, 0, 1, 1], prefixes=[28, 5])
    np.testing.assert_allclose(as_numpy(restatement(wl)), brute(wl, dense=True),
                               rtol=2e-5, atol=2e-6)


# ----------------------------------------------------------------- closed forms
# Each pin takes the attention under test, the head dim of its cases and an
# absolute tolerance (None: the fp32 oracles' own); the HIP path runs the same
# pins in bf16 (tests/test_gpu_pins.py).

def _visible_slots(wl, b, t):
    """Slot ids visible to new token t of request b (positions 0 .. P + t)."""
    L = wl.batch.max_seq_len if wl.batch.batch_size == 1 else wl.seq_lens[b]
    P = L - wl.ext_lens[b]
    rtt = wl.batch.req_to_token.cpu().numpy()
    return [max(int(rtt[wl.rows[b], k]), 0) for k in range(P + t + 1)]


def pin_single_key_returns_value(attn, d=16, atol=None):
    wl = small_case([1, 1, 1], [1, 1, 1], hq=4, hkv=2, d=d, seed=4)
    out = attn(wl)
    vp = wl.v_pool.numpy()
    for b in range(3):
        slot = _visible_slots(wl, b, 0)[0]
        for h in range(4):
            if not np.allclose(out[b, h], vp[slot, h // 2], atol=1e-6 if atol is None else atol):
                return False
    return True


def pin_equal_keys_average_visible_values(attn, d=16, atol=None):
    wl = small_case([10, 7, 13], [4, 1, 6], hq=4, hkv=2, d=d, seed=5)
    wl.k_pool[:] = wl.k_pool[1:2].clone()          # every key row identical
    out = attn(wl)
    vp = wl.v_pool.numpy().astype(np.float64)
    row = 0
    for b in range(3):
        for t in range(wl.ext_lens[b]):
            slots = _visible_slots(wl, b, t)
            for h in range(4):
                want = vp[slots, h // 2].mean(axis=0)
                if not np.allclose(out[row, h], want, atol=1e-5 if atol is None else atol):
                    return False
            row += 1
    return True


def pin_dominant_key_selects_its_value(attn, d=16, atol=None):
    """q of head h aligned with one key of kv head h // G: softmax ~ one-hot."""
    wl = small_case([9, 12], [3, 1], hq=4, hkv=2, d=d, seed=6)
    rng = np.random.default_rng(0)
    row = 0
    targets = []
    for b in range(2):
        for t in range(wl.ext_lens[b]):
            slots = _visible_slots(wl, b, t)
            for h in range(4):
                s = slots[int(rng.integers(len(slots)))]
                key = wl.k_pool[s, h // 2]
                wl.q[row, h] = key / key.norm() * 400.0
                targets.append((row, h, s))
            row += 1
    # Give the chosen keys a large norm so they dominate every other key.
    for _, h, s in targets:
        wl.k_pool[s, h // 2] = wl.k_pool[s, h // 2] / wl.k_pool[s, h // 2].norm() * 4.0
    for row, h, s in targets:
        key = wl.k_pool[s, h // 2]
        wl.q[row, h] = key / key.norm() * 400.0
    out = attn(wl)
    vp = wl.v_pool.numpy()
    tol = 1e-4 if atol is None else atol
    return all(np.allclose(out[row, h], vp[s, h // 2], atol=tol) for row, h, s in targets)


def pin_slot_permutation_invariance(attn, d=16, atol=None):
    wl = small_case([11, 6], [4, 1], hq=4, hkv=1, d=d, seed=7, pool=64)
    base = attn(wl)
    perm = torch.randperm(63, generator=torch.Generator().manual_seed(3)) + 1
    new_of_old = torch.zeros(64, dtype=torch.long)
    new_of_old[1:] = perm
    kp, vp = wl.k_pool.clone(), wl.v_pool.clone()
    wl.k_pool[new_of_old] = kp
    wl.v_pool[new_of_old] = vp
    rtt = wl.batch.req_to_token
    live = rtt >= 0
    rtt[live] = new_of_old[rtt[live]]
    return np.allclose(attn(wl), base, atol=1e-6 if atol is None else atol)


def pin_prefix_extend_equals_full_prefill_rows(attn, d=16, atol=None):
    """A request whose first P positions are a cached prefix gives the same rows
    as a fresh prefill of all P + N tokens (the reference's own equivalence)."""
    P, N = 9, 5
    full = small_case([P + N], [P + N], hq=4, hkv=2, d=d, seed=8)
    ref = attn(full)
    ext = rebatch(full, [P + N], [N], full.q[P:].clone())
    return np.allclose(attn(ext), ref[P:], atol=1e-6 if atol is None else atol)


def pin_chunked_extend_equals_one_shot(attn, d=16, atol=None):
    P, N1, N2 = 6, 4, 3
    one = small_case([P + N1 + N2, 5], [N1 + N2, 1], hq=4, hkv=1, d=d, seed=9)
    ref = attn(one)
    a = rebatch(one, [P + N1, 5], [N1, 1], torch.cat([one.q[:N1], one.q[N1 + N2:]]))
    b = rebatch(one, [P + N1 + N2, 5], [N2, 1], torch.cat([one.q[N1:N1 + N2],
                                                           one.q[N1 + N2:]]))
    got = np.concatenate([attn(a)[:N1], attn(b)[:N2]])
    return np.allclose(got, ref[:N1 + N2], atol=1e-6 if atol is None else atol)


def pin_decode_equals_last_prefill_row(attn, d=16, atol=None):
    L = 10
    pre = small_case([L, 4], [L, 1], hq=4, hkv=2, d=d, seed=10)
    ref = attn(pre)
    dec = rebatch(pre, [L, 4], [1, 1], torch.stack([pre.q[L - 1], pre.q[L]]))
    return np.allclose(attn(dec)[0], ref[L - 1], atol=1e-6 if atol is None else atol)


def pin_two_keys_logistic_weight(attn, d=16, atol=None):
    """Two visible keys and a one-hot query: the weight of key 0 is the logistic
    function 1 / (1 + exp(scale * c * (x1 - x0))) of the score gap."""
    import math
    wl = small_case([2, 2], [1, 1], hq=2, hkv=1, d=d, seed=12, scale=0.3)
    rtt = wl.batch.req_to_token.numpy()
    for b in range(2):
        s0, s1 = (int(rtt[wl.rows[b], k]) for k in range(2))
        wl.k_pool[s0, 0, 0] = 1.5 + b
        wl.k_pool[s1, 0, 0] = -0.5
        wl.q[b] = 0.0
        wl.q[b, :, 0] = torch.tensor([2.0, -1.0])
    out = attn(wl)
    vp = wl.v_pool.double().numpy()
    for b in range(2):
        s0, s1 = (int(rtt[wl.rows[b], k]) for k in range(2))
        x0, x1 = float(wl.k_pool[s0, 0, 0]), float(wl.k_pool[s1, 0, 0])
        for h, c in enumerate((2.0, -1.0)):
            w0 = 1.0 / (1.0 + math.exp(0.3 * c * (x1 - x0)))
            want = w0 * vp[s0, 0] + (1 - w0) * vp[s1, 0]
            if not np.allclose(out[b, h], want, atol=1e-5 if atol is None else atol):
                return False
    return True


PINS = [pin_single_key_returns_value, pin_equal_keys_average_visible_values,
        pin_two_keys_logistic_weight,
        pin_dominant_key_selects_its_value, pin_slot_permutation_invariance,
        pin_prefix_extend_equals_full_prefill_rows, pin_chunked_extend_equals_one_shot,
        pin_decode_equals_last_prefill_row]


def _restatement_np(wl):
    return as_numpy(restatement(wl))


def _brute_np(wl):
    return brute(wl)


@pytest.mark.parametrize("pin", PINS, ids=lambda f: f.__name__)
@pytest.mark.parametrize("impl", [_restatement_np, _brute_np], ids=["restatement", "brute"])
def test_oracle_satisfies_pin(pin, impl):
    assert pin(impl)


# ----------------------------------------------------------------- planted mistakes

def _mutant(kind):
    """A float64 attention with one deliberate mistake (pins must reject it)."""

    def attn(wl):
        q = wl.q.double().numpy()
        kp = wl.k_pool.double().numpy()
        vp = wl.v_pool.double().numpy()
        rtt = wl.batch.req_to_token.numpy()
        n_q, n_kv = wl.num_q_heads, wl.num_kv_heads
        group = n_q // n_kv
        seq = [wl.batch.max_seq_len] if wl.batch.batch_size == 1 else wl.seq_lens
        out = np.zeros_like(q)
        base = 0
        for b, row in enumerate(wl.rows):
            L, e = seq[b], wl.ext_lens[b]
            P = L - e
            for t in range(e):
                last = P + t + (1 if kind == "causal_off_by_one" else 0)
                last = min(last, L - 1) if kind != "no_length_mask" else L - 1
                if kind == "causal_off_by_one" and e > 1:
                    last = P + t - 1 if t > 0 else P + t
                slots = [max(int(x), 0) for x in rtt[row, :last + 1]]
                for h in range(n_q):
                    kvh = (h % n_kv) if kind == "gqa_modulo" else h // group
                    sc = kp[slots, kvh] @ q[base + t, h]
                    if kind != "no_scale":
                        sc = sc * wl.scale
                    w = np.exp(sc - sc.max())
                    out[base + t, h] = (w / w.sum()) @ vp[slots, kvh]
            base += e
        return out

    return attn


@pytest.mark.parametrize("kind", ["gqa_modulo", "causal_off_by_one", "no_scale"])
def test_planted_mistake_fails_a_pin(kind):
    attn = _mutant(kind)
    failed = [p.__name__ for p in PINS if not p(attn)]
    assert failed, f"mutation {kind} passed every pin"


def test_unmutated_mutant_harness_passes_all_pins():
    attn = _mutant("none")
    assert all(p(attn) for p in PINS)


# ----------------------------------------------------------------- slot gather

def test_gather_ref_matches_explicit_loops_and_clamps_padding():
    wl = small_case([5, 9, 2], [1, 1, 1], hq=2, hkv=2, d=8, seed=11)
    got = gather_kv_ref(wl.k_pool, wl.batch.req_to_token, wl.batch.req_pool_indices,
                        wl.batch.max_seq_len).numpy()
    rtt = wl.batch.req_to_token.numpy()
    kp = wl.k_pool.numpy()
    for b, row in enumerate(wl.rows):
        for t in range(wl.batch.max_seq_len):
            sid = rtt[row, t]
            want = kp[0] if sid < 0 else kp[sid]
            assert (sid >= 0) == (t < wl.seq_lens[b])
            np.testing.assert_array_equal(got[b, t], want)


@pytest.mark.parametrize("entry", [-1, -3])
def test_negative_slot_ids_follow_each_branch(entry):
    """A negative req_to_token entry v: the bsz == 1 branch indexes the pool
    directly, reading slot S + v (torch indexing, full_attention.py:188-190);
    the batched branches clamp it to slot 0 (:217-219).  With one visible key
    the output is exactly that key's V row (G = 2 heads per kv head)."""
    S = 40
    one = small_case([1], [1], hq=4, hkv=2, d=8, seed=21, pool=S)
    one.batch.req_to_token[one.rows[0], 0] = entry
    got = restatement(one)
    want = one.v_pool[S + entry].repeat_interleave(2, dim=0)
    torch.testing.assert_close(got[0], want, rtol=0, atol=0)
    two = small_case([1, 1], [1, 1], hq=4, hkv=2, d=8, seed=22, pool=S)
    two.batch.req_to_token[two.rows[0], 0] = entry
    got = restatement(two)
    torch.testing.assert_close(got[0], two.v_pool[0].repeat_interleave(2, dim=0), rtol=0,
                               atol=0)
    slot = int(two.batch.req_to_token[two.rows[1], 0])
    torch.testing.assert_close(got[1], two.v_pool[slot].repeat_interleave(2, dim=0), rtol=0,
                               atol=0)


def test_forward_batch_defaults_follow_reference_rules():
    from tokenfactory_amd import ForwardBatch
    fb = ForwardBatch(batch_size=2, req_pool_indices=torch.tensor([3, 1]),
                      seq_lens=torch.tensor([7, 12]), prefix_lens=torch.tensor([6, 9]),
                      extend_lens=[1, 3], out_cache_loc=torch.arange(4),
                      req_to_token=torch.full((4, 16), -1))
    assert fb.max_extend_len == 3 and fb.max_seq_len == 12
    assert fb.extend_lens_tensor.tolist() == [1, 3]
    assert fb.req_pool_indices_list == [3, 1]


def _ocp_e4m3_value(code: int) -> float:
    """OCP 8-bit float E4M3 (FN) decoding from the format definition: sign bit,
    4 exponent bits (bias 7), 3 mantissa bits, subnormals at exponent 0, no
    infinities, S.1111.111 is NaN."""
    sign = -1.0 if code & 0x80 else 1.0
    exp = (code >> 3) & 0xF
    man = code & 0x7
    if exp == 0xF and man == 0x7:
        return float("nan")
    if exp == 0:
        return sign * man / 8.0 * 2.0 ** -6
    return sign * (1.0 + man / 8.0) * 2.0 ** (exp - 7)


def test_e4m3_oracle_matches_ocp_definition():
    """The fp8 oracle's dequantisation of every code equals the OCP formula, and
    its quantisation is round-to-nearest-even onto that table with saturation at
    +-448 (checked on random values, exact table values and every midpoint)."""
    from oracle.kv_quant import dequantize_e4m3, quantize_e4m3
    codes = torch.arange(256, dtype=torch.uint8).view(torch.float8_e4m3fn)
    got = dequantize_e4m3(codes, 1.0).numpy()
    want = np.array([_ocp_e4m3_value(c) for c in range(256)])
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan], want[~nan])

    table = np.unique(want[~nan])                    # sorted finite values
    assert table.max() == 448.0 and table.min() == -448.0
    mids = (table[1:] + table[:-1]) / 2
    rng = np.random.default_rng(5)
    xs = np.concatenate([rng.normal(0, 100, 4000), rng.uniform(-600, 600, 2000), table, mids,
                         [1e-9, -1e-9, 2.0 ** -10, 500.0, -1e6]]).astype(np.float32)

    def rne(x):
        x = min(max(float(x), -448.0), 448.0)
        i = np.searchsorted(table, x)
        if i < len(table) and table[i] == x:
            return x
        lo, hi = table[i - 1], table[i]
        if x - lo != hi - x:
            return lo if x - lo < hi - x else hi
        # tie: the even code (mantissa lsb 0)
        code_lo = int(np.nonzero(want == lo)[0][0])
        return lo if (code_lo & 1) == 0 else hi

    q = dequantize_e4m3(quantize_e4m3(torch.from_numpy(xs), 1.0), 1.0).numpy()
    ref = np.array([rne(x) for x in xs])
    assert np.array_equal(q, ref)
    # a scale divides before rounding
    q2 = dequantize_e4m3(quantize_e4m3(torch.from_numpy(xs[:100]), 0.5), 0.5).numpy()
    assert np.array_equal(q2, np.array([rne(x / 0.5) for x in xs[:100]]) * 0.5)
