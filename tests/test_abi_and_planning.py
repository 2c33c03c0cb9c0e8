"""C-ABI surface and host-side planning (CPU only: no kernel is launched)."""
import ctypes
import re
import subprocess
from pathlib import Path

import numpy as np
import pytest

from tokenfactory_amd import _native
from tokenfactory_amd.planning import EXTEND_TILE_ROWS, plan_decode_items, plan_extend

HEADER = Path(__file__).resolve().parent.parent / "include" / "tf_attn.h"


def declared_functions():
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(tf_[a-z0-9_]+)\s*\(", text)))


def test_library_loads_with_matching_abi():
    lib = _native.load()
    assert lib.tf_attn_abi_version() == _native.ABI_VERSION


def test_every_declared_symbol_is_exported_and_bound():
    names = declared_functions()
    assert len(names) >= 9, names
    out = subprocess.run(["nm", "-D", "--defined-only", str(_native.LIB_PATH)],
                         capture_output=True, text=True, check=True).stdout
    exported = {ln.split()[-1] for ln in out.splitlines() if ln.strip()}
    missing = [n for n in names if n not in exported]
    assert not missing, missing
    unbound = [n for n in names if n not in _native.SIGNATURES]
    assert not unbound, unbound


def test_decode_workspace_size_and_unsupported_arguments():
    # One partial slot per (unit) + one per workgroup: index b + u is unique.
    n = _native.decode_workspace_bytes(64, 24, 4, 256, 8192, 512)
    assert n >= (64 * 4 + 512) * 16 * 256 * 4
    # other head dims run the one-wave-per-row kernel, which needs no workspace
    assert _native.decode_workspace_bytes(4, 16, 2, 128, 512, 0) == 0
    assert _native.decode_workspace_bytes(4, 16, 2, 32, 512, 0) == 0
    with pytest.raises(NotImplementedError):
        _native.decode_workspace_bytes(4, 16, 2, 36, 512, 0)        # not a multiple of 8
    with pytest.raises(NotImplementedError):
        _native.decode_workspace_bytes(4, 16, 2, 264, 512, 0)       # above 256
    with pytest.raises(NotImplementedError):
        _native.decode_workspace_bytes(4096, 16, 2, 256, 512, 0)    # > 2048 requests
    with pytest.raises(ValueError):
        _native.decode_workspace_bytes(4, 16, 3, 256, 512, 0)       # 16 % 3 != 0
    with pytest.raises(ValueError):
        _native.decode_workspace_bytes(4, 16, 2, 256, 512, -1)


def test_gdn_extend_workspace_covers_rows_and_chunk_records():
    # Per token row: conv outputs (bf16), split q / k (4 x 128 bf16 per key
    # head), gates (2 fp32 per value head), the row's request (int32); then
    # one 9 KB record per (32-token chunk slot, value head), with
    # n_tokens / 32 + batch + 1 slots; then the 16 KB SiLU table.
    lib = _native.load()
    hk, hv = 16, 48
    row = (2 * hk * 128 + hv * 128) * 2 + hk * 4 * 128 * 2 + hv * 8 + 4
    for n_tok, bsz in [(1, 1), (8320, 132), (70, 3)]:
        got = lib.tf_gdn_extend_workspace_bytes(n_tok, bsz, hk, hv)
        assert got >= n_tok * row + (n_tok // 32 + bsz + 1) * hv * 2304 * 4 + 16384
        assert got <= n_tok * row + 80 + (n_tok // 32 + bsz + 1) * hv * 2304 * 4 + 16384
    assert lib.tf_gdn_extend_workspace_bytes(100, 5, hk, hv) < \
        lib.tf_gdn_extend_workspace_bytes(100, 6, hk, hv)
    assert lib.tf_gdn_extend_workspace_bytes(10, -1, hk, hv) == _native.TF_ERR_INVALID
    assert lib.tf_gdn_extend_workspace_bytes(10, 1, 0, hv) == _native.TF_ERR_INVALID


def test_entry_points_reject_bad_arguments_before_launching():
    lib = _native.load()
    rc = lib.tf_attn_decode(None, 0, None, None, 16, 0, None, None, None, 1, 16, 16,
                            None, None, 0, None, None, 1, 16, 2, 256, 0.0625, None, 0,
                            None, 0, 16, 0, None, 0, 0, None, None)
    assert rc == _native.TF_ERR_INVALID
    assert b"null" in lib.tf_attn_last_error()
    rc = lib.tf_attn_extend(None, 0, None, None, 16, 5, None, None, None, 1, 16, 16,
                            None, None, 0, None, 3, 16, 2, 256, 0.0625, None, 0,
                            None, 0, 0, None, None)
    assert rc == _native.TF_ERR_UNSUPPORTED
    # A misaligned output gate is rejected before anything is launched.
    rc = lib.tf_attn_extend(16, 6144, 16, 16, 16, 0, None, None, 16, 1, 16, 16,
                            16, 16, 0, 16, 3, 24, 4, 256, 0.0625, 16, 6144,
                            8, 12288, 512, None, None)
    assert rc == _native.TF_ERR_INVALID and b"gate" in lib.tf_attn_last_error()
    rc = lib.tf_kv_write(None, None, 0, 0, None, 4, None, None, 16, 0, None, None, 2, 256,
                         None)
    assert rc == _native.TF_ERR_INVALID
    # Zero-sized work is a no-op that succeeds without touching any pointer.
    assert lib.tf_kv_write(None, None, 0, 0, None, 0, None, None, 16, 0, None, None, 2, 256,
                           None) == 0
    assert lib.tf_gather_kv(None, 0, 16, 512, None, 1, 16, 16, None, 0, 5, None, None) == 0


def test_gdn_decode_workspace_holds_conv_outputs_and_gates():
    """The decode workspace is the bf16 conv outputs [B, conv_dim] followed by
    the fp32 gates [B, Hv, 2], 16-byte aligned; a smaller or misaligned one is
    rejected before anything is launched (the pointers below are never used)."""
    lib = _native.load()
    bsz, hk, hv = 4, 16, 48
    conv_dim = 2 * hk * 128 + hv * 128
    need = bsz * (conv_dim * 2 + hv * 8)
    assert lib.tf_gdn_decode_workspace_bytes(bsz, hk, hv) == need
    p = 1 << 20   # a 16-byte aligned stand-in address for every tensor

    def call(ws, ws_bytes):
        return lib.tf_gdn_decode(p, conv_dim, p, p, hv, p, hv * 128, p, p, p, p, 1e-6,
                                 p, 3 * conv_dim, p, hv * 128 * 128, p, bsz, 8, hk, hv, 128,
                                 128, 4, p, hv * 128, None, 0, ws, ws_bytes, None)

    assert call(p, need - 1) == _native.TF_ERR_INVALID        # no room for the gates
    assert b"workspace" in lib.tf_attn_last_error()
    assert call(p + 8, need) == _native.TF_ERR_INVALID        # 8-byte aligned only
    assert b"16-byte aligned" in lib.tf_attn_last_error()


def _expected_extend_items(lens, hq, hkv, skip_decode):
    g = hq // hkv
    starts = np.concatenate([[0], np.cumsum(lens)[:-1]])
    order = sorted([b for b in range(len(lens)) if not (skip_decode and lens[b] == 1)],
                   key=lambda b: -lens[b])
    items = []
    for b in order:
        tiles = -(-lens[b] * g // EXTEND_TILE_ROWS)
        for t in reversed(range(tiles)):
            for h in range(hkv):
                items.append([b, h, t * EXTEND_TILE_ROWS, starts[b], lens[b], 0, 0, 0])
    return np.array(items, dtype=np.int32).reshape(-1, 8)


@pytest.mark.parametrize("lens", [[1], [5], [3, 1, 700, 1, 22], [2048] * 4 + [1] * 128])
@pytest.mark.parametrize("skip", [False, True])
def test_plan_extend_covers_every_row_once(lens, skip):
    hq, hkv = 24, 4
    work = plan_extend(lens, hq, hkv, skip)
    np.testing.assert_array_equal(work, _expected_extend_items(lens, hq, hkv, skip))
    # Coverage: each (request, kv head, row) appears in exactly one tile.
    g = hq // hkv
    cover = {}
    for b, h, r0, qs, e, *_ in work.tolist():
        for r in range(r0, min(r0 + EXTEND_TILE_ROWS, e * g)):
            cover[(b, h, r)] = cover.get((b, h, r), 0) + 1
    want = {(b, h, r) for b, e in enumerate(lens) if not (skip and e == 1)
            for h in range(hkv) for r in range(e * g)}
    assert set(cover) == want and all(v == 1 for v in cover.values())


def test_plan_decode_items_lists_single_token_requests():
    items, rows = plan_decode_items([4, 1, 1, 7, 1])
    assert items.tolist() == [1, 2, 4]
    assert rows.tolist() == [4, 5, 13]
    with pytest.raises(ValueError):
        plan_decode_items([3, 0])
