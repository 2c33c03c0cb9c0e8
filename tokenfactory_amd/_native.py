"""ctypes binding of ``libtf_attn.so`` (declared in ``include/tf_attn.h``).

The library is loaded from ``tokenfactory_amd/_lib/`` only; there is no
fallback of any kind: if it is missing or fails to load, every entry point
raises ``NativeLibraryError``.
"""
from __future__ import annotations

import ctypes
import threading
from pathlib import Path
from typing import Optional

LIB_PATH = Path(__file__).resolve().parent / "_lib" / "libtf_attn.so"
ABI_VERSION = 12

TF_DTYPE_BF16 = 0
TF_DTYPE_FP8_E4M3 = 1
TF_DTYPE_FP32 = 2

TF_OK = 0
TF_ERR_INVALID = -1
TF_ERR_UNSUPPORTED = -2
TF_ERR_HIP = -3

TF_FP8_QUANT_WORKSPACE_BYTES = 4096

# Exported symbols and their ctypes signatures (restype, argtypes).
_p = ctypes.c_void_p
_i32 = ctypes.c_int32
_i64 = ctypes.c_int64
_f32 = ctypes.c_float

SIGNATURES = {
    "tf_attn_abi_version": (_i32, []),
    "tf_attn_last_error": (ctypes.c_char_p, []),
    "tf_attn_decode_workspace_bytes": (_i64, [_i32, _i32, _i32, _i32, _i32, _i32]),
    "tf_attn_decode": (_i32, [
        _p, _i64,                      # q, q_row_stride
        _p, _p, _i64, _i32, _p, _p,    # k_pool, v_pool, pool_slots, kv_dtype, k_scale, v_scale
        _p, _i64, _i64, _i64,          # req_to_token, rtt_rows, rtt_row_stride, rtt_cols
        _p, _p, _i32,                  # req_pool_indices, seq_lens, seq_len_override
        _p, _p, _i32,                  # items, q_rows, n_items
        _i32, _i32, _i32, _f32,        # num_q_heads, num_kv_heads, head_dim, scale
        _p, _i64,                      # out, out_row_stride
        _p, _i64, _i32, _i32,          # workspace, workspace_bytes, max_seq_len, num_workgroups
        _p, _i64, _i64,                # gate, gate_row_stride, gate_head_stride
        _p, _p,                        # out_amax, stream
    ]),
    "tf_attn_decode_noalloc": (_i32, [
        _p, _i64,                      # q, q_row_stride
        _p, _p, _i64, _i32, _p, _p,    # k_pool, v_pool, pool_slots, kv_dtype, k_scale, v_scale
        _p, _i64, _i64, _i64,          # req_to_token, rtt_rows, rtt_row_stride, rtt_cols
        _p, _p, _i32,                  # req_pool_indices, seq_lens, seq_len_override
        _p, _p, _i32,                  # items, q_rows, n_items
        _i32, _i32, _i32, _f32,        # num_q_heads, num_kv_heads, head_dim, scale
        _p, _i64,                      # out, out_row_stride
        _i32, _i32,                    # max_seq_len, num_workgroups
        _p, _i64, _i64,                # gate, gate_row_stride, gate_head_stride
        _p, _p,                        # out_amax, stream
    ]),
    "tf_attn_decode_partial": None,   # same signature as tf_attn_decode
    "tf_attn_decode_merge": None,
    "tf_attn_extend": (_i32, [
        _p, _i64,
        _p, _p, _i64, _i32, _p, _p,
        _p, _i64, _i64, _i64,
        _p, _p, _i32,
        _p, _i32,                      # work, n_work
        _i32, _i32, _i32, _f32,
        _p, _i64,
        _p, _i64, _i64,                # gate, gate_row_stride, gate_head_stride
        _p, _p,                        # out_amax, stream
    ]),
    "tf_attn_plan_extend": (_i32, [_p, _i32, _i32, _i32, _i32, _p, _i32]),
    "tf_attn_plan_device_capacity": (_i64, [_i64, _i32, _i32, _i32]),
    "tf_attn_plan_device": (_i32, [
        _p, _i32, _i32, _i32, _i32,    # extend_lens (device int64), batch, heads, decode_to_decode
        _p, _i32,                      # work, work_capacity
        _p, _p, _i32,                  # dec_items, dec_rows, dec_capacity
        _p, _p,                        # status, stream
    ]),
    "tf_attn_plan_decode_items": (_i32, [_p, _i32, _p, _p, _i32]),
    "tf_req_to_token_sync": (_i32, [
        _p, _i64, _i64, _i64,          # req_to_token, rtt_rows, rtt_row_stride, rtt_cols
        _p, _p, _p,                    # req_pool_indices, prefix_lens, seq_lens
        _p, _i64,                      # out_cache_loc, out_cache_loc_len
        _p, _p, _p, _i64,              # patch_from, patch_offsets, patch_vals, patch_vals_len
        _i32, _i32, _p,                # batch_size, num_workgroups, stream
    ]),
    "tf_kv_write": (_i32, [
        _p, _p, _i64, _i32,            # k, v, src_row_stride, src_dtype
        _p, _i64,                      # out_cache_loc, n_tokens
        _p, _p, _i64, _i32, _p, _p,    # k_pool, v_pool, pool_slots, kv_dtype, k_scale, v_scale
        _i32, _i32, _p,                # num_kv_heads, head_dim, stream
    ]),
    "tf_qk_norm_rope_kv_write": (_i32, [
        _p, _i64, _i64,                # q, q_token_stride, q_head_stride
        _p, _i64, _p, _i64,            # k, k_token_stride, v, v_token_stride
        _i64, _i32, _i32, _i32,        # n_tokens, num_q_heads, num_kv_heads, head_dim
        _p, _p, _f32,                  # q_norm_weight, k_norm_weight, eps
        _p, _i32, _i64,                # positions, position_rows, position_row_stride
        _p, _i32, _i32, _i32, _i32,    # inv_freq, rotary_dim, mrope sections
        _i32,                          # mrope_interleaved
        _p, _i64,                      # q_out, q_out_token_stride
        _p, _p, _p, _i64, _i32,        # out_cache_loc, k_pool, v_pool, pool_slots, kv_dtype
        _p, _p, _p,                    # k_scale, v_scale, stream
    ]),
    "tf_fp8_act_quant": (_i32, [
        _p, _i32, _i64, _i64, _i64,    # x, x_dtype, rows, cols, x_row_stride
        _p, _i64, _p,                  # xq, xq_row_stride, x_scale
        _p, _i64, _p,                  # workspace, workspace_bytes, stream
    ]),
    "tf_fp8_act_quant_amax": (_i32, [
        _p, _i32, _i64, _i64, _i64,    # x, x_dtype, rows, cols, x_row_stride
        _p, _i64, _p,                  # xq, xq_row_stride, x_scale
        _p, _p,                        # amax_bits, stream
    ]),
    "tf_fp8_block_gemm": (_i32, [
        _p, _i64, _p,                  # xq, xq_row_stride, x_scale
        _p, _i64,                      # w, w_row_stride
        _p, _i64, _i64, _i32, _i32,    # w_scale, its row / col strides, block_h, block_w
        _p, _i64, _i64, _i64,          # bias, m, n, k
        _p, _i64,                      # out, out_row_stride
        _p, _i64, _p,                  # workspace, workspace_bytes, stream
    ]),
    "tf_fp8_block_gemm_workspace_bytes": (_i64, [_i64, _i64, _i64]),
    "tf_gdn_decode": (_i32, [
        _p, _i64, _p, _p, _i64,        # qkv, qkv_row_stride, a, b, ab_row_stride
        _p, _i64,                      # z, z_row_stride
        _p, _p, _p, _p, _f32,          # conv_weight, a_log, dt_bias, norm_weight, eps
        _p, _i64, _p, _i64,            # conv_state, its slot stride, ssm_state, its slot stride
        _p, _i32, _i64,                # req_indices, batch_size, n_slots
        _i32, _i32, _i32, _i32, _i32,  # num_k_heads, num_v_heads, head_k/v_dim, conv_kernel
        _p, _i64, _p, _i64,            # out, out_row_stride, core_out, core_row_stride
        _p, _i64, _p,                  # workspace, workspace_bytes, stream
    ]),
    "tf_gdn_decode_workspace_bytes": (_i64, [_i32, _i32, _i32]),
    "tf_gdn_extend": (_i32, [
        _p, _i64, _p, _p, _i64,        # qkv, qkv_row_stride, a, b, ab_row_stride
        _p, _i64,                      # z, z_row_stride
        _p, _p, _p, _p, _f32,          # conv_weight, a_log, dt_bias, norm_weight, eps
        _p, _i64, _p, _i64,            # conv_state, its slot stride, ssm_state, its slot stride
        _p, _p, _i32, _i64, _i32, _i64,  # req_indices, token_offsets, batch, n_tokens,
                                         # max_extend_len, n_slots
        _i32, _i32, _i32, _i32, _i32,  # num_k_heads, num_v_heads, head_k/v_dim, conv_kernel
        _p, _i64, _p, _i64,            # out, out_row_stride, core_out, core_row_stride
        _p, _i64, _p,                  # workspace, workspace_bytes, stream
    ]),
    "tf_gdn_extend_workspace_bytes": (_i64, [_i64, _i32, _i32, _i32]),
    "tf_gather_kv": (_i32, [
        _p, _i32, _i64, _i64,          # pool, kv_dtype, pool_slots, row_elems
        _p, _i64, _i64, _i64,          # req_to_token, rtt_rows, rtt_row_stride, rtt_cols
        _p, _i32, _i32, _p, _p,        # req_pool_indices, batch_size, max_len, out, stream
    ]),
}


SIGNATURES["tf_attn_decode_partial"] = SIGNATURES["tf_attn_decode"]
SIGNATURES["tf_attn_decode_merge"] = SIGNATURES["tf_attn_decode"]


class NativeLibraryError(RuntimeError):
    """libtf_attn.so is missing, stale or failed to load."""


class NativeCallError(RuntimeError):
    """A libtf_attn entry point returned an error status."""

    def __init__(self, fn: str, code: int, message: str):
        super().__init__(f"{fn} failed with status {code}: {message}")
        self.code = code


_lock = threading.Lock()
_lib: Optional[ctypes.CDLL] = None


def load(path: Optional[Path] = None) -> ctypes.CDLL:
    """Loads (once) and returns the library with every signature declared."""
    global _lib
    with _lock:
        if _lib is not None and path is None:
            return _lib
        target = Path(path) if path is not None else LIB_PATH
        if not target.exists():
            raise NativeLibraryError(
                f"{target} not found: build it with `python -m tokenfactory_amd.build` "
                "(the attention path has no non-native fallback)")
        try:
            lib = ctypes.CDLL(str(target))
        except OSError as exc:
            raise NativeLibraryError(f"cannot load {target}: {exc}") from exc
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        ver = lib.tf_attn_abi_version()
        if ver != ABI_VERSION:
            raise NativeLibraryError(f"{target}: ABI version {ver}, expected {ABI_VERSION}")
        if path is None:
            _lib = lib
        return lib


def call(name: str, *args) -> int:
    """Calls an int32-status entry point and raises on a negative status."""
    lib = load()
    rc = getattr(lib, name)(*args)
    if rc < 0:
        msg = lib.tf_attn_last_error().decode(errors="replace")
        if rc == TF_ERR_INVALID:
            raise ValueError(f"{name}: {msg}")
        if rc == TF_ERR_UNSUPPORTED:
            raise NotImplementedError(f"{name}: {msg}")
        raise NativeCallError(name, rc, msg)
    return rc


def plan_device_capacity(total_tokens, batch_size, num_q_heads, num_kv_heads) -> int:
    """Work-list entries tf_attn_plan_device fills for T tokens and B requests."""
    n = load().tf_attn_plan_device_capacity(total_tokens, batch_size, num_q_heads, num_kv_heads)
    if n < 0:
        raise ValueError(load().tf_attn_last_error().decode(errors="replace"))
    return int(n)


def decode_workspace_bytes(n_items, num_q_heads, num_kv_heads, head_dim, max_seq_len,
                           num_workgroups=0) -> int:
    lib = load()
    n = lib.tf_attn_decode_workspace_bytes(n_items, num_q_heads, num_kv_heads, head_dim,
                                           max_seq_len, num_workgroups)
    if n < 0:
        msg = lib.tf_attn_last_error().decode(errors="replace")
        if n == TF_ERR_UNSUPPORTED:
            raise NotImplementedError(msg)
        raise ValueError(msg)
    return int(n)
