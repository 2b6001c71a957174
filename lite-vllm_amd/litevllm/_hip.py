"""ctypes binding of liblitevllm_hip.so (the C ABI in include/litevllm_hip.h).

The library is loaded lazily on first use.  There is no fallback: if the
library is missing or cannot be loaded, every hot-path op raises
``RuntimeError`` (the reference's Triton sampler silently fell back to torch,
litevllm/layers/sampler.py:38-55; this build fails loudly instead so a GPU
run can never pass on a non-native path).
"""

from __future__ import annotations

import ctypes
import threading
from pathlib import Path

LIB_NAME = "liblitevllm_hip.so"
LIB_PATH = Path(__file__).resolve().parent / LIB_NAME

LV_F32, LV_F16, LV_BF16 = 0, 1, 2
LV_ACT_NONE, LV_ACT_SILU_MUL = 0, 1
ABI_VERSION = 7
LV_ERR_DEVICE_INDEX = -5
LV_DEVERR_BLOCK_ID, LV_DEVERR_SLOT = 1, 2

# Every symbol the header declares, with (restype, argtypes).
_c_i32, _c_i64, _c_f32, _c_p, _c_sz = (
    ctypes.c_int32, ctypes.c_int64, ctypes.c_float, ctypes.c_void_p, ctypes.c_size_t)

SIGNATURES: dict[str, tuple] = {
    "lv_last_error": (ctypes.c_char_p, []),
    "lv_abi_version": (ctypes.c_int, []),
    "lv_device_errors": (ctypes.c_int, [ctypes.POINTER(ctypes.c_uint32), _c_i32]),
    "lv_pack_inputs": (ctypes.c_int, [
        _c_p, _c_i32,            # descs, num_seqs
        _c_p, _c_i64,            # block_ids, num_block_ids
        _c_p, _c_i64,            # token_ids, num_token_ids
        _c_p, _c_i64,            # device_tokens, num_device_tokens
        _c_i64, _c_i32, _c_i32,  # num_tokens, block_size, max_blocks
        _c_p, _c_p, _c_p,        # input_ids, positions, slot_mapping
        _c_p, _c_p, _c_p, _c_p,  # cu_seqlens, seq_start, context_lens, block_tables
        _c_p,                    # stream
    ]),
    "lv_kv_scatter": (ctypes.c_int, [
        _c_p, _c_i64, _c_p, _c_i64,   # key, key_stride_t, value, value_stride_t
        _c_p, _c_p,                   # key_cache, value_cache
        _c_p, _c_i64,                 # slot_mapping, num_tokens
        _c_i32, _c_i32, _c_i32,       # num_kv_heads, head_dim, block_size
        _c_i64, ctypes.c_int, _c_p,   # num_blocks, dtype, stream
    ]),
    "lv_paged_attention_workspace_size": (_c_sz, [
        _c_i32, _c_i32, _c_i64, _c_i32, _c_i32, _c_i32, _c_i32, _c_i32, ctypes.c_int,
    ]),
    "lv_paged_attention": (ctypes.c_int, [
        _c_p, _c_i64,                 # query, q_stride_t
        _c_p, _c_p, _c_i64,           # key_cache, value_cache, num_cache_blocks
        _c_p, _c_i32,                 # block_tables, max_blocks
        _c_p, _c_p,                   # cu_seqlens, context_lens
        _c_i32, _c_i32, _c_i64,       # num_seqs, num_decodes, num_tokens
        _c_i32,                       # max_query_len
        _c_i32, _c_i32, _c_i32,       # num_heads, num_kv_heads, head_dim
        _c_i32, _c_f32,               # block_size, scale
        _c_p, _c_i64,                 # out, out_stride_t
        _c_p, _c_sz,                  # workspace, workspace_bytes
        ctypes.c_int, _c_p,           # dtype, stream
    ]),
    "lv_paged_attention_prefix_workspace_size": (_c_sz, [_c_i32, _c_i32, _c_i32]),
    "lv_paged_attention_prefix": (ctypes.c_int, [
        _c_p, _c_i64,                 # query, q_stride_t
        _c_p, _c_p, _c_i64,           # key_cache, value_cache, num_cache_blocks
        _c_p, _c_i32,                 # block_tables, max_blocks
        _c_p, _c_p,                   # cu_seqlens, context_lens
        _c_i32, _c_i32, _c_i64,       # num_seqs, num_decodes, num_tokens
        _c_i32,                       # max_query_len
        _c_i32, _c_i32, _c_i32,       # num_heads, num_kv_heads, head_dim
        _c_i32, _c_f32,               # block_size, scale
        _c_p, _c_i64,                 # out, out_stride_t
        _c_p, _c_sz,                  # workspace, workspace_bytes
        _c_p, _c_p, _c_i32,           # prefix_blocks, prefix_items, max_items
        _c_p, _c_i32,                 # prefix_members, num_members
        _c_p, _c_sz,                  # prefix_workspace, its bytes
        ctypes.c_int, _c_p,           # dtype, stream
    ]),
    "lv_sample_workspace_size": (ctypes.c_size_t, [_c_i64, _c_i64]),
    "lv_sample": (ctypes.c_int, [
        _c_p, _c_i64, _c_i64, _c_i64,  # logits, num_rows, vocab_size, row_stride
        _c_p, _c_p, _c_p,              # temperature, uniform, out_ids
        _c_p, ctypes.c_size_t,         # workspace, workspace_bytes
        ctypes.c_int, _c_p,            # dtype, stream
    ]),
    "lv_sample_noalloc": (ctypes.c_int, [
        _c_p, _c_i64, _c_i64, _c_i64,  # logits, num_rows, vocab_size, row_stride
        _c_p, _c_p, _c_p,              # temperature, uniform, out_ids
        ctypes.c_int, _c_p,            # dtype, stream
    ]),
    "lv_add_rms_norm": (ctypes.c_int, [
        _c_p, _c_i64, _c_p, _c_i64,    # x, x_stride, residual, residual_stride
        _c_p, _c_p, _c_i64,            # weight, out, out_stride
        _c_i64, _c_i32, ctypes.c_float,  # num_tokens, hidden, eps
        ctypes.c_int, _c_p,            # dtype, stream
    ]),
    "lv_qk_norm_rope_cache": (ctypes.c_int, [
        _c_p, _c_i64, _c_p, _c_p,      # qkv, qkv_stride, q_norm_w, k_norm_w
        _c_p, _c_p, _c_i64,            # cos, sin, max_position
        _c_p, _c_p,                    # positions, slot_mapping
        _c_p, _c_i64, _c_p, _c_p,      # q_out, q_out_stride, key_cache, value_cache
        _c_i64, _c_i32, _c_i64,        # num_blocks, block_size, num_tokens
        _c_i32, _c_i32, _c_i32,        # num_heads, num_kv_heads, head_dim
        ctypes.c_float, ctypes.c_int, _c_p,  # eps, dtype, stream
    ]),
    "lv_silu_mul": (ctypes.c_int, [
        _c_p, _c_i64, _c_p, _c_i64,    # gate_up, in_stride, out, out_stride
        _c_i64, _c_i32,                # num_tokens, intermediate
        ctypes.c_int, _c_p,            # dtype, stream
    ]),
    "lv_linear_supported": (ctypes.c_int, [_c_i64, _c_i64, _c_i64, _c_i32, ctypes.c_int]),
    "lv_linear": (ctypes.c_int, [
        _c_p, _c_i64, _c_p, _c_i64,    # x, x_stride, weight, weight_stride
        _c_p, _c_i64,                  # y, y_stride
        _c_i64, _c_i64, _c_i64,        # m, n, k
        _c_i32, ctypes.c_int, _c_p,    # activation, dtype, stream
    ]),
}

_lock = threading.Lock()
_lib: ctypes.CDLL | None = None


def load() -> ctypes.CDLL:
    """Load and bind the library (once per process); raise if unavailable."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is not None:
            return _lib
        if not LIB_PATH.exists():
            raise RuntimeError(
                f"{LIB_NAME} is not built (expected at {LIB_PATH}); build it with "
                "`python -m litevllm._build` or __graft_entry__.build()")
        lib = ctypes.CDLL(str(LIB_PATH))
        for name, (restype, argtypes) in SIGNATURES.items():
            fn = getattr(lib, name)  # AttributeError if a symbol is missing
            fn.restype = restype
            fn.argtypes = argtypes
        v = lib.lv_abi_version()
        if v != ABI_VERSION:
            raise RuntimeError(f"{LIB_NAME} ABI version {v} != expected {ABI_VERSION}")
        _lib = lib
        return lib


def check(rc: int, what: str) -> None:
    if rc != 0:
        msg = load().lv_last_error().decode(errors="replace")
        raise RuntimeError(f"{what} failed (status {rc}): {msg}")
