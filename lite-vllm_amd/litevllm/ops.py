"""Tensor-level wrappers of the HIP hot path (one function per C entry point).

Each wrapper checks shapes, dtypes and devices on the host, passes raw
pointers plus the current HIP stream to liblitevllm_hip.so, and raises
``RuntimeError`` with the library's message on failure.  Inputs must be
tensors on a ROCm ("cuda") device: there is no CPU path behind these calls.
"""

from __future__ import annotations

import ctypes
import os
from typing import NamedTuple, Optional

import torch

from . import _hip

_DTYPE_CODES = {
    torch.float32: _hip.LV_F32,
    torch.float16: _hip.LV_F16,
    torch.bfloat16: _hip.LV_BF16,
}

# Field order of lv_seq_desc (include/litevllm_hip.h).
SEQ_DESC_FIELDS = ("num_computed", "query_len", "num_blocks", "block_offset",
                   "token_offset", "token_index")


def _dtype_code(t: torch.Tensor) -> int:
    try:
        return _DTYPE_CODES[t.dtype]
    except KeyError:
        raise RuntimeError(f"unsupported dtype {t.dtype}; expected fp32, fp16 or bf16") from None


def _require_device(name: str, t: Optional[torch.Tensor], device: torch.device) -> None:
    if t is None:
        return
    if t.device.type != "cuda":
        raise RuntimeError(
            f"litevllm HIP op: `{name}` is on {t.device}; the hot path runs only on a "
            "ROCm device (there is no CPU implementation)")
    if t.device != device:
        raise RuntimeError(f"litevllm HIP op: `{name}` on {t.device}, expected {device}")


def _ptr(t: Optional[torch.Tensor]) -> Optional[int]:
    return None if t is None else t.data_ptr()


def _stream(device: torch.device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


def _check_int(name: str, t: torch.Tensor, dtype: torch.dtype, dim: int) -> None:
    if t.dtype != dtype or t.dim() != dim or not t.is_contiguous():
        raise RuntimeError(f"`{name}` must be a contiguous {dim}-d {dtype} tensor, "
                           f"got {t.dtype} {tuple(t.shape)} contiguous={t.is_contiguous()}")


# ---------------------------------------------------------------------------
# Device-side index errors
# ---------------------------------------------------------------------------

DEVICE_ERROR_NAMES = {
    _hip.LV_DEVERR_BLOCK_ID: "block-table entry outside [0, num_cache_blocks)",
    _hip.LV_DEVERR_SLOT: "slot_mapping entry >= num_blocks * block_size",
}


def device_errors(device: Optional[torch.device] = None, clear: bool = True) -> int:
    """Bits (LV_DEVERR_*) of the out-of-range indices the kernels met on
    `device` since the last clear; they were clamped (a block id outside the
    cache read block 0, a slot past the cache was not written).  Waits for
    the device.  lv_device_errors in include/litevllm_hip.h."""
    lib = _hip.load()
    flags = ctypes.c_uint32(0)
    with torch.cuda.device(device if device is not None else torch.cuda.current_device()):
        rc = lib.lv_device_errors(ctypes.byref(flags), 1 if clear else 0)
    if rc not in (0, _hip.LV_ERR_DEVICE_INDEX):
        _hip.check(rc, "lv_device_errors")
    return int(flags.value)


def check_device_errors(device: Optional[torch.device] = None) -> None:
    """Raise RuntimeError if a kernel met an out-of-range index on `device`
    (as the reference's torch indexing raises, layers/attention.py:80-84,
    111-119); clears the report."""
    bits = device_errors(device, clear=True)
    if bits:
        names = [n for b, n in DEVICE_ERROR_NAMES.items() if bits & b]
        raise RuntimeError("litevllm kernels met out-of-range indices (clamped, results "
                           "invalid): " + "; ".join(names))


# ---------------------------------------------------------------------------
# (2) KV scatter
# ---------------------------------------------------------------------------

def kv_scatter(key: torch.Tensor, value: torch.Tensor, key_cache: torch.Tensor,
               value_cache: torch.Tensor, slot_mapping: torch.Tensor) -> None:
    """key_cache[slot // bs, slot % bs] = key (same for value), in place.

    Reference: litevllm/layers/attention.py:17-33 and 79-84.
    key/value: [T, Hkv, D] (token stride free, heads contiguous);
    caches: contiguous [N, bs, Hkv, D]; slot_mapping: int64 [T].
    """
    dev = key_cache.device
    for n, t in (("key", key), ("value", value), ("key_cache", key_cache),
                 ("value_cache", value_cache), ("slot_mapping", slot_mapping)):
        _require_device(n, t, dev)
    if key_cache.dim() != 4 or not key_cache.is_contiguous() or not value_cache.is_contiguous():
        raise RuntimeError("caches must be contiguous [num_blocks, block_size, num_kv_heads, head_dim]")
    if value_cache.shape != key_cache.shape:
        raise RuntimeError("key_cache and value_cache shapes differ")
    n_blocks, bs, hkv, d = key_cache.shape
    T = slot_mapping.shape[0]
    _check_int("slot_mapping", slot_mapping, torch.int64, 1)
    for n, t in (("key", key), ("value", value)):
        if tuple(t.shape) != (T, hkv, d):
            raise RuntimeError(f"`{n}` shape {tuple(t.shape)} != {(T, hkv, d)}")
        if t.dtype != key_cache.dtype:
            raise RuntimeError(f"`{n}` dtype {t.dtype} != cache dtype {key_cache.dtype}")
        if T > 0 and (t.stride(2) != 1 or t.stride(1) != d):
            raise RuntimeError(f"`{n}` must have contiguous heads (strides {t.stride()})")
    if T == 0:
        return
    lib = _hip.load()
    rc = lib.lv_kv_scatter(_ptr(key), key.stride(0), _ptr(value), value.stride(0),
                           _ptr(key_cache), _ptr(value_cache), _ptr(slot_mapping), T,
                           hkv, d, bs, n_blocks, _dtype_code(key_cache), _stream(dev))
    _hip.check(rc, "lv_kv_scatter")


# ---------------------------------------------------------------------------
# (3) paged attention
# ---------------------------------------------------------------------------

_workspaces: dict[tuple[int, int, str], torch.Tensor] = {}


def _workspace(device: torch.device, nbytes: int, kind: str = "attn") -> Optional[torch.Tensor]:
    """Per-(device, stream, kind) scratch buffer, grown on demand and reused."""
    if nbytes == 0:
        return None
    key = (device.index if device.index is not None else torch.cuda.current_device(),
           _stream(device), kind)
    ws = _workspaces.get(key)
    if ws is None or ws.numel() < nbytes:
        ws = torch.empty(max(nbytes, 1 << 20), dtype=torch.uint8, device=device)
        _workspaces[key] = ws
    return ws


# Shared-prefix pass geometry (lv_paged_attention_prefix): keys per split,
# most prefix blocks, and query rows (members x GQA heads) per work item.
PREFIX_KEYS_PER_SPLIT = 128
PREFIX_MAX_BLOCKS = 128
PREFIX_ROWS_PER_ITEM = 128
PREFIX_MAX_SPLITS = 16
PREFIX_MAX_DECODES = 7000


class PrefixPlan(NamedTuple):
    """Device description of the decode rows' shared prefixes (the three
    arrays lv_paged_attention_prefix reads)."""
    blocks: torch.Tensor    # int32 [num_decodes]: leading blocks of each row in its group's prefix
    items: torch.Tensor     # int32 [max_items, 4]: leader, first member, members, split
    members: torch.Tensor   # int32: member rows, one group after another


def prefix_plan_arrays(groups, num_decodes: int, group_size: int, block_size: int = 16,
                       max_items: Optional[int] = None, max_members: Optional[int] = None):
    """Host (numpy) arrays of a PrefixPlan.

    ``groups``: iterable of (rows, prefix_blocks) -- decode rows whose block
    tables start with the same ``prefix_blocks`` physical blocks; rows[0] is
    the leader whose table the prefix pass reads.  ``group_size`` = num_heads
    // num_kv_heads.  One item per (group, slice of 128 // group_size rows,
    128-key split); ``max_items`` / ``max_members`` pad the arrays to a fixed
    size (unused items have leader -1) so they can live in graph-static
    buffers.  Groups with one row or an empty prefix are dropped.
    """
    import numpy as np
    per_item = PREFIX_ROWS_PER_ITEM // group_size
    blocks = np.zeros(num_decodes, np.int32)
    items: list[tuple[int, int, int, int]] = []
    parts = []
    base = 0
    for rows, pblocks in groups:
        rows = np.asarray(rows, dtype=np.int32).reshape(-1)
        pblocks = int(pblocks)
        if pblocks < 0 or pblocks > PREFIX_MAX_BLOCKS:
            raise ValueError(f"prefix of {pblocks} blocks outside [0, {PREFIX_MAX_BLOCKS}]")
        n = rows.shape[0]
        if n < 2 or pblocks == 0:
            continue
        parts.append(rows)
        blocks[rows] = pblocks
        nsplit = -(-pblocks * block_size // PREFIX_KEYS_PER_SPLIT)
        leader = int(rows[0])
        for s0 in range(0, n, per_item):
            cnt = min(per_item, n - s0)
            items.extend((leader, base + s0, cnt, sp) for sp in range(nsplit))
        base += n
    members = np.concatenate(parts) if parts else np.zeros(0, np.int32)
    if members.size and (members.min() < 0 or members.max() >= num_decodes
                         or np.unique(members).size != members.size):
        raise ValueError("a group row is out of range or in two groups")
    if max_items is not None:
        if len(items) > max_items:
            raise ValueError(f"{len(items)} prefix items exceed max_items={max_items}")
        items += [(-1, 0, 0, 0)] * (max_items - len(items))
    if max_members is not None:
        if members.size > max_members:
            raise ValueError(f"{members.size} members exceed max_members={max_members}")
        members = np.concatenate([members, np.zeros(max_members - members.size, np.int32)])
    items_a = np.asarray(items, np.int32).reshape(-1, 4)
    members_a = members.astype(np.int32) if members.size else np.zeros(1, np.int32)
    check_prefix_plan(blocks, items_a, members_a, group_size, block_size)
    return blocks, items_a, members_a


def check_prefix_plan(blocks, items, members, group_size: int, block_size: int = 16) -> None:
    """Raise ValueError unless host arrays (numpy) form a plan that
    lv_paged_attention_prefix computes correctly: every used item's (leader
    >= 0) leader, split and member slice in range; every member of a
    slice shares the leader's prefix length; and every row with a prefix
    covered by exactly one item for each 128-key split of it.  (The kernels
    skip out-of-range items, but a row left uncovered would merge a stale
    partial.)"""
    import numpy as np
    blocks = np.asarray(blocks, np.int64)
    items = np.asarray(items, np.int64).reshape(-1, 4)
    members = np.asarray(members, np.int64).reshape(-1)
    n = blocks.shape[0]
    it = items[items[:, 0] >= 0]
    leader, first, cnt, split = it[:, 0], it[:, 1], it[:, 2], it[:, 3]
    per_item = PREFIX_ROWS_PER_ITEM // group_size
    if ((leader >= n) | (split < 0) | (split >= PREFIX_MAX_SPLITS)
            | (cnt < 1) | (cnt > per_item) | (first < 0) | (first + cnt > members.size)).any():
        raise ValueError("prefix plan: an item's leader, split or member slice is out of range")
    if ((blocks < 0) | (blocks > PREFIX_MAX_BLOCKS)).any():
        raise ValueError(f"prefix plan: prefix lengths must lie in [0, {PREFIX_MAX_BLOCKS}]")
    nsplit = -(-blocks * block_size // PREFIX_KEYS_PER_SPLIT)
    if (blocks[leader] <= 0).any() or (split >= nsplit[leader]).any():
        raise ValueError("prefix plan: an item's split lies past its leader's prefix")
    def ranks(counts):   # 0..c-1 for each count c, concatenated
        return np.arange(int(counts.sum())) - np.repeat(np.cumsum(counts) - counts, counts)
    rows = members[np.repeat(first, cnt) + ranks(cnt)]
    splits = np.repeat(split, cnt)
    leads = np.repeat(leader, cnt)
    if ((rows < 0) | (rows >= n)).any() or (blocks[rows] != blocks[leads]).any():
        raise ValueError("prefix plan: a member row is out of range or has another prefix length")
    covered = rows * 32 + splits
    need = np.repeat(np.arange(n), nsplit) * 32 + ranks(nsplit)
    if covered.size != need.size or not np.array_equal(np.sort(covered), np.sort(need)):
        raise ValueError("prefix plan: every (row, split) of a prefix must be covered by "
                         "exactly one item")


def prefix_attention_supported(num_heads: int, num_kv_heads: int, head_dim: int,
                               block_size: int, dtype: torch.dtype) -> bool:
    """Shapes lv_paged_attention_prefix serves (else LV_ERR_UNSUPPORTED)."""
    g = num_heads // max(num_kv_heads, 1)
    return (dtype in (torch.bfloat16, torch.float16) and head_dim in (64, 128)
            and block_size == 16 and num_heads % max(num_kv_heads, 1) == 0
            and g in (1, 2, 4, 8) and 1 <= num_kv_heads <= 8
            and os.environ.get("LV_ATTN_DECODE_KERNEL", "")[:1] != "r")


def prefix_workspace_size(num_decodes: int, num_heads: int, head_dim: int) -> int:
    """Bytes of prefix scratch lv_paged_attention_prefix needs."""
    return int(_hip.load().lv_paged_attention_prefix_workspace_size(num_decodes, num_heads,
                                                                    head_dim))


def prefix_items_needed(groups, group_size: int, block_size: int = 16) -> int:
    """Work items prefix_plan_arrays makes for these groups."""
    per_item = PREFIX_ROWS_PER_ITEM // group_size
    return sum(-(-len(rows) // per_item) * -(-int(pb) * block_size // PREFIX_KEYS_PER_SPLIT)
               for rows, pb in groups if len(rows) >= 2 and pb > 0)


def prefix_plan(groups, num_decodes: int, group_size: int, device, block_size: int = 16,
                max_items: Optional[int] = None, max_members: Optional[int] = None) -> PrefixPlan:
    """PrefixPlan on ``device`` (see prefix_plan_arrays)."""
    blocks, items, members = prefix_plan_arrays(groups, num_decodes, group_size, block_size,
                                                max_items, max_members)
    return PrefixPlan(torch.from_numpy(blocks).to(device), torch.from_numpy(items).to(device),
                      torch.from_numpy(members).to(device))


def paged_attention(query: torch.Tensor, key_cache: torch.Tensor, value_cache: torch.Tensor,
                    block_tables: torch.Tensor, context_lens: torch.Tensor, *,
                    num_kv_heads: Optional[int] = None, scale: float,
                    cu_seqlens: Optional[torch.Tensor] = None,
                    num_decodes: Optional[int] = None, max_query_len: int = 1,
                    out: Optional[torch.Tensor] = None,
                    workspace: Optional[torch.Tensor] = None,
                    prefix: Optional[PrefixPlan] = None,
                    prefix_workspace: Optional[torch.Tensor] = None) -> torch.Tensor:
    """Attention of every query row over its sequence's paged K/V.

    Reference: litevllm/layers/attention.py:91-139 (decode) and 141-151
    (prefill, here generalised to chunks at an offset).  query: [T, H, D];
    block_tables int32 [B, max_blocks]; context_lens int32 [B] (tokens in
    cache incl. this step's); cu_seqlens int32 [B+1] (None => T == B, all
    decodes); the first ``num_decodes`` sequences must be 1-token decodes.
    ``workspace`` (uint8, at least paged_attention_workspace_size bytes) is
    used instead of the per-stream scratch buffer when given: a captured HIP
    graph must own the memory its kernels read.  ``prefix`` (a PrefixPlan)
    selects lv_paged_attention_prefix: the decode rows' shared prefixes are
    read once per group; ``prefix_workspace`` is its scratch as above.
    """
    dev = key_cache.device
    for n, t in (("query", query), ("key_cache", key_cache), ("value_cache", value_cache),
                 ("block_tables", block_tables), ("context_lens", context_lens),
                 ("cu_seqlens", cu_seqlens), ("out", out)):
        _require_device(n, t, dev)
    if query.dim() != 3 or query.stride(2) != 1 or query.stride(1) != query.shape[2]:
        raise RuntimeError(f"query must be [T, H, D] with contiguous heads, got "
                           f"{tuple(query.shape)} strides {query.stride()}")
    T, H, D = query.shape
    n_blocks, bs, hkv, d = key_cache.shape
    if num_kv_heads is not None and num_kv_heads != hkv:
        raise RuntimeError(f"num_kv_heads={num_kv_heads} but cache has {hkv}")
    if d != D or value_cache.shape != key_cache.shape:
        raise RuntimeError("cache head_dim / shapes do not match the query")
    if query.dtype != key_cache.dtype or value_cache.dtype != key_cache.dtype:
        raise RuntimeError("query and caches must share one dtype")
    if not key_cache.is_contiguous() or not value_cache.is_contiguous():
        raise RuntimeError("caches must be contiguous")
    _check_int("block_tables", block_tables, torch.int32, 2)
    _check_int("context_lens", context_lens, torch.int32, 1)
    B, max_blocks = block_tables.shape
    if context_lens.shape[0] != B:
        raise RuntimeError("context_lens and block_tables disagree on the batch size")
    if cu_seqlens is None:
        if T != B:
            raise RuntimeError("without cu_seqlens every sequence must have exactly one query row")
        num_decodes = B if num_decodes is None else num_decodes
    else:
        _check_int("cu_seqlens", cu_seqlens, torch.int32, 1)
        if cu_seqlens.shape[0] != B + 1:
            raise RuntimeError("cu_seqlens must have num_seqs + 1 entries")
        num_decodes = 0 if num_decodes is None else num_decodes
    if out is None:
        out = torch.empty_like(query, memory_format=torch.contiguous_format)
    elif out.shape != query.shape or out.dtype != query.dtype or out.stride(2) != 1 \
            or out.stride(1) != D:
        raise RuntimeError("`out` must match query's shape/dtype with contiguous heads")
    if B == 0:
        return out
    lib = _hip.load()
    dt = _dtype_code(query)
    ws_bytes = lib.lv_paged_attention_workspace_size(B, num_decodes, T, H, D, bs, max_blocks,
                                                     max_query_len, dt)
    if workspace is not None:
        _require_device("workspace", workspace, dev)
        if workspace.dtype != torch.uint8 or not workspace.is_contiguous() or \
                workspace.numel() < ws_bytes:
            raise RuntimeError(f"workspace must be a contiguous uint8 tensor of >= {ws_bytes} bytes")
        ws = workspace if ws_bytes > 0 else None
    else:
        ws = _workspace(dev, ws_bytes)
    if prefix is None:
        rc = lib.lv_paged_attention(
            _ptr(query), query.stride(0), _ptr(key_cache), _ptr(value_cache), n_blocks,
            _ptr(block_tables), max_blocks, _ptr(cu_seqlens), _ptr(context_lens),
            B, num_decodes, T, max_query_len, H, hkv, D, bs, float(scale),
            _ptr(out), out.stride(0), _ptr(ws), 0 if ws is None else ws.numel(), dt,
            _stream(dev))
        _hip.check(rc, "lv_paged_attention")
        return out
    for n, t in zip(("prefix.blocks", "prefix.items", "prefix.members"), prefix):
        _require_device(n, t, dev)
    _check_int("prefix.blocks", prefix.blocks, torch.int32, 1)
    _check_int("prefix.items", prefix.items, torch.int32, 2)
    _check_int("prefix.members", prefix.members, torch.int32, 1)
    if prefix.blocks.shape[0] != num_decodes or prefix.items.shape[1] != 4:
        raise RuntimeError("prefix.blocks must have num_decodes entries and prefix.items 4 columns")
    pws_bytes = int(lib.lv_paged_attention_prefix_workspace_size(num_decodes, H, D))
    if prefix_workspace is not None:
        _require_device("prefix_workspace", prefix_workspace, dev)
        if prefix_workspace.dtype != torch.uint8 or not prefix_workspace.is_contiguous() or \
                prefix_workspace.numel() < pws_bytes:
            raise RuntimeError(
                f"prefix_workspace must be a contiguous uint8 tensor of >= {pws_bytes} bytes")
        pws = prefix_workspace
    else:
        pws = _workspace(dev, pws_bytes, "prefix")
    rc = lib.lv_paged_attention_prefix(
        _ptr(query), query.stride(0), _ptr(key_cache), _ptr(value_cache), n_blocks,
        _ptr(block_tables), max_blocks, _ptr(cu_seqlens), _ptr(context_lens),
        B, num_decodes, T, max_query_len, H, hkv, D, bs, float(scale),
        _ptr(out), out.stride(0), _ptr(ws), 0 if ws is None else ws.numel(),
        _ptr(prefix.blocks), _ptr(prefix.items), prefix.items.shape[0], _ptr(prefix.members),
        prefix.members.shape[0], _ptr(pws), 0 if pws is None else pws.numel(), dt, _stream(dev))
    _hip.check(rc, "lv_paged_attention_prefix")
    return out


def paged_attention_workspace_size(num_seqs: int, num_decodes: int, num_tokens: int,
                                   num_heads: int, head_dim: int, block_size: int,
                                   max_blocks: int, max_query_len: int,
                                   dtype: torch.dtype) -> int:
    """Bytes of scratch one lv_paged_attention call with these sizes needs."""
    lib = _hip.load()
    return int(lib.lv_paged_attention_workspace_size(num_seqs, num_decodes, num_tokens,
                                                     num_heads, head_dim, block_size, max_blocks,
                                                     max_query_len, _DTYPE_CODES[dtype]))


# ---------------------------------------------------------------------------
# (1) packing
# ---------------------------------------------------------------------------

def pack_inputs(descs: torch.Tensor, block_ids: torch.Tensor, token_ids: torch.Tensor,
                num_tokens: int, block_size: int, max_blocks: int,
                device_tokens: Optional[torch.Tensor] = None,
                out: Optional[dict[str, torch.Tensor]] = None) -> dict[str, torch.Tensor]:
    """Expand per-sequence descriptors into the packed step tensors on the GPU.

    Reference: ModelRunner.prepare_inputs, litevllm/engine/model_runner.py:180-260.
    descs: int32 [B, 6] device tensor in lv_seq_desc field order
    (SEQ_DESC_FIELDS); block_ids int32 [*]; token_ids int64 [*];
    device_tokens int64 [*] or None.
    Returns input_ids/positions/slot_mapping (int64 [T]), cu_seqlens
    (int32 [B+1]), seq_start/context_lens (int32 [B]) and block_tables
    (int32 [B, max_blocks]); with ``out`` given (same keys, exactly those
    shapes, contiguous) they are written in place.
    """
    dev = descs.device
    for n, t in (("descs", descs), ("block_ids", block_ids), ("token_ids", token_ids),
                 ("device_tokens", device_tokens)):
        _require_device(n, t, dev)
    _check_int("descs", descs, torch.int32, 2)
    if descs.shape[1] != len(SEQ_DESC_FIELDS):
        raise RuntimeError("descs must be [B, 6] int32")
    _check_int("block_ids", block_ids, torch.int32, 1)
    _check_int("token_ids", token_ids, torch.int64, 1)
    if device_tokens is not None:
        _check_int("device_tokens", device_tokens, torch.int64, 1)
    B = descs.shape[0]
    T = int(num_tokens)
    shapes = {"input_ids": ((T,), torch.int64), "positions": ((T,), torch.int64),
              "slot_mapping": ((T,), torch.int64), "cu_seqlens": ((B + 1,), torch.int32),
              "seq_start": ((B,), torch.int32), "context_lens": ((B,), torch.int32),
              "block_tables": ((B, max_blocks), torch.int32)}
    if out is None:
        out = {k: torch.empty(shp, dtype=dt, device=dev) for k, (shp, dt) in shapes.items()}
    else:
        for k, (shp, dt) in shapes.items():
            t = out[k]
            _require_device(k, t, dev)
            if tuple(t.shape) != shp or t.dtype != dt or not t.is_contiguous():
                raise RuntimeError(f"out[{k!r}] must be a contiguous {dt} tensor of shape {shp}")
    lib = _hip.load()
    rc = lib.lv_pack_inputs(
        _ptr(descs), B, _ptr(block_ids), block_ids.numel(), _ptr(token_ids), token_ids.numel(),
        _ptr(device_tokens), 0 if device_tokens is None else device_tokens.numel(),
        T, block_size, max_blocks,
        _ptr(out["input_ids"]), _ptr(out["positions"]), _ptr(out["slot_mapping"]),
        _ptr(out["cu_seqlens"]), _ptr(out["seq_start"]), _ptr(out["context_lens"]),
        _ptr(out["block_tables"]), _stream(dev))
    _hip.check(rc, "lv_pack_inputs")
    return out


# ---------------------------------------------------------------------------
# (4) sampler
# ---------------------------------------------------------------------------

def sample(logits: torch.Tensor, temperature: torch.Tensor,
           uniform: Optional[torch.Tensor] = None,
           out: Optional[torch.Tensor] = None,
           workspace: Optional[torch.Tensor] = None) -> torch.Tensor:
    """Greedy (temperature 0) or inverse-CDF temperature sampling per row.

    Reference: litevllm/layers/sampler.py:60-187.  logits [B, V] (unit
    stride along V); temperature / uniform: float32 [B] (uniform in [0, 1),
    may be None when every row is greedy).  Returns int64 [B].  ``workspace``
    (uint8, >= lv_sample_workspace_size bytes) replaces the per-stream
    scratch buffer when given.
    """
    dev = logits.device
    for n, t in (("logits", logits), ("temperature", temperature), ("uniform", uniform),
                 ("out", out)):
        _require_device(n, t, dev)
    if logits.dim() != 2 or logits.stride(1) != 1:
        raise RuntimeError("logits must be [B, V] with unit stride along V")
    B, V = logits.shape
    _check_int("temperature", temperature, torch.float32, 1)
    if temperature.shape[0] != B:
        raise RuntimeError("temperature must have one entry per row")
    if uniform is None:
        uniform = torch.zeros(B, dtype=torch.float32, device=dev)
    _check_int("uniform", uniform, torch.float32, 1)
    if uniform.shape[0] != B:
        raise RuntimeError("uniform must have one entry per row")
    if out is None:
        out = torch.empty(B, dtype=torch.int64, device=dev)
    else:
        _check_int("out", out, torch.int64, 1)
    if B == 0:
        return out
    lib = _hip.load()
    ws_bytes = int(lib.lv_sample_workspace_size(B, V))
    if workspace is not None:
        _require_device("workspace", workspace, dev)
        if workspace.dtype != torch.uint8 or not workspace.is_contiguous() or \
                workspace.numel() < ws_bytes:
            raise RuntimeError(f"workspace must be a contiguous uint8 tensor of >= {ws_bytes} bytes")
        ws = workspace
    else:
        ws = _workspace(dev, ws_bytes)
    rc = lib.lv_sample(_ptr(logits), B, V, logits.stride(0), _ptr(temperature), _ptr(uniform),
                       _ptr(out), _ptr(ws), 0 if ws is None else ws.numel(),
                       _dtype_code(logits), _stream(dev))
    _hip.check(rc, "lv_sample")
    return out


# ---------------------------------------------------------------------------
# fused layer work: residual add + RMSNorm, attention prologue, SiLU gate
# ---------------------------------------------------------------------------

def _check_rows(name: str, t: torch.Tensor, width: int, dtype: torch.dtype) -> None:
    if t.dim() != 2 or t.shape[1] < width or t.stride(1) != 1:
        raise RuntimeError(f"`{name}` must be [T, >={width}] with unit column stride, got "
                           f"{tuple(t.shape)} strides {t.stride()}")
    if t.dtype != dtype:
        raise RuntimeError(f"`{name}` dtype {t.dtype} != {dtype}")


def add_rms_norm(x: torch.Tensor, weight: torch.Tensor, eps: float,
                 residual: Optional[torch.Tensor] = None,
                 out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """out = weight * to_dtype(s * rsqrt(mean(s^2) + eps)) with s = x, or,
    when `residual` is given, s = residual := x + residual (updated in place).

    Reference: litevllm/models/llama.py:24-27 (RMSNorm) and the residual adds
    of the decoder layer (models/qwen3.py:131-140).  x/residual/out: [T, hidden].
    """
    dev = x.device
    for n, t in (("x", x), ("weight", weight), ("residual", residual), ("out", out)):
        _require_device(n, t, dev)
    T, hidden = x.shape
    _check_rows("x", x, hidden, x.dtype)
    if weight.shape != (hidden,) or not weight.is_contiguous() or weight.dtype != x.dtype:
        raise RuntimeError(f"`weight` must be a contiguous [{hidden}] {x.dtype} tensor")
    if residual is not None:
        _check_rows("residual", residual, hidden, x.dtype)
        if residual.shape[0] != T:
            raise RuntimeError("`residual` rows != x rows")
    if out is None:
        out = torch.empty((T, hidden), dtype=x.dtype, device=dev)
    _check_rows("out", out, hidden, x.dtype)
    if T == 0:
        return out
    lib = _hip.load()
    rc = lib.lv_add_rms_norm(_ptr(x), x.stride(0), _ptr(residual),
                             residual.stride(0) if residual is not None else 0, _ptr(weight),
                             _ptr(out), out.stride(0), T, hidden, float(eps), _dtype_code(x),
                             _stream(dev))
    _hip.check(rc, "lv_add_rms_norm")
    return out


def qk_norm_rope_cache(qkv: torch.Tensor, num_heads: int, num_kv_heads: int, head_dim: int,
                       cos_cache: torch.Tensor, sin_cache: torch.Tensor,
                       positions: torch.Tensor, slot_mapping: torch.Tensor,
                       key_cache: torch.Tensor, value_cache: torch.Tensor,
                       q_norm_weight: Optional[torch.Tensor] = None,
                       k_norm_weight: Optional[torch.Tensor] = None, eps: float = 1e-6,
                       q_out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """Split a fused q|k|v projection, RMSNorm q and k per head (when the
    weights are given), rotate both with the module's cos/sin caches, write
    the query to q_out [T, H, D] and K/V into the paged cache at slot_mapping.

    Reference: models/qwen3.py:75-84, layers/rotary_emb.py:92-117,
    layers/attention.py:79-84.
    """
    dev = qkv.device
    for n, t in (("qkv", qkv), ("cos_cache", cos_cache), ("sin_cache", sin_cache),
                 ("positions", positions), ("slot_mapping", slot_mapping),
                 ("key_cache", key_cache), ("value_cache", value_cache),
                 ("q_norm_weight", q_norm_weight), ("k_norm_weight", k_norm_weight),
                 ("q_out", q_out)):
        _require_device(n, t, dev)
    H, Hkv, D = num_heads, num_kv_heads, head_dim
    T = qkv.shape[0]
    _check_rows("qkv", qkv, (H + 2 * Hkv) * D, key_cache.dtype)
    _check_int("positions", positions, torch.int64, 1)
    _check_int("slot_mapping", slot_mapping, torch.int64, 1)
    if positions.shape[0] != T or slot_mapping.shape[0] != T:
        raise RuntimeError("positions / slot_mapping length != number of tokens")
    n_blocks, bs, hkv, d = key_cache.shape
    if (hkv, d) != (Hkv, D) or value_cache.shape != key_cache.shape or \
            not key_cache.is_contiguous() or not value_cache.is_contiguous():
        raise RuntimeError(f"caches must be contiguous [N, bs, {Hkv}, {D}] and equal in shape")
    for n, t in (("cos_cache", cos_cache), ("sin_cache", sin_cache)):
        if t.dim() != 2 or t.shape[1] != D // 2 or not t.is_contiguous() or t.dtype != qkv.dtype:
            raise RuntimeError(f"`{n}` must be a contiguous [max_pos, {D // 2}] {qkv.dtype} tensor")
    for n, t in (("q_norm_weight", q_norm_weight), ("k_norm_weight", k_norm_weight)):
        if t is not None and (t.shape != (D,) or not t.is_contiguous() or t.dtype != qkv.dtype):
            raise RuntimeError(f"`{n}` must be a contiguous [{D}] {qkv.dtype} tensor")
    if q_out is None:
        q_out = torch.empty((T, H, D), dtype=qkv.dtype, device=dev)
    if q_out.shape != (T, H, D) or q_out.stride(2) != 1 or q_out.stride(1) != D:
        raise RuntimeError("`q_out` must be [T, H, D] with contiguous heads")
    if T == 0:
        return q_out
    lib = _hip.load()
    rc = lib.lv_qk_norm_rope_cache(
        _ptr(qkv), qkv.stride(0), _ptr(q_norm_weight), _ptr(k_norm_weight), _ptr(cos_cache),
        _ptr(sin_cache), cos_cache.shape[0], _ptr(positions), _ptr(slot_mapping), _ptr(q_out),
        q_out.stride(0), _ptr(key_cache), _ptr(value_cache), n_blocks, bs, T, H, Hkv, D,
        float(eps), _dtype_code(qkv), _stream(dev))
    _hip.check(rc, "lv_qk_norm_rope_cache")
    return q_out


def silu_mul(gate_up: torch.Tensor, out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """out = to_dtype(silu(gate)) * up for gate_up = [gate | up] per row.

    Reference: models/llama.py:37-38.
    """
    dev = gate_up.device
    _require_device("gate_up", gate_up, dev)
    _require_device("out", out, dev)
    T, two_i = gate_up.shape
    inter = two_i // 2
    _check_rows("gate_up", gate_up, 2 * inter, gate_up.dtype)
    if out is None:
        out = torch.empty((T, inter), dtype=gate_up.dtype, device=dev)
    _check_rows("out", out, inter, gate_up.dtype)
    if T == 0:
        return out
    lib = _hip.load()
    rc = lib.lv_silu_mul(_ptr(gate_up), gate_up.stride(0), _ptr(out), out.stride(0), T, inter,
                         _dtype_code(gate_up), _stream(dev))
    _hip.check(rc, "lv_silu_mul")
    return out


_ACTIVATIONS = {None: _hip.LV_ACT_NONE, "silu_mul": _hip.LV_ACT_SILU_MUL}
_linear_ok: dict = {}


def linear_supported(m: int, n: int, k: int, dtype: torch.dtype,
                     activation: Optional[str] = None) -> bool:
    """Whether lv_linear has a kernel for this shape (bf16/fp16, n % 32 == 0,
    k % 128 == 0; n is the output width); cached per (n, k, dtype,
    activation)."""
    if dtype not in (torch.bfloat16, torch.float16) or m < 1:
        return False
    key = (n, k, dtype, activation)
    ok = _linear_ok.get(key)
    if ok is None:
        ok = bool(_hip.load().lv_linear_supported(m, n, k, _ACTIVATIONS[activation],
                                                  _DTYPE_CODES[dtype]))
        _linear_ok[key] = ok
    return ok


def linear(x: torch.Tensor, weight: torch.Tensor, activation: Optional[str] = None,
           out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """y = x @ weight.T (nn.Linear without bias) for decode-sized x ([M, K],
    M up to a few hundred) on the MFMA kernel; with activation="silu_mul" and
    weight = [gate; up] ([2N, K]): y = silu_mul(x @ weight.T), the same
    values lv_silu_mul gives on the plain product.  Raises for shapes it has
    no kernel for (see linear_supported).

    Reference: layers/linear.py:15-65 (ColumnParallelLinear /
    RowParallelLinear = nn.Linear), models/llama.py:38.
    """
    dev = x.device
    for name, t in (("x", x), ("weight", weight), ("out", out)):
        _require_device(name, t, dev)
    M, K = x.shape
    rows = weight.shape[0]
    N = rows // 2 if activation == "silu_mul" else rows
    _check_rows("x", x, K, x.dtype)
    _check_rows("weight", weight, K, x.dtype)
    if weight.shape[1] != K or (activation == "silu_mul" and rows % 2):
        raise RuntimeError(f"weight {tuple(weight.shape)} does not match x {tuple(x.shape)}")
    if out is None:
        out = torch.empty((M, N), dtype=x.dtype, device=dev)
    _check_rows("out", out, N, x.dtype)
    if M == 0:
        return out
    lib = _hip.load()
    rc = lib.lv_linear(_ptr(x), x.stride(0), _ptr(weight), weight.stride(0), _ptr(out),
                       out.stride(0), M, N, K, _ACTIVATIONS[activation], _dtype_code(x),
                       _stream(dev))
    _hip.check(rc, "lv_linear")
    return out
