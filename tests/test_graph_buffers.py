"""Graph-static buffers of DecodeGraphs, built on the CPU (no kernel runs):
for every padded batch size a decode graph can replay, the attention
workspace, the shared-prefix scratch and the prefix-plan buffer cover what
the C ABI's size functions ask for.  (What the decode kernels address is
modelled against those size functions in tests/host_model/capi_host_check.cpp.)"""

from __future__ import annotations

from types import SimpleNamespace

import numpy as np
import pytest
import torch

from litevllm import ops, workloads
from litevllm.config.config import CacheConfig, ModelConfig
from litevllm.engine.model_runner import GRAPH_BATCHES, PREFIX_MAX_ITEMS, DecodeGraphs


def _runner(max_model_len: int, shape: dict):
    mc = ModelConfig(model="shape-only", dtype="bfloat16", max_model_len=max_model_len,
                     load_format="dummy", hf_overrides=dict(shape))
    mc.resolve()
    return SimpleNamespace(model_config=mc, device="cpu",
                           config=SimpleNamespace(cache_config=CacheConfig(block_size=16)))


@pytest.mark.parametrize("max_batch", [1, 7, 200, 256, 512])
@pytest.mark.parametrize("shape", ["qwen3", "gqa4"])
def test_static_buffers_cover_every_padded_batch(max_batch, shape):
    spec = dict(workloads.QWEN3_06B_SHAPE)
    if shape == "gqa4":
        spec.update(num_attention_heads=32, num_key_value_heads=8)
    r = _runner(40960, spec)
    mc = r.model_config
    g = DecodeGraphs(r, max_batch)
    H, D, bs = mc.num_attention_heads, mc.head_dim, 16
    assert g.max_blocks == 40960 // bs
    # every batch of B <= max_batch rows has a captured size b >= B
    assert g.batches == sorted(g.batches) and g.batches[-1] == max_batch
    assert all(b in GRAPH_BATCHES or b == max_batch for b in g.batches)
    for B in range(1, max_batch + 1):
        assert any(b >= B for b in g.batches)
    for b in g.batches:
        need = ops.paged_attention_workspace_size(b, b, b, H, D, bs, g.max_blocks, 1,
                                                  mc.torch_dtype)
        assert g.workspace.numel() >= need, (b, g.workspace.numel(), need)
        for name, t in g._views(b).items():
            want = b + 1 if name == "cu_seqlens" else b
            assert t.shape[0] == want, name
        assert g._views(b)["block_tables"].shape[1] == g.max_blocks
    assert g.use_prefix
    n = max_batch
    for b in g.batches:
        assert g.pfx_workspace.numel() >= ops.prefix_workspace_size(b, H, D)
    # plan buffer: blocks [n] padded to 4, items [PREFIX_MAX_ITEMS, 4] 16-byte
    # aligned, members [n]; unused items are marked -1
    p = g.pfx_plan
    assert p.blocks.shape[0] == n and p.members.shape[0] == n
    assert p.items.shape == (PREFIX_MAX_ITEMS, 4)
    assert (p.items.data_ptr() - g.pfx_buf.data_ptr()) % 16 == 0
    assert p.items.data_ptr() - g.pfx_buf.data_ptr() == g.pfx_npad * 4
    assert p.members.data_ptr() - g.pfx_buf.data_ptr() == (g.pfx_npad + 4 * PREFIX_MAX_ITEMS) * 4
    assert bool((p.items[:, 0] == -1).all())
    # the plan the engine writes for a batch of n rows in groups of 16 that
    # share 32 blocks fills exactly the static buffer (blocks, padding,
    # items, members), with at most PREFIX_MAX_ITEMS items
    from litevllm.engine.model_runner import find_shared_prefixes
    nblk = 40
    descs = np.zeros((n, 6), np.int32)
    descs[:, 0] = nblk * 16 - 1
    descs[:, 1] = 1
    descs[:, 2] = nblk
    descs[:, 3] = np.arange(n) * nblk
    block_ids = np.arange(n * nblk, dtype=np.int32) + 1
    for i in range(n):                        # rows of a group share blocks 0..31
        lead = (i // 16) * 16
        block_ids[i * nblk:i * nblk + 32] = block_ids[lead * nblk:lead * nblk + 32]
    groups = find_shared_prefixes(descs, block_ids, n, 16, g.group_size, min_saved=0)
    blocks, items, members = ops.prefix_plan_arrays(groups, n, g.group_size, 16,
                                                    max_items=PREFIX_MAX_ITEMS, max_members=n)
    assert blocks.size == n and items.shape == (PREFIX_MAX_ITEMS, 4) and members.size == n
    assert g.pfx_npad + items.size + members.size == g.pfx_buf.numel()
    if n >= 32:
        assert groups and int((items[:, 0] >= 0).sum()) <= PREFIX_MAX_ITEMS
