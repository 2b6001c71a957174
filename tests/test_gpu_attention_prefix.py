"""GPU parity of the shared-prefix (cascade) decode attention,
lv_paged_attention_prefix, against the CPU oracle.

Decode rows are put in groups whose block tables start with the same
physical blocks; the kernel reads those blocks once per group and merges the
partial softmax with each row's own remaining blocks.  The oracle
(oracle/attention.py, the reference's _decode_fast restated) gathers every
row's whole context, so agreement shows the split and merge change nothing
beyond fp32 rounding: same bar as the plain path (max-abs 2e-2, mean-abs
1e-3, relative L2 1e-2), plus closeness to lv_paged_attention's own output.
"""

from __future__ import annotations

import pytest
import torch

from litevllm import ops, workloads
from oracle import attention as oatt

pytestmark = pytest.mark.gpu

ATOL_MAX, ATOL_MEAN, REL_L2 = 2e-2, 1e-3, 1e-2


def _say(msg):
    print(f"[case] {msg}", flush=True)


def _check(got: torch.Tensor, ref: torch.Tensor, what: str):
    got = got.float().cpu()
    err = (got - ref).abs()
    rel = (got - ref).norm() / ref.norm().clamp_min(1e-30)
    assert torch.isfinite(got).all(), f"{what}: non-finite output"
    assert err.max() <= ATOL_MAX, f"{what}: max-abs {err.max():.3e}"
    assert err.mean() <= ATOL_MEAN, f"{what}: mean-abs {err.mean():.3e}"
    assert rel <= REL_L2, f"{what}: rel-L2 {rel:.3e}"


def _share(batch: workloads.PagedBatch, groups):
    """Copy each group leader's first prefix blocks into its members' tables
    (the layout a prefix-cache hit on a common prompt produces)."""
    bt = batch.block_tables.clone()
    for rows, pblocks in groups:
        for r in rows[1:]:
            bt[r, :pblocks] = bt[rows[0], :pblocks]
    batch.block_tables = bt
    return batch


def _oracle(b: workloads.PagedBatch):
    return oatt.mixed_attention(b.query, b.key_cache, b.value_cache, b.block_tables,
                                b.cu_seqlens, b.context_lens, b.scale)


def _run(b: workloads.PagedBatch, device, plan=None, use_cu=False, **kw):
    d = b.to(device)
    return ops.paged_attention(d.query, d.key_cache, d.value_cache, d.block_tables,
                               d.context_lens, scale=d.scale,
                               cu_seqlens=d.cu_seqlens if use_cu else None,
                               num_decodes=d.num_decodes, max_query_len=d.max_query_len,
                               prefix=plan, **kw)


def _groups_for(ctx: torch.Tensor, spans, bs=16):
    """spans: (first row, rows, prefix blocks or None = largest the group's
    shortest context allows, capped at 128)."""
    out = []
    for r0, n, pb in spans:
        rows = list(range(r0, r0 + n))
        cap = min(int(ctx[r0:r0 + n].min()) // bs, ops.PREFIX_MAX_BLOCKS)
        out.append((rows, cap if pb is None else min(pb, cap)))
    return out


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("heads", [(16, 8, 128), (4, 2, 64), (8, 8, 128), (32, 4, 64),
                                   (16, 2, 128), (32, 8, 128), (16, 4, 64)])
def test_prefix_shapes(device, dtype, heads):
    H, Hkv, D = heads
    _say(f"prefix shapes dtype={dtype} H={H} Hkv={Hkv} D={D}")
    b = workloads.paged_decode(seed=31, num_seqs=160, num_heads=H, num_kv_heads=Hkv,
                               head_dim=D, ctx_lo=40, ctx_hi=1500, dtype=dtype,
                               scale_inputs=False, tail_fill=float("nan"))
    # a big group (several member slices for every G), a small one, one of
    # two rows, a prefix of one block, a prefix not a multiple of 128 keys
    groups = _groups_for(b.context_lens, [(0, 70, None), (70, 5, 5), (80, 2, 1),
                                          (90, 30, 13)])
    b = _share(b, groups)
    plan = ops.prefix_plan(groups, b.num_decodes, H // Hkv, device)
    got = _run(b, device, plan)
    _check(got, _oracle(b), f"prefix {dtype} {heads}")
    plain = _run(b, device)
    assert (got.float() - plain.float()).abs().max() <= 2e-2


def test_prefix_config2_shape(device):
    """The Qwen3 decode shape at config-2 size: half the rows share 32 blocks
    (512 tokens), a quarter share 8 blocks, the rest are on their own."""
    _say("prefix config2 shape")
    b = workloads.paged_decode(seed=0, num_seqs=256, ctx_lo=600, ctx_hi=2048)
    groups = [(list(range(0, 128)), 32), (list(range(128, 192)), 8)]
    b = _share(b, groups)
    plan = ops.prefix_plan(groups, b.num_decodes, 2, device)
    _check(_run(b, device, plan), _oracle(b), "config2 prefix")


def test_prefix_covers_whole_context(device):
    """Rows whose whole context is the shared prefix (nothing left to walk:
    the merge has only prefix partials), including the 128-block maximum."""
    _say("prefix covers the whole context")
    b = workloads.paged_decode(seed=4, num_seqs=40, ctx_lo=300, ctx_hi=2100,
                               scale_inputs=False,
                               ctx_head=[2048] * 6 + [160] * 4 + [2048] * 3)
    groups = [([0, 1, 2, 3, 4, 5], 128), ([6, 7, 8, 9], 10), ([10, 11, 12], 128)]
    b = _share(b, groups)
    plan = ops.prefix_plan(groups, b.num_decodes, 2, device)
    _check(_run(b, device, plan), _oracle(b), "whole-context prefix")


def test_prefix_long_rows_many_pieces(device):
    """Long rows (each spread over many workgroup ranges) with a shared
    prefix of more than four 128-key splits, rows whose whole context is
    that prefix, a row with one block past it, and long rows without a
    prefix: the reduce kernel's general merge (pieces from their slots,
    splits in a loop) for every combination."""
    _say("prefix long rows, many pieces and splits")
    b = workloads.paged_decode(seed=17, num_seqs=12, ctx_lo=5000, ctx_hi=9000,
                               scale_inputs=False,
                               ctx_head=[1024, 1024, 7000, 9000, 1030, 6000])
    groups = [(list(range(0, 6)), 64), ([6, 7, 8], 20)]
    b = _share(b, groups)
    plan = ops.prefix_plan(groups, b.num_decodes, 2, device)
    got = _run(b, device, plan)
    _check(got, _oracle(b), "long rows with prefix")
    plain = _run(b, device)
    assert (got.float() - plain.float()).abs().max() <= 2e-2


def test_prefix_padding_and_workspace_reuse(device):
    """A padded plan (unused items) and back-to-back calls with different
    plans on the same workspaces: stale partials are never read."""
    _say("prefix padding and workspace reuse")
    for seed, n, spans in ((41, 300, [(0, 100, 20), (100, 100, None)]),
                           (42, 17, [(3, 9, 2)]),
                           (43, 64, [(0, 64, None)])):
        b = workloads.paged_decode(seed=seed, num_seqs=n, ctx_lo=100, ctx_hi=2500,
                                   scale_inputs=False)
        groups = _groups_for(b.context_lens, spans)
        b = _share(b, groups)
        plan = ops.prefix_plan(groups, b.num_decodes, 2, device, max_items=64, max_members=400)
        _check(_run(b, device, plan), _oracle(b), f"reuse seed={seed}")


def test_prefix_with_prefill_chunks(device):
    """Decode rows with shared prefixes next to prefill chunks in one call:
    the chunk rows are computed exactly as without a prefix plan."""
    _say("prefix with prefill chunks")
    step = workloads.mixed_step(seed=5, num_decodes=48, dec_lo=300, dec_hi=1500, num_chunks=3,
                                chunk_len=70, off_hi=400, num_cache_slots=16 * 3000)
    b = step.batch
    groups = _groups_for(b.context_lens, [(0, 30, 16), (30, 10, None)])
    b = _share(b, groups)
    plan = ops.prefix_plan(groups, b.num_decodes, 2, device)
    got = _run(b, device, plan, use_cu=True)
    _check(got, _oracle(b), "prefix + chunks")
    plain = _run(b, device, use_cu=True)
    nd = b.num_decodes
    assert torch.equal(got[nd:].cpu(), plain[nd:].cpu())


@pytest.mark.parametrize("dtype,heads", [(torch.bfloat16, (16, 8, 128)),
                                         (torch.float16, (8, 8, 64)),
                                         (torch.bfloat16, (32, 4, 128))])
def test_prefix_interleaved_groups_and_leaders(device, dtype, heads):
    """Groups whose rows interleave (even rows share one prefix, rows
    1 mod 4 another), leaders that are not the group's first row, and
    more members than one item slice holds: each member's query row is
    found through prefix_members."""
    H, Hkv, D = heads
    _say(f"prefix interleaved groups {dtype} {heads}")
    b = workloads.paged_decode(seed=12, num_seqs=200, num_heads=H, num_kv_heads=Hkv,
                               head_dim=D, ctx_lo=400, ctx_hi=1800, dtype=dtype,
                               scale_inputs=False)
    even = list(range(0, 200, 2))
    odd = list(range(1, 200, 4))
    groups = [([even[37]] + even[:37] + even[38:], 20), ([odd[-1]] + odd[:-1], 9)]
    b = _share(b, groups)
    plan = ops.prefix_plan(groups, b.num_decodes, H // Hkv, device)
    got = _run(b, device, plan)
    _check(got, _oracle(b), f"interleaved {dtype} {heads}")


def test_prefix_out_of_range_entries_are_skipped(device):
    """Items naming rows or splits outside their ranges do nothing (the rows
    of valid items are still right)."""
    _say("prefix out-of-range items")
    b = workloads.paged_decode(seed=6, num_seqs=20, ctx_lo=400, ctx_hi=900, scale_inputs=False)
    groups = [(list(range(0, 8)), 16)]
    b = _share(b, groups)
    blocks, items, members = ops.prefix_plan_arrays(groups, 20, 2)
    bad = [[25, 0, 8, 0], [0, 0, 8, 16], [-1, 0, 8, 0], [0, 0, 0, 0]]
    items = torch.cat([torch.from_numpy(items), torch.tensor(bad, dtype=torch.int32)])
    plan = ops.PrefixPlan(torch.from_numpy(blocks).to(device), items.to(device),
                          torch.from_numpy(members).to(device))
    _check(_run(b, device, plan), _oracle(b), "out-of-range items")


def test_prefix_unsupported_raises(device):
    _say("prefix unsupported")
    b = workloads.paged_decode(seed=7, num_seqs=8, ctx_lo=100, ctx_hi=200, dtype=torch.float32)
    plan = ops.prefix_plan([([0, 1], 4)], 8, 2, device)
    with pytest.raises(RuntimeError, match="shared-prefix"):
        _run(b, device, plan)
