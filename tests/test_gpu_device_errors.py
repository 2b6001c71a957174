"""Out-of-range indices reach the kernels: they clamp them (nothing is read
or written outside a buffer) and report them through lv_device_errors.

The reference's torch indexing raises on such an index
(litevllm/layers/attention.py:80-84 slot_mapping into the caches, 111-119
block_table into the caches).  Here one invalid slot (lv_kv_scatter,
lv_qk_norm_rope_cache) must leave the cache untouched for that token and
raise LV_DEVERR_SLOT; one invalid block id (decode rows on the persistent
and the row kernel, prefill-chunk rows, the shared-prefix pass) must be
read as block 0 and raise LV_DEVERR_BLOCK_ID.  Every test starts and ends
with a clean report."""

from __future__ import annotations

import pytest
import torch

from litevllm import _hip, ops, workloads
from oracle import attention as oatt
from oracle import layers as L

pytestmark = pytest.mark.gpu

ATOL_MAX, ATOL_MEAN, REL_L2 = 2e-2, 1e-3, 1e-2


def _say(msg):
    print(f"[case] {msg}", flush=True)


@pytest.fixture(autouse=True)
def clean_report(device):
    # every earlier test of the session left nothing behind
    assert ops.device_errors(device, clear=True) == 0
    yield
    assert ops.device_errors(device, clear=True) == 0


def _close(got, ref, what):
    got = got.float().cpu()
    err = (got - ref).abs()
    assert torch.isfinite(got).all(), what
    assert err.max() <= ATOL_MAX and err.mean() <= ATOL_MEAN, f"{what}: {err.max():.3e}"
    assert (got - ref).norm() / ref.norm() <= REL_L2, what


def test_scatter_reports_slot_past_the_cache(device):
    _say("scatter: one slot past the cache, one padding slot")
    g = torch.Generator().manual_seed(5)
    N, bs, Hkv, D, T = 40, 16, 8, 128, 100
    slots = torch.randperm(N * bs, generator=g)[:T].to(torch.int64)
    slots[17] = N * bs               # first slot past the cache
    slots[60] = -1                   # padding: skipped, not an error
    k = torch.randn(T, Hkv, D, generator=g).to(torch.bfloat16)
    v = torch.randn(T, Hkv, D, generator=g).to(torch.bfloat16)
    kc = torch.full((N, bs, Hkv, D), 5.0, dtype=torch.bfloat16, device=device)
    vc = torch.full((N, bs, Hkv, D), -5.0, dtype=torch.bfloat16, device=device)
    ops.kv_scatter(k.to(device), v.to(device), kc, vc, slots.to(device))
    assert ops.device_errors(device, clear=False) == _hip.LV_DEVERR_SLOT
    with pytest.raises(RuntimeError, match="slot_mapping entry"):
        ops.check_device_errors(device)
    assert ops.device_errors(device) == 0            # the check cleared it
    ok = (slots >= 0) & (slots < N * bs)
    fk, fv = kc.view(N * bs, Hkv, D).cpu(), vc.view(N * bs, Hkv, D).cpu()
    assert torch.equal(fk[slots[ok]], k[ok]) and torch.equal(fv[slots[ok]], v[ok])
    untouched = torch.ones(N * bs, dtype=torch.bool)
    untouched[slots[ok]] = False
    assert bool((fk[untouched] == 5.0).all()) and bool((fv[untouched] == -5.0).all())
    # a valid call afterwards reports nothing
    ops.kv_scatter(k[ok].to(device), v[ok].to(device), kc, vc, slots[ok].to(device))
    assert ops.device_errors(device) == 0


def test_qk_norm_rope_cache_reports_slot_past_the_cache(device):
    _say("qk_norm_rope_cache: one slot past the cache")
    g = torch.Generator().manual_seed(6)
    H, Hkv, D, T, bs, nb, P = 16, 8, 128, 33, 16, 10, 2048
    dt = torch.bfloat16
    qkv = torch.randn(T, (H + 2 * Hkv) * D, generator=g).to(dt)
    inv = 1.0 / (1e6 ** (torch.arange(0, D, 2, dtype=torch.float32) / D))
    f = torch.outer(torch.arange(P, dtype=torch.float32), inv)
    cos, sin = f.cos().to(dt), f.sin().to(dt)
    pos = torch.randint(0, P, (T,), generator=g)
    slots = torch.randperm(nb * bs, generator=g)[:T]
    bad = slots.clone()
    bad[9] = nb * bs + 3
    qw = (torch.rand(D, generator=g) + 0.5).to(dt)
    kw = (torch.rand(D, generator=g) + 0.5).to(dt)
    kc = torch.full((nb, bs, Hkv, D), 3.0, dtype=dt)
    vc = torch.full((nb, bs, Hkv, D), 3.0, dtype=dt)
    kc_d, vc_d = kc.to(device), vc.to(device)
    ref_slots = slots.clone()
    ref_slots[9] = -1                 # the oracle writes no row for that token
    L.qk_norm_rope_cache(qkv, H, Hkv, D, cos, sin, pos, ref_slots, kc, vc, qw, kw, 1e-6)
    ops.qk_norm_rope_cache(qkv.to(device), H, Hkv, D, cos.to(device), sin.to(device),
                           pos.to(device), bad.to(device), kc_d, vc_d,
                           q_norm_weight=qw.to(device), k_norm_weight=kw.to(device), eps=1e-6)
    assert ops.device_errors(device) == _hip.LV_DEVERR_SLOT
    # the token's cache row was not written (still the fill value); every
    # other row is the oracle's to within the kernel's 1-2 ulp
    fk, fv = kc_d.view(nb * bs, Hkv, D).cpu(), vc_d.view(nb * bs, Hkv, D).cpu()
    assert bool((fk[slots[9]] == 3.0).all()) and bool((fv[slots[9]] == 3.0).all())
    assert torch.equal(fv, vc.view(nb * bs, Hkv, D))
    kref = kc.view(nb * bs, Hkv, D)
    assert (fk.float() - kref.float()).abs().max() <= 0.05


def _decode_batch():
    return workloads.paged_decode(seed=8, num_seqs=24, ctx_lo=40, ctx_hi=900,
                                  scale_inputs=False, ctx_head=[300, 17, 600])


@pytest.mark.parametrize("kernel", ["persistent", "rows"])
def test_decode_reports_block_id_outside_the_cache(device, kernel, monkeypatch):
    _say(f"decode ({kernel}): one block id outside the cache")
    if kernel == "rows":
        monkeypatch.setenv("LV_ATTN_DECODE_KERNEL", "rows")
    b = _decode_batch()
    nblk = b.key_cache.shape[0]
    bt = b.block_tables.clone()
    bt[0, 5] = nblk + 11              # inside row 0's context (300 tokens)
    bt[2, 20] = -4                    # inside row 2's context (600 tokens)
    d = b.to(device)
    got = ops.paged_attention(d.query, d.key_cache, d.value_cache, bt.to(device),
                              d.context_lens, scale=b.scale)
    assert ops.device_errors(device) == _hip.LV_DEVERR_BLOCK_ID
    ref_bt = bt.clone()
    ref_bt[0, 5] = 0                  # what the clamp reads instead
    ref_bt[2, 20] = 0
    ref = oatt.mixed_attention(b.query, b.key_cache, b.value_cache, ref_bt, b.cu_seqlens,
                               b.context_lens, b.scale)
    _close(got, ref, f"decode {kernel} clamped")
    # the same call with a valid table reports nothing
    ops.paged_attention(d.query, d.key_cache, d.value_cache, d.block_tables, d.context_lens,
                        scale=b.scale)
    assert ops.device_errors(device) == 0


def test_chunk_rows_report_block_id_outside_the_cache(device):
    _say("prefill chunks: one block id outside the cache")
    step = workloads.mixed_step(seed=12, num_decodes=3, dec_lo=50, dec_hi=300, num_chunks=2,
                                chunk_len=70, off_lo=100, off_hi=200, num_cache_slots=16 * 200)
    b = step.batch
    nblk = b.key_cache.shape[0]
    bt = b.block_tables.clone()
    bt[3, 2] = nblk                   # first chunk sequence, a block of its cached prefix
    d = b.to(device)
    got = ops.paged_attention(d.query, d.key_cache, d.value_cache, bt.to(device),
                              d.context_lens, scale=b.scale, cu_seqlens=d.cu_seqlens,
                              num_decodes=b.num_decodes, max_query_len=b.max_query_len)
    assert ops.device_errors(device) == _hip.LV_DEVERR_BLOCK_ID
    ref_bt = bt.clone()
    ref_bt[3, 2] = 0
    ref = oatt.mixed_attention(b.query, b.key_cache, b.value_cache, ref_bt, b.cu_seqlens,
                               b.context_lens, b.scale)
    _close(got, ref, "chunks clamped")


def test_prefix_pass_reports_block_id_outside_the_cache(device):
    _say("shared-prefix pass: one block id outside the cache in the shared prefix")
    b = workloads.paged_decode(seed=9, num_seqs=32, ctx_lo=400, ctx_hi=900, scale_inputs=False)
    nblk = b.key_cache.shape[0]
    bt = b.block_tables.clone()
    bt[1:8, :16] = bt[0, :16]         # rows 0-7 share 16 blocks (256 tokens)
    bt[0:8, 4] = nblk + 2             # one of them outside the cache, in every member
    plan = ops.prefix_plan([(list(range(8)), 16)], 32, 2, device)
    d = b.to(device)
    got = ops.paged_attention(d.query, d.key_cache, d.value_cache, bt.to(device),
                              d.context_lens, scale=b.scale, prefix=plan)
    assert ops.device_errors(device) == _hip.LV_DEVERR_BLOCK_ID
    ref_bt = bt.clone()
    ref_bt[0:8, 4] = 0
    ref = oatt.mixed_attention(b.query, b.key_cache, b.value_cache, ref_bt, b.cu_seqlens,
                               b.context_lens, b.scale)
    _close(got, ref, "prefix clamped")
