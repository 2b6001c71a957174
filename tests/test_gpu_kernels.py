"""GPU parity of the four hot-path kernels against the CPU oracle.

Bars: packing, slot_mapping and KV scatter bit-exact; greedy argmax
bit-exact; temperature sampling bit-exact against oracle/sampler_ref.c at
the same uniforms; attention within 2e-2 max-abs and 1e-3 mean-abs of the
fp32 oracle on the same bf16 inputs (plus relative L2 <= 1e-2).
"""

from __future__ import annotations

import json
import math
import sys
from pathlib import Path

import numpy as np
import pytest
import torch

from litevllm import ops, workloads
from oracle import attention as oatt
from oracle import packing as opack
from oracle import sampler as osamp
from oracle import scatter as oscat

pytestmark = pytest.mark.gpu

ATOL_MAX, ATOL_MEAN, REL_L2 = 2e-2, 1e-3, 1e-2


def _say(msg):
    print(f"[case] {msg}", flush=True)


def _check_attention(got: torch.Tensor, ref: torch.Tensor, what: str):
    got = got.float().cpu()
    err = (got - ref).abs()
    rel = (got - ref).norm() / ref.norm().clamp_min(1e-30)
    assert torch.isfinite(got).all(), f"{what}: non-finite output"
    assert err.max() <= ATOL_MAX, f"{what}: max-abs {err.max():.3e}"
    assert err.mean() <= ATOL_MEAN, f"{what}: mean-abs {err.mean():.3e}"
    assert rel <= REL_L2, f"{what}: rel-L2 {rel:.3e}"


# ---------------------------------------------------------------------------
# KV scatter
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("strided", [False, True])
def test_kv_scatter_bit_exact(device, dtype, strided):
    _say(f"kv_scatter dtype={dtype} strided={strided}")
    g = torch.Generator().manual_seed(11)
    N, bs, Hkv, D, T = 64, 16, 8, 128, 300
    kc = torch.full((N, bs, Hkv, D), 3.5, dtype=dtype)
    vc = torch.full((N, bs, Hkv, D), -3.5, dtype=dtype)
    slots = torch.randperm(N * bs, generator=g)[:T].to(torch.int64)
    slots[::37] = -1
    if strided:
        qkv = torch.randn(T, (16 + 2 * Hkv) * D, generator=g).to(dtype)
        k = qkv[:, 16 * D:(16 + Hkv) * D].view(T, Hkv, D)
        v = qkv[:, (16 + Hkv) * D:].view(T, Hkv, D)
    else:
        k = torch.randn(T, Hkv, D, generator=g).to(dtype)
        v = torch.randn(T, Hkv, D, generator=g).to(dtype)
    kc_d, vc_d = kc.to(device), vc.to(device)
    if strided:
        qkv_d = qkv.to(device)
        k_d = qkv_d[:, 16 * D:(16 + Hkv) * D].view(T, Hkv, D)
        v_d = qkv_d[:, (16 + Hkv) * D:].view(T, Hkv, D)
    else:
        k_d, v_d = k.to(device), v.to(device)
    ops.kv_scatter(k_d, v_d, kc_d, vc_d, slots.to(device))
    torch.cuda.synchronize()
    kn, vn = kc.clone(), vc.clone()
    oscat.kv_scatter(k.contiguous().view(torch.int16).numpy() if dtype != torch.float32 else k.contiguous().numpy(),
                     v.contiguous().view(torch.int16).numpy() if dtype != torch.float32 else v.contiguous().numpy(),
                     kn.view(torch.int16).numpy() if dtype != torch.float32 else kn.numpy(),
                     vn.view(torch.int16).numpy() if dtype != torch.float32 else vn.numpy(),
                     slots.numpy())
    assert torch.equal(kc_d.cpu().view(torch.uint8), kn.view(torch.uint8))
    assert torch.equal(vc_d.cpu().view(torch.uint8), vn.view(torch.uint8))


def test_kv_scatter_config3_round_trip(device):
    _say("kv_scatter config3 round trip")
    step = workloads.mixed_step(seed=3)
    b = step.batch
    kc = torch.zeros_like(b.key_cache, device=device)
    vc = torch.zeros_like(b.value_cache, device=device)
    kc.fill_(7.0)
    vc.fill_(-7.0)
    slots = step.slot_mapping.to(device)
    ops.kv_scatter(step.key.to(device), step.value.to(device), kc, vc, slots)
    nb, bs = kc.shape[0], kc.shape[1]
    flat_k = kc.view(nb * bs, *kc.shape[2:])
    flat_v = vc.view(nb * bs, *vc.shape[2:])
    assert torch.equal(flat_k[slots].cpu(), step.key)
    assert torch.equal(flat_v[slots].cpu(), step.value)
    touched = torch.zeros(nb * bs, dtype=torch.bool, device=device)
    touched[slots] = True
    assert bool((flat_k[~touched] == 7.0).all()) and bool((flat_v[~touched] == -7.0).all())


# ---------------------------------------------------------------------------
# paged attention
# ---------------------------------------------------------------------------

def _run_attention(batch: workloads.PagedBatch, device, use_cu: bool):
    b = batch.to(device)
    return ops.paged_attention(b.query, b.key_cache, b.value_cache, b.block_tables,
                               b.context_lens, scale=b.scale,
                               cu_seqlens=b.cu_seqlens if use_cu else None,
                               num_decodes=b.num_decodes, max_query_len=b.max_query_len)


def _oracle(batch: workloads.PagedBatch):
    return oatt.mixed_attention(batch.query, batch.key_cache, batch.value_cache,
                                batch.block_tables, batch.cu_seqlens, batch.context_lens,
                                batch.scale)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("heads", [(16, 8, 128), (4, 2, 64), (8, 8, 128), (32, 4, 64),
                                   (16, 2, 128), (32, 8, 128), (16, 4, 64)])
def test_decode_small_shapes(device, dtype, heads):
    H, Hkv, D = heads
    _say(f"decode small dtype={dtype} H={H} Hkv={Hkv} D={D}")
    batch = workloads.paged_decode(seed=5, num_seqs=24, num_heads=H, num_kv_heads=Hkv,
                                   head_dim=D, ctx_lo=1, ctx_hi=700, dtype=dtype,
                                   scale_inputs=False, tail_fill=float("nan"),
                                   ctx_head=[1, 15, 16, 17, 256, 257, 512, 513])
    got = _run_attention(batch, device, use_cu=False)
    _check_attention(got, _oracle(batch), f"decode {dtype} {heads}")


@pytest.mark.parametrize("scaled", [True, False])
def test_decode_config2(device, scaled):
    _say(f"decode config2 scaled={scaled}")
    batch = workloads.paged_decode(seed=0, scale_inputs=scaled)
    got = _run_attention(batch, device, use_cu=False)
    _check_attention(got, _oracle(batch), f"config2 scaled={scaled}")


def test_decode_workspace_reuse_and_counter_reset(device):
    """Back-to-back calls of different shapes share one workspace; each is
    correct (stale partials of an earlier call are never read)."""
    _say("decode workspace reuse")
    for seed, n, lo, hi in ((21, 300, 1, 3000), (22, 7, 2000, 9000), (23, 64, 1, 40)):
        batch = workloads.paged_decode(seed=seed, num_seqs=n, ctx_lo=lo, ctx_hi=hi,
                                       scale_inputs=False)
        got = _run_attention(batch, device, use_cu=False)
        _check_attention(got, _oracle(batch), f"reuse seed={seed}")


def test_decode_long_contexts(device):
    """Rows of 16k-32k tokens among short ones: each workgroup walks many
    64-block groups, and a long row spreads over dozens of workgroup ranges,
    so the reduce takes its general (many-piece) merge path."""
    _say("decode long contexts")
    batch = workloads.paged_decode(seed=17, num_seqs=40, ctx_lo=1, ctx_hi=600,
                                   scale_inputs=False, tail_fill=float("nan"),
                                   ctx_head=[32768, 20000, 16385, 31999, 1])
    got = _run_attention(batch, device, use_cu=False)
    _check_attention(got, _oracle(batch), "long contexts")


@pytest.mark.parametrize("heads", [(16, 8, 128), (8, 1, 64), (32, 4, 128)])
def test_decode_lockstep_interval_bit_identical(device, heads, monkeypatch):
    """The persistent kernel's wavefront lockstep barrier (LV_ATTN_SYNC,
    default every 4 blocks) moves no data: outputs are bit-identical with it
    off, at the default and at every 2 blocks; each run must also finish
    (every wavefront of a workgroup reaches the same barriers)."""
    H, Hkv, D = heads
    _say(f"decode lockstep interval H={H} Hkv={Hkv} D={D}")
    batch = workloads.paged_decode(seed=31, num_seqs=200, num_heads=H, num_kv_heads=Hkv,
                                   head_dim=D, ctx_lo=1, ctx_hi=1500, scale_inputs=False,
                                   ctx_head=[1, 2, 17, 33, 1024])
    outs = {}
    for sync in ("default", "0", "2"):
        if sync == "default":
            monkeypatch.delenv("LV_ATTN_SYNC", raising=False)
        else:
            monkeypatch.setenv("LV_ATTN_SYNC", sync)
        outs[sync] = _run_attention(batch, device, use_cu=False).cpu()
    monkeypatch.delenv("LV_ATTN_SYNC", raising=False)
    _check_attention(outs["default"], _oracle(batch), f"lockstep {heads}")
    assert torch.equal(outs["default"].view(torch.int16), outs["0"].view(torch.int16))
    assert torch.equal(outs["default"].view(torch.int16), outs["2"].view(torch.int16))


@pytest.mark.parametrize("knobs", [
    {"LV_ATTN_NBUF": "4"}, {"LV_ATTN_NT": "0"}, {"LV_ATTN_PERSIST_WGS": "97"},
    {"LV_ATTN_PERSIST_WGS": "1"}, {"LV_ATTN_PERSIST_WGS": "1024"},
    {"LV_ATTN_DECODE_KERNEL": "rows"},
    {"LV_ATTN_DECODE_KERNEL": "rows", "LV_ATTN_PART_TOKENS": "128"},
    {"LV_ATTN_CHUNK_KERNEL": "rows"}])
def test_attention_tuning_knobs(device, knobs, monkeypatch):
    """The per-call tuning knobs of lv_paged_attention (register buffers,
    load type, persistent grid -- one workgroup: every row whole; 1024: the
    40 rows cut into ranges of a few blocks, most rows in three or more
    pieces -- the fallback row kernels and their partition size) keep a
    mixed step within the attention bar; the two that change only prefetch
    depth or load type leave it bit-identical."""
    _say(f"attention knobs {knobs}")
    step = workloads.mixed_step(seed=13, num_decodes=40, dec_lo=1, dec_hi=2500, num_chunks=3,
                                chunk_len=90, off_hi=700, num_cache_slots=16 * 3000)
    base = _run_attention(step.batch, device, use_cu=True).cpu()
    for k, v in knobs.items():
        monkeypatch.setenv(k, v)
    got = _run_attention(step.batch, device, use_cu=True).cpu()
    for k in knobs:
        monkeypatch.delenv(k)
    _check_attention(got, _oracle(step.batch), f"knobs {knobs}")
    if set(knobs) <= {"LV_ATTN_NBUF", "LV_ATTN_NT"}:
        assert torch.equal(got.view(torch.int16), base.view(torch.int16))


def test_decode_matches_reference_restatement(device):
    """The literal _decode_fast restatement (gather over max_s, mask, einsum)."""
    _say("decode vs literal _decode_fast restatement")
    batch = workloads.paged_decode(seed=9, num_seqs=12, ctx_lo=1, ctx_hi=300, scale_inputs=False)
    got = _run_attention(batch, device, use_cu=False)
    ref = oatt.decode_attention(batch.query.float(), batch.key_cache.float(),
                                batch.value_cache.float(), batch.block_tables,
                                batch.context_lens, batch.scale)
    _check_attention(got, ref, "literal restatement")


@pytest.mark.parametrize("seed", [0, 1])
def test_mixed_step_small(device, seed):
    _say(f"mixed step small seed={seed}")
    step = workloads.mixed_step(seed=seed, num_decodes=12, dec_lo=1, dec_hi=600, num_chunks=4,
                                chunk_len=67, off_hi=300, num_cache_slots=16 * 400)
    got = _run_attention(step.batch, device, use_cu=True)
    _check_attention(got, _oracle(step.batch), f"mixed small seed={seed}")


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("heads", [(16, 8, 128), (4, 2, 64), (8, 8, 128), (32, 4, 64),
                                   (16, 2, 128), (32, 8, 128), (16, 4, 64)])
def test_chunks_all_shapes(device, dtype, heads):
    """Prefill chunks at unaligned offsets (MFMA path for bf16/fp16, per-row
    path for fp32), mixed with decodes, against the fp32 oracle."""
    H, Hkv, D = heads
    _say(f"chunks dtype={dtype} H={H} Hkv={Hkv} D={D}")
    step = workloads.mixed_step(seed=7, num_decodes=5, dec_lo=1, dec_hi=300, num_chunks=5,
                                chunk_len=97, off_lo=0, off_hi=400, num_heads=H,
                                num_kv_heads=Hkv, head_dim=D, num_cache_slots=16 * 300,
                                dtype=dtype)
    got = _run_attention(step.batch, device, use_cu=True)
    _check_attention(got, _oracle(step.batch), f"chunks {dtype} {heads}")


def test_chunk_lengths_and_offsets(device):
    """Chunk lengths 1..70 (ragged last query tile), offsets that are and
    are not block-aligned, a chunk ending exactly on a block edge."""
    _say("chunk lengths / offsets")
    g = torch.Generator().manual_seed(3)
    for chunk_len, off in ((1, 0), (2, 15), (31, 16), (32, 17), (33, 0), (64, 5), (70, 64), (16, 48)):
        step = workloads.mixed_step(seed=chunk_len * 100 + off, num_decodes=0, num_chunks=2,
                                    chunk_len=chunk_len, off_lo=off, off_hi=off,
                                    num_cache_slots=16 * 64)
        got = _run_attention(step.batch, device, use_cu=True)
        _check_attention(got, _oracle(step.batch), f"chunk len={chunk_len} off={off}")


def test_chunks_beyond_64_tiles(device):
    """Chunk rows whose keys run past 64 tiles of 64 keys (contexts beyond
    4096 tokens): the block ids each wavefront prefetches 64 tiles at a time
    are refilled mid-row.  One pair of chunks straddles the 4096-key edge,
    the other runs to ~12k keys (two refills)."""
    for seed, off_lo, off_hi, L in ((41, 3990, 3990, 130), (42, 8000, 12000, 96)):
        _say(f"chunks beyond 64 tiles off={off_lo}..{off_hi} len={L}")
        step = workloads.mixed_step(seed=seed, num_decodes=4, dec_lo=1, dec_hi=6000,
                                    num_chunks=2, chunk_len=L, off_lo=off_lo, off_hi=off_hi,
                                    num_cache_slots=16 * 4096)
        assert int(step.batch.context_lens.max()) > 64 * 64
        got = _run_attention(step.batch, device, use_cu=True)
        _check_attention(got, _oracle(step.batch), f"long chunks off={off_lo}")


def test_mixed_config3_full(device):
    """The full config-3 step: 192 decodes + 15 chunks of 512 at offsets up
    to 3072, 200k-slot cache, N(0,1) values."""
    _say("mixed config3 full")
    step = workloads.mixed_step(seed=0)
    got = _run_attention(step.batch, device, use_cu=True)
    _check_attention(got, _oracle(step.batch), "config3")


def test_prefill_only_offset_zero(device):
    _say("prefill only, offset 0")
    step = workloads.mixed_step(seed=4, num_decodes=0, num_chunks=3, chunk_len=100, off_lo=0,
                                off_hi=0, num_cache_slots=16 * 64)
    got = _run_attention(step.batch, device, use_cu=True)
    _check_attention(got, _oracle(step.batch), "prefill offset 0")


# ---------------------------------------------------------------------------
# sampler
# ---------------------------------------------------------------------------

def test_sampler_config4(device):
    _say("sampler config4")
    sb = workloads.sampler_batch(seed=0)
    got = ops.sample(sb.logits.to(device), sb.temperature.to(device), sb.uniform.to(device)).cpu()
    x = sb.logits.float().numpy()
    half = sb.logits.shape[0] // 2
    # greedy rows: the planted maximum, bit-exact with argmax
    assert torch.equal(got[:half], sb.planted[:half])
    assert np.array_equal(got[:half].numpy(), osamp.greedy(x[:half]))
    # temperature rows: bit-exact with the C restatement at the same uniforms
    ref = osamp.sample(x[half:], sb.temperature[half:].numpy(), sb.uniform[half:].numpy())
    assert np.array_equal(got[half:].numpy(), ref)


_SAMPLER_CHILD = r"""
import sys, numpy as np, torch
sys.path[:0] = sys.argv[1:3]
from litevllm import ops, workloads
sb = workloads.sampler_batch(seed=0)
d = torch.device("cuda:0")
ids = ops.sample(sb.logits.to(d), sb.temperature.to(d), sb.uniform.to(d)).cpu().numpy()
np.save(sys.argv[3], ids)
"""


@pytest.mark.parametrize("per_cu", ["1", "3", "32"])
def test_sampler_grid_knob_bit_identical(device, per_cu, tmp_path):
    """LV_SAMPLER_WGS_PER_CU (workgroups of the items kernel per CU, read
    once per process) only changes how segments are spread over
    wavefronts: config 4's ids are bit-identical to this process's default
    grid.  One child process per setting (the value is cached at first
    use)."""
    import os
    import subprocess
    import sys
    _say(f"sampler LV_SAMPLER_WGS_PER_CU={per_cu} (child process)")
    sb = workloads.sampler_batch(seed=0)
    want = ops.sample(sb.logits.to(device), sb.temperature.to(device),
                      sb.uniform.to(device)).cpu().numpy()
    root = Path(__file__).resolve().parent.parent
    out = tmp_path / "ids.npy"
    env = dict(os.environ, LV_SAMPLER_WGS_PER_CU=per_cu)
    subprocess.run([sys.executable, "-c", _SAMPLER_CHILD, str(root), str(root / "lite-vllm_amd"),
                    str(out)], env=env, check=True, timeout=240)
    assert np.array_equal(np.load(out), want)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("V", [1, 7, 511, 512, 513, 32000, 151936])
def test_sampler_shapes(device, dtype, V):
    _say(f"sampler dtype={dtype} V={V}")
    g = torch.Generator().manual_seed(V)
    B = 12
    x = (torch.randn(B, V + 5, generator=g) * 3).to(dtype)[:, :V]   # row stride V + 5
    if V > 4:
        x[0, 1] = x[0, 3] = x[0].float().max() + 1   # tie: first index wins
        x[1, : V // 2] = float("-inf")
    temp = torch.tensor([0.0] * 4 + [0.6, 1.0, 1.7, 0.05, 1e-4, 2.0, 1.0, 1.0], dtype=torch.float32)
    uni = torch.rand(B, generator=g)
    uni[-2] = 0.0
    uni[-1] = float(np.nextafter(np.float32(1), np.float32(0)))
    xd = torch.empty(B, V + 5, dtype=dtype, device=device)[:, :V]
    xd.copy_(x)
    got = ops.sample(xd, temp.to(device), uni.to(device)).cpu().numpy()
    ref = osamp.sample(x.float().numpy(), temp.numpy(), uni.numpy())
    assert np.array_equal(got, ref)


# ---------------------------------------------------------------------------
# packing
# ---------------------------------------------------------------------------

KAT = json.loads((Path(__file__).parent / "golden" / "packing_kat.json").read_text())


def _pack_on_gpu(device, descs, blocks, toks, bs, max_blocks, dev_toks=None):
    T = int(np.asarray(descs)[:, 1].sum())
    out = ops.pack_inputs(torch.as_tensor(descs, dtype=torch.int32).to(device),
                          torch.as_tensor(blocks, dtype=torch.int32).to(device),
                          torch.as_tensor(toks, dtype=torch.int64).to(device), T, bs, max_blocks,
                          device_tokens=None if dev_toks is None else
                          torch.as_tensor(dev_toks, dtype=torch.int64).to(device))
    return {k: v.cpu().numpy() for k, v in out.items()}


@pytest.mark.parametrize("case", KAT["cases"], ids=lambda c: c["name"])
def test_pack_kat(device, case):
    _say(f"pack kat {case['name']}")
    recs = [opack.SeqRecord(s["prompt"], s["output"], s["num_computed"], s["blocks"])
            for s in case["seqs"]]
    descs, blocks, toks = opack.descriptors_from_records(recs)
    got = _pack_on_gpu(device, descs, blocks, toks, KAT["block_size"], case["packed"]["max_blocks"])
    for k in ("input_ids", "positions", "slot_mapping"):
        assert got[k].tolist() == case["reference"][k], k
    for k in ("cu_seqlens", "seq_start", "context_lens", "block_tables"):
        assert got[k].tolist() == case["packed"][k], k


@pytest.mark.parametrize("seed", range(4))
def test_pack_random(device, seed):
    _say(f"pack random seed={seed}")
    rng = np.random.default_rng(seed)
    B = int(rng.integers(1, 300))
    bs = 16
    descs, blocks, toks = [], [], []
    dev_toks = rng.integers(0, 151936, 50)
    for _ in range(B):
        if rng.random() < 0.6:
            n, q = int(rng.integers(0, 4000)), 1
        else:
            n, q = int(rng.integers(0, 3000)), int(rng.integers(1, 600))
        nb = (n + q + bs - 1) // bs - int(rng.random() < 0.1)
        tidx = int(rng.integers(0, 50)) if (q == 1 and rng.random() < 0.5) else -1
        descs.append([n, q, max(nb, 0), len(blocks), len(toks), tidx])
        blocks.extend(rng.integers(0, 12500, max(nb, 0)).tolist())
        toks.extend(rng.integers(0, 151936, q).tolist())
    descs = np.array(descs, dtype=np.int32)
    blocks = np.array(blocks, dtype=np.int32)
    toks = np.array(toks, dtype=np.int64)
    mb = int(descs[:, 2].max()) if B else 0
    got = _pack_on_gpu(device, descs, blocks, toks, bs, mb, dev_toks)
    ref = opack.expand_descriptors(descs, blocks, toks, bs, mb, device_tokens=dev_toks)
    for k in ref:
        assert np.array_equal(got[k], ref[k]), k


sys.path.insert(0, str(Path(__file__).parent / "golden"))
import packing_fixture  # noqa: E402


def test_pack_reference_fixtures(device):
    """Every schedule whose packed arrays the reference's own
    ModelRunner.prepare_inputs wrote (tests/golden/reference_packing.npz:
    40 decode-only and 40 prefill-only batches, block tables from its
    BlockManager, block sizes 8/16/32), replayed through lv_pack_inputs:
    bit-exact."""
    cases = packing_fixture.load_cases()
    _say(f"pack: {len(cases)} reference prepare_inputs fixtures")
    for case in cases:
        descs, blocks, toks = opack.descriptors_from_records(case["seqs"])
        mb = max(len(s.block_ids) for s in case["seqs"])
        got = _pack_on_gpu(device, descs, blocks, toks, case["block_size"], mb)
        for k in ("input_ids", "positions", "slot_mapping"):
            assert np.array_equal(got[k], case[k]), (case["name"], k)
        if not case["is_prefill"]:
            assert np.array_equal(got["block_tables"], case["block_tables"]), case["name"]
            assert np.array_equal(got["context_lens"], case["context_lens"]), case["name"]


def test_pack_config3(device):
    _say("pack config3")
    step = workloads.mixed_step(seed=2)
    mb = step.batch.block_tables.shape[1]
    got = _pack_on_gpu(device, step.descs.numpy(), step.block_ids.numpy(),
                       step.token_ids.numpy(), 16, mb)
    assert np.array_equal(got["slot_mapping"], step.slot_mapping.numpy())
    assert np.array_equal(got["positions"], step.positions.numpy())
    assert np.array_equal(got["input_ids"], step.token_ids.numpy())
    assert np.array_equal(got["cu_seqlens"], step.batch.cu_seqlens.numpy())
    assert np.array_equal(got["context_lens"], step.batch.context_lens.numpy())
    assert np.array_equal(got["block_tables"], step.batch.block_tables.numpy())
