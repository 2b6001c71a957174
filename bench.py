#!/usr/bin/env python3
"""Benchmark of the MI355X continuous-batching hot path (one GPU).

Default workload (``--workload e2e``): LLM.generate over 256 requests on a
random-init Qwen3-0.6B-shaped model in bf16 (prompts U[100,1024], half of
them behind a shared 512-token prefix with prefix caching on, 1024 greedy
output tokens each, ignore EOS); value = output tokens/s, one "step" = one
generate() over the whole workload.  Its roofline is the decode-attention
kernel measured live inside that run; the config-2 microbench of the same
kernel is reported beside it.  Kernel workloads: ``decode`` (paged decode
attention at the Qwen3-0.6B attention shape, 256 sequences, context
U[128, 2048], one lv_paged_attention call per step), ``mixed``
(chunked-prefill step: pack + scatter + attention), ``sampler`` (fused
sampler on [256, 151936] bf16 logits), ``copy`` (counter calibration).

Prints ONE JSON line with the throughput, the roofline of the dominant
kernel (algorithmic bytes / average duration measured with HIP events on
the launch stream) and a CPU baseline: the oracle's restatement of the
reference algorithm timed on a bounded sample on this host's cores.
"""

from __future__ import annotations

import argparse
import json
import os
import statistics
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
for p in (str(ROOT), str(ROOT / "lite-vllm_amd")):
    if p not in sys.path:
        sys.path.insert(0, p)

METRIC = "output tok/s (Qwen3-0.6B shape, 256 seqs, 1 GPU); paged-decode attn HBM GB/s"
HBM_PEAK_GBPS = 8000.0
MFMA_BF16_PEAK_TFLOPS = 2500.0   # dense bf16 MFMA, MI355X


def _log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def _cpu_threads() -> int:
    try:
        return len(os.sched_getaffinity(0))
    except AttributeError:
        return os.cpu_count() or 1


def _cpu_model() -> str:
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


TRAFFIC_SOURCE = ("profiles/traffic.json: HBM bytes per call from separate rocprofv3 --pmc "
                  "FETCH_SIZE / WRITE_SIZE runs of this workload, scaled by the plain-copy "
                  "calibration (not measured in this run)")


def _time_gpu(fn, steps: int, warmup: int):
    """Run fn warmup+steps times; return (total ms over the timed steps,
    per-step event durations in ms)."""
    import torch
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
           for _ in range(steps)]
    t_start = torch.cuda.Event(enable_timing=True)
    t_end = torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    t_start.record()
    for a, b in evs:
        a.record()
        fn()
        b.record()
    t_end.record()
    torch.cuda.synchronize()
    return t_start.elapsed_time(t_end), [a.elapsed_time(b) for a, b in evs]


def _time_back_to_back(fn, calls: int = 20, reps: int = 5, warmup: int = 3) -> float:
    """Average time per call (ms) of `calls` back-to-back launches of fn
    between one pair of HIP events on the launch stream (median of reps):
    the kernels' own duration, without the cost of an event pair around
    every call (2-6 us on this part, a large share of a 10-25 us kernel)."""
    import torch
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    ts = []
    for _ in range(reps):
        a = torch.cuda.Event(enable_timing=True)
        b = torch.cuda.Event(enable_timing=True)
        a.record()
        for _ in range(calls):
            fn()
        b.record()
        torch.cuda.synchronize()
        ts.append(a.elapsed_time(b) / calls)
    return statistics.median(ts)


B2B_NOTE = ("avg_launch_us: 20 back-to-back calls between one pair of HIP events on the launch "
            "stream (median of 5); per_call_event_us: one event pair around every call")


def _median_cpu(fn, reps: int = 5) -> float:
    fn()  # warmup
    ts = []
    for _ in range(reps):
        t0 = time.perf_counter()
        fn()
        ts.append(time.perf_counter() - t0)
    return statistics.median(ts)


def _traffic(workload: str):
    """Measured HBM bytes per call for `workload` from profiles/traffic.json
    (rocprofv3 FETCH_SIZE / WRITE_SIZE scaled by the copy calibration), or
    None when no measurement is recorded."""
    f = ROOT / "profiles" / "traffic.json"
    if not f.exists():
        return None
    d = json.loads(f.read_text())
    w = d.get(workload)
    if not w or w.get("fetch_kib") is None or w.get("write_kib") is None:
        return None
    return int(w["fetch_kib"] * 1024 * d["fetch_scale"] + w["write_kib"] * 1024 * d["write_scale"])


def decode_bytes(batch) -> int:
    """Algorithmic HBM bytes of one decode-attention pass: each live K/V row
    once, q and out once, the used block-table entries and context lengths."""
    import torch
    ctx = batch.context_lens.to(torch.int64)
    B, H, D = batch.query.shape
    es = batch.query.element_size()
    kv = batch.kv_bytes_read()
    qo = 2 * B * H * D * es
    tables = int(((ctx + batch.key_cache.shape[1] - 1) // batch.key_cache.shape[1]).sum()) * 4
    return kv + qo + tables + B * 4


def bench_decode(args):
    import torch
    from litevllm import ops, workloads
    dev = torch.device("cuda:0")
    cpu_batch = workloads.paged_decode(seed=0)
    b = cpu_batch.to(dev)
    out = torch.empty_like(b.query)

    def step():
        ops.paged_attention(b.query, b.key_cache, b.value_cache, b.block_tables, b.context_lens,
                            scale=b.scale, num_decodes=b.num_decodes, out=out)

    total_ms, per = _time_gpu(step, args.steps, args.warmup)
    nbytes = decode_bytes(cpu_batch)
    kern_ms = _time_back_to_back(step)
    achieved = nbytes / (kern_ms * 1e-3) / 1e9
    result = {
        "value": round(achieved, 1),
        "unit": "GB/s",
        "ms_per_step": round(total_ms / args.steps, 4),
        "config": {
            "workload": "config2 paged decode attention: 256 seqs, ctx U[128,2048] (seed 0), "
                        "16 q / 8 kv heads, head_dim 128, block_size 16, bf16 in / fp32 accumulate",
            "num_seqs": 256, "sum_ctx": int(cpu_batch.context_lens.sum()),
            "kernel": "lv_paged_attention (attn_decode_persistent_kernel + "
                      "attn_persist_reduce_kernel)",
        },
        "roofline": {
            "bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBPS,
            "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBPS, 4),
            "traffic": _traffic("decode"), "traffic_source": TRAFFIC_SOURCE,
            "algorithmic_bytes": nbytes, "avg_launch_us": round(kern_ms * 1e3, 2),
            "per_call_event_us": round(statistics.mean(per) * 1e3, 2), "timing": B2B_NOTE,
        },
    }
    if not args.no_cpu_baseline:
        result["cpu_baseline"] = cpu_baseline_decode(cpu_batch)
    return result


def cpu_baseline_decode(cpu_batch, n_seqs: int = 64):
    """The reference's _decode_fast restated (oracle.attention), fp32, on the
    first n_seqs sequences of the same batch; reported in the same unit."""
    import torch
    from oracle.attention import decode_attention
    threads = _cpu_threads()
    torch.set_num_threads(threads)
    ctx = cpu_batch.context_lens[:n_seqs]
    bs = cpu_batch.key_cache.shape[1]
    mb = int(((ctx + bs - 1) // bs).max())
    tables = cpu_batch.block_tables[:n_seqs, :mb].contiguous()
    q = cpu_batch.query[:n_seqs].float()
    kc = cpu_batch.key_cache.float()
    vc = cpu_batch.value_cache.float()
    secs = _median_cpu(lambda: decode_attention(q, kc, vc, tables, ctx, cpu_batch.scale))
    sub = type(cpu_batch)(cpu_batch.query[:n_seqs], cpu_batch.key_cache, cpu_batch.value_cache,
                          tables, ctx, cpu_batch.cu_seqlens[:n_seqs + 1], n_seqs, 1,
                          cpu_batch.scale)
    return {
        "value": round(decode_bytes(sub) / secs / 1e9, 3), "unit": "GB/s (algorithmic, bf16 bytes)",
        "cores": threads, "cpu_model": _cpu_model(), "kind": "port",
        "sample": f"config2 sequences 0..{n_seqs - 1} (sum ctx {int(ctx.sum())}), fp32 "
                  f"_decode_fast restatement (oracle.attention.decode_attention), median of 5 "
                  f"after 1 warmup: {secs * 1e3:.1f} ms",
    }


def bench_sampler(args):
    import torch
    from litevllm import ops, workloads
    dev = torch.device("cuda:0")
    sb = workloads.sampler_batch(seed=0)
    logits = sb.logits.to(dev)
    temp = sb.temperature.to(dev)
    if args.sampler_rows == "greedy":
        temp = torch.zeros_like(temp)
    elif args.sampler_rows == "temperature":
        temp = torch.full_like(temp, 0.75)
    uni = sb.uniform.to(dev)
    out = torch.empty(logits.shape[0], dtype=torch.int64, device=dev)
    call = lambda: ops.sample(logits, temp, uni, out=out)
    total_ms, per = _time_gpu(call, args.steps, args.warmup)
    B, V = logits.shape
    nbytes = B * V * logits.element_size() + B * (4 + 4 + 8)
    kern_ms = _time_back_to_back(call)
    achieved = nbytes / (kern_ms * 1e-3) / 1e9
    res = {
        "value": round(B / (kern_ms * 1e-3), 1), "unit": "sampled rows/s",
        "ms_per_step": round(total_ms / args.steps, 4),
        "config": {"workload": ("config4 fused sampler: [256, 151936] bf16 logits N(0,16), "
                                "rows 0-127 greedy, 128-255 T~U[0.5,1], supplied uniforms"
                                if args.sampler_rows == "config4" else
                                f"config4 logits, all rows {args.sampler_rows} (diagnostic)"),
                   "kernel": "lv_sample (sampler_items_kernel + sampler_finish_kernel; "
                             "the roofline figures are over the whole call)"},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBPS,
                     "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBPS, 4),
                     "traffic": _traffic("sampler"), "traffic_source": TRAFFIC_SOURCE,
                     "algorithmic_bytes": nbytes, "avg_launch_us": round(kern_ms * 1e3, 2),
                     "per_call_event_us": round(statistics.mean(per) * 1e3, 2),
                     "timing": B2B_NOTE},
    }
    if not args.no_cpu_baseline:
        from oracle import sampler as osamp
        threads = _cpu_threads()
        x = sb.logits[:32].float().numpy()
        t = sb.temperature[96:128 + 32].numpy()
        secs = _median_cpu(lambda: (osamp.greedy(x[:16]),
                                    osamp.sample(sb.logits[128:144].float().numpy(),
                                                 sb.temperature[128:144].numpy(),
                                                 sb.uniform[128:144].numpy())))
        res["cpu_baseline"] = {"value": round(32 / secs, 2), "unit": "sampled rows/s",
                               "cores": 1, "cpu_model": _cpu_model(), "kind": "port",
                               "sample": "16 greedy + 16 temperature rows of config4 through "
                                         "oracle.sampler (numpy argmax, C inverse-CDF), median of 5"}
        del x, t
    return res


def bench_mixed(args):
    import torch
    from litevllm import ops, workloads
    dev = torch.device("cuda:0")
    step_cpu = workloads.mixed_step(seed=0)
    b = step_cpu.batch.to(dev)
    key, value = step_cpu.key.to(dev), step_cpu.value.to(dev)
    descs = step_cpu.descs.to(dev)
    block_ids = step_cpu.block_ids.to(dev)
    token_ids = step_cpu.token_ids.to(dev)
    T = step_cpu.token_ids.shape[0]
    mb = b.block_tables.shape[1]
    out = torch.empty_like(b.query)

    def step():
        packed = ops.pack_inputs(descs, block_ids, token_ids, T, 16, mb)
        ops.kv_scatter(key, value, b.key_cache, b.value_cache, packed["slot_mapping"])
        ops.paged_attention(b.query, b.key_cache, b.value_cache, packed["block_tables"],
                            packed["context_lens"], scale=b.scale,
                            cu_seqlens=packed["cu_seqlens"], num_decodes=b.num_decodes,
                            max_query_len=b.max_query_len, out=out)

    total_ms, per = _time_gpu(step, args.steps, args.warmup)
    kern_ms = statistics.mean(per)
    result = {
        "value": round(T / (kern_ms * 1e-3), 1), "unit": "packed tokens/s",
        "ms_per_step": round(total_ms / args.steps, 4),
        "config": {"workload": "config3 mixed step: 192 decodes ctx U[256,4096] + 15 chunks x 512 "
                               "at offset U[0,3072], 200k-slot cache, bf16",
                   "num_tokens": T},
    }
    if args.no_secondary:      # (keeps a kernel trace of this run to the step itself)
        return result

    # The chunk rows alone (decode rows come first in the batch), same cache,
    # tables and lengths: the MFMA kernel's rate, HIP events on the launch
    # stream around each call.  FLOPs = 4·H·D·Σ(L·o + L(L+1)/2) over the
    # chunk sequences (L query tokens at offset o).
    nd = b.num_decodes
    H, D = b.query.shape[1], b.query.shape[2]
    cu_cpu = step_cpu.batch.cu_seqlens.tolist()
    ctx_cpu = step_cpu.batch.context_lens.tolist()
    flops = 0
    for i in range(nd, len(ctx_cpu)):
        L = cu_cpu[i + 1] - cu_cpu[i]
        o = ctx_cpu[i] - L
        flops += 4 * H * D * (L * o + L * (L + 1) // 2)
    packed = ops.pack_inputs(descs, block_ids, token_ids, T, 16, mb)
    q_c = b.query[nd:]
    bt_c = packed["block_tables"][nd:]
    ctx_c = packed["context_lens"][nd:]
    cu_c = (packed["cu_seqlens"][nd:] - nd).contiguous()
    out_c = torch.empty_like(q_c)

    def chunk_call():
        ops.paged_attention(q_c, b.key_cache, b.value_cache, bt_c, ctx_c, scale=b.scale,
                            cu_seqlens=cu_c, num_decodes=0, max_query_len=b.max_query_len,
                            out=out_c)

    _, per_c = _time_gpu(chunk_call, args.steps, args.warmup)
    chunk_ms = statistics.mean(per_c)
    tflops = flops / (chunk_ms * 1e-3) / 1e12
    result["chunk_roofline"] = {
        "bound": "mfma", "achieved": round(tflops, 1), "peak": MFMA_BF16_PEAK_TFLOPS,
        "unit": "TFLOP/s", "frac": round(tflops / MFMA_BF16_PEAK_TFLOPS, 4),
        "algorithmic_flops": flops, "avg_launch_us": round(chunk_ms * 1e3, 2),
        "kernel": "attn_chunk_mfma_kernel (lv_paged_attention on the chunk rows alone)",
        "note": "repeated chunk-only calls keep the chunks' K/V (~140 MB) in the MALL, so "
                "they read faster than the chunk kernel inside the step (rocprof trace of "
                "this workload with --no-secondary)",
    }
    return result


def mixed_kernel_rooflines(steps: int = 20, warmup: int = 5):
    """Config 3 split into its kernels, each bracketed by HIP events on the
    launch stream, in step order: packing, KV scatter, the prefill-chunk
    rows (lv_paged_attention on the chunk sequences alone: the MFMA chunk
    kernel) and the decode rows (lv_paged_attention on the decode sequences
    alone: the persistent decode kernel + its reduce).  Returns the three
    roofline entries of the bench line's `secondary` list."""
    import torch
    from litevllm import ops, workloads
    dev = torch.device("cuda:0")
    step_cpu = workloads.mixed_step(seed=0)
    b = step_cpu.batch.to(dev)
    key, value = step_cpu.key.to(dev), step_cpu.value.to(dev)
    descs, block_ids = step_cpu.descs.to(dev), step_cpu.block_ids.to(dev)
    token_ids = step_cpu.token_ids.to(dev)
    T = step_cpu.token_ids.shape[0]
    mb = b.block_tables.shape[1]
    nd = b.num_decodes
    H, D = b.query.shape[1], b.query.shape[2]
    hkv = b.key_cache.shape[2]
    packed = ops.pack_inputs(descs, block_ids, token_ids, T, 16, mb)
    q_c, q_d = b.query[nd:], b.query[:nd]
    out_c, out_d = torch.empty_like(q_c), torch.empty_like(q_d)
    cu_c = (packed["cu_seqlens"][nd:] - nd).contiguous()
    segs = ("pack", "scatter", "chunks", "decodes")
    evs = {k: [] for k in segs}

    def run(record):
        marks = [torch.cuda.Event(enable_timing=True) for _ in range(5)] if record else None
        if record:
            marks[0].record()
        p = ops.pack_inputs(descs, block_ids, token_ids, T, 16, mb, out=packed)
        if record:
            marks[1].record()
        ops.kv_scatter(key, value, b.key_cache, b.value_cache, p["slot_mapping"])
        if record:
            marks[2].record()
        ops.paged_attention(q_c, b.key_cache, b.value_cache, p["block_tables"][nd:],
                            p["context_lens"][nd:], scale=b.scale, cu_seqlens=cu_c,
                            num_decodes=0, max_query_len=b.max_query_len, out=out_c)
        if record:
            marks[3].record()
        ops.paged_attention(q_d, b.key_cache, b.value_cache, p["block_tables"][:nd],
                            p["context_lens"][:nd], scale=b.scale, out=out_d)
        if record:
            marks[4].record()
            for i, k in enumerate(segs):
                evs[k].append((marks[i], marks[i + 1]))

    for _ in range(warmup):
        run(False)
    torch.cuda.synchronize()
    for _ in range(steps):
        run(True)
    torch.cuda.synchronize()
    us = {k: statistics.mean(a.elapsed_time(c) for a, c in v) * 1e3 for k, v in evs.items()}
    # the scatter (~10 us) timed back to back as well: the event pair around
    # each in-step call costs a large share of it
    scatter_b2b = _time_back_to_back(
        lambda: ops.kv_scatter(key, value, b.key_cache, b.value_cache, packed["slot_mapping"])) * 1e3
    cu_cpu = step_cpu.batch.cu_seqlens.tolist()
    ctx_cpu = step_cpu.batch.context_lens.tolist()
    flops = 0
    for i in range(nd, len(ctx_cpu)):
        L = cu_cpu[i + 1] - cu_cpu[i]
        flops += 4 * H * D * (L * (ctx_cpu[i] - L) + L * (L + 1) // 2)
    scatter_bytes = T * hkv * D * 2 * 2 * b.key_cache.element_size() + T * 8
    sub = workloads.PagedBatch(step_cpu.batch.query[:nd], step_cpu.batch.key_cache,
                               step_cpu.batch.value_cache, step_cpu.batch.block_tables[:nd],
                               step_cpu.batch.context_lens[:nd],
                               step_cpu.batch.cu_seqlens[:nd + 1], nd, 1, step_cpu.batch.scale)
    dec_bytes = decode_bytes(sub)
    wl = ("config3 mixed step (192 decodes ctx U[256,4096] + 15 chunks x 512 at offset "
          "U[0,3072], 200k-slot cache, bf16), kernels timed one by one in step order, "
          f"{steps} steps after {warmup} warmup")

    def hbm(nbytes, t_us, in_step_us, timing, traffic_key):
        a = nbytes / (t_us * 1e-6) / 1e9
        return {"bound": "hbm", "achieved": round(a, 1), "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                "frac": round(a / HBM_PEAK_GBPS, 4), "traffic": _traffic(traffic_key),
                "traffic_source": TRAFFIC_SOURCE,
                "algorithmic_bytes": int(nbytes), "avg_launch_us": round(t_us, 2),
                "in_step_event_us": round(in_step_us, 2), "timing": timing}
    in_step = ("avg_launch_us: one pair of HIP events around each call in the step "
               f"({steps} steps)")
    tf = flops / (us["chunks"] * 1e-6) / 1e12
    return [
        {"metric": "KV scatter HBM GB/s (config 3)", "kernel": "lv_kv_scatter (kv_scatter_kernel)",
         "value": round(scatter_bytes / (scatter_b2b * 1e-6) / 1e9, 1), "unit": "GB/s",
         "roofline": hbm(scatter_bytes, scatter_b2b, us["scatter"],
                         "avg_launch_us: 20 back-to-back calls between one pair of HIP events "
                         "(median of 5); in_step_event_us: an event pair around the call in "
                         "the step", "scatter_config3"),
         "config": wl, "pack_in_step_event_us": round(us["pack"], 2)},
        {"metric": "prefill-chunk attention MFMA TFLOP/s (config 3)",
         "kernel": "lv_paged_attention chunk rows (attn_chunk_mfma_kernel)",
         "value": round(tf, 1), "unit": "TFLOP/s",
         "roofline": {"bound": "mfma", "achieved": round(tf, 1), "peak": MFMA_BF16_PEAK_TFLOPS,
                      "unit": "TFLOP/s", "frac": round(tf / MFMA_BF16_PEAK_TFLOPS, 4),
                      "traffic": _traffic("chunk_config3"), "traffic_source": TRAFFIC_SOURCE,
                      "algorithmic_flops": flops,
                      "avg_launch_us": round(us["chunks"], 2), "timing": in_step},
         "config": wl},
        {"metric": "paged-decode attn HBM GB/s (config 3 decode rows)",
         "kernel": "lv_paged_attention decode rows (attn_decode_persistent_kernel + "
                   "attn_persist_reduce_kernel)",
         "value": round(dec_bytes / (us["decodes"] * 1e-6) / 1e9, 1), "unit": "GB/s",
         "roofline": hbm(dec_bytes, us["decodes"], us["decodes"], in_step,
                         "decode_rows_config3"), "config": wl},
    ]


def bench_e2e(args):
    """Config 5: LLM.generate over 256 Qwen3-0.6B-shaped requests (random
    init, bf16), prefix caching on, 8192-token step budget, chunk 512.  One
    step = one generate() of the whole workload; value = output tokens / wall
    time.  The decode-attention launches of decode-only steps are bracketed
    by HIP events on the launch stream for the roofline."""
    import torch
    from litevllm import LLM, SamplingParams, _hip, workloads
    from litevllm.engine import model_runner as mr

    mc = workloads.QWEN3_06B_SHAPE
    prompts, sharers = workloads.e2e_prompts(seed=0)
    warm_prompts, _ = workloads.e2e_prompts(seed=1)
    hkv, D, H = mc["num_key_value_heads"], mc["head_dim"], mc["num_attention_heads"]

    # -- instrumentation of decode attention in decode-only steps: HIP events
    # on the launch stream right around the C-ABI call (lv_paged_attention /
    # lv_paged_attention_prefix, which enqueues the call's kernels) of an
    # eager step, so the interval is the kernels' GPU time, not the Python
    # wrapper's.  A captured graph cannot hold timing events on ROCm, so with
    # graphs on, one decode step in SAMPLE_EVERY runs eagerly (same kernels,
    # same data) and is the timing sample; the others replay graphs.
    SAMPLE_EVERY = 32
    probe = {"on": False, "meta": None, "durs": [], "bytes": 0, "decode_steps": 0,
             "saved": [], "shared": {}, "arena": None, "arena_at": 0}
    import ctypes
    _hiprt = ctypes.CDLL("libamdhip64.so")
    _hiprt.hipMemcpyAsync.restype = ctypes.c_int
    _hiprt.hipMemcpyAsync.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t,
                                      ctypes.c_int, ctypes.c_void_p]

    def hip_memcpy_d2d(dst, src, n):
        # stream-ordered after the call that read these inputs (kind 3:
        # device to device); no host synchronisation
        if _hiprt.hipMemcpyAsync(dst, src, n, 3, torch.cuda.current_stream().cuda_stream) != 0:
            raise RuntimeError("hipMemcpyAsync failed")
    orig_exec = mr.ModelRunner.execute_model
    orig_accepts = mr.DecodeGraphs.accepts
    lib = _hip.load()
    orig_c = {n: getattr(lib, n) for n in ("lv_paged_attention", "lv_paged_attention_prefix")}

    def step_bytes(meta):
        """K/V rows each read once per row -- a block that the step's
        shared-prefix pass reads once for a group counts once -- plus q,
        out, table entries, context lengths, and the prefix pass's fp32
        partials (written, then read by the merge)."""
        B = meta.num_decodes
        kv_tokens = meta.num_context_tokens - meta.prefix_saved_blocks * 16
        return (kv_tokens * hkv * D * 2 * 2 + 2 * B * H * D * 2
                + meta.num_context_blocks * 4 + B * 4
                + meta.prefix_partial_rows * H * (D + 2) * 4 * 2)

    def exec_probe(self, meta):
        probe["meta"] = meta
        return orig_exec(self, meta)

    # Graph-replay timing of the same calls: the serving loop runs decode
    # steps as HIP-graph replays, where the call's kernels follow each other
    # without the eager launch gaps.  Each sampled call's inputs (query, block
    # tables, context lengths, shared-prefix plan; the layer's KV cache stays
    # in place) are copied aside; after the timed region each call is
    # captured as a one-call graph on its saved inputs and replayed, and the
    # second replay is timed with HIP events.
    # Copies go to one arena allocated before the timed region (no
    # allocation inside it); a sample that does not fit is not saved.
    def dev_copy(ptr, nbytes):
        n = (max(int(nbytes), 1) + 255) // 256 * 256
        at = probe["arena_at"]
        if at + n > probe["arena"].numel():
            return None
        t = probe["arena"][at:at + n]
        probe["arena_at"] = at + n
        if ptr and nbytes:
            hip_memcpy_d2d(t.data_ptr(), ptr, int(nbytes))
        return t

    def save_call(name, args, nbytes):
        a = list(args)
        B, mb, T = a[9], a[6], a[11]
        step_key = probe["decode_steps"]
        shared = probe["shared"].get(step_key)
        if shared is None:      # tables, lengths and plan: the same for every layer of a step
            shared = {"bt": dev_copy(a[5], B * mb * 4), "ctx": dev_copy(a[8], B * 4)}
            if name == "lv_paged_attention_prefix":
                shared["pb"] = dev_copy(a[22], a[10] * 4)
                shared["pi"] = dev_copy(a[23], a[24] * 16)
                shared["pm"] = dev_copy(a[25], a[26] * 4)
            probe["shared"] = {step_key: shared}
        q = dev_copy(a[0], T * a[1] * (4 if a[-2] == _hip.LV_F32 else 2))
        if q is None or any(v is None for v in shared.values()):
            return
        probe["saved"].append((name, a, shared, q, nbytes))

    REPLAY_COPIES = 8

    def replay_saved():
        times, nbytes = [], 0
        for name, a, sh, q, nb in probe["saved"]:
            a = list(a)
            out = torch.empty(max(a[11] * a[19] * (4 if a[-2] == _hip.LV_F32 else 2), 1),
                              dtype=torch.uint8, device="cuda")
            ws = torch.zeros(max(a[21], 1), dtype=torch.uint8, device="cuda")
            a[0], a[5], a[8], a[18], a[20] = q.data_ptr(), sh["bt"].data_ptr(), \
                sh["ctx"].data_ptr(), out.data_ptr(), ws.data_ptr()
            if name == "lv_paged_attention_prefix":
                pws = torch.zeros(max(a[28], 1), dtype=torch.uint8, device="cuda")
                a[22], a[23], a[25], a[27] = sh["pb"].data_ptr(), sh["pi"].data_ptr(), \
                    sh["pm"].data_ptr(), pws.data_ptr()
            fn = orig_c[name]
            g = torch.cuda.CUDAGraph()
            with torch.inference_mode(), torch.cuda.graph(g):
                a[-1] = torch.cuda.current_stream().cuda_stream
                for _ in range(REPLAY_COPIES):
                    _hip.check(fn(*a), name)
            g.replay()
            e0 = torch.cuda.Event(enable_timing=True)
            e1 = torch.cuda.Event(enable_timing=True)
            e0.record()
            g.replay()
            e1.record()
            torch.cuda.synchronize()
            times.append(e0.elapsed_time(e1) / REPLAY_COPIES)
            nbytes += nb
            del g
        return times, nbytes

    def c_probe(name):
        fn = orig_c[name]

        def call(*args):
            meta = probe["meta"]
            if not probe["on"] or meta is None or meta.num_decodes != len(meta.seq_ids):
                return fn(*args)
            e0 = torch.cuda.Event(enable_timing=True)
            e1 = torch.cuda.Event(enable_timing=True)
            e0.record()
            rc = fn(*args)
            e1.record()
            probe["durs"].append((e0, e1))
            nb = step_bytes(meta)
            probe["bytes"] += nb
            if len(probe["saved"]) < 32 * mc["num_hidden_layers"]:
                save_call(name, args, nb)
            return rc
        return call

    def accepts_probe(self, st):
        ok = orig_accepts(self, st)
        if ok and probe["on"]:
            probe["decode_steps"] += 1
            if probe["decode_steps"] % SAMPLE_EVERY == 0:
                return False            # this step runs eagerly: timing sample
        return ok

    mr.ModelRunner.execute_model = exec_probe
    for n in orig_c:
        setattr(lib, n, c_probe(n))
    mr.DecodeGraphs.accepts = accepts_probe
    llm = LLM("qwen3-0.6b-shape", dtype="bfloat16", load_format="dummy", hf_overrides=mc,
              skip_tokenizer_init=True, enable_prefix_caching=True, max_num_batched_tokens=8192,
              chunk_size=512, block_size=16, max_num_seqs=256, seed=0,
              enforce_eager=args.eager)
    eng = llm.engine
    sp = SamplingParams(temperature=0.0, max_tokens=args.output_len, ignore_eos=True)

    def reset_prefix_cache():
        pc = eng.prefix_cache
        pc.evict_unused(len(pc.cache))

    warm_sp = SamplingParams(temperature=0.0, max_tokens=8, ignore_eos=True)
    _log("e2e: model and KV cache ready")
    for _ in range(args.warmup):
        llm.generate(prompt_token_ids=warm_prompts, sampling_params=warm_sp)
        reset_prefix_cache()
        _log("e2e: warmup generate done")
    # 32 sampled steps x (28 queries of up to 256 x 16 x 128 bf16 + tables
    # of the graphs' 2560-block width): ~1 GiB, allocated before timing
    probe["arena"] = torch.empty(1 << 30, dtype=torch.uint8, device="cuda")
    torch.cuda.synchronize()
    probe["on"] = True
    hits0 = eng.prefix_cache.hit_tokens
    t0 = time.perf_counter()
    n_out = 0
    outs = []
    for i in range(args.steps):
        outs = llm.generate(prompt_token_ids=prompts, sampling_params=sp)
        n_out += sum(o.num_output_tokens for o in outs)
        _log(f"e2e: timed generate {i + 1}/{args.steps} done")
        if i + 1 < args.steps:
            reset_prefix_cache()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    probe["on"] = False
    mr.ModelRunner.execute_model = orig_exec
    for n, fn in orig_c.items():
        setattr(lib, n, fn)
    mr.DecodeGraphs.accepts = orig_accepts
    durs = [a.elapsed_time(b) for a, b in probe["durs"]]
    if args.no_graph_timing:          # (keeps a kernel trace of this run to the serving run)
        gdurs, gbytes = [], 0
    else:
        _log(f"e2e: graph replays of the {len(probe['saved'])} sampled attention calls")
        gdurs, gbytes = replay_saved()
    probe["saved"].clear()
    probe["shared"].clear()
    probe["arena"] = None
    cpu_state = cpu_cfg = None
    by_prompt = {tuple(o.prompt_token_ids): list(o.output_token_ids) for o in outs}
    streams = [by_prompt[tuple(p)] for p in prompts[:8]]
    if not args.no_cpu_baseline:
        cpu_state = {k: v.detach().to("cpu", torch.float32)
                     for k, v in eng.model_runner.model.state_dict().items()}
        cpu_cfg = eng.config.model_config
    attn_ms = sum(durs)
    achieved_eager = probe["bytes"] / (attn_ms * 1e-3) / 1e9 if durs else 0.0
    gattn_ms = sum(gdurs)
    if not gdurs:                      # --no-graph-timing: the eager figure only
        gdurs, gattn_ms, gbytes = [0.0] * len(durs), attn_ms, probe["bytes"]
    achieved = gbytes / (gattn_ms * 1e-3) / 1e9 if gattn_ms else 0.0
    result = {
        "value": round(n_out / wall, 1), "unit": "output tok/s",
        "ms_per_step": round(wall * 1e3 / args.steps, 2),
        "config": {
            "workload": "config5 e2e: LLM.generate, Qwen3-0.6B shape (28 layers, hidden 1024, "
                        "MLP 3072, 16q/8kv, D128, qk-norm, theta 1e6, vocab 151936, untied), "
                        "random init seed 0, bf16; 256 prompts U[100,1024] (128 share a 512-token "
                        "prefix, length max(drawn,528)), prefix caching on, "
                        f"{args.output_len} output tokens ignore_eos, greedy, "
                        "max_num_batched_tokens 8192, chunk 512, block 16",
            "num_seqs": len(prompts), "prompt_tokens": sum(map(len, prompts)),
            "output_tokens": n_out, "prefix_hit_tokens": eng.prefix_cache.hit_tokens - hits0,
            "num_gpu_blocks": eng.config.cache_config.num_gpu_blocks,
            "kernel": "lv_paged_attention_prefix decode (shared-prefix pass "
                      "attn_chunk_mfma_kernel<PFX> + attn_decode_persistent_kernel + "
                      "attn_persist_reduce_kernel), decode-only steps",
            "decode_graphs": not args.eager,
            "roofline_sample": ("every decode-only step" if args.eager else
                                f"every {SAMPLE_EVERY}th decode-only step runs eagerly with HIP "
                                "events around each attention launch; the others replay graphs"),
        },
        "roofline": {
            "bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBPS,
            "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBPS, 4),
            "traffic": _traffic("e2e_decode"), "traffic_source": TRAFFIC_SOURCE,
            "algorithmic_bytes": int(gbytes / max(len(gdurs), 1)),
            "avg_launch_us": round(gattn_ms * 1e3 / max(len(gdurs), 1), 2),
            "launches": len(gdurs),
            "timing": "HIP events around each eager call (--no-graph-timing)"
            if args.no_graph_timing else
                      ("graph replay (as the serving loop runs decode steps) of every "
                       "attention call of the sampled steps, on copies of that call's inputs "
                       "(query, block tables, context lengths, shared-prefix plan; KV cache in "
                       "place): after the timed region each call is captured 8 times back to "
                       "back in one HIP graph, HIP events around the second replay, time / 8 "
                       "(a single bracketed call adds ~10 us of launch and event overhead that "
                       "a call inside the decode-step graph does not pay)"),
            "eager": {
                "achieved": round(achieved_eager, 1),
                "frac": round(achieved_eager / HBM_PEAK_GBPS, 4),
                "avg_launch_us": round(attn_ms * 1e3 / max(len(durs), 1), 2),
                "launches": len(durs),
                "timing": "HIP events around each call in the eagerly run sample steps "
                          "(includes the eager launch gaps between the call's kernels)"},
            "attention_share_of_wall_est": round(
                attn_ms / max(len(durs), 1) * 1e-3 * mc["num_hidden_layers"]
                * probe["decode_steps"] / wall, 4) if not args.eager else round(attn_ms * 1e-3 / wall, 4),
        },
    }
    del llm, eng
    torch.cuda.empty_cache()
    if args.no_secondary:
        if not args.no_cpu_baseline:
            result["cpu_baseline"], result["parity"] = cpu_baseline_e2e(
                cpu_state, cpu_cfg, prompts, streams)
        return result
    # Every hot-path kernel's roofline beside the headline, in this run:
    # config 2 decode attention, config 3 split into its kernels, config 4
    # sampler (all HIP events on the launch stream).
    _log("e2e: config-2 decode-attention microbench")
    dec = bench_decode(argparse.Namespace(steps=50, warmup=10, no_cpu_baseline=True))
    secondary = [{
        "metric": "paged-decode attn HBM GB/s (config 2, 50 launches after 10 warmup)",
        "kernel": dec["config"]["kernel"],
        "value": dec["value"], "unit": dec["unit"], "roofline": dec["roofline"],
        "config": dec["config"]["workload"]}]
    _log("e2e: config-3 kernels")
    secondary += mixed_kernel_rooflines()
    _log("e2e: config-4 sampler")
    smp = bench_sampler(argparse.Namespace(steps=50, warmup=10, no_cpu_baseline=True,
                                           sampler_rows="config4"))
    secondary.append({
        "metric": "fused sampler HBM GB/s (config 4, 50 calls after 10 warmup)",
        "kernel": smp["config"]["kernel"], "value": smp["roofline"]["achieved"], "unit": "GB/s",
        "roofline": smp["roofline"], "config": smp["config"]["workload"]})
    result["secondary"] = secondary
    if not args.no_cpu_baseline:
        result["cpu_baseline"], result["parity"] = cpu_baseline_e2e(
            cpu_state, cpu_cfg, prompts, streams)
    return result


def cpu_baseline_e2e(state, model_config, prompts, streams, n_seqs: int = 8, n_steps: int = 64,
                     margin_bar: float = 0.1):
    """The reference's CPU model path restated (oracle.model, fp32, the same
    random weights): prefill the first n_seqs prompts of the workload
    (untimed), then time n_steps batched greedy decode steps.

    The decode steps are fed the engine's own tokens for those prompts
    (``streams``, from the timed run), so the same pass also checks them:
    each of the first n_steps + 1 engine tokens must be the oracle's argmax
    where the oracle's top-2 margin is at least margin_bar, and within
    margin_bar of the oracle's maximum everywhere (the bf16 bar of the
    config-5 GPU test).  Returns (cpu_baseline, parity)."""
    import torch
    from oracle.model import OracleDecoder
    threads = _cpu_threads()
    torch.set_num_threads(threads)
    o = OracleDecoder(state, model_config, use_qk_norm=True)
    n_steps = max(0, min(n_steps, min(len(s) for s in streams[:n_seqs]) - 1))
    checked = exact = 0
    max_gap = 0.0

    def check(logits, t):
        nonlocal checked, exact, max_gap
        top2 = torch.topk(logits, 2, dim=-1).values
        for r in range(logits.shape[0]):
            tok = streams[r][t]
            gap = float(top2[r, 0] - logits[r, tok])
            max_gap = max(max_gap, gap)
            if float(top2[r, 0] - top2[r, 1]) >= margin_bar:
                exact += int(tok == int(torch.argmax(logits[r])))
                checked += 1

    kvs, first, pos = [], [], []
    for p in prompts[:n_seqs]:
        kv: list = []
        first.append(o.forward(p, 0, kv))
        kvs.append(kv)
        pos.append(len(p))
    check(torch.stack(first), 0)
    _log("e2e cpu baseline: prefill done")
    secs = 0.0
    for t in range(n_steps):
        t0 = time.perf_counter()
        logits = o.decode_batch([s[t] for s in streams[:n_seqs]], pos, kvs)
        secs += time.perf_counter() - t0
        check(logits, t + 1)
        pos = [x + 1 for x in pos]
    base = {"value": round(n_seqs * n_steps / max(secs, 1e-9), 2), "unit": "output tok/s",
            "cores": threads, "cpu_model": _cpu_model(), "kind": "port",
            "sample": f"config5 prompts 0..{n_seqs - 1} ({sum(map(len, prompts[:n_seqs]))} prompt "
                      f"tokens, prefill untimed), {n_steps} batched greedy decode steps of "
                      f"oracle.model.OracleDecoder (fp32 restatement of the reference model "
                      f"path): {secs:.2f} s"}
    parity = {"rows": n_seqs, "tokens_per_row": n_steps + 1,
              "clear_margin_tokens": checked, "argmax_match": exact,
              "max_gap_below_oracle_max": round(max_gap, 4), "bar": margin_bar,
              "ok": exact == checked and max_gap <= margin_bar,
              "check": f"engine tokens of the timed run (prompts 0-{n_seqs - 1}, first "
                       f"{n_steps + 1} tokens) vs the fp32 oracle decoder teacher-forced on them: "
                       "argmax where the oracle's top-2 margin >= bar, within bar of its max "
                       "everywhere"}
    return base, parity


def bench_copy(args):
    """Plain device copy of 1 GiB (torch copy_): the calibration kernel for
    the HBM byte counters and the achievable-bandwidth reference."""
    import torch
    dev = torch.device("cuda:0")
    n = 1 << 29  # bf16 elements = 1 GiB
    src = torch.empty(n, dtype=torch.bfloat16, device=dev).normal_()
    dst = torch.empty_like(src)
    total_ms, per = _time_gpu(lambda: dst.copy_(src), args.steps, args.warmup)
    kern_ms = statistics.mean(per)
    nbytes = 2 * n * 2
    achieved = nbytes / (kern_ms * 1e-3) / 1e9
    return {"value": round(achieved, 1), "unit": "GB/s", "ms_per_step": round(total_ms / args.steps, 4),
            "config": {"workload": "calibration: torch copy_ of 1 GiB bf16 (1 GiB read + 1 GiB write)",
                       "bytes_read": n * 2, "bytes_written": n * 2},
            "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBPS,
                         "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBPS, 4), "traffic": None,
                         "algorithmic_bytes": nbytes, "avg_launch_us": round(kern_ms * 1e3, 2)}}


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=None,
                    help="timed steps (default: 1 for e2e, 50 for the kernel workloads)")
    ap.add_argument("--warmup", type=int, default=None,
                    help="untimed warmup steps (default: 1 for e2e, 10 otherwise)")
    ap.add_argument("--workload", choices=["e2e", "decode", "sampler", "mixed", "copy"],
                    default="e2e")
    ap.add_argument("--output-len", type=int, default=1024,
                    help="e2e: output tokens per request")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--sampler-rows", choices=["config4", "greedy", "temperature"],
                    default="config4",
                    help="sampler workload rows: config 4's half/half mix (the bench line), "
                         "all greedy, or all at T = 0.75 (same logits; a diagnostic)")
    ap.add_argument("--eager", action="store_true",
                    help="e2e: no HIP graphs for decode steps")
    ap.add_argument("--no-graph-timing", action="store_true",
                    help="e2e: skip the graph replays of the sampled attention calls (the "
                         "roofline then holds the eager per-call figure; for kernel traces)")
    ap.add_argument("--no-secondary", action="store_true",
                    help="e2e: skip the config-2 decode-attention microbench; mixed: skip "
                         "the chunk-rows-alone timing")
    args = ap.parse_args()
    if args.steps is None:
        args.steps = 1 if args.workload == "e2e" else 50
    if args.warmup is None:
        args.warmup = 1 if args.workload == "e2e" else 10
    if args.steps < 1 or args.warmup < 0:
        print("--steps must be >= 1 and --warmup >= 0", file=sys.stderr)
        return 2
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (this build has no multi-GPU path); got --gpus "
              f"{args.gpus}", file=sys.stderr)
        return 2
    import torch
    if not torch.cuda.is_available():
        print("bench.py needs a ROCm GPU", file=sys.stderr)
        return 2
    fn = {"e2e": bench_e2e, "decode": bench_decode, "sampler": bench_sampler, "mixed": bench_mixed,
          "copy": bench_copy}[args.workload]
    res = fn(args)
    line = {
        "metric": METRIC, "value": res["value"], "unit": res["unit"], "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": res["ms_per_step"],
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "bf16",
        "data": "synthetic (seeded torch.Generator, seed 0)", "config": res["config"],
    }
    for k in ("roofline", "chunk_roofline", "cpu_baseline", "parity", "secondary"):
        if k in res:
            line[k] = res[k]
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
