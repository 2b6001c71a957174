#!/usr/bin/env python3
"""Benchmark of the MI355X continuous-batching hot path (one GPU).

Default workload (``--workload decode``): paged decode attention at the
Qwen3-0.6B attention shape, 256 sequences, context U[128, 2048], 16 q / 8 kv
heads, head_dim 128, block_size 16, bf16 (fp32 accumulate).  One "step" is
one lv_paged_attention call over the whole batch with every input resident
in HBM.  Other workloads: ``mixed`` (chunked-prefill step: pack + scatter +
attention), ``sampler`` (fused sampler on [256, 151936] bf16 logits).

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
MFMA_BF16_PEAK_TFLOPS = 2500.0


def _cpu_threads() -> int:
    try:
        return len(os.sched_getaffinity(0))
    except AttributeError:
        return os.cpu_count() or 1


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
    kern_ms = statistics.mean(per)
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
            "traffic": _traffic("decode"),
            "algorithmic_bytes": nbytes, "avg_launch_us": round(kern_ms * 1e3, 2),
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
        "cores": threads, "kind": "port",
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
    uni = sb.uniform.to(dev)
    out = torch.empty(logits.shape[0], dtype=torch.int64, device=dev)
    total_ms, per = _time_gpu(lambda: ops.sample(logits, temp, uni, out=out), args.steps,
                              args.warmup)
    B, V = logits.shape
    nbytes = B * V * logits.element_size() + B * (4 + 4 + 8)
    kern_ms = statistics.mean(per)
    achieved = nbytes / (kern_ms * 1e-3) / 1e9
    res = {
        "value": round(B / (kern_ms * 1e-3), 1), "unit": "sampled rows/s",
        "ms_per_step": round(total_ms / args.steps, 4),
        "config": {"workload": "config4 fused sampler: [256, 151936] bf16 logits N(0,16), "
                               "rows 0-127 greedy, 128-255 T~U[0.5,1], supplied uniforms",
                   "kernel": "lv_sample (sampler_kernel)"},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBPS,
                     "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBPS, 4),
                     "traffic": _traffic("sampler"),
                     "algorithmic_bytes": nbytes, "avg_launch_us": round(kern_ms * 1e3, 2)},
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
                               "cores": 1, "kind": "port",
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
    return {
        "value": round(T / (kern_ms * 1e-3), 1), "unit": "packed tokens/s",
        "ms_per_step": round(total_ms / args.steps, 4),
        "config": {"workload": "config3 mixed step: 192 decodes ctx U[256,4096] + 15 chunks x 512 "
                               "at offset U[0,3072], 200k-slot cache, bf16",
                   "num_tokens": T},
    }


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
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--workload", choices=["decode", "sampler", "mixed", "copy"], default="decode")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (this build has no multi-GPU path); got --gpus "
              f"{args.gpus}", file=sys.stderr)
        return 2
    import torch
    if not torch.cuda.is_available():
        print("bench.py needs a ROCm GPU", file=sys.stderr)
        return 2
    fn = {"decode": bench_decode, "sampler": bench_sampler, "mixed": bench_mixed,
          "copy": bench_copy}[args.workload]
    res = fn(args)
    line = {
        "metric": METRIC, "value": res["value"], "unit": res["unit"], "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": res["ms_per_step"],
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "bf16",
        "data": "synthetic (seeded torch.Generator, seed 0)", "config": res["config"],
    }
    for k in ("roofline", "cpu_baseline"):
        if k in res:
            line[k] = res[k]
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
