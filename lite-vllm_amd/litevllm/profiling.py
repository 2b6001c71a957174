"""Summaries of rocprofv3 kernel traces (the SQLite ``*_results.db`` that
``rocprofv3 --kernel-trace -d DIR -o NAME`` writes).

``python -m litevllm.profiling DIR [--top N]`` prints a markdown table of
kernels by total time, the GPU busy time against the trace span, and, for
an engine run, the average duration of the decode-attention kernels over
decode-only steps (a step starts at each ``pack_kernel`` dispatch; it is
decode-only when no ``attn_chunk_mfma_kernel`` runs in it).

``python -m litevllm.profiling --counters DIR`` reads the
``*counter_collection.csv`` of a ``rocprofv3 --pmc ... --output-format csv``
run and prints, per counter, the mean value per decode-attention launch
pair (persistent kernel + its reduce kernel) over decode-only steps, and the
mean per dispatch of every other kernel.
"""

from __future__ import annotations

import argparse
import glob
import re
import sqlite3
import statistics
from pathlib import Path


def _rows(db: str) -> list[tuple[str, int, int]]:
    cur = sqlite3.connect(db).cursor()
    return cur.execute("select name, start, end from kernels order by start").fetchall()


def _short(name: str, width: int = 100) -> str:
    return name.split("(")[0][:width]


def summarize(trace_dir: str, top: int = 25) -> str:
    dbs = sorted(glob.glob(str(Path(trace_dir) / "**" / "*.db"), recursive=True))
    if not dbs:
        raise FileNotFoundError(f"no rocprofv3 database under {trace_dir}")
    out: list[str] = []
    for db in dbs:
        rows = _rows(db)
        if not rows:
            continue
        per: dict[str, list[int]] = {}
        for name, s, e in rows:
            per.setdefault(name, []).append(e - s)
        busy, cs, ce = 0, None, None
        for _, s, e in rows:
            if cs is None:
                cs, ce = s, e
            elif s > ce:
                busy += ce - cs
                cs, ce = s, e
            else:
                ce = max(ce, e)
        busy += ce - cs
        total = sum(sum(v) for v in per.values())
        span = rows[-1][2] - rows[0][1]
        out.append(f"kernels {len(rows)}; sum of durations {total / 1e6:.1f} ms; GPU busy "
                   f"{busy / 1e6:.1f} ms; trace span {span / 1e6:.1f} ms\n")
        out.append("| kernel | calls | avg us | total ms | share |")
        out.append("|---|---|---|---|---|")
        for name, d in sorted(per.items(), key=lambda kv: -sum(kv[1]))[:top]:
            out.append(f"| `{_short(name)}` | {len(d)} | {sum(d) / len(d) / 1e3:.2f} | "
                       f"{sum(d) / 1e6:.1f} | {sum(d) / total:.3f} |")
        dec = _decode_only(rows)
        if dec:
            out.append("")
            out.append("Decode-only steps (no chunk-attention kernel between two packing "
                       f"dispatches): {dec['steps']} steps")
            for k, v in dec["kernels"].items():
                out.append(f"* `{k}`: {v[0]} launches, mean {v[1]:.2f} us, median {v[2]:.2f} us")
    return "\n".join(out)


def _decode_only(rows) -> dict:
    steps, cur = [], None
    for name, s, e in rows:
        if "pack_kernel" in name:
            if cur is not None:
                steps.append(cur)
            cur = []
        elif cur is not None:
            cur.append((name, e - s))
    if cur:
        steps.append(cur)
    keep = [st for st in steps if st and not any("attn_chunk_mfma_kernel" in n for n, _ in st)]
    acc: dict[str, list[int]] = {}
    for st in keep:
        for n, d in st:
            if "attn_decode_persistent_kernel" in n or "attn_persist_reduce_kernel" in n:
                acc.setdefault(_short(n, 80), []).append(d)
    if not acc:
        return {}
    return {"steps": len(keep),
            "kernels": {k: (len(v), sum(v) / len(v) / 1e3, statistics.median(v) / 1e3)
                        for k, v in acc.items()}}


def summarize_counters(pmc_dir: str) -> str:
    import csv
    files = sorted(glob.glob(str(Path(pmc_dir) / "**" / "*counter_collection.csv"),
                             recursive=True))
    if not files:
        raise FileNotFoundError(f"no counter_collection.csv under {pmc_dir}")
    # dispatch id -> (kernel name, {counter: value})
    disp: dict[int, tuple[str, dict[str, float]]] = {}
    for f in files:
        for r in csv.DictReader(open(f)):
            d = int(r.get("Dispatch_Id") or r["Correlation_Id"])
            name, vals = disp.setdefault(d, (r["Kernel_Name"], {}))
            vals[r["Counter_Name"]] = vals.get(r["Counter_Name"], 0.0) + float(r["Counter_Value"])
    order = sorted(disp)
    counters = sorted({c for _, v in disp.values() for c in v})
    steps, cur = [], None
    for d in order:
        name, vals = disp[d]
        if "pack_kernel" in name:
            if cur is not None:
                steps.append(cur)
            cur = []
        elif cur is not None:
            cur.append((name, vals))
    if cur:
        steps.append(cur)
    def is_prefix_pass(n: str) -> bool:
        # attn_chunk_mfma_kernel<T, D, G, BS, W, BPW, true> (names may carry
        # the argument list after the template arguments)
        return re.search(r"attn_chunk_mfma_kernel<[^<>]*,\s*true>", n) is not None

    def is_chunk(n: str) -> bool:
        return "attn_chunk_mfma_kernel" in n and not is_prefix_pass(n)

    # One decode-attention call: [shared-prefix pass] + persistent kernel +
    # reduce kernel, summed.
    pairs: list[dict[str, float]] = []
    for st in steps:
        if any(is_chunk(n) for n, _ in st):
            continue
        acc, walked = None, False
        for n, vals in st:
            if is_prefix_pass(n) or ("attn_decode_persistent_kernel" in n and walked) or \
                    ("attn_decode_persistent_kernel" in n and acc is None):
                if acc is not None:
                    pairs.append(acc)
                acc, walked = dict(vals), "attn_decode_persistent_kernel" in n
            elif acc is not None and ("attn_decode_persistent_kernel" in n
                                      or "attn_persist_reduce_kernel" in n):
                walked = walked or "attn_decode_persistent_kernel" in n
                for c, v in vals.items():
                    acc[c] = acc.get(c, 0.0) + v
        if acc is not None:
            pairs.append(acc)
    out = [f"dispatches with counters: {len(order)}; decode-only steps: "
           f"{sum(1 for st in steps if not any(is_chunk(n) for n, _ in st))}; "
           f"decode-attention calls in them: {len(pairs)}", ""]
    if pairs:
        out.append("| counter | mean per decode-attention call (decode-only steps) |")
        out.append("|---|---|")
        for c in counters:
            vals = [p[c] for p in pairs if c in p]
            if vals:
                out.append(f"| {c} | {statistics.mean(vals):.1f} |")
        out.append("")
    per: dict[str, dict[str, list[float]]] = {}
    for d in order:
        name, vals = disp[d]
        for c, v in vals.items():
            per.setdefault(_short(name, 80), {}).setdefault(c, []).append(v)
    out.append("| kernel | counter | dispatches | mean per dispatch |")
    out.append("|---|---|---|---|")
    for k in sorted(per):
        for c, v in sorted(per[k].items()):
            out.append(f"| `{k}` | {c} | {len(v)} | {statistics.mean(v):.1f} |")
    return "\n".join(out)


def main() -> None:
    ap = argparse.ArgumentParser(description=__doc__)
    ap.add_argument("trace_dir")
    ap.add_argument("--top", type=int, default=25)
    ap.add_argument("--counters", action="store_true",
                    help="trace_dir holds a rocprofv3 --pmc csv run")
    args = ap.parse_args()
    if args.counters:
        print(summarize_counters(args.trace_dir))
    else:
        print(summarize(args.trace_dir, args.top))


if __name__ == "__main__":
    main()
