"""Summaries of rocprofv3 kernel traces (the SQLite ``*_results.db`` that
``rocprofv3 --kernel-trace -d DIR -o NAME`` writes).

``python -m litevllm.profiling DIR [--top N]`` prints a markdown table of
kernels by total time, the GPU busy time against the trace span, and, for
an engine run, the average duration of the decode-attention kernels over
decode-only steps (a step starts at each ``pack_kernel`` dispatch; it is
decode-only when no ``attn_chunk_mfma_kernel`` runs in it).
"""

from __future__ import annotations

import argparse
import glob
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


def main() -> None:
    ap = argparse.ArgumentParser(description=__doc__)
    ap.add_argument("trace_dir")
    ap.add_argument("--top", type=int, default=25)
    args = ap.parse_args()
    print(summarize(args.trace_dir, args.top))


if __name__ == "__main__":
    main()
