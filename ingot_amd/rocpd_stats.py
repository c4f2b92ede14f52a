"""Per-kernel duration statistics from a rocprofv3 output database (rocpd SQLite).

    python -m ingot_amd.rocpd_stats gpurun_out/prof_bench/bench_results.db

Prints calls, mean / median / min duration (us) and total time per kernel,
largest total first: the same figures rocprofv3 --stats reports per kernel.
"""
from __future__ import annotations

import re
import sqlite3
import sys
from collections import defaultdict


def kernel_stats(db_path: str):
    cur = sqlite3.connect(db_path).cursor()
    cols = [r[1] for r in cur.execute("pragma table_info(kernels)")]
    ci = {c: i for i, c in enumerate(cols)}
    agg = defaultdict(list)
    for r in cur.execute("select * from kernels"):
        agg[r[ci["name"]]].append((r[ci["end"]] - r[ci["start"]]) / 1000.0)
    out = []
    for name, v in agg.items():
        v.sort()
        out.append({"kernel": re.sub(r"\(.*", "", name), "calls": len(v), "mean_us": sum(v) / len(v),
                    "median_us": v[len(v) // 2], "min_us": v[0], "total_ms": sum(v) / 1000.0})
    return sorted(out, key=lambda d: -d["total_ms"])


def main(argv):
    rows = kernel_stats(argv[1])
    print(f"| kernel | calls | mean us | median us | min us | total ms |")
    print(f"|---|---:|---:|---:|---:|---:|")
    for d in rows:
        print(f"| `{d['kernel']}` | {d['calls']} | {d['mean_us']:.2f} | {d['median_us']:.2f} | {d['min_us']:.2f} | "
              f"{d['total_ms']:.2f} |")


if __name__ == "__main__":
    main(sys.argv)
