"""Summarise rocprofv3 output into the short text files kept under profiles/.

    python h3.c_amd/rocprof_summary.py stats <results.db> [top]
        per-kernel calls / total / average / min / max duration (us)
    python h3.c_amd/rocprof_summary.py pmc <counter_collection.csv> <kernel-substring>
        per-dispatch average of every counter for the kernels matching the
        substring, and for the calibration kernel (hk_elementwise<2>, add_bf16)
"""
import csv
import sqlite3
import sys
from collections import defaultdict


def stats(db, top=25):
    c = sqlite3.connect(db)
    rows = c.execute(
        "select name, count(*), sum(duration), avg(duration), min(duration), "
        "max(duration) from kernels group by name order by sum(duration) desc"
    ).fetchall()
    total = sum(r[2] for r in rows) or 1
    print(f"{'kernel':60s} {'calls':>6s} {'total_us':>12s} {'avg_us':>10s} "
          f"{'min_us':>10s} {'max_us':>10s} {'pct':>6s}")
    for name, n, tot, avg, mn, mx in rows[:top]:
        print(f"{name[:60]:60s} {n:6d} {tot / 1e3:12.1f} {avg / 1e3:10.1f} "
              f"{mn / 1e3:10.1f} {mx / 1e3:10.1f} {100 * tot / total:6.2f}")


def pmc(path, match):
    per = defaultdict(list)
    for r in csv.DictReader(open(path)):
        name = r["Kernel_Name"]
        if match in name or "hk_elementwise<2>" in name:
            per[(name, r["Counter_Name"])].append(float(r["Counter_Value"]))
    for (name, counter), vals in sorted(per.items()):
        print(f"{name[:48]:48s} {counter:16s} dispatches {len(vals):4d} "
              f"avg {sum(vals) / len(vals):16.1f}")


if __name__ == "__main__":
    if sys.argv[1] == "stats":
        stats(sys.argv[2], int(sys.argv[3]) if len(sys.argv) > 3 else 25)
    else:
        pmc(sys.argv[2], sys.argv[3])
