"""Summarise rocprofv3 output into the short text files kept under profiles/.

    python h3.c_amd/rocprof_summary.py stats <results.db> [top]
        per-kernel calls / total / average / min / max duration (us)
    python h3.c_amd/rocprof_summary.py pmc <counter_collection.csv> <kernel-substring>
        per-dispatch average of every counter for the kernels matching the
        substring, and for the calibration kernel (hk_elementwise8<2>, add_bf16)
    python h3.c_amd/rocprof_summary.py traffic <fetch.csv> <write.csv> <kernel-substring> <calib-elements>
        HBM-side bytes per launch of the matching kernel as JSON: FETCH_SIZE
        and WRITE_SIZE (KiB per dispatch) scaled by what they read for the
        last add_bf16 dispatch, which moves exactly 2 x 2 x calib-elements
        bytes in and 2 x calib-elements bytes out
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
        if match in name or "hk_elementwise8<2>" in name:
            per[(name, r["Counter_Name"])].append(float(r["Counter_Value"]))
    for (name, counter), vals in sorted(per.items()):
        print(f"{name[:48]:48s} {counter:16s} dispatches {len(vals):4d} "
              f"avg {sum(vals) / len(vals):16.1f}")


def _dispatches(path, match):
    out = []
    for r in csv.DictReader(open(path)):
        if match in r["Kernel_Name"]:
            out.append((int(r["Dispatch_Id"]), int(r["Grid_Size"]),
                        float(r["Counter_Value"])))
    return sorted(out)


def traffic(fetch_csv, write_csv, match, calib_elements):
    import json
    calib_in = 4 * calib_elements
    calib_out = 2 * calib_elements
    f_cal = _dispatches(fetch_csv, "hk_elementwise8<2>")[-1][2] * 1024
    w_cal = _dispatches(write_csv, "hk_elementwise8<2>")[-1][2] * 1024
    f_scale, w_scale = calib_in / f_cal, calib_out / w_cal
    fetch = _dispatches(fetch_csv, match)
    write = _dispatches(write_csv, match)
    per_launch = [(fv * 1024 * f_scale, wv * 1024 * w_scale)
                  for (_, _, fv), (_, _, wv) in zip(fetch, write)]
    n = len(per_launch)
    total_f = sum(f for f, _ in per_launch)
    total_w = sum(w for _, w in per_launch)
    both = [f + w for f, w in per_launch]
    print(json.dumps({
        "kernel": match,
        "dispatches": n,
        "calibration": {"kernel": "hk_elementwise8<2> (add_bf16)",
                        "elements": calib_elements,
                        "fetch_scale": round(f_scale, 5),
                        "write_scale": round(w_scale, 5)},
        "fetch_bytes_per_launch": round(total_f / n),
        "write_bytes_per_launch": round(total_w / n),
        "bytes_per_launch": round((total_f + total_w) / n),
        "bytes_per_launch_min": round(min(both)),
        "bytes_per_launch_max": round(max(both)),
    }, indent=1))


if __name__ == "__main__":
    if sys.argv[1] == "stats":
        stats(sys.argv[2], int(sys.argv[3]) if len(sys.argv) > 3 else 25)
    elif sys.argv[1] == "traffic":
        traffic(sys.argv[2], sys.argv[3], sys.argv[4], int(sys.argv[5]))
    else:
        pmc(sys.argv[2], sys.argv[3])
