"""Summarise rocprofv3 output into the short text files kept under profiles/.

    python h3.c_amd/rocprof_summary.py stats <results.db> [top]
        per-kernel calls / total / average / min / max duration (us)
    python h3.c_amd/rocprof_summary.py stats_csv <run_kernel_stats.csv> [top]
        the same from rocprofv3's csv output
    python h3.c_amd/rocprof_summary.py pmc <counter_collection.csv> <kernel-substring>
        per-dispatch average of every counter for the kernels matching the
        substring, and for the calibration kernel (hk_elementwise8<2>, add_bf16)
    python h3.c_amd/rocprof_summary.py traffic <fetch.csv> <write.csv> <kernel-substring> <calib-elements>
        HBM-side bytes per launch of the matching kernel as JSON: FETCH_SIZE
        and WRITE_SIZE (KiB per dispatch) scaled by what they read for the
        last add_bf16 dispatch, which moves exactly 2 x 2 x calib-elements
        bytes in and 2 x calib-elements bytes out
    python h3.c_amd/rocprof_summary.py kernels <kernel_trace.csv> <mfma.csv> <fetch.csv> <write.csv> <calib-elements>
        per kernel (name and grid size; the flash kernel's alternating self /
        cross launches of the forward apart): launches, average duration from
        the kernel trace, MfmaUtil (SQ_VALU_MFMA_BUSY_CYCLES over all SIMDs
        against GRBM_GUI_ACTIVE, as rocprofv3 derives it), FETCH_SIZE and
        WRITE_SIZE per launch calibrated as in `traffic`, and the HBM GB/s
        they make over the average duration
    python h3.c_amd/rocprof_summary.py forward <mfma_raw.csv>
        MFMA busy % of the one forward bench.py --profile-pass measures, from
        SQ_VALU_MFMA_BUSY_CYCLES / GRBM_GUI_ACTIVE / SQ_INSTS_VALU_MFMA_MOPS_BF16
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


def stats_csv(path, top=25):
    """The same table from rocprofv3's run_kernel_stats.csv."""
    rows = list(csv.DictReader(open(path)))
    total = sum(float(r["TotalDurationNs"]) for r in rows) or 1.0
    print(f"{'kernel':60s} {'calls':>6s} {'total_us':>12s} {'avg_us':>10s} "
          f"{'min_us':>10s} {'max_us':>10s} {'pct':>6s}")
    for r in rows[:top]:
        name = _short(r["Name"])
        tot = float(r["TotalDurationNs"])
        print(f"{name[:60]:60s} {int(r['Calls']):6d} {tot / 1e3:12.1f} "
              f"{float(r['AverageNs']) / 1e3:10.1f} "
              f"{float(r['MinNs']) / 1e3:10.1f} "
              f"{float(r['MaxNs']) / 1e3:10.1f} {100 * tot / total:6.2f}")


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


def _groups(path, value="Counter_Value"):
    """(kernel name, grid size, role) -> list of values, in dispatch order.
    Self attention is the 8-wave flash kernel and short cross attention
    the 4-wave one; traces of the single-instance kernel, whose launches
    alternate self / cross with one grid size, are told apart by order."""
    rows = []
    for r in csv.DictReader(open(path)):
        grid = (int(r["Grid_Size"]) if "Grid_Size" in r else
                int(r["Grid_Size_X"]) * int(r["Grid_Size_Y"]) *
                int(r["Grid_Size_Z"]))
        rows.append((int(r["Dispatch_Id"]), r["Kernel_Name"], grid, r))
    rows.sort(key=lambda t: t[0])
    seen = defaultdict(int)
    out = defaultdict(list)
    for _, name, grid, r in rows:
        role = ""
        if "hk_flash_fwd<false, false, 4>" in name:
            role = "cross"
        elif "hk_flash_fwd<false, false, 8>" in name:
            role = "self"
        elif "hk_flash_fwd<false, false>" in name:
            i = seen[(name, grid)]
            seen[(name, grid)] += 1
            role = "self" if i % 2 == 0 else "cross"
        v = (float(r[value]) if value in r else
             (int(r["End_Timestamp"]) - int(r["Start_Timestamp"])))
        out[(name, grid, role)].append(v)
    return out


def _mfma_groups(path, simds=1024, xcds=8):
    """(kernel, grid, role) -> MFMA busy % per dispatch: rocprofv3's derived
    MfmaUtil where the run collected it, else SQ_VALU_MFMA_BUSY_CYCLES over
    GRBM_GUI_ACTIVE (summed over the XCDs) x SIMDs, the same derivation."""
    rows = list(csv.DictReader(open(path)))
    if any(r["Counter_Name"] == "MfmaUtil" for r in rows):
        return _groups(path)
    per = defaultdict(dict)
    meta = {}
    for r in rows:
        i = int(r["Dispatch_Id"])
        per[i][r["Counter_Name"]] = float(r["Counter_Value"])
        meta[i] = r
    tmp = "/tmp/_mfma_util.csv"
    with open(tmp, "w", newline="") as f:
        w = csv.DictWriter(f, fieldnames=list(rows[0].keys()))
        w.writeheader()
        for i, c in per.items():
            if "SQ_VALU_MFMA_BUSY_CYCLES" not in c or not c.get(
                    "GRBM_GUI_ACTIVE"):
                continue
            r = dict(meta[i])
            r["Counter_Name"] = "MfmaUtil"
            r["Counter_Value"] = 100.0 * c["SQ_VALU_MFMA_BUSY_CYCLES"] / (
                c["GRBM_GUI_ACTIVE"] / xcds * simds)
            w.writerow(r)
    return _groups(tmp)


def _short(name):
    name = name.replace("void ", "")
    cut = name.find("(")
    return name[:cut] if cut > 0 else name


def forward_util(mfma_raw_csv, simds=1024, xcds=8):
    """MFMA busy fraction of one whole forward: SQ_VALU_MFMA_BUSY_CYCLES
    summed over the forward's dispatches against their summed
    GRBM_GUI_ACTIVE (reported summed over the XCDs) x SIMDs.  The forward
    is the run between the two F32 fills that bench.py --profile-pass
    launches around it."""
    per = defaultdict(dict)
    names = {}
    for r in csv.DictReader(open(mfma_raw_csv)):
        i = int(r["Dispatch_Id"])
        per[i][r["Counter_Name"]] = float(r["Counter_Value"])
        names[i] = r["Kernel_Name"]
    seps = [i for i in sorted(names) if "hk_fill_normal_kernel<float>" in
            names[i]]
    lo, hi = seps[-2], seps[-1]
    busy = sum(per[i]["SQ_VALU_MFMA_BUSY_CYCLES"] for i in per
               if lo < i < hi)
    active = sum(per[i]["GRBM_GUI_ACTIVE"] / xcds for i in per
                 if lo < i < hi)
    flops = sum(per[i]["SQ_INSTS_VALU_MFMA_MOPS_BF16"] * 512 for i in per
                if lo < i < hi)
    return {"dispatches": hi - lo - 1,
            "mfma_busy_pct": round(100.0 * busy / (active * simds), 2),
            "mfma_bf16_flop": flops}


def kernels(trace_csv, mfma_csv, fetch_csv, write_csv, calib_elements):
    dur = _groups(trace_csv, "duration")
    mfma = _mfma_groups(mfma_csv)
    fetch = _groups(fetch_csv)
    write = _groups(write_csv)
    cal = [k for k in fetch if "hk_elementwise8<2>" in k[0]]
    f_cal = fetch[cal[0]][-1] * 1024
    w_cal = write[cal[0]][-1] * 1024
    f_scale = 4 * calib_elements / f_cal
    w_scale = 2 * calib_elements / w_cal
    print(f"calibration: add_bf16 of {calib_elements} elements; FETCH_SIZE x "
          f"{f_scale:.5f}, WRITE_SIZE x {w_scale:.5f}\n")
    print("| kernel | grid | role | launches | avg us | MFMA busy % | "
          "fetch MB | write MB | HBM GB/s |")
    print("|---|---|---|---|---|---|---|---|---|")
    keys = sorted(dur, key=lambda k: -sum(dur[k]))
    for key in keys:
        d = dur[key]
        if sum(d) / 1e3 < 20 and "skinny" not in key[0]:
            continue
        avg = sum(d) / len(d) / 1e3
        mu = mfma.get(key)
        fb = fetch.get(key)
        wb = write.get(key)
        f_mb = sum(fb) / len(fb) * 1024 * f_scale / 1e6 if fb else None
        w_mb = sum(wb) / len(wb) * 1024 * w_scale / 1e6 if wb else None
        gbs = ((f_mb + w_mb) * 1e6 / (avg * 1e-6) / 1e9
               if f_mb is not None and w_mb is not None else None)

        def fmt(v, p=1):
            return "-" if v is None else f"{v:.{p}f}"
        print(f"| `{_short(key[0])[:56]}` | {key[1]} | {key[2] or '-'} | "
              f"{len(d)} | {avg:.1f} | "
              f"{fmt(sum(mu) / len(mu) if mu else None)} | {fmt(f_mb)} | "
              f"{fmt(w_mb)} | {fmt(gbs, 0)} |")


if __name__ == "__main__":
    if sys.argv[1] == "stats_csv":
        stats_csv(sys.argv[2], int(sys.argv[3]) if len(sys.argv) > 3 else 25)
    elif sys.argv[1] == "stats":
        stats(sys.argv[2], int(sys.argv[3]) if len(sys.argv) > 3 else 25)
    elif sys.argv[1] == "forward":
        import json
        print(json.dumps(forward_util(sys.argv[2])))
    elif sys.argv[1] == "kernels":
        kernels(sys.argv[2], sys.argv[3], sys.argv[4], sys.argv[5],
                int(sys.argv[6]))
    elif sys.argv[1] == "traffic":
        traffic(sys.argv[2], sys.argv[3], sys.argv[4], int(sys.argv[5]))
    else:
        pmc(sys.argv[2], sys.argv[3])
