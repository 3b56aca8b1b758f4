"""Summaries of rocprofv3 CSV output for the verify pass.

A model pass starts with its token-embedding kernel (k_embed, one workgroup per pass row), so
a kernel trace or a counter collection splits into passes at each k_embed dispatch and the
row count of a pass is that dispatch's workgroup count.  The summaries below keep only this
library's kernels of the passes with a given row count (9 = y plus an 8-token chain draft).

    python -m momij_amd.profiling trace    <run_kernel_trace.csv>       --rows 9 [--last N]
    python -m momij_amd.profiling counters <run_counter_collection.csv> --rows 9 --scale F
    python -m momij_amd.profiling traffic  <fetch.csv> <write.csv> --rows 9 --kernel NAME
                                           --copy-mb 512 [--out FILE.json]
    python -m momij_amd.profiling multi    <run_counter_collection.csv> --rows 9 (0: all)

`trace` prints, per kernel and grid size, launches per pass and the mean / median duration;
`--last N` restricts it to the last N passes of that row count (the eager, event-timed passes
bench.py runs after its graph-replayed steps).  `counters` prints the mean counter value per
dispatch in MB, multiplied by `--scale` (the calibration factor of the counter: the ratio of a
plain copy's known bytes to what the counter reports for it).  `traffic` takes a FETCH_SIZE and
a WRITE_SIZE collection of runs that end with one plain device copy of `--copy-mb` MiB
(bench.py --copy-calib-mb), derives each counter's factor from that copy, and reports the HBM
bytes per dispatch of the kernel whose name starts with NAME.  `multi` prints the mean per
dispatch of every counter of a collection (e.g. SQ_VALU_MFMA_BUSY_CYCLES with GRBM_GUI_ACTIVE),
per kernel.
"""
from __future__ import annotations

import argparse
import collections
import csv
import statistics


def _ours(name: str) -> bool:
    # k_hold only delays a profiled pass (it runs before the pass's k_embed); not pass work
    return (name.startswith("k_") or name.startswith("void k_")) and not name.startswith("k_hold")


def _key(name: str, grid: int, wg: int) -> str:
    return f"{name.split('(')[0]} [{grid // max(wg, 1)} wg]"


def split_passes(rows, grid_col: str, wg_col: str):
    """[(rows of the pass, [csv rows of its kernels])] in dispatch order."""
    passes, cur = [], None
    for r in rows:
        name = r["Kernel_Name"]
        if name.startswith("k_embed"):
            cur = (int(r[grid_col]) // int(r[wg_col]), [])
            passes.append(cur)
        if cur is not None and _ours(name):
            cur[1].append(r)
    return passes


def trace_summary(path: str, n_rows: int, last: int | None = None) -> str:
    rows = list(csv.DictReader(open(path)))
    rows.sort(key=lambda r: int(r["Start_Timestamp"]))
    passes = [p for p in split_passes(rows, "Grid_Size_X", "Workgroup_Size_X") if p[0] == n_rows]
    if last:
        passes = passes[-last:]
    if not passes:
        return f"no passes with {n_rows} rows"
    stat = collections.defaultdict(list)
    spans = []
    for _, ks in passes:
        t0 = int(ks[0]["Start_Timestamp"])
        t1 = max(int(k["End_Timestamp"]) for k in ks)
        spans.append((t1 - t0) / 1e3)
        for k in ks:
            d = (int(k["End_Timestamp"]) - int(k["Start_Timestamp"])) / 1e3
            stat[_key(k["Kernel_Name"], int(k["Grid_Size_X"]), int(k["Workgroup_Size_X"]))].append(d)
    n = len(passes)
    out = [f"passes with {n_rows} rows: {n}; pass span (first start to last end) median "
           f"{statistics.median(spans):.1f} us",
           f"{'kernel [workgroups]':44s} {'per pass':>8s} {'mean us':>9s} {'median us':>9s} "
           f"{'us/pass':>9s}"]
    total = 0.0
    for k, v in sorted(stat.items(), key=lambda kv: -sum(kv[1])):
        per = len(v) / n
        total += statistics.mean(v) * per
        out.append(f"{k:44s} {per:8.1f} {statistics.mean(v):9.2f} {statistics.median(v):9.2f} "
                   f"{statistics.mean(v) * per:9.1f}")
    out.append(f"{'sum of kernel time per pass':44s} {'':8s} {'':9s} {'':9s} {total:9.1f}")
    return "\n".join(out)


def counter_summary(path: str, n_rows: int, scale: float) -> str:
    rows = list(csv.DictReader(open(path)))
    rows.sort(key=lambda r: int(r["Dispatch_Id"]))
    counter = rows[0]["Counter_Name"] if rows else "?"
    passes = [p for p in split_passes(rows, "Grid_Size", "Workgroup_Size") if p[0] == n_rows]
    by = collections.defaultdict(list)
    for _, ks in passes:
        for r in ks:
            by[_key(r["Kernel_Name"], int(r["Grid_Size"]), int(r["Workgroup_Size"]))].append(
                float(r["Counter_Value"]) * scale * 1024 / 1e6)
    out = [f"{counter} x {scale:g} per dispatch, passes with {n_rows} rows: {len(passes)}",
           f"{'kernel [workgroups]':44s} {'dispatches':>10s} {'mean MB':>10s} {'median MB':>10s}"]
    for k, v in sorted(by.items(), key=lambda kv: -statistics.mean(kv[1])):
        out.append(f"{k:44s} {len(v):10d} {statistics.mean(v):10.3f} {statistics.median(v):10.3f}")
    return "\n".join(out)


def multi_counter_summary(path: str, n_rows: int | None) -> str:
    """Mean value per dispatch of every counter in a collection, per kernel (passes of
    `n_rows` rows, or every dispatch of this library's kernels when n_rows is None)."""
    rows = list(csv.DictReader(open(path)))
    rows.sort(key=lambda r: int(r["Dispatch_Id"]))
    if n_rows is None:
        ks = [r for r in rows if _ours(r["Kernel_Name"])]
    else:
        ks = [r for n, p in split_passes(rows, "Grid_Size", "Workgroup_Size") if n == n_rows
              for r in p]
    per = collections.defaultdict(lambda: collections.defaultdict(float))  # (key, id) -> ctr
    keys = {}
    names = []
    for r in ks:
        k = _key(r["Kernel_Name"], int(r["Grid_Size"]), int(r["Workgroup_Size"]))
        d = int(r["Dispatch_Id"])
        keys[d] = k
        c = r["Counter_Name"]
        if c not in names:
            names.append(c)
        per[d][c] += float(r["Counter_Value"])
    by = collections.defaultdict(list)
    for d, vals in per.items():
        by[keys[d]].append(vals)
    out = [f"mean per dispatch; dispatches counted: {len(per)}",
           f"{'kernel [workgroups]':44s} {'n':>5s} " + " ".join(f"{c:>28s}" for c in names)]
    for k, v in sorted(by.items()):
        out.append(f"{k:44s} {len(v):5d} " +
                   " ".join(f"{statistics.mean(x.get(c, 0.0) for x in v):28.1f}" for c in names))
    return "\n".join(out)


def copy_scale(path: str, copy_bytes: int) -> float:
    """Known bytes / counted bytes of the largest plain copy dispatch in a collection."""
    rows = [r for r in csv.DictReader(open(path)) if "copyBuffer" in r["Kernel_Name"]]
    if not rows:
        raise SystemExit(f"{path}: no copy dispatch to calibrate against")
    counted = max(float(r["Counter_Value"]) * 1024 for r in rows)
    return copy_bytes / counted


def kernel_bytes(path: str, n_rows: int, kernel: str, scale: float) -> tuple[float, int]:
    rows = list(csv.DictReader(open(path)))
    rows.sort(key=lambda r: int(r["Dispatch_Id"]))
    vals = [float(r["Counter_Value"]) * 1024 * scale
            for n, ks in split_passes(rows, "Grid_Size", "Workgroup_Size") if n == n_rows
            for r in ks if r["Kernel_Name"].startswith(kernel)]
    if not vals:
        raise SystemExit(f"{path}: no dispatch of {kernel!r} in passes of {n_rows} rows")
    return statistics.mean(vals), len(vals)


def traffic_summary(fetch_csv: str, write_csv: str, n_rows: int, kernel: str,
                    copy_mb: int) -> dict:
    copy_bytes = copy_mb << 20
    fs, ws = copy_scale(fetch_csv, copy_bytes), copy_scale(write_csv, copy_bytes)
    fb, nf = kernel_bytes(fetch_csv, n_rows, kernel, fs)
    wb, nw = kernel_bytes(write_csv, n_rows, kernel, ws)
    return {"kernel": kernel, "rows": n_rows, "fetch_bytes_per_launch": round(fb),
            "write_bytes_per_launch": round(wb), "traffic_bytes_per_launch": round(fb + wb),
            "fetch_scale": round(fs, 4), "write_scale": round(ws, 4),
            "dispatches": [nf, nw], "copy_bytes": copy_bytes}


def main():
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("kind", choices=["trace", "counters", "traffic", "multi"])
    ap.add_argument("csv")
    ap.add_argument("csv2", nargs="?")
    ap.add_argument("--kernel", default="void k_moe_fused<64, false, 16>")
    ap.add_argument("--copy-mb", type=int, default=512)
    ap.add_argument("--out", default=None)
    ap.add_argument("--rows", type=int, default=9)
    ap.add_argument("--last", type=int, default=None)
    ap.add_argument("--scale", type=float, default=1.0)
    a = ap.parse_args()
    if a.kind == "trace":
        print(trace_summary(a.csv, a.rows, a.last))
    elif a.kind == "counters":
        print(counter_summary(a.csv, a.rows, a.scale))
    elif a.kind == "multi":
        print(multi_counter_summary(a.csv, a.rows if a.rows > 0 else None))
    else:
        import json

        t = traffic_summary(a.csv, a.csv2, a.rows, a.kernel, a.copy_mb)
        print(json.dumps(t, indent=1))
        if a.out:
            with open(a.out, "w") as f:
                json.dump(t, f, indent=1)
                f.write("\n")


if __name__ == "__main__":
    main()
