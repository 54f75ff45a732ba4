#!/usr/bin/env python3
"""Summaries of rocprofv3 CSV output (`--output-format csv`) for the profiles of this library.

  rocprof_summary.py trace DIR
      per-kernel calls, total and average duration from DIR's *_kernel_stats.csv
  rocprof_summary.py traffic FETCH_DIR WRITE_DIR KERNEL [--copy k_copy_calibrate --copy-bytes N]
                                   [--units N]
      HBM bytes per dispatch of KERNEL (a substring of the kernel's name) from a FETCH_SIZE
      pass and a WRITE_SIZE pass, or, with --units N, the sum over every dispatch of the
      kernels KERNEL names (comma-separated substrings) divided by N: each
      counter's mean per dispatch, scaled by (known copy bytes / the counter's mean over the
      plain copy kernel's dispatches in the same pass)
  rocprof_summary.py mfma DIR [--simds N --xcds N]
      per-kernel MFMA busy fraction, SQ_VALU_MFMA_BUSY_CYCLES / (active cycles x SIMDs), and
      MFMA FLOPs from the SQ_INSTS_VALU_MFMA_MOPS_* counters (x 512), plus the totals over
      every kernel of the pass. The profiler sums GRBM_GUI_ACTIVE over the XCDs (each counts
      the dispatch's cycles), so active cycles = GRBM_GUI_ACTIVE / XCDs

Each prints a markdown table and, with --json FILE, writes the figures as JSON.
"""
import argparse
import csv
import glob
import json
import os
import sys
from collections import defaultdict


def _csvs(d, suffix):
    files = sorted(glob.glob(os.path.join(d, "**", "*" + suffix), recursive=True))
    if not files:
        raise SystemExit(f"no *{suffix} under {d}")
    return files


def _short(name):
    """Kernel name without return type, anonymous namespace and argument list."""
    name = name.strip().replace("(anonymous namespace)::", "")
    if name.startswith("void "):
        name = name[5:]
    return name.split("(")[0] if "(" in name else name


def kernel_stats(d):
    rows = []
    for f in _csvs(d, "_kernel_stats.csv"):
        with open(f, newline="") as fh:
            for r in csv.DictReader(fh):
                rows.append({"kernel": _short(r["Name"]), "calls": int(r["Calls"]),
                             "total_ms": float(r["TotalDurationNs"]) / 1e6,
                             "avg_us": float(r["AverageNs"]) / 1e3,
                             "min_us": float(r["MinNs"]) / 1e3, "max_us": float(r["MaxNs"]) / 1e3})
    rows.sort(key=lambda r: -r["total_ms"])
    return rows


def counters(d):
    """{kernel: {counter: [value per dispatch]}} from DIR's *_counter_collection.csv."""
    out = defaultdict(lambda: defaultdict(dict))
    for f in _csvs(d, "_counter_collection.csv"):
        with open(f, newline="") as fh:
            for r in csv.DictReader(fh):
                k = _short(r["Kernel_Name"])
                out[k][r["Counter_Name"]][(f, r["Dispatch_Id"])] = float(r["Counter_Value"])
    return {k: {c: list(v.values()) for c, v in cs.items()} for k, cs in out.items()}


def mean(v):
    return sum(v) / len(v) if v else float("nan")


def cmd_trace(a):
    rows = kernel_stats(a.dir)
    print("| kernel | calls | total ms | average µs | min µs | max µs |")
    print("|---|---:|---:|---:|---:|---:|")
    for r in rows[: a.top]:
        print(f"| `{r['kernel']}` | {r['calls']} | {r['total_ms']:.3f} | {r['avg_us']:.1f} | "
              f"{r['min_us']:.1f} | {r['max_us']:.1f} |")
    return {"kernels": rows}


def cmd_traffic(a):
    fc, wc = counters(a.fetch_dir), counters(a.write_dir)

    def per_dispatch(cs, kernel, counter):
        for k, v in cs.items():
            if kernel in k and counter in v:
                return mean(v[counter]), len(v[counter])
        raise SystemExit(f"{counter} for {kernel} not found")

    def per_unit(cs, names, counter):
        tot, n = 0.0, 0
        for k, v in cs.items():
            if counter in v and any(x in k for x in names) and a.copy not in k:
                tot += sum(v[counter])
                n += len(v[counter])
        if not n:
            raise SystemExit(f"{counter} for {names} not found")
        return tot / a.units, n

    if a.units:
        names = [x for x in a.kernel.split(",") if x]
        fk, nf = per_unit(fc, names, "FETCH_SIZE")
        wk, nw = per_unit(wc, names, "WRITE_SIZE")
    else:
        fk, nf = per_dispatch(fc, a.kernel, "FETCH_SIZE")
        wk, nw = per_dispatch(wc, a.kernel, "WRITE_SIZE")
    fcp, ncf = per_dispatch(fc, a.copy, "FETCH_SIZE")
    wcp, ncw = per_dispatch(wc, a.copy, "WRITE_SIZE")
    fs, ws = a.copy_bytes / fcp, a.copy_bytes / wcp
    res = {"kernel": {"name": a.kernel, "FETCH_SIZE_kib": fk, "WRITE_SIZE_kib": wk,
                      "dispatches": min(nf, nw)},
           "copy": {"kernel": a.copy, "bytes_read": a.copy_bytes, "bytes_written": a.copy_bytes,
                    "FETCH_SIZE_kib": fcp, "WRITE_SIZE_kib": wcp, "dispatches": min(ncf, ncw)},
           "scale": {"FETCH_SIZE_bytes_per_kib": fs, "WRITE_SIZE_bytes_per_kib": ws},
           "result": {"read_bytes": round(fk * fs), "write_bytes": round(wk * ws),
                      "traffic_bytes": round(fk * fs + wk * ws)}}
    if a.algorithmic:
        res["result"]["algorithmic_bytes"] = a.algorithmic
        res["result"]["traffic_over_algorithmic"] = round((fk * fs + wk * ws) / a.algorithmic, 4)
    unit = f"per {a.units}th of the sum" if a.units else "per dispatch"
    print(f"| kernel | dispatches | FETCH_SIZE {unit} | WRITE_SIZE {unit} |")
    print("|---|---:|---:|---:|")
    print(f"| {a.copy} ({a.copy_bytes} B copy) | {min(ncf, ncw)} | {fcp:,.1f} | {wcp:,.1f} |")
    print(f"| {a.kernel} | {min(nf, nw)} | {fk:,.1f} | {wk:,.1f} |")
    print()
    print(f"scale: FETCH_SIZE {fs:.2f} B per unit, WRITE_SIZE {ws:.2f} B per unit")
    print()
    print(f"| {'per unit' if a.units else 'per dispatch'} | bytes |")
    print("|---|---:|")
    for k in ("read_bytes", "write_bytes", "traffic_bytes", "algorithmic_bytes", "traffic_over_algorithmic"):
        if k in res["result"]:
            v = res["result"][k]
            print(f"| {k} | {v:,} |" if isinstance(v, int) else f"| {k} | {v} |")
    return res


def cmd_mfma(a):
    cs = counters(a.dir)
    rows, tot_busy, tot_active, tot_flops = [], 0.0, 0.0, 0.0
    for k, v in cs.items():
        if "SQ_VALU_MFMA_BUSY_CYCLES" not in v or "GRBM_GUI_ACTIVE" not in v:
            continue
        busy, active = sum(v["SQ_VALU_MFMA_BUSY_CYCLES"]), sum(v["GRBM_GUI_ACTIVE"]) / a.xcds
        mops = sum(sum(x) for c, x in v.items() if c.startswith("SQ_INSTS_VALU_MFMA_MOPS_"))
        rows.append({"kernel": k, "dispatches": len(v["GRBM_GUI_ACTIVE"]), "mfma_busy": busy,
                     "gui_active": active, "busy_frac": busy / (active * a.simds) if active else 0.0,
                     "mfma_flops": mops * 512})
        tot_busy += busy
        tot_active += active
        tot_flops += mops * 512
    rows.sort(key=lambda r: -r["gui_active"])
    print("| kernel | dispatches | MFMA busy / (active cycles x SIMDs) | MFMA FLOP per dispatch |")
    print("|---|---:|---:|---:|")
    for r in rows[: a.top]:
        print(f"| `{r['kernel']}` | {r['dispatches']} | {r['busy_frac']:.4f} | "
              f"{r['mfma_flops'] / r['dispatches']:.3e} |")
    allf = tot_busy / (tot_active * a.simds) if tot_active else 0.0
    print(f"| all kernels | {sum(r['dispatches'] for r in rows)} | {allf:.4f} | "
          f"{tot_flops:.3e} (total) |")
    return {"kernels": rows, "all": {"busy_frac": allf, "mfma_flops": tot_flops,
                                     "mfma_busy": tot_busy, "gui_active": tot_active}}


def main():
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    sub = ap.add_subparsers(dest="cmd", required=True)
    t = sub.add_parser("trace")
    t.add_argument("dir")
    t.add_argument("--top", type=int, default=20)
    f = sub.add_parser("traffic")
    f.add_argument("fetch_dir")
    f.add_argument("write_dir")
    f.add_argument("kernel")
    f.add_argument("--copy", default="k_copy_calibrate")
    f.add_argument("--copy-bytes", type=int, default=1 << 30)
    f.add_argument("--algorithmic", type=int, default=0, help="algorithmic bytes per dispatch (unit)")
    f.add_argument("--units", type=int, default=0, help="divide the matched kernels' sum by this")
    m = sub.add_parser("mfma")
    m.add_argument("dir")
    m.add_argument("--simds", type=int, default=1024, help="SIMDs on the device (4 per CU)")
    m.add_argument("--xcds", type=int, default=8, help="XCDs whose GRBM_GUI_ACTIVE the profiler sums")
    m.add_argument("--top", type=int, default=20)
    for p in (t, f, m):
        p.add_argument("--json", default="")
    a = ap.parse_args()
    res = {"trace": cmd_trace, "traffic": cmd_traffic, "mfma": cmd_mfma}[a.cmd](a)
    if a.json:
        with open(a.json, "w") as fh:
            json.dump(res, fh, indent=1)
    return 0


if __name__ == "__main__":
    sys.exit(main())
