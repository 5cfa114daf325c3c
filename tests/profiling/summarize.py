#!/usr/bin/env python3
"""Summarises the rocprofv3 CSV output that run_rocprof.sh collects.

Reads <dir>/trace/*_kernel_stats.csv, <dir>/{fetch,write,busy,cache}/
*_counter_collection.csv and <dir>/calib_{fetch,write}/, and writes
<dir>/summary.md and <dir>/traffic.json:
  * kernel duration statistics of the selected kernel;
  * HBM traffic per launch: FETCH_SIZE and WRITE_SIZE (KiB per dispatch),
    each divided by what the same counter reads per byte for a 1 GiB copy;
  * achieved algorithmic GB/s and measured HBM GB/s at the trace average;
  * VALU busy %, MFMA busy %, instruction counts per wave.
"""
import argparse
import csv
import glob
import json
import os
import re
import statistics

CU_NUM = 256
SIMD_NUM = 1024
# GRBM_GUI_ACTIVE counts the cycles of each XCD's graphics block and the
# counter sums the 8 XCDs of an MI355X: the kernel's cycles are an eighth of
# it (at C2 that gives 1.25e6 cycles in 607 µs, a 2.07 GHz clock).
XCD_NUM = 8


def _rows(pattern):
    out = []
    for p in glob.glob(pattern, recursive=True):
        with open(p) as f:
            out.extend(csv.DictReader(f))
    return out


def counters(d, kernel_re):
    """{counter: [value per matching dispatch]} from a counter_collection CSV."""
    per = {}
    for r in _rows(os.path.join(d, "**", "*counter_collection.csv")):
        if not re.search(kernel_re, r["Kernel_Name"]):
            continue
        key = (r["Counter_Name"], r["Dispatch_Id"])
        per[key] = per.get(key, 0.0) + float(r["Counter_Value"])
    res = {}
    for (name, _), v in per.items():
        res.setdefault(name, []).append(v)
    return res


def trace_stats(d, kernel_re):
    durs = []
    for r in _rows(os.path.join(d, "**", "*kernel_trace.csv")):
        if re.search(kernel_re, r["Kernel_Name"]):
            durs.append((int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1000.0)
    return durs


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("dir")
    ap.add_argument("--kernel", default="fmha_decode_fwd_kernel")
    ap.add_argument("--bytes", type=float, required=True, help="algorithmic bytes per launch")
    ap.add_argument("--label", default="")
    ap.add_argument("--command", default="")
    a = ap.parse_args()

    durs = trace_stats(os.path.join(a.dir, "trace"), a.kernel)
    names = set()
    for r in _rows(os.path.join(a.dir, "trace", "**", "*kernel_trace.csv")):
        if re.search(a.kernel, r["Kernel_Name"]):
            names.add(r["Kernel_Name"])
    out = {"label": a.label, "kernel": sorted(names), "algorithmic_bytes_per_launch": a.bytes}
    lines = [f"# {a.label}", "", "Command:", "", "    " + a.command, ""]
    if durs:
        avg = statistics.mean(durs)
        out.update(calls=len(durs), avg_us=avg, median_us=statistics.median(durs), min_us=min(durs),
                   max_us=max(durs), achieved_gbs=a.bytes / (avg * 1e-6) / 1e9)
        lines += [f"Kernel(s): {', '.join(sorted(names))}", "",
                  "| calls | avg µs | median µs | min µs | max µs | algorithmic GB/s at avg | % of 8 TB/s |",
                  "|---|---|---|---|---|---|---|",
                  f"| {len(durs)} | {avg:.1f} | {statistics.median(durs):.1f} | {min(durs):.1f} | "
                  f"{max(durs):.1f} | {out['achieved_gbs']:.0f} | {out['achieved_gbs'] / 80:.1f} |", ""]
    cf = counters(os.path.join(a.dir, "calib_fetch"), r"copy|elementwise|Copy")
    cw = counters(os.path.join(a.dir, "calib_write"), r"copy|elementwise|Copy")
    kf = counters(os.path.join(a.dir, "fetch"), a.kernel)
    kw = counters(os.path.join(a.dir, "write"), a.kernel)
    gib_kib = float(1 << 20)
    if cf.get("FETCH_SIZE") and cw.get("WRITE_SIZE") and kf.get("FETCH_SIZE") and kw.get("WRITE_SIZE"):
        f_scale = statistics.median(cf["FETCH_SIZE"]) / gib_kib
        w_scale = statistics.median(cw["WRITE_SIZE"]) / gib_kib
        fetch = statistics.median(kf["FETCH_SIZE"]) / f_scale * 1024
        write = statistics.median(kw["WRITE_SIZE"]) / w_scale * 1024
        out.update(fetch_scale=f_scale, write_scale=w_scale, fetch_bytes=fetch, write_bytes=write,
                   hbm_bytes_per_launch=fetch + write,
                   traffic_over_algorithmic=(fetch + write) / a.bytes)
        lines += ["HBM traffic per launch (rocprofv3 --pmc, one counter per run):", "",
                  "| counter | raw KiB/dispatch (median) | calibration KiB per copied KiB | bytes/launch |",
                  "|---|---|---|---|",
                  f"| FETCH_SIZE | {statistics.median(kf['FETCH_SIZE']):.0f} | {f_scale:.4f} | {fetch:.4g} |",
                  f"| WRITE_SIZE | {statistics.median(kw['WRITE_SIZE']):.0f} | {w_scale:.4f} | {write:.4g} |",
                  "",
                  f"Measured HBM bytes per launch {fetch + write:.4g} vs algorithmic {a.bytes:.4g} "
                  f"(ratio {(fetch + write) / a.bytes:.4f}).  Calibration: a 1 GiB device-to-device copy "
                  f"(tests/profiling/calib_copy.py) reads and writes 2^20 KiB per dispatch.", ""]
        if durs:
            out["hbm_gbs"] = (fetch + write) / (statistics.mean(durs) * 1e-6) / 1e9
            lines += [f"Measured HBM GB/s at the trace average: {out['hbm_gbs']:.0f}", ""]
    busy = counters(os.path.join(a.dir, "busy"), a.kernel)
    if busy:
        med = {k: statistics.median(v) for k, v in busy.items()}
        g = med.get("GRBM_GUI_ACTIVE")
        if g:
            cycles = g / XCD_NUM
            out["kernel_cycles"] = cycles
            if durs:
                out["clock_ghz"] = cycles / (statistics.median(durs) * 1e-6) / 1e9
            # SQ_ACTIVE_INST_VALU counts quad-cycles summed over the SIMDs;
            # SQ_VALU_MFMA_BUSY_CYCLES cycles summed over the SIMDs.
            if "SQ_ACTIVE_INST_VALU" in med:
                out["valu_busy_pct"] = 100 * 4 * med["SQ_ACTIVE_INST_VALU"] / (SIMD_NUM * cycles)
            if "SQ_VALU_MFMA_BUSY_CYCLES" in med:
                out["mfma_busy_pct"] = 100 * med["SQ_VALU_MFMA_BUSY_CYCLES"] / (SIMD_NUM * cycles)
        w = med.get("SQ_WAVES")
        lines += ["Busy counters (median over dispatches):", "", "| counter | value | per wave |", "|---|---|---|"]
        for k in sorted(med):
            pw = f"{med[k] / w:.1f}" if w and k.startswith("SQ_INSTS") else ""
            lines.append(f"| {k} | {med[k]:.6g} | {pw} |")
        if "valu_busy_pct" in out:
            clk = f", {out['clock_ghz']:.2f} GHz over the median kernel time" if "clock_ghz" in out else ""
            lines += ["", f"VALUBusy = {out['valu_busy_pct']:.1f}%  "
                          f"MfmaUtil = {out.get('mfma_busy_pct', 0):.2f}%  "
                          f"(per SIMD and kernel cycle; kernel cycles = GRBM_GUI_ACTIVE / {XCD_NUM} XCDs = "
                          f"{out['kernel_cycles']:.4g}{clk}; VALUBusy = 4 SQ_ACTIVE_INST_VALU / "
                          f"({SIMD_NUM} SIMDs x cycles), MfmaUtil = SQ_VALU_MFMA_BUSY_CYCLES / ({SIMD_NUM} x cycles))"]
        out["busy"] = med
        lines.append("")
    cache = counters(os.path.join(a.dir, "cache"), a.kernel)
    if cache:
        med = {k: statistics.median(v) for k, v in cache.items()}
        out["cache"] = med
        lines += ["Cache / LDS counters (median over dispatches):", "", "| counter | value |", "|---|---|"]
        lines += [f"| {k} | {med[k]:.6g} |" for k in sorted(med)]
        lines.append("")
    with open(os.path.join(a.dir, "summary.md"), "w") as f:
        f.write("\n".join(lines) + "\n")
    with open(os.path.join(a.dir, "traffic.json"), "w") as f:
        json.dump(out, f, indent=1)
    print("\n".join(lines))


if __name__ == "__main__":
    main()
