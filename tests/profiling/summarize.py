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


def _short(name):
    """A kernel's name without the return type and namespace."""
    return re.sub(r"^void\s+", "", name).replace("fmha_decode::", "")


def _bench_json(path):
    """The JSON line the profiled program printed (splitkv_bench.py), if any."""
    if not path or not os.path.exists(path):
        return None
    for line in open(path, errors="replace"):
        line = line.strip()
        if line.startswith("{") and "us_per_call_median" in line:
            try:
                return json.loads(line)
            except ValueError:
                pass
    return None


def per_kernel(a):
    """Per-pass table of a call made of several kernels (split-KV): each
    kernel's average duration, HBM bytes per dispatch (FETCH_SIZE and
    WRITE_SIZE, copy-calibrated) and VALU/MFMA busy; the call's total against
    the algorithmic bytes (Q + K + V + O) and the workspace bytes the plan
    moves."""
    names = sorted({r["Kernel_Name"] for r in _rows(os.path.join(a.dir, "trace", "**", "*kernel_trace.csv"))
                    if re.search(a.kernel, r["Kernel_Name"])})
    cf = counters(os.path.join(a.dir, "calib_fetch"), r"copy|elementwise|Copy")
    cw = counters(os.path.join(a.dir, "calib_write"), r"copy|elementwise|Copy")
    gib_kib = float(1 << 20)
    f_scale = statistics.median(cf["FETCH_SIZE"]) / gib_kib if cf.get("FETCH_SIZE") else None
    w_scale = statistics.median(cw["WRITE_SIZE"]) / gib_kib if cw.get("WRITE_SIZE") else None
    bench = _bench_json(a.bench_log)
    ws = bench.get("workspace_traffic_bytes", 0) if bench else 0
    rows, tot_us, tot_bytes = [], 0.0, 0.0
    for n in names:
        kre = "^" + re.escape(n) + "$"
        durs = trace_stats(os.path.join(a.dir, "trace"), kre)
        avg = statistics.mean(durs) if durs else float("nan")
        kf = counters(os.path.join(a.dir, "fetch"), kre).get("FETCH_SIZE")
        kw = counters(os.path.join(a.dir, "write"), kre).get("WRITE_SIZE")
        fetch = statistics.median(kf) / f_scale * 1024 if kf and f_scale else float("nan")
        write = statistics.median(kw) / w_scale * 1024 if kw and w_scale else float("nan")
        busy = {k: statistics.median(v) for k, v in counters(os.path.join(a.dir, "busy"), kre).items()}
        cyc = busy.get("GRBM_GUI_ACTIVE", 0) / XCD_NUM
        valu = 100 * 4 * busy["SQ_ACTIVE_INST_VALU"] / (SIMD_NUM * cyc) if cyc and "SQ_ACTIVE_INST_VALU" in busy else None
        mfma = (100 * busy["SQ_VALU_MFMA_BUSY_CYCLES"] / (SIMD_NUM * cyc)
                if cyc and "SQ_VALU_MFMA_BUSY_CYCLES" in busy else None)
        tot_us += avg
        tot_bytes += fetch + write
        rows.append({"kernel": _short(n), "calls": len(durs), "avg_us": avg, "fetch_bytes": fetch,
                     "write_bytes": write, "hbm_gbs": (fetch + write) / (avg * 1e-6) / 1e9 if durs else None,
                     "valu_busy_pct": valu, "mfma_busy_pct": mfma, "waves": busy.get("SQ_WAVES")})
    out = {"label": a.label, "per_kernel": rows, "algorithmic_bytes_per_call": a.bytes,
           "workspace_bytes_per_call": ws, "kernel_us_per_call": tot_us, "hbm_bytes_per_call": tot_bytes,
           "traffic_over_algorithmic": tot_bytes / a.bytes,
           "traffic_over_algorithmic_plus_workspace": tot_bytes / (a.bytes + ws),
           "achieved_gbs": a.bytes / (tot_us * 1e-6) / 1e9, "bench": bench}
    lines = [f"# {a.label}", "", "Command:", "", "    " + a.command, ""]
    if bench:
        lines += [f"Plan (fmha_decode_last_plan): {'; '.join(bench.get('plan', []))}", "",
                  f"Timed call (HIP events, median of the program's own loop): "
                  f"{bench['us_per_call_median']} µs, {bench['tb_s']} TB/s algorithmic", ""]
    lines += ["| kernel | dispatches | avg µs | FETCH bytes | WRITE bytes | HBM GB/s | VALUBusy % | MfmaUtil % |",
              "|---|---|---|---|---|---|---|---|"]
    fmt = lambda x, f: "-" if x is None or x != x else format(x, f)
    for r in rows:
        lines.append(f"| `{r['kernel']}` | {r['calls']} | {fmt(r['avg_us'], '.1f')} | {fmt(r['fetch_bytes'], '.4g')} | "
                     f"{fmt(r['write_bytes'], '.4g')} | {fmt(r['hbm_gbs'], '.0f')} | {fmt(r['valu_busy_pct'], '.1f')} | "
                     f"{fmt(r['mfma_busy_pct'], '.2f')} |")
    lines += ["", f"Per call: kernel time {tot_us:.1f} µs (sum of the passes' averages); algorithmic bytes "
                  f"{a.bytes:.4g} (Q + K + V + O, fmha_host.cpp:428-430) -> {out['achieved_gbs']:.0f} GB/s, "
                  f"{out['achieved_gbs'] / 80:.1f}% of 8 TB/s; workspace bytes by the plan {ws:.4g}; measured HBM "
                  f"bytes {tot_bytes:.4g} = {out['traffic_over_algorithmic']:.4f} x algorithmic, "
                  f"{out['traffic_over_algorithmic_plus_workspace']:.4f} x (algorithmic + workspace).", "",
              "FETCH_SIZE and WRITE_SIZE (KiB per dispatch, one counter per run) are scaled by what they read for "
              "a 1 GiB device-to-device copy (tests/profiling/calib_copy.py); VALUBusy = 4 SQ_ACTIVE_INST_VALU / "
              f"({SIMD_NUM} SIMDs x GRBM_GUI_ACTIVE / {XCD_NUM}), MfmaUtil = SQ_VALU_MFMA_BUSY_CYCLES / "
              f"({SIMD_NUM} x the same cycles), medians over dispatches.", ""]
    with open(os.path.join(a.dir, "summary.md"), "w") as f:
        f.write("\n".join(lines) + "\n")
    with open(os.path.join(a.dir, "traffic.json"), "w") as f:
        json.dump(out, f, indent=1)
    print("\n".join(lines))


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("dir")
    ap.add_argument("--kernel", default="fmha_decode_fwd_kernel")
    ap.add_argument("--bytes", type=float, required=True, help="algorithmic bytes per launch")
    ap.add_argument("--label", default="")
    ap.add_argument("--command", default="")
    ap.add_argument("--per-kernel", action="store_true", help="one row per kernel (multi-pass calls)")
    ap.add_argument("--bench-log", default="", help="the profiled program's output (its JSON line)")
    a = ap.parse_args()
    if a.per_kernel:
        per_kernel(a)
        return

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
