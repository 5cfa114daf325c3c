#!/usr/bin/env python3
"""Streaming ceiling of each BASELINE configuration next to the decode kernel.

For C1..C5 runs, on the same GPU and in turn:
  * the decode kernel (tests/fmha_host.py, timing only);
  * tests/profiling/_build/stream_ceiling: the kernel's exact loads and
    stores without its arithmetic;
  * the same without the O stores (reads only);
and prints a markdown table: µs per call, algorithmic TB/s, and the kernel's
share of its own traffic's ceiling.  C1 runs over 4 input sets in rotation
(its 503 MB would otherwise partly stay in the 256 MB MALL).

    python3 tests/profiling/ceiling.py [--iters N] > summary.md
"""
import argparse
import json
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
BIN = os.path.join(HERE, "_build", "stream_ceiling")
CONFIGS = {1: (30720, 16, 16, 1, 128), 2: (30720, 16, 16, 16, 128), 3: (30720, 16, 16, 5, 256),
           4: (30720, 32, 16, 16, 128), 5: (30720, 32, 32, 16, 256)}


def run_json(cmd):
    out = subprocess.run(cmd, check=True, capture_output=True, text=True).stdout
    return [json.loads(l) for l in out.splitlines() if l.startswith("{")]


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--iters", type=int, default=50)
    ap.add_argument("--configs", default="1,2,3,4,5")
    a = ap.parse_args()
    if not os.path.exists(BIN):
        sys.exit(f"{BIN} is not built (make -C tests/profiling)")
    rows = []
    for c in [int(x) for x in a.configs.split(",")]:
        B, hq, hkv, S, D = CONFIGS[c]
        sets = 4 if c == 1 else 1
        k = run_json([sys.executable, os.path.join(ROOT, "tests", "fmha_host.py"), str(c), "--suite", "baseline",
                      "--validate", "none", "--iters", str(a.iters), "--rotate", str(sets)])[0]
        base = [BIN, str(B), str(hq), str(hkv), str(S), str(D), "--sets", str(sets), "--iters", str(a.iters)]
        rw = run_json(base)[0]
        ro = run_json(base + ["--no-write"])[0]
        rows.append((c, B, hq, hkv, S, D, sets, k, rw, ro))
        print(f"C{c}: kernel {k['us_per_call_median']} us, ceiling {rw['us_per_call_median']} us, "
              f"reads only {ro['us_per_call_median']} us", file=sys.stderr, flush=True)
    print("TB/s counts the algorithmic bytes (Q + K + V + O); in the last column, which")
    print("stores nothing, it counts the bytes read (Q + K + V).")
    print()
    print("| config | input sets | decode kernel µs (TB/s) | same traffic, no arithmetic µs (TB/s) | "
          "ceiling µs / kernel µs | same without the O stores µs (TB/s read) |")
    print("|---|---|---|---|---|---|")
    for c, B, hq, hkv, S, D, sets, k, rw, ro in rows:
        read_bytes = 2 * B * hq * D + 4 * B * S * hkv * D
        print(f"| C{c} B={B} Hq={hq} Hkv={hkv} S={S} D={D} | {sets} | {k['us_per_call_median']} ({k['tb_s_median']:.2f}) "
              f"| {rw['us_per_call_median']} ({rw['tb_s']:.2f}) | {rw['us_per_call_median'] / k['us_per_call_median']:.3f} "
              f"| {ro['us_per_call_median']} ({read_bytes / ro['us_per_call_median'] / 1e6:.2f}) |")


if __name__ == "__main__":
    main()
