#!/bin/bash
# Counter capture for the decode-attention kernel on one GPU.
#
#   ./run_rocprof.sh [OUTDIR] [WORKLOAD]
#     OUTDIR    default gpurun_out/rocprof
#     WORKLOAD  bench (default: bench.py's headline workload, BASELINE C2),
#               bN (BASELINE config N, 1..5), b1rot (C1 over 8 input sets in
#               turn: 504 MB, beyond the 256 MB MALL), bNv (the same through the
#               cu_seqlens entry point fmha_decode_fwd), rN (the reference's
#               config N, 0..4, Poisson lengths through fmha_decode_fwd) or gN
#               (tests/fmha_host.py's GQA suite, config N, 1..8), or
#               s:B:Hq:Hkv:S:D[:LAYOUT] (one shape through
#               tests/profiling/splitkv_bench.py: lengths beyond 16 through
#               the split-KV entry points, LAYOUT packed, bhsd or pagedN;
#               summarised per kernel, with the workspace bytes apart)
#     KERNEL    (environment) regular expression of the kernel summarised,
#               default fmha_decode:: (every kernel of the library)
#
# Runs rocprofv3 once per pass (kernel trace; FETCH_SIZE; WRITE_SIZE; busy
# counters; cache/LDS counters; FETCH_SIZE and WRITE_SIZE of a 1 GiB copy for
# calibration), each under its own time limit, then writes OUTDIR/summary.md
# and OUTDIR/traffic.json (tests/profiling/summarize.py): kernel µs, achieved
# algorithmic GB/s, measured HBM bytes per launch, VALU/MFMA busy.
set -u
ROOT=$(cd "$(dirname "$0")" && pwd)
OUT=${1:-$ROOT/gpurun_out/rocprof}
case "$OUT" in /*) ;; *) OUT="$ROOT/$OUT" ;; esac
WL=${2:-bench}
mkdir -p "$OUT"
cd /tmp && export TMPDIR=/tmp

case "$WL" in
  bench) CMD=(python3 "$ROOT/bench.py" --no-cpu --rotate 1); TRACE_ARGS=(--steps 50 --warmup 5); PMC_ARGS=(--steps 3 --warmup 1) ;;
  b[1-5]) CMD=(python3 "$ROOT/tests/fmha_host.py" "${WL#b}" --suite baseline --validate none)
          TRACE_ARGS=(--iters 50 --warmup 5); PMC_ARGS=(--iters 3 --warmup 1) ;;
  b[1-5]v) N=${WL#b}; CMD=(python3 "$ROOT/tests/fmha_host.py" "${N%v}" --suite baseline --validate none --varlen)
          TRACE_ARGS=(--iters 50 --warmup 5); PMC_ARGS=(--iters 3 --warmup 1) ;;
  g[1-8]) CMD=(python3 "$ROOT/tests/fmha_host.py" "${WL#g}" --suite gqa --validate none)
          TRACE_ARGS=(--iters 50 --warmup 5); PMC_ARGS=(--iters 3 --warmup 1) ;;
  r[0-4]) CMD=(python3 "$ROOT/tests/fmha_host.py" "${WL#r}" --suite reference --validate none)
          TRACE_ARGS=(--iters 50 --warmup 5); PMC_ARGS=(--iters 3 --warmup 1) ;;
  b1rot) CMD=(python3 "$ROOT/tests/fmha_host.py" 1 --suite baseline --validate none --rotate 8)
          TRACE_ARGS=(--iters 64 --warmup 8); PMC_ARGS=(--iters 16 --warmup 8) ;;
  s:*) IFS=: read -r _ SB SHQ SHKV SS SD SLAYOUT <<< "$WL"
       CMD=(python3 "$ROOT/tests/profiling/splitkv_bench.py" --shapes "$SB:$SHQ:$SHKV:$SS:$SD" --layout "${SLAYOUT:-packed}")
       TRACE_ARGS=(--iters 50 --warmup 5); PMC_ARGS=(--iters 3 --warmup 1) ;;
  *) echo "unknown workload $WL"; exit 2 ;;
esac
BYTES=$(python3 - "$ROOT" "$WL" <<'PY'
import sys
sys.path.insert(0, sys.argv[1])
wl = sys.argv[2]
from tests.fmha_host import SUITES, algorithmic_bytes
if wl == "bench":
    B, Hq, Hkv, S, D, _ = SUITES["baseline"][2]
elif wl == "b1rot":
    B, Hq, Hkv, S, D, _ = SUITES["baseline"][1]
elif wl.startswith("s:"):
    B, Hq, Hkv, S, D = (int(x) for x in wl.split(":")[1:6])
else:
    suite = {"b": "baseline", "r": "reference", "g": "gqa"}[wl[0]]
    B, Hq, Hkv, S, D, _ = SUITES[suite][int(wl[1:].rstrip("v"))]
if S is None:
    import oracle
    rows = int(oracle.generate_seqlens(B, 16).sum())
else:
    rows = B * S
print(algorithmic_bytes(B, Hq, Hkv, rows, D))
PY
)

pass_() {  # name, timeout, rocprof args..., -- command...
  local name=$1 t=$2; shift 2
  echo "== $name" >&2
  timeout -k 10 -s KILL "$t" rocprofv3 "$@" > "$OUT/$name.log" 2>&1
  local rc=$?
  [ $rc -eq 0 ] || { echo "pass $name failed rc=$rc" >&2; tail -5 "$OUT/$name.log" >&2; exit $rc; }
}
pass_ trace 300 --kernel-trace --stats --output-format csv -d "$OUT/trace" -o run -- "${CMD[@]}" "${TRACE_ARGS[@]}"
pass_ fetch 120 --pmc FETCH_SIZE --output-format csv -d "$OUT/fetch" -o run -- "${CMD[@]}" "${PMC_ARGS[@]}"
pass_ write 120 --pmc WRITE_SIZE --output-format csv -d "$OUT/write" -o run -- "${CMD[@]}" "${PMC_ARGS[@]}"
pass_ busy 120 --pmc SQ_WAVES SQ_INSTS_VALU SQ_INSTS_VMEM_RD SQ_INSTS_SALU SQ_ACTIVE_INST_VALU SQ_VALU_MFMA_BUSY_CYCLES SQ_BUSY_CU_CYCLES GRBM_GUI_ACTIVE --output-format csv -d "$OUT/busy" -o run -- "${CMD[@]}" "${PMC_ARGS[@]}"
pass_ cache 120 --pmc TCC_HIT_sum TCC_MISS_sum SQ_INSTS_LDS SQ_LDS_BANK_CONFLICT --output-format csv -d "$OUT/cache" -o run -- "${CMD[@]}" "${PMC_ARGS[@]}"
pass_ calib_fetch 120 --pmc FETCH_SIZE --output-format csv -d "$OUT/calib_fetch" -o run -- python3 "$ROOT/tests/profiling/calib_copy.py"
pass_ calib_write 120 --pmc WRITE_SIZE --output-format csv -d "$OUT/calib_write" -o run -- python3 "$ROOT/tests/profiling/calib_copy.py"
KRE=${KERNEL:-fmha_decode::}
EXTRA=()
case "$WL" in s:*) EXTRA=(--per-kernel --bench-log "$OUT/trace.log") ;; esac
python3 "$ROOT/tests/profiling/summarize.py" "$OUT" --bytes "$BYTES" --kernel "$KRE" --label "workload $WL" \
  --command "./run_rocprof.sh gpurun_out/rocprof_${WL//:/_} $WL" "${EXTRA[@]}"
