#!/usr/bin/env python3
"""Benchmark of the decode-attention hot path on one MI355X.

One step = one call of the HIP kernel over the headline workload (BASELINE.json
B=30720, Hq=Hkv=16, seqlen_q=1, seqlen_kv=16, D=128, bf16 Q/K/V
drawn N(0,1) from a fixed seed, fp32 accumulation, fp16 output), with every
input resident in HBM before the timed region.

Prints one JSON line:
  value         algorithmic TB/s of the timed region: K back-to-back calls of
                fmha_decode_fwd_uniform between one HIP-event pair on the
                launch stream, as the reference's harness times them
                (fmha_host.cpp:377-397); bytes per call as the reference
                counts them (fmha_host.cpp:428-430).  At this group size
                (Hq/Hkv = 1) the call computes the reference CPU loop's
                arithmetic step for step: its outputs are that loop's
                (fmha_host.cpp:179-244), bit for bit;
  roofline      the kernel alone: algorithmic bytes per launch over the mean
                of per-launch HIP-event durations, from a second loop of K
                calls, each between its own event pair on the launch stream
                (those events add a few µs between launches, so they stay out
                of the value loop), against the 8 TB/s HBM peak; traffic =
                measured HBM bytes per launch from the committed rocprofv3
                counter summary, when present;
  rotated_inputs  the same calls over --rotate input/output sets used in
                turn (no call finds Q or O of the previous call in the MALL);
                the timed loop above reuses one set, as the reference's
                harness does (fmha_host.cpp:377-389);
  cu_seqlens    the same workload and bytes through fmha_decode_fwd, the
                entry point the reference's host program reaches
                (fmha_host.cpp:367/382/437 through launch_fmha_mfma_4x4x4):
                lengths from a device cu_seqlens array, timed as `value` is
                after the warm-up calls (whose first call runs under the
                default wave cap, its time reported as first_call_us); the
                same numerics as value;
  fast          the same workload through fmha_decode_fwd_uniform_fast
                (tree-order sums: within the comparison gate of the loop,
                not its bits), timed as value;
  cpu_baseline  the reference's own CPU loop (fmha_host.cpp:158-284, built from
                /root/reference into oracle/_ref) -- or the restated oracle
                when that build is absent -- timed single-threaded on this
                host over a bounded sample of the same workload, plus the
                restated loop on up to 16 host cores (port_all_cores).
"""
import argparse
import contextlib
import json
import math
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0
METRIC = "µs/call + achieved HBM TB/s (% of peak) at B=30720,H=16,Skv=16,d=128"
WORKLOAD = dict(batch=30720, num_heads_q=16, num_heads_kv=16, seqlen_kv=16, head_dim=128, std=1.0)
SEED = 0xF3A00000 + 16 * 2
TRAFFIC_FILE = os.path.join(ROOT, "profiles", "fmha_decode_c2_traffic.json")


def algorithmic_bytes(B, Hq, Hkv, S, D):
    # Q (bf16) + K and V (bf16) + O (fp16), fmha_host.cpp:428-430 with Hkv heads for K/V.
    return 2 * B * Hq * D + 2 * (2 * B * S * Hkv * D) + 2 * B * Hq * D


@contextlib.contextmanager
def _quiet_stdout():
    """Silence fd 1 (the reference loop prints while it validates)."""
    sys.stdout.flush()
    saved = os.dup(1)
    with open(os.devnull, "w") as dn:
        os.dup2(dn.fileno(), 1)
        try:
            yield
        finally:
            sys.stdout.flush()
            os.dup2(saved, 1)
            os.close(saved)


def cpu_baseline(q, k, v, o, B, Hq, Hkv, S, D, scale, max_batches):
    """Time the reference CPU loop on the first `max_batches` batches."""
    import numpy as np
    import torch
    import oracle

    nb = min(B, max_batches)
    qh = q.view(B, Hq, D)[:nb].contiguous().view(torch.int16).cpu().numpy().view(np.uint16)
    kh = k.view(B * S, Hkv, D)[: nb * S].contiguous().view(torch.int16).cpu().numpy().view(np.uint16)
    vh = v.view(B * S, Hkv, D)[: nb * S].contiguous().view(torch.int16).cpu().numpy().view(np.uint16)
    oh = o.view(B, Hq, D)[:nb].contiguous().view(torch.int16).cpu().numpy().view(np.uint16)
    cu = np.arange(0, (nb + 1) * S, S, dtype=np.int32)
    nbytes = algorithmic_bytes(nb, Hq, Hkv, S, D)
    if oracle.ref_available() and Hq == Hkv:
        kind = "reference"
        with _quiet_stdout():
            t0 = time.perf_counter()
            _, passed = oracle.ref_do_validation(qh, kh, vh, cu, Hq, Hkv, D, gpu_o=oh)
            dt = time.perf_counter() - t0
        extra = {"reference_check_of_gpu_output": "passed" if passed else "failed"}
    else:
        kind = "port"
        t0 = time.perf_counter()
        oracle.decode(qh, kh, vh, cu, Hq, Hkv, D, scale, nthreads=1)
        dt = time.perf_counter() - t0
        extra = {}
    out = {
        "value": nbytes / dt / 1e12,
        "unit": "TB/s",
        "cores": 1,
        "kind": kind,
        "sample": f"first {nb} of {B} batches of the timed workload (all heads, S={S}), one pass, "
                  f"single thread: {dt:.2f} s; us_per_call scaled to the full batch = "
                  f"{dt * 1e6 * B / nb:.0f}",
        "us_per_call_full_batch": dt * 1e6 * B / nb,
    }
    out.update(extra)
    # The same sample through the restated loop (oracle/), OpenMP over batches
    # on the host's cores (at most 16, the GPU box's share).
    threads = max(1, min(16, os.cpu_count() or 1))
    t0 = time.perf_counter()
    oracle.decode(qh, kh, vh, cu, Hq, Hkv, D, scale, nthreads=threads)
    dt_mt = time.perf_counter() - t0
    out["port_all_cores"] = {"value": nbytes / dt_mt / 1e12, "unit": "TB/s", "cores": threads, "kind": "port",
                             "seconds": round(dt_mt, 3), "us_per_call_full_batch": dt_mt * 1e6 * B / nb}
    return out


def main():
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--cpu-batches", type=int, default=30720,
                    help="batches of the workload the CPU baseline runs (bounded sample)")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--rotate", type=int, default=2,
                    help="input/output sets of the second timed leg (1 = skip that leg)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py: this build runs on one GPU only (asked for --gpus {args.gpus}); "
              "the decode path shards by batch or KV head without communication, so the "
              "one-GPU figure is the per-GPU figure", file=sys.stderr)
        sys.exit(2)

    import torch
    import fmha_amd

    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    W = WORKLOAD
    B, Hq, Hkv, S, D = W["batch"], W["num_heads_q"], W["num_heads_kv"], W["seqlen_kv"], W["head_dim"]
    gen = torch.Generator(device=dev).manual_seed(SEED)
    q = torch.randn(B, Hq, 1, D, generator=gen, device=dev, dtype=torch.bfloat16)
    k = torch.randn(B, S, Hkv, D, generator=gen, device=dev, dtype=torch.bfloat16)
    v = torch.randn(B, S, Hkv, D, generator=gen, device=dev, dtype=torch.bfloat16)
    o = torch.empty(B, Hq, 1, D, device=dev, dtype=torch.float16)
    scale = 1.0 / math.sqrt(D)
    stream = torch.cuda.current_stream(dev)
    sptr = stream.cuda_stream
    qp, kp, vp, op = q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr()

    def step(ptrs=(qp, kp, vp, op)):
        fmha_amd.launch_fmha_decode_uniform(sptr, *ptrs, S, B, Hq, Hkv, 1, D, D, scale)

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()

    K = args.steps
    ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(K)]
    e_start, e_end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)

    def timed_loop(ptr_sets, call=step):
        """K back-to-back calls between one event pair: ms per call."""
        torch.cuda.synchronize()
        e_start.record(stream)
        for i in range(K):
            call(ptr_sets[i % len(ptr_sets)])
        e_end.record(stream)
        torch.cuda.synchronize()
        return e_start.elapsed_time(e_end) / K

    def per_launch_loop(ptr_sets, call=step):
        """K calls, each between its own event pair: per-launch ms."""
        torch.cuda.synchronize()
        for i in range(K):
            ev[i][0].record(stream)
            call(ptr_sets[i % len(ptr_sets)])
            ev[i][1].record(stream)
        torch.cuda.synchronize()
        return [a.elapsed_time(b) for a, b in ev]

    one_set = [(qp, kp, vp, op)]
    wall0 = time.perf_counter()
    ms_per_step = timed_loop(one_set)
    wall = time.perf_counter() - wall0
    per = per_launch_loop(one_set)                      # ms, each launch alone
    kern_ms = sum(per) / K
    nbytes = algorithmic_bytes(B, Hq, Hkv, S, D)
    value_tbs = nbytes / (ms_per_step * 1e-3) / 1e12
    achieved_gbs = nbytes / (kern_ms * 1e-3) / 1e9
    per_sorted = sorted(per)

    # Second leg: the same calls over --rotate input/output sets used in
    # turn.  In the leg above the next call finds part of Q (read with the
    # default policy) and the rewritten O in the 256 MB MALL; here every call
    # reads and writes buffers the previous call did not touch.
    rotated = None
    if args.rotate > 1:
        sets = [(qp, kp, vp, op)]
        keep = []
        for _ in range(args.rotate - 1):
            t = (torch.randn(B, Hq, 1, D, generator=gen, device=dev, dtype=torch.bfloat16),
                 torch.randn(B, S, Hkv, D, generator=gen, device=dev, dtype=torch.bfloat16),
                 torch.randn(B, S, Hkv, D, generator=gen, device=dev, dtype=torch.bfloat16),
                 torch.empty(B, Hq, 1, D, device=dev, dtype=torch.float16))
            keep.append(t)
            sets.append(tuple(x.data_ptr() for x in t))
        for i in range(args.warmup):
            step(sets[i % len(sets)])
        rot_ms = timed_loop(sets)
        rot_kern_ms = sum(per_launch_loop(sets)) / K
        rotated = {
            "input_sets": len(sets),
            "us_per_call": round(rot_ms * 1e3, 2),
            "us_per_call_kernel_mean": round(rot_kern_ms * 1e3, 2),
            "tb_s": round(nbytes / (rot_ms * 1e-3) / 1e12, 4),
            "pct_of_peak": round(100.0 * nbytes / (rot_ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 2),
        }
        del keep

    # Third leg: the drop-in entry point on the same inputs, lengths from a
    # device cu_seqlens array.  Its wave cap comes from the mean length the
    # previous call on this device reported (the first call, timed alone
    # here, has none and runs under the default cap).
    cu = torch.arange(0, (B + 1) * S, S, dtype=torch.int32, device=dev)
    cup = cu.data_ptr()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)

    def step_cu(ptrs=(qp, kp, vp, op)):
        fmha_amd.launch_fmha_decode(sptr, *ptrs, cup, B, Hq, Hkv, 1, D, D, scale)

    torch.cuda.synchronize()
    e0.record(stream)
    step_cu()
    e1.record(stream)
    torch.cuda.synchronize()
    first_cu_ms = e0.elapsed_time(e1)
    for _ in range(args.warmup):
        step_cu()
    cu_ms = timed_loop(one_set, step_cu)
    cu_kern_ms = sum(per_launch_loop(one_set, step_cu)) / K
    cu_leg = {
        "entry_point": "fmha_decode_fwd (cu_seqlens)",
        "us_per_call": round(cu_ms * 1e3, 2),
        "us_per_call_kernel_mean": round(cu_kern_ms * 1e3, 2),
        "tb_s": round(nbytes / (cu_ms * 1e-3) / 1e12, 4),
        "pct_of_peak": round(100.0 * nbytes / (cu_ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 2),
        "vs_uniform_entry": round(ms_per_step / cu_ms, 4),
        "first_call_us": round(first_cu_ms * 1e3, 2),
    }

    # Fourth leg: the tree-order entry point on the same inputs.
    def step_fast(ptrs=(qp, kp, vp, op)):
        fmha_amd.launch_fmha_decode_uniform_fast(sptr, *ptrs, S, B, Hq, Hkv, 1, D, D, scale)

    for _ in range(args.warmup):
        step_fast()
    fast_ms = timed_loop(one_set, step_fast)
    fast_leg = {
        "entry_point": "fmha_decode_fwd_uniform_fast (tree-order sums)",
        "us_per_call": round(fast_ms * 1e3, 2),
        "tb_s": round(nbytes / (fast_ms * 1e-3) / 1e12, 4),
        "pct_of_peak": round(100.0 * nbytes / (fast_ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 2),
        "value_entry_time_over_this": round(ms_per_step / fast_ms, 4),
    }

    traffic = None
    if os.path.exists(TRAFFIC_FILE):
        with open(TRAFFIC_FILE) as f:
            traffic = json.load(f).get("hbm_bytes_per_launch")

    cpu = None
    if not args.no_cpu:
        cpu = cpu_baseline(q, k, v, o, B, Hq, Hkv, S, D, scale, args.cpu_batches)

    line = {
        "metric": METRIC,
        "value": round(value_tbs, 4),
        "unit": "TB/s",
        "n_gpus": 1,
        "steps": K,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 5),
        "us_per_call": round(ms_per_step * 1e3, 2),
        "us_per_call_kernel_mean": round(kern_ms * 1e3, 2),
        "us_per_call_kernel_median": round(per_sorted[K // 2] * 1e3, 2),
        "pct_of_peak": round(100.0 * value_tbs * 1e3 / HBM_PEAK_GBS, 2),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "accumulate": "f32",
        "data": "synthetic: seeded N(0,1) bf16 generated on the GPU",
        "config": {
            "workload": "BASELINE configs[1]: decode attention B=30720 Hq=Hkv=16 seqlen_q=1 "
                        "seqlen_kv=16 D=128, bf16 in, fp16 out",
            "batch": B, "num_heads_q": Hq, "num_heads_kv": Hkv, "seqlen_q": 1, "seqlen_kv": S,
            "head_dim": D, "bytes_per_call": nbytes, "parallelism": "single GPU",
        },
        "roofline": {
            "bound": "hbm",
            "achieved": round(achieved_gbs, 1),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(achieved_gbs / HBM_PEAK_GBS, 4),
            "traffic": traffic,
        },
        "rotated_inputs": rotated,
        "numerics": "the reference CPU loop's arithmetic step for step (outputs bit-equal to "
                    "fmha_host.cpp:179-244 with nearest-float exponentials)",
        "cu_seqlens": cu_leg,
        "fast": fast_leg,
        "cpu_baseline": cpu,
        "wall_s_timed_region": round(wall, 4),
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
