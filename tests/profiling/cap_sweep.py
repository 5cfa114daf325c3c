#!/usr/bin/env python3
"""Wave-cap sweep of the short kernels (lengths up to 16), for the in-flight
budget model that picks each launch's waves per CU
(fmha_amd/csrc/fmha_decode_caps.hpp: budget_waves, tree_order_budget; fmha_decode_api.hip:
waves_per_cu_for, waves_per_cu_exact).

For each shape, times the call with FMHA_DECODE_WAVE_CAP set to every cap
of --caps and once without it (the model's own cap, read back from
fmha_decode_last_plan), each the minimum over --rounds rounds of --iters
calls between two HIP events on the launch stream, and prints one JSON line:
µs per cap, the model's cap and µs, the best cap and how far the model's
time is from the best (model_over_best).

    python3 tests/profiling/cap_sweep.py --shapes B:Hq:Hkv:S:D[:mode],... [--caps 3,4,...]
    python3 tests/profiling/cap_sweep.py --preset budget

--preset budget: the 102 shapes the budget model's fitted parameters come
from (the 4-head kernel at G = 3, 4 and the 8-head one at G = 5-8, D = 64,
128, 256, S = 1-16; B=30720, 15360 at D = 256; Hkv = 16 at D = 128, else 8).

mode: uniform (default; fmha_decode_fwd_uniform, the lengths known on the
host: tree-order numerics above two query heads per KV head, the reference
loop's arithmetic up to two), cu (fmha_decode_fwd with cu_seqlens_kv on the
device, uniform lengths), fast (fmha_decode_fwd_uniform_fast) or
fastcu (fmha_decode_fwd_fast).  bf16 N(0, 1) inputs; all batches have S rows.
"""
import argparse
import json
import math
import os
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)


def budget_shapes():
    """The shapes of --preset budget."""
    sh = []
    for g in (3, 4):
        sh += [f"30720:{16 * g}:16:{s}:128" for s in (1, 2, 3, 4, 6, 8, 12, 16)]
    for g in (3, 4):
        sh += [f"30720:{8 * g}:8:{s}:64" for s in (1, 2, 3, 4, 6, 8, 12, 16)]
        sh += [f"15360:{8 * g}:8:{s}:256" for s in (1, 2, 3, 4, 6, 8, 12, 16)]
    for g in (5, 6, 7, 8):
        sh += [f"30720:{8 * g}:8:{s}:64" for s in (1, 2, 4, 6, 8, 12, 16)]
    for g in (5, 6, 8):
        sh += [f"15360:{8 * g}:8:{s}:256" for s in (2, 4, 6, 8, 12, 16)]
    for g in (5, 8):
        sh += [f"30720:{16 * g}:16:{s}:128" for s in (2, 4, 8, 16)]
    return ",".join(sh)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--shapes", default="")
    ap.add_argument("--preset", choices=["budget"], default=None)
    ap.add_argument("--caps", default="3,4,5,6,7,8,10,12,16")
    ap.add_argument("--iters", type=int, default=10)
    ap.add_argument("--rounds", type=int, default=3)
    a = ap.parse_args()
    if a.preset == "budget":
        a.shapes = budget_shapes()
    if not a.shapes:
        ap.error("give --shapes or --preset")
    import torch
    import fmha_amd

    caps = [int(c) for c in a.caps.split(",")]
    dev = torch.device("cuda", 0)
    stream = torch.cuda.current_stream(dev)
    for spec in a.shapes.split(","):
        f = spec.split(":")
        B, hq, hkv, S, D = (int(x) for x in f[:5])
        mode = f[5] if len(f) > 5 else "uniform"
        g = torch.Generator(device=dev).manual_seed(B + hq + S + D)
        q = torch.randn(B, hq, 1, D, generator=g, device=dev, dtype=torch.bfloat16)
        k = torch.randn(B * S, hkv, D, generator=g, device=dev, dtype=torch.bfloat16)
        v = torch.randn(B * S, hkv, D, generator=g, device=dev, dtype=torch.bfloat16)
        o = torch.empty(B, hq, 1, D, device=dev, dtype=torch.float16)
        cu = torch.arange(0, (B + 1) * S, S, dtype=torch.int32, device=dev)
        scale = 1.0 / math.sqrt(D)
        fast = mode in ("fast", "fastcu")
        if mode in ("cu", "fastcu"):
            def call():
                fmha_amd.fmha_decode(q, k, v, cu_seqlens_kv=cu, softmax_scale=scale, out=o, fast=fast)
        else:
            def call():
                fmha_amd.fmha_decode(q, k, v, seqlen_kv=S, softmax_scale=scale, out=o, fast=fast)

        def timed():
            for _ in range(3):
                call()
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record(stream)
            for _ in range(a.iters):
                call()
            e1.record(stream)
            e1.synchronize()
            return e0.elapsed_time(e1) * 1e3 / a.iters

        res = {}
        model_cap = None
        for _ in range(a.rounds):
            for c in caps + [0]:
                if c:
                    os.environ["FMHA_DECODE_WAVE_CAP"] = str(c)
                else:
                    os.environ.pop("FMHA_DECODE_WAVE_CAP", None)
                us = timed()
                res.setdefault(c, []).append(us)
                if not c:
                    plan = fmha_amd.last_plan()
                    fields = dict(kv.split("=", 1) for kv in plan[-1].partition("(")[2].rstrip(")").split() if "=" in kv)
                    model_cap = int(fields.get("waves_per_cu", 0))
        os.environ.pop("FMHA_DECODE_WAVE_CAP", None)
        best = {c: round(min(t), 1) for c, t in res.items() if c}
        model_us = round(min(res[0]), 1)
        best_cap = min(best, key=best.get)
        nbytes = 2 * B * hq * D * 2 + 2 * B * S * hkv * D * 2
        print(json.dumps({"shape": [B, hq, hkv, S, D], "mode": mode, "us_by_cap": best, "model_cap": model_cap,
                          "model_us": model_us, "best_cap": best_cap, "best_us": best[best_cap],
                          "model_over_best": round(model_us / best[best_cap], 4),
                          "best_tb_s": round(nbytes / best[best_cap] / 1e6, 3), "plan": fmha_amd.last_plan()}),
              flush=True)
        del q, k, v, o, cu, call
        torch.cuda.empty_cache()


if __name__ == "__main__":
    main()
