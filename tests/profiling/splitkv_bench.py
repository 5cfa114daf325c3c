#!/usr/bin/env python3
"""Timing of the split-KV entry point (fmha_decode_fwd_splitkv) on
long-context shapes, for the profile under profiles/.

For each shape (uniform lengths, bf16 N(0,1) inputs on the GPU), calls the
library at least --warmup times and for at least 0.1 s (tests/common.py:
gpu_warmup), then times --iters calls with a HIP event pair per
call on the launch stream and prints one JSON line: median µs per call and
algorithmic TB/s (Q + K + V + O as the reference counts them,
fmha_host.cpp:428-430, with Hkv heads for K/V), the plan the library reports
for the call (fmha_decode_last_plan) and the bytes that plan moves through
the workspace (workspace_traffic_bytes, counted apart).  Run it under
`rocprofv3 --kernel-trace --stats` for the per-kernel split
(run_rocprof.sh's s:... workloads).

    python3 tests/profiling/splitkv_bench.py [--iters N] [--shapes B:Hq:Hkv:S:D,... | --preset layouts]
        [--layout packed|bhsd|pagedN]

--preset layouts: 85 shapes for comparing layouts, B sized for about 512 MB
of K and V: D = 128 with Hq/Hkv 8/8, 32/8, 64/8, 128/8, 4/1, 8/1, 16/2 and
D = 64, 256 with 8/8, 32/8, 64/8, 4/1, 8/1, each at S = 24, 48, 128, 512,
4096.

--layout bhsd stores K/V as [B, Hkv, S, D] (fmha_decode_strided on the
transposed view); pagedN as pages of N rows handed out in a random order
with an [B, S/N] block table (fmha_decode_paged with max_seqlen_kv = S).
S <= 16 then runs the short kernels of those layouts.
"""
import argparse
import json
import math
import os
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)

from tests.common import gpu_warmup  # noqa: E402

# Long rows over few sequences (split path), many sequences of 24-256 rows
# (single pass; the last one below its threshold), and the 16-row headline
# batch through this entry point (short kernel).
SHAPES = [(64, 32, 8, 4096, 128), (8, 32, 8, 32768, 128), (256, 64, 8, 1024, 128), (1, 32, 8, 131072, 128),
          (2048, 32, 8, 128, 128), (4096, 32, 8, 64, 128), (16384, 32, 8, 24, 128), (8192, 16, 16, 64, 128),
          (512, 32, 8, 128, 128), (256, 32, 8, 256, 128), (128, 32, 8, 256, 128), (30720, 16, 16, 16, 128)]


def layout_shapes():
    """The shapes of --preset layouts."""
    heads = [(128, h) for h in ((8, 8), (32, 8), (64, 8), (128, 8), (4, 1), (8, 1), (16, 2))]
    heads += [(d, h) for d in (64, 256) for h in ((8, 8), (32, 8), (64, 8), (4, 1), (8, 1))]
    shapes = []
    for D, (hq, hkv) in heads:
        for S in (24, 48, 128, 512, 4096):
            B = max(1, round(512e6 / (S * hkv * D * 4)))
            shapes.append((B, hq, hkv, S, D))
    return shapes


def workspace_traffic(plan, B, hq, hkv, D):
    """Bytes the split-KV passes move through the workspace per call, from the
    plan the library reports: the scores T (written by the scores pass, read
    by P.V), the per-block max and sum (written, read by the statistics
    pass), the per-head max and sum (written, read by P.V) and, with more
    than one chunk per row, the fp32 partial outputs (written by P.V, read by
    the combine).  0 for the single pass and the short kernels."""
    total = 0
    for entry in plan:
        kind, _, rest = entry.partition("(")
        if kind not in ("split", "split_matrix_core"):
            continue
        f = dict(kv.split("=") for kv in rest.rstrip(")").split())
        heads = B * max(hq, hkv * int(f["G"]))
        nblk, chunks = int(f["blocks"]), int(f["chunks"])
        total += 2 * heads * nblk * 16 * 4 + 2 * 2 * heads * nblk * 4 + 2 * heads * 2 * 4
        if chunks > 1:
            total += 2 * heads * chunks * D * 4
    return total


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--iters", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--shapes", default="")
    ap.add_argument("--preset", choices=["layouts"], default=None)
    ap.add_argument("--layout", default="packed")
    a = ap.parse_args()
    import torch
    import fmha_amd

    if a.preset == "layouts":
        shapes = layout_shapes()
    else:
        shapes = [tuple(int(x) for x in s.split(":")) for s in a.shapes.split(",")] if a.shapes else SHAPES
    dev = torch.device("cuda", 0)
    stream = torch.cuda.current_stream(dev)
    for B, hq, hkv, S, D in shapes:
        g = torch.Generator(device=dev).manual_seed(B * 7 + S)
        q = torch.randn(B, hq, 1, D, generator=g, device=dev, dtype=torch.bfloat16)
        k = torch.randn(B * S, hkv, D, generator=g, device=dev, dtype=torch.bfloat16)
        v = torch.randn(B * S, hkv, D, generator=g, device=dev, dtype=torch.bfloat16)
        cu = torch.arange(0, (B + 1) * S, S, dtype=torch.int32, device=dev)
        o = torch.empty(B, hq, 1, D, device=dev, dtype=torch.float16)
        ws = torch.empty(max(fmha_amd.splitkv_workspace_size(B, hq, hkv, S, D), 1), dtype=torch.uint8, device=dev)
        scale = 1.0 / math.sqrt(D)

        if a.layout == "packed":
            def call():
                fmha_amd.fmha_decode_splitkv(q, k, v, cu, S, softmax_scale=scale, out=o, workspace=ws)
        elif a.layout == "bhsd":
            kt = k.view(B, S, hkv, D).transpose(1, 2).contiguous().transpose(1, 2)
            vt = v.view(B, S, hkv, D).transpose(1, 2).contiguous().transpose(1, 2)
            del k, v

            def call():
                fmha_amd.fmha_decode_strided(q, kt, vt, softmax_scale=scale, out=o, workspace=ws)
        elif a.layout.startswith("paged"):
            ps = int(a.layout[5:])
            npg = B * ((S + ps - 1) // ps)
            perm = torch.randperm(npg, generator=torch.Generator().manual_seed(S)).to(torch.int32)
            bt = perm.view(B, -1).to(dev)
            kc = torch.zeros(npg, ps, hkv, D, device=dev, dtype=torch.bfloat16)
            vc = torch.zeros(npg, ps, hkv, D, device=dev, dtype=torch.bfloat16)
            rows = torch.arange(B * S, device=dev)
            b_of, j_of = rows // S, rows % S
            page = bt[b_of, j_of // ps].long()
            kc[page, j_of % ps] = k
            vc[page, j_of % ps] = v
            del k, v, rows, b_of, j_of, page
            lens = torch.full((B,), S, dtype=torch.int32, device=dev)

            def call():
                fmha_amd.fmha_decode_paged(q, kc, vc, bt, lens, softmax_scale=scale, out=o,
                                           max_seqlen_kv=S, workspace=ws)
        else:
            raise SystemExit(f"unknown layout {a.layout}")

        gpu_warmup(call, min_calls=a.warmup)
        ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(a.iters)]
        for e0, e1 in ev:
            e0.record(stream)
            call()
            e1.record(stream)
        torch.cuda.synchronize()
        per = sorted(e0.elapsed_time(e1) * 1e3 for e0, e1 in ev)
        med = per[len(per) // 2]
        nbytes = 2 * B * hq * D * 2 + 4 * B * S * hkv * D
        plan = fmha_amd.last_plan()
        print(json.dumps({"layout": a.layout, "B": B, "Hq": hq, "Hkv": hkv, "S": S, "D": D,
                          "us_per_call_median": round(med, 1),
                          "tb_s": round(nbytes / med / 1e6, 3), "workspace_bytes": ws.numel(), "plan": plan,
                          "workspace_traffic_bytes": workspace_traffic(plan, B, hq, hkv, D)}), flush=True)
        del q, o, ws, call
        torch.cuda.empty_cache()


if __name__ == "__main__":
    main()
