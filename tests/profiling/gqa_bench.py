#!/usr/bin/env python3
"""Timing of the short-KV decode kernels across GQA group sizes, for the
profile under profiles/.

For each shape (uniform lengths, bf16 N(0,1) inputs generated on the GPU)
and each kernel choice (FMHA_DECODE_GQA_KERNEL=valu: the VALU kernel, for
G <= 8, G = 3 and 5-7 on its 4- and 8-head instantiations; =mfma: the
matrix-core kernel; default: the library's own choice), calls
fmha_decode_fwd_uniform at least --warmup times and for at least 0.1 s
(tests/common.py: gpu_warmup), then times --iters calls with a HIP
event pair per call on the launch stream, and prints one JSON line: median
µs per call and algorithmic TB/s (Q + K + V + O as the reference counts
them, fmha_host.cpp:428-430, with Hkv heads for K/V).  Run it under
`rocprofv3 --kernel-trace --stats` (or `--pmc ...`) for the per-kernel view.

    python3 tests/profiling/gqa_bench.py [--iters N] [--shapes B:Hq:Hkv:S:D,...] [--modes valu,mfma,default]
"""
import argparse
import json
import math
import os
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)

from tests.common import gpu_warmup  # noqa: E402

# Hkv = 16, S = 16, D = 128 (the headline batch) with G = 1..16, MQA, short
# rows, and the other head dims.
SHAPES = [(30720, 16 * g, 16, 16, 128) for g in (1, 2, 3, 4, 5, 6, 7, 8, 12, 16)] + [
    (30720, 32, 1, 16, 128), (30720, 64, 8, 4, 128), (30720, 48, 16, 8, 128), (30720, 48, 16, 4, 128),
    (30720, 112, 16, 8, 128), (30720, 112, 16, 2, 128), (30720, 24, 8, 16, 64), (30720, 40, 8, 16, 64),
    (30720, 56, 8, 16, 64), (15360, 24, 8, 16, 256), (15360, 48, 8, 16, 256)]


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--iters", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--shapes", default="")
    ap.add_argument("--modes", default="valu,mfma,default")
    a = ap.parse_args()
    import torch
    import fmha_amd

    shapes = [tuple(int(x) for x in s.split(":")) for s in a.shapes.split(",")] if a.shapes else SHAPES
    modes = a.modes.split(",")
    dev = torch.device("cuda", 0)
    stream = torch.cuda.current_stream(dev)
    for B, hq, hkv, S, D in shapes:
        g = torch.Generator(device=dev).manual_seed(B * 7 + hq)
        q = torch.randn(B, hq, 1, D, generator=g, device=dev, dtype=torch.bfloat16)
        k = torch.randn(B, S, hkv, D, generator=g, device=dev, dtype=torch.bfloat16)
        v = torch.randn(B, S, hkv, D, generator=g, device=dev, dtype=torch.bfloat16)
        o = torch.empty(B, hq, 1, D, device=dev, dtype=torch.float16)
        nbytes = 2 * B * hq * D * 2 + 2 * B * S * hkv * D * 2
        G = hq // hkv
        row = {"B": B, "Hq": hq, "Hkv": hkv, "G": G, "S": S, "D": D}
        for mode in modes:
            if mode == "valu" and G > 8:
                continue
            if mode == "default":
                os.environ.pop("FMHA_DECODE_GQA_KERNEL", None)
            else:
                os.environ["FMHA_DECODE_GQA_KERNEL"] = mode
            call = lambda: fmha_amd.fmha_decode(q, k, v, seqlen_kv=S, out=o)
            gpu_warmup(call, min_calls=a.warmup)
            times = []
            for _ in range(a.iters):
                e0 = torch.cuda.Event(enable_timing=True)
                e1 = torch.cuda.Event(enable_timing=True)
                e0.record(stream)
                call()
                e1.record(stream)
                e1.synchronize()
                times.append(e0.elapsed_time(e1) * 1000.0)
            times.sort()
            us = times[len(times) // 2]
            row[mode] = {"us": round(us, 1), "tb_s": round(nbytes / us / 1e6, 3)}
        os.environ.pop("FMHA_DECODE_GQA_KERNEL", None)
        print(json.dumps(row), flush=True)
        del q, k, v, o


if __name__ == "__main__":
    main()
