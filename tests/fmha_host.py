#!/usr/bin/env python3
"""Host benchmark and validation driver for the decode-attention library --
the counterpart of the reference's `./fmha [config_index]` (fmha_host.cpp:
477-533), run by validate.sh and run_rocprof.sh.

It lives under tests/ because it validates against the CPU oracle.  For each
selected configuration it:
  * builds seeded inputs on the GPU (N(0, std) rounded to bf16), with every
    length taken from the configuration (uniform) or from the reference's
    own generator (Poisson(4) rejected outside [2, max], mt19937(42),
    fmha_host.cpp:58-72) for the reference-suite configurations;
  * times `--iters` calls (HIP events per call on the launch stream, after
    at least `--warmup` calls and 0.1 s of them, tests/common.py: gpu_warmup;
    with --rotate N, N input sets used in turn so that a
    small configuration is not served from the 256 MB MALL) and reports
    µs/call, algorithmic TB/s and % of the 8 TB/s HBM peak, counting bytes
    as fmha_host.cpp:428-430 does;
  * zeroes O, runs once more and checks the whole output against the oracle
    with the gate in tests/common.py (or a seeded sample of batches);
  * prints one JSON line per configuration and exits non-zero if any check
    fails (the reference always exits 0, fmha_host.cpp:532).

Suites:
  baseline   C1..C5 of BASELINE.json (uniform lengths), indices 1..5
  reference  the reference's own table (fmha_host.cpp:511-517): index 0 is
             B=10, H=16, D=128; 1..4 are B=30720 with H in {16, 32} and
             D in {128, 256}; all with Poisson lengths in [2, 16]
  gqa        full-size group sizes outside {1, 2, 4, 8} (the reference has
             no GQA): G = 3, 5, 7, 12, MQA G = 32, G = 5 with Poisson
             lengths, G = 6 at D = 256 with std 2, G = 5 at D = 64; the
             library's kernel choice runs 4 and 5 (G > 8) on the
             matrix-core kernel and 1, 2, 3, 6, 7, 8 on the VALU kernel's
             padded 4- and 8-head instantiations
"""
import argparse
import json
import math
import os
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)

HBM_PEAK_TBS = 8.0

# name: (B, Hq, Hkv, S or None for Poisson lengths, D, std)
SUITES = {
    "baseline": {
        1: (30720, 16, 16, 1, 128, 1.0),
        2: (30720, 16, 16, 16, 128, 1.0),
        3: (30720, 16, 16, 5, 256, 1.0),
        4: (30720, 32, 16, 16, 128, 1.0),
        5: (30720, 32, 32, 16, 256, 2.0),
    },
    "reference": {
        0: (10, 16, 16, None, 128, 1.0),
        1: (30720, 16, 16, None, 128, 1.0),
        2: (30720, 16, 16, None, 256, 1.0),
        3: (30720, 32, 32, None, 128, 1.0),
        4: (30720, 32, 32, None, 256, 1.0),
    },
    "gqa": {
        1: (30720, 48, 16, 16, 128, 1.0),
        2: (30720, 80, 16, 16, 128, 1.0),
        3: (30720, 112, 16, 16, 128, 1.0),
        4: (30720, 192, 16, 16, 128, 1.0),
        5: (30720, 32, 1, 16, 128, 1.0),
        6: (30720, 40, 8, None, 128, 1.0),
        7: (15360, 48, 8, 16, 256, 2.0),
        8: (30720, 40, 8, 16, 64, 1.0),
    },
}

SEED_OFFSET = {"baseline": 0, "reference": 8, "gqa": 12}


def algorithmic_bytes(B, Hq, Hkv, rows, D):
    return 2 * B * Hq * D + 2 * 2 * rows * Hkv * D + 2 * B * Hq * D


def run_config(suite, idx, args):
    import numpy as np
    import torch

    import fmha_amd
    import oracle
    from tests.common import ATOL, RTOL, gpu_warmup

    B, Hq, Hkv, S, D, std = SUITES[suite][idx]
    dev = torch.device("cuda", 0)
    if S is None:
        seqlens = oracle.generate_seqlens(B, 16)
    else:
        seqlens = np.full(B, S, np.int32)
    cu_h = np.concatenate([[0], np.cumsum(seqlens)]).astype(np.int32)
    rows = int(cu_h[-1])
    seed = 0xF3A00000 + 16 * idx + SEED_OFFSET[suite]
    gen = torch.Generator(device=dev).manual_seed(seed)
    # --rotate N: N independent input/output sets used in turn, so that a
    # small configuration cannot be served from the 256 MB MALL between calls.
    sets = []
    for _ in range(max(1, args.rotate)):
        q = torch.randn(B, Hq, 1, D, generator=gen, device=dev, dtype=torch.bfloat16)
        k = torch.randn(rows, Hkv, D, generator=gen, device=dev, dtype=torch.bfloat16)
        v = torch.randn(rows, Hkv, D, generator=gen, device=dev, dtype=torch.bfloat16)
        if std != 1.0:
            q.mul_(std), k.mul_(std), v.mul_(std)
        o = torch.empty(B, Hq, 1, D, device=dev, dtype=torch.float16)
        sets.append((q, k, v, o))
    q, k, v, o = sets[0]
    cu = torch.from_numpy(cu_h).to(dev)
    scale = 1.0 / math.sqrt(D)
    stream = torch.cuda.current_stream(dev)
    sp = stream.cuda_stream
    uniform = S is not None and not args.varlen

    def call(i=0):
        qq, kk, vv, oo = sets[i % len(sets)]
        if uniform:
            fmha_amd.launch_fmha_decode_uniform(sp, qq.data_ptr(), kk.data_ptr(), vv.data_ptr(), oo.data_ptr(),
                                                S, B, Hq, Hkv, 1, D, D, scale)
        else:
            fmha_amd.launch_fmha_decode(sp, qq.data_ptr(), kk.data_ptr(), vv.data_ptr(), oo.data_ptr(),
                                        cu.data_ptr(), B, Hq, Hkv, 1, D, D, scale)

    n_warm = [0]

    def warm_call():
        call(n_warm[0])
        n_warm[0] += 1

    gpu_warmup(warm_call, min_calls=args.warmup)
    ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
          for _ in range(args.iters)]
    for i, (a, b) in enumerate(ev):
        a.record(stream)
        call(i)
        b.record(stream)
    torch.cuda.synchronize()
    per = sorted(a.elapsed_time(b) * 1e3 for a, b in ev)  # µs
    mean_us = sum(per) / len(per)
    med_us = per[len(per) // 2]
    nbytes = algorithmic_bytes(B, Hq, Hkv, rows, D)
    res = {
        "suite": suite, "config": idx, "batch": B, "num_heads_q": Hq, "num_heads_kv": Hkv,
        "seqlen_kv": S if S is not None else "poisson(4) in [2,16]", "head_dim": D, "std": std,
        "path": "uniform" if uniform else "cu_seqlens", "rows": rows, "bytes_per_call": nbytes,
        "input_sets": len(sets),
        "us_per_call_median": round(med_us, 2), "us_per_call_mean": round(mean_us, 2),
        "tb_s_median": round(nbytes / (med_us * 1e-6) / 1e12, 4),
        "pct_of_peak_median": round(100 * nbytes / (med_us * 1e-6) / 1e12 / HBM_PEAK_TBS, 2),
    }

    if args.validate != "none":
        o.zero_()
        call()
        torch.cuda.synchronize()
        bits = lambda t: t.contiguous().view(torch.int16).cpu().numpy().view(np.uint16)
        if args.validate == "full" or B <= 1024:
            sel = np.arange(B)
            qs, os_ = bits(q.view(B, Hq, D)), bits(o.view(B, Hq, D))
            ks, vs, cus = bits(k), bits(v), cu_h
        else:
            rng = np.random.default_rng(idx)
            sel = np.unique(np.concatenate([[0, B - 1], rng.choice(B, 512, replace=False)]))
            idx_t = torch.from_numpy(sel).to(dev)
            qs, os_ = bits(q.view(B, Hq, D)[idx_t]), bits(o.view(B, Hq, D)[idx_t])
            parts_k, parts_v = [], []
            for b in sel:
                parts_k.append(k[cu_h[b]:cu_h[b + 1]])
                parts_v.append(v[cu_h[b]:cu_h[b + 1]])
            ks, vs = bits(torch.cat(parts_k)), bits(torch.cat(parts_v))
            cus = np.concatenate([[0], np.cumsum(seqlens[sel])]).astype(np.int32)
        r, slack = oracle.decode(qs, ks, vs, cus, Hq, Hkv, D, scale, with_slack=True)
        st = oracle.compare(os_, r, slack, ATOL, RTOL)
        ok = st["fails"] == 0 and st["ref_rule_fails"] == 0 and st["nonfinite"] == 0
        res["validation"] = {"batches_checked": int(len(sel)), "passed": ok,
                             **{k_: st[k_] for k_ in ("n", "fails", "ref_rule_fails", "ref_rule_fails_raw", "nonfinite",
                                                      "slack_elems", "max_abs", "max_rel")}}
    return res


def main():
    ap = argparse.ArgumentParser(description="decode-attention benchmark + validation")
    ap.add_argument("config", nargs="?", default="all", help="config index or 'all'")
    ap.add_argument("--suite", choices=sorted(SUITES), default="baseline")
    ap.add_argument("--iters", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--validate", choices=["full", "sample", "none"], default="sample")
    ap.add_argument("--rotate", type=int, default=1,
                    help="independent input sets used in turn (defeats MALL residency for small configs)")
    ap.add_argument("--varlen", action="store_true",
                    help="launch uniform configurations through the cu_seqlens entry point")
    args = ap.parse_args()
    suite = SUITES[args.suite]
    idxs = sorted(suite) if args.config == "all" else [int(args.config)]
    for i in idxs:
        if i not in suite:
            sys.exit(f"config {i} is not in suite {args.suite} ({sorted(suite)})")
    failed = False
    for i in idxs:
        res = run_config(args.suite, i, args)
        print(json.dumps(res), flush=True)
        if "validation" in res and not res["validation"]["passed"]:
            failed = True
    sys.exit(1 if failed else 0)


if __name__ == "__main__":
    main()
