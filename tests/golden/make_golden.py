#!/usr/bin/env python3
"""Writes the golden fixtures in tests/golden/ (run where /root/reference is
mounted and `make -C oracle` has built oracle/_ref).

Every expected output here is produced by the reference's own code or by an
independent library routine, never by the oracle under test:
  * seqlens_ref.json: the reference's length generator
    (FMHAConfig::generate_seqlens_kv, fmha_host.cpp:58-72) for batch 64, max 16;
  * mha_*.npz: inputs plus the fp16 output of the reference's CPU loop
    (do_validation, fmha_host.cpp:158-284), for MHA shapes where its indexing
    is correct;
  * gqa_sdpa_*.npz: inputs plus torch.nn.functional.scaled_dot_product_attention
    in float64 on the CPU (K/V heads repeated per group), the float64 truth for
    grouped-query shapes, which the reference cannot produce (it indexes K/V
    with the query head, fmha_host.cpp:190-192).
Inputs are seeded N(0, 1) rounded to bf16; uint16 arrays hold bit patterns.
"""
import json
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)


def bf16_normal(rng, shape, std=1.0):
    import torch
    x = torch.from_numpy(rng.standard_normal(shape).astype(np.float32) * np.float32(std))
    return x.to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)


def main():
    import torch
    import oracle
    if not oracle.ref_available():
        sys.exit("oracle/_ref/libfmha_ref.so is not built (needs /root/reference; make -C oracle)")

    seq = oracle.ref_generate_seqlens(64, 16)
    with open(os.path.join(HERE, "seqlens_ref.json"), "w") as f:
        json.dump({"source": "fmha_host.cpp:58-72 generate_seqlens_kv, batch=64, max_seqlen_kv=16",
                   "seqlens": [int(x) for x in seq]}, f)

    rng = np.random.default_rng(20261201)
    mha_cases = [("mha_d128_varlen", 6, 4, 128, list(seq[:6]), 1.0),
                 ("mha_d256_s5", 3, 4, 256, [5, 5, 5], 1.0),
                 ("mha_d128_s1_s16", 4, 2, 128, [1, 16, 1, 16], 2.0)]
    for name, B, H, D, seqlens, std in mha_cases:
        cu = np.concatenate([[0], np.cumsum(seqlens)]).astype(np.int32)
        q = bf16_normal(rng, (B, H, D), std)
        k = bf16_normal(rng, (int(cu[-1]), H, D), std)
        v = bf16_normal(rng, (int(cu[-1]), H, D), std)
        ref_o, _ = oracle.ref_do_validation(q, k, v, cu, H, H, D)
        np.savez(os.path.join(HERE, name + ".npz"), q=q, k=k, v=v, cu=cu, o=ref_o,
                 meta=np.array([B, H, H, D], np.int32))

    gqa_cases = [("gqa_sdpa_g2_d128", 3, 4, 2, 128, [3, 16, 7]),
                 ("gqa_sdpa_g4_d64", 2, 8, 2, 64, [16, 1]),
                 # group sizes outside {1, 2, 4, 8} (the matrix-core kernel's)
                 ("gqa_sdpa_g5_d128", 3, 10, 2, 128, [16, 5, 1]),
                 ("gqa_sdpa_g3_d256", 2, 6, 2, 256, [9, 16])]
    for name, B, Hq, Hkv, D, seqlens in gqa_cases:
        cu = np.concatenate([[0], np.cumsum(seqlens)]).astype(np.int32)
        q = bf16_normal(rng, (B, Hq, D))
        k = bf16_normal(rng, (int(cu[-1]), Hkv, D))
        v = bf16_normal(rng, (int(cu[-1]), Hkv, D))
        f = lambda a: torch.from_numpy(a.astype(np.uint32) << 16).view(torch.float32).double()
        out = np.zeros((B, Hq, D), np.float64)
        for b in range(B):
            kb = f(k[cu[b]:cu[b + 1]]).repeat_interleave(Hq // Hkv, dim=1).transpose(0, 1)  # [Hq, S, D]
            vb = f(v[cu[b]:cu[b + 1]]).repeat_interleave(Hq // Hkv, dim=1).transpose(0, 1)
            qb = f(q[b]).unsqueeze(1)                                                     # [Hq, 1, D]
            o = torch.nn.functional.scaled_dot_product_attention(qb, kb, vb, scale=1.0 / np.sqrt(D))
            out[b] = o[:, 0, :].numpy()
        np.savez(os.path.join(HERE, name + ".npz"), q=q, k=k, v=v, cu=cu, o=out,
                 meta=np.array([B, Hq, Hkv, D], np.int32))
    print("fixtures written to", HERE)


if __name__ == "__main__":
    main()
