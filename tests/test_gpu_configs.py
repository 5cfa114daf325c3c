"""The five BASELINE.json configurations at full size on the GPU.

At B=30720 the whole oracle run is too slow for a test, so each config is
checked through size-independent properties plus the oracle on a seeded
sample of batches:
  * every output is finite;
  * the default entry points (fmha_decode_fwd_uniform, and fmha_decode_fwd
    with a cu_seqlens array) give identical bits;
  * on a seeded sample of batches (plus the first and last) they equal the
    oracle's restated reference loop (fmha_host.cpp:179-244, grouped-query
    head mapping, nearest-float exponentials: oracle.decode(p_mode=2)) bit
    for bit, with no gate and no slack;
  * the tree-order entry point (fmha_decode_fwd_uniform_fast) passes the
    gate against the oracle on the same sample (the gate is documented in
    tests/common.py), and both lie within the bf16-weight bound of float64
    truth, with no tie slack (tests/common.py: f64_bound);
  * config 1 (S=1): the whole output equals fp16(V) bit for bit.
"""
import numpy as np
import pytest

import oracle
from tests.common import CONFIGS, assert_pass, cu_from_seqlens, default_scale, f64_bound, f64_check

pytestmark = pytest.mark.gpu


def _gen(shape, seed, std, device):
    import torch
    g = torch.Generator(device=device).manual_seed(seed)
    x = torch.randn(*shape, generator=g, device=device, dtype=torch.bfloat16)
    return x * std if std != 1.0 else x


def _bits(t):
    import torch
    return t.contiguous().view(torch.int16).cpu().numpy().view(np.uint16)


@pytest.mark.parametrize("cfg", [1, 2, 3, 4, 5])
def test_baseline_config(cfg):
    import torch
    import fmha_amd
    B, Hq, Hkv, S, D, std = CONFIGS[cfg]
    dev = "cuda"
    print(f"config {cfg}: B={B} Hq={Hq} Hkv={Hkv} S={S} D={D} std={std}", flush=True)
    q = _gen((B, Hq, 1, D), 0xF3A00000 + 16 * cfg + 0, std, dev)
    k = _gen((B, S, Hkv, D), 0xF3A00000 + 16 * cfg + 1, std, dev)
    v = _gen((B, S, Hkv, D), 0xF3A00000 + 16 * cfg + 2, std, dev)
    scale = default_scale(D)
    o_u = fmha_amd.fmha_decode(q, k, v, seqlen_kv=S, softmax_scale=scale)
    cu = torch.arange(0, (B + 1) * S, S, dtype=torch.int32, device=dev)
    o_c = fmha_amd.fmha_decode(q, k.view(B * S, Hkv, D), v.view(B * S, Hkv, D), cu_seqlens_kv=cu,
                               softmax_scale=scale)
    o_f = fmha_amd.fmha_decode(q, k, v, seqlen_kv=S, softmax_scale=scale, fast=True)
    torch.cuda.synchronize()
    assert bool(torch.isfinite(o_u).all()) and bool(torch.isfinite(o_f).all())
    assert torch.equal(o_u.view(torch.int16), o_c.view(torch.int16))
    if S == 1:
        assert torch.equal(o_u.view(B, Hq, D), v.view(B, Hkv, D).to(torch.float16))
        assert torch.equal(o_f.view(B, Hq, D), v.view(B, Hkv, D).to(torch.float16))
    rng = np.random.default_rng(cfg)
    sample = np.unique(np.concatenate([[0, B - 1], rng.choice(B, size=192, replace=False)]))
    idx = torch.from_numpy(sample).to(dev)
    qs = _bits(q.view(B, Hq, D)[idx])
    ks = _bits(k[idx].reshape(-1, Hkv, D))
    vs = _bits(v[idx].reshape(-1, Hkv, D))
    os_ = _bits(o_u.view(B, Hq, D)[idx])
    of_ = _bits(o_f.view(B, Hq, D)[idx])
    cus = cu_from_seqlens(np.full(len(sample), S, np.int32))
    r2, _ = oracle.decode(qs, ks, vs, cus, Hq, Hkv, D, scale, p_mode=2)
    diff = int(np.count_nonzero(os_.reshape(r2.shape) != r2))
    print(f"config {cfg}: sampled {len(sample)} batches, default entry points: {diff} of {r2.size} outputs "
          f"differ from the restated loop", flush=True)
    assert diff == 0, f"config {cfg}: {diff} outputs differ from oracle p_mode=2"
    r, slack = oracle.decode(qs, ks, vs, cus, Hq, Hkv, D, scale, with_slack=True)
    st = oracle.compare(of_, r, slack)
    print(f"config {cfg}: sampled {len(sample)} batches, fast entry point: {st}", flush=True)
    assert_pass(st, f"config {cfg} (fast)")
    t, bound = f64_bound(qs, ks, vs, cus, Hq, Hkv, D, scale)
    for name, o in (("default", os_), ("fast", of_)):
        sf = f64_check(o, t, bound)
        print(f"config {cfg}: {name} entry point against float64, no slack: {sf}", flush=True)
        assert sf["f64_violations"] == 0, f"config {cfg} ({name}): outside the bf16-weight bound of float64: {sf}"
