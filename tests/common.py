"""Shared helpers for the tests: seeded inputs, launching through the C ABI,
checking against the oracle with the documented gate.

Gate (written here, used by every parity test): an output element o passes
against the oracle value r when

    |o - r| <= ATOL + RTOL * |r| + slack

with ATOL = 2e-3, RTOL = 1e-2 (read allclose-style)
and slack = sum_j |bf16(p_j(1+eps)) - bf16(p_j(1-eps))| * |V_jd|: non-zero
only where a softmax weight sits next to a bf16 rounding midpoint, where any
float32 difference flips the reference's bf16 rounding of that weight
(fmha_host.cpp:225) by one bf16 step.  eps is computed per head by the oracle:
max(2^-19, 4 * (2 * max_j |t_j - t_j exact| + |L - L exact| / L)), i.e. four
times the oracle's own float32 error in the scores t and the normaliser L
against float64 -- an implementation summing in another order is uncertain by
about as much.  The reference's own rule |o - r| <= 1e-2 + 1e-2|r|
(fmha_host.cpp:260) is required with the same slack; its count without slack
is reported (ref_rule_fails_raw).
"""
import math

import numpy as np

import oracle

ATOL = 2e-3
RTOL = 1e-2

# (B, Hq, Hkv, S, D, std)
CONFIGS = {
    1: (30720, 16, 16, 1, 128, 1.0),
    2: (30720, 16, 16, 16, 128, 1.0),
    3: (30720, 16, 16, 5, 256, 1.0),
    4: (30720, 32, 16, 16, 128, 1.0),
    5: (30720, 32, 32, 16, 256, 2.0),
}


def default_scale(d):
    # fmha_host.cpp:371 passes 1.0f / sqrt(head_dim); in float32 this equals
    # 1.0f / sqrtf(head_dim) (fmha_host.cpp:211) for every supported D.
    return float(np.float32(1.0) / np.sqrt(np.float32(d)))


def cu_from_seqlens(seqlens):
    return np.concatenate([[0], np.cumsum(np.asarray(seqlens, dtype=np.int64))]).astype(np.int32)


def bf16_normal(shape, gen, std=1.0):
    """Seeded N(0, std) rounded to bf16 (torch RNE), as uint16 bits."""
    import torch
    x = torch.randn(*shape, generator=gen, dtype=torch.float32) * std
    return x.to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)


def make_inputs(B, Hq, Hkv, D, seqlens, seed, std=1.0):
    import torch
    gen = torch.Generator().manual_seed(seed)
    cu = cu_from_seqlens(seqlens)
    rows = int(cu[-1])
    q = bf16_normal((B, Hq, D), gen, std)
    k = bf16_normal((rows, Hkv, D), gen, std)
    v = bf16_normal((rows, Hkv, D), gen, std)
    return q, k, v, cu


def to_dev(bits, device="cuda"):
    import torch
    t = torch.from_numpy(np.ascontiguousarray(bits).view(np.int16)).to(device)
    return t.view(torch.bfloat16)


def run_gpu(q, k, v, cu, Hq, Hkv, D, scale=None, uniform_s=None, device="cuda", fast=False, exact=False):
    """Launch the HIP kernel through the C ABI (fmha_decode_fwd, or
    fmha_decode_fwd_uniform with uniform_s; their _fast forms with fast;
    fmha_decode_fwd_exact with exact); returns O as fp16 bits."""
    import torch
    import fmha_amd
    scale = default_scale(D) if scale is None else scale
    B = q.shape[0]
    qd, kd, vd = to_dev(q, device), to_dev(k, device), to_dev(v, device)
    if uniform_s is None:
        cud = torch.from_numpy(np.ascontiguousarray(cu)).to(device)
        o = fmha_amd.fmha_decode(qd, kd, vd, cu_seqlens_kv=cud, softmax_scale=scale, fast=fast, exact=exact)
    else:
        o = fmha_amd.fmha_decode(qd, kd.view(B, uniform_s, Hkv, D), vd.view(B, uniform_s, Hkv, D),
                                 seqlen_kv=uniform_s, softmax_scale=scale, fast=fast)
    torch.cuda.synchronize()
    return o.view(torch.int16).cpu().numpy().view(np.uint16)


def last_plan():
    """The launches of the most recent library call on this thread, as the
    library reports them (fmha_decode_last_plan): [(kind, {key: int or
    str})], e.g. ("onepass", {"D": 128, "G": 8, "layout": "paged16_lanes",
    ...})."""
    import fmha_amd
    out = []
    for entry in fmha_amd.last_plan():
        kind, _, rest = entry.partition("(")
        fields = {}
        for kv in rest.rstrip(")").split():
            key, _, val = kv.partition("=")
            fields[key] = int(val) if val.lstrip("-").isdigit() else val
        out.append((kind, fields))
    return out


def plan_kinds():
    """The kernel kinds of the most recent call, in launch order."""
    return [k for k, _ in last_plan()]


def plan_launch(kind):
    """The fields of the one launch of this kind in the most recent call."""
    found = [f for k, f in last_plan() if k == kind]
    assert len(found) == 1, f"expected one {kind} launch, plan: {last_plan()}"
    return found[0]


def check(o, q, k, v, cu, Hq, Hkv, D, scale=None):
    """Compare GPU output bits with the oracle; returns the stats dict."""
    scale = default_scale(D) if scale is None else scale
    r, slack = oracle.decode(q, k, v, cu, Hq, Hkv, D, scale, p_mode=0, with_slack=True)
    st = oracle.compare(o.reshape(r.shape), r, slack, ATOL, RTOL)
    return st


def assert_exact(o, q, k, v, cu, Hq, Hkv, D, ctx="", scale=None):
    """o (fp16 bits) equals the oracle's restated reference loop with
    nearest-float exponentials (oracle.decode(p_mode=2)) bit for bit: the
    numerics of the default entry points up to 2 query heads per KV head,
    and of fmha_decode_fwd_exact."""
    scale = default_scale(D) if scale is None else scale
    r, _ = oracle.decode(q, k, v, cu, Hq, Hkv, D, scale, p_mode=2)
    diff = int(np.count_nonzero(np.asarray(o).reshape(r.shape) != r))
    assert diff == 0, f"{ctx}: {diff} of {r.size} outputs differ from the restated loop (p_mode=2)"


def check_entry_points(q, k, v, cu, Hq, Hkv, D, uniform_s=None, ctx=""):
    """Both numerics on the same inputs: the default entry point (bit for
    bit against the restated loop up to 2 query heads per KV head, through
    the gate above that) and the _fast one (through the gate).  Returns the
    default entry point's output bits."""
    o = run_gpu(q, k, v, cu, Hq, Hkv, D, uniform_s=uniform_s)
    if Hq // Hkv <= 2:
        assert_exact(o, q, k, v, cu, Hq, Hkv, D, ctx + " (default)")
    else:
        assert_pass(check(o, q, k, v, cu, Hq, Hkv, D), ctx + " (default)")
    of = run_gpu(q, k, v, cu, Hq, Hkv, D, uniform_s=uniform_s, fast=True)
    assert_pass(check(of, q, k, v, cu, Hq, Hkv, D), ctx + " (fast)")
    return o


def assert_pass(st, ctx=""):
    assert st["nonfinite"] == 0, f"{ctx}: non-finite outputs {st}"
    assert st["fails"] == 0, f"{ctx}: gate failures {st}"
    assert st["ref_rule_fails"] == 0, f"{ctx}: reference-rule failures {st}"


def f64_bound(q, k, v, cu, Hq, Hkv, D, scale=None):
    """float64 truth t [B,Hq,D] and a per-element bound on |o - t| that any
    bf16-weight implementation with float32 arithmetic meets, with no tie
    slack (the bf16 rounding of a weight may go either way): 2^-8 M (the
    weights' bf16 rounding, M = max_j |V_jd|) + 2 dt M (float32 scores) +
    2^-10 |t| (the fp16 output) + 1e-5 (1 + M) (float32 sums); the oracle
    computes it beside t (head_f64 in oracle/fmha_oracle.cpp)."""
    scale = default_scale(D) if scale is None else scale
    seqlens = np.diff(np.asarray(cu, dtype=np.int64))
    return oracle.decode_f64(q, k, v, cu, Hq, Hkv, D, scale, max_seqlen=int(seqlens.max(initial=0)),
                             with_bound=True)


def f64_check(o_bits, t, bound):
    """Elements of o (fp16 bits) outside t +- bound, and the largest
    |o - t| / bound."""
    o = oracle.f16_to_f32(np.asarray(o_bits).reshape(t.shape)).astype(np.float64)
    err = np.abs(o - t)
    err[~np.isfinite(o)] = np.inf
    return {"f64_violations": int((err > bound).sum()), "f64_max_ratio": float((err / bound).max()),
            "f64_max_abs": float(err.max()), "f64_mean_abs": float(err.mean())}


def gpu_warmup(call, min_calls=10, min_seconds=0.1):
    """Untimed calls until at least min_calls have run and min_seconds of
    wall time have passed, synchronising every 16 calls.  A GPU that has
    just started working runs short kernels slower for its first tens of
    milliseconds (Hq=40 Hkv=8 with Poisson lengths, about 0.2 ms per call:
    70.8% of peak after 10 warm-up calls, 81.1% after 200 and 81.4% after
    2000), so a count alone under-warms short kernels."""
    import time

    import torch
    t0 = time.perf_counter()
    n = 0
    while n < min_calls or time.perf_counter() - t0 < min_seconds:
        call()
        n += 1
        if n % 16 == 0:
            torch.cuda.synchronize()
    torch.cuda.synchronize()
    return n
