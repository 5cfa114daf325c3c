"""GPU parity of the exact-arithmetic numerics: the reference CPU loop's
arithmetic step for step (fmha_host.cpp:179-244), extended to grouped-query
attention with KV head h / (Hq / Hkv).

These are the numerics of the default entry points (fmha_decode_fwd and
fmha_decode_fwd_uniform) up to 2 query heads per KV head, and of
fmha_decode_fwd_exact for every call (up to 8).  Their outputs must equal, bit for bit
and with no gate or slack, the oracle's bf16-weight loop with nearest-float
exponentials (oracle.decode(p_mode=2)); the loop with the C library's expf
(p_mode=0, the reference's own) then differs from it only through the few
exponentials that expf misrounds (tests/test_oracle.py pins that).
Covered: every length 0..16 through both entry points, head dims
64/128/256, group sizes 1-8 (3 and 5-7 on padded query groups), head counts
below and above what one wave holds (the R-batch kernel and the one-batch
kernel), logit spreads, invalid lengths (NaN), the rejected group sizes,
and BASELINE configurations at full size on a seeded sample of batches.
"""
import numpy as np
import pytest

import oracle
from tests.common import CONFIGS, cu_from_seqlens, default_scale, make_inputs, to_dev

pytestmark = pytest.mark.gpu


def _bits(t):
    import torch
    return t.contiguous().view(torch.int16).cpu().numpy().view(np.uint16)


def _run(q, k, v, cu, Hq, Hkv, D, out=None, entry="exact"):
    """O through fmha_decode_fwd_exact ("exact") or fmha_decode_fwd
    ("default"), fp16 bits."""
    import torch
    import fmha_amd
    o = fmha_amd.fmha_decode(to_dev(q), to_dev(k), to_dev(v), cu_seqlens_kv=torch.from_numpy(cu).cuda(),
                             softmax_scale=default_scale(D), out=out, exact=entry == "exact")
    torch.cuda.synchronize()
    return _bits(o)


def _run_uniform(q, k, v, S, D, fast=False):
    """O through fmha_decode_fwd_uniform (or its _fast form): K/V as
    [B, S, Hkv, D]."""
    import torch
    import fmha_amd
    B, Hq = q.shape[0], q.shape[1]
    Hkv = k.shape[1]
    kd = to_dev(k).view(B, S, Hkv, D)
    vd = to_dev(v).view(B, S, Hkv, D)
    o = fmha_amd.fmha_decode(to_dev(q), kd, vd, seqlen_kv=S, softmax_scale=default_scale(D), fast=fast)
    torch.cuda.synchronize()
    return _bits(o)


def _assert_bit_exact(o, q, k, v, cu, Hq, Hkv, D, ctx):
    r, _ = oracle.decode(q, k, v, cu, Hq, Hkv, D, default_scale(D), p_mode=2)
    o = o.reshape(r.shape)
    diff = int(np.count_nonzero(o != r))
    r0, _ = oracle.decode(q, k, v, cu, Hq, Hkv, D, default_scale(D), p_mode=0)
    print(f"{ctx}: {o.size} outputs, {diff} differ from the nearest-exp loop, "
          f"{int(np.count_nonzero(o != r0))} from the expf loop", flush=True)
    assert diff == 0, f"{ctx}: {diff} outputs differ from the oracle (p_mode=2)"


# (Hq, Hkv): one query head per KV head with few and many KV heads (the
# R-batch kernel below a wave's heads, the one-batch kernel above), then
# group sizes 2-8 likewise.
HEADS = [(1, 1), (2, 2), (16, 16), (32, 32), (2, 1), (8, 4), (32, 16), (3, 1), (12, 4), (48, 16), (4, 1),
         (64, 16), (5, 1), (40, 8), (6, 1), (7, 1), (56, 8), (8, 1), (64, 8), (128, 16)]


@pytest.mark.parametrize("D", [64, 128, 256])
@pytest.mark.parametrize("Hq,Hkv", HEADS)
def test_all_lengths_bit_exact(D, Hq, Hkv):
    seqlens = np.array(list(range(17)) * 3, dtype=np.int32)
    np.random.default_rng(D + 7 * Hq + Hkv).shuffle(seqlens)
    q, k, v, cu = make_inputs(len(seqlens), Hq, Hkv, D, seqlens, seed=900 + D + Hq + 3 * Hkv)
    print(f"exact: D={D} Hq={Hq} Hkv={Hkv} B={len(seqlens)}", flush=True)
    o = _run(q, k, v, cu, Hq, Hkv, D)
    _assert_bit_exact(o, q, k, v, cu, Hq, Hkv, D, f"D={D} Hq={Hq} Hkv={Hkv}")
    if Hq // Hkv <= 2:  # fmha_decode_fwd computes the same numerics there
        assert np.array_equal(_run(q, k, v, cu, Hq, Hkv, D, entry="default"), o)


@pytest.mark.parametrize("D", [64, 128, 256])
@pytest.mark.parametrize("Hq,Hkv", [(1, 1), (16, 16), (32, 32), (2, 1), (8, 4), (32, 16)])
@pytest.mark.parametrize("S", [0, 1, 2, 3, 5, 8, 9, 16])
def test_uniform_bit_exact(D, Hq, Hkv, S):
    """The uniform entry point (known-length kernels, one bucket per call;
    the R-batch kernel below a wave's heads) against the oracle on
    [B, S, Hkv, D] inputs, for the group sizes it takes these numerics for."""
    B = 37
    seqlens = np.full(B, S, np.int32)
    q, k, v, cu = make_inputs(B, Hq, Hkv, D, seqlens, seed=940 + D + Hq + S)
    print(f"exact uniform: D={D} Hq={Hq} Hkv={Hkv} S={S}", flush=True)
    o = _run_uniform(q, k, v, S, D)
    _assert_bit_exact(o, q, k, v, cu, Hq, Hkv, D, f"uniform D={D} Hq={Hq} Hkv={Hkv} S={S}")


@pytest.mark.parametrize("std", [0.25, 2.0, 4.0])
@pytest.mark.parametrize("D", [128, 256])
@pytest.mark.parametrize("Hq,Hkv", [(16, 16), (32, 16), (64, 16)])
def test_logit_spread_bit_exact(std, D, Hq, Hkv):
    seqlens = oracle.generate_seqlens(300, 16)
    q, k, v, cu = make_inputs(300, Hq, Hkv, D, seqlens, seed=910, std=std)
    print(f"exact: std={std} D={D} Hq={Hq} Hkv={Hkv}", flush=True)
    _assert_bit_exact(_run(q, k, v, cu, Hq, Hkv, D), q, k, v, cu, Hq, Hkv, D, f"std={std} D={D} Hq={Hq}")


@pytest.mark.parametrize("Hq,Hkv", [(2, 2), (16, 16), (4, 2), (32, 16), (24, 4)])
def test_invalid_lengths_give_nan(Hq, Hkv):
    """A length outside [0, 16] turns that batch's outputs into NaN; the
    other batches stay exact."""
    D = 128
    seqlens = np.array([5, 16, 3, 9, 1, 0, 12, 7], np.int32)
    q, k, v, cu = make_inputs(len(seqlens), Hq, Hkv, D, seqlens, seed=920)
    bad = cu.copy()
    bad[2] += 1  # batch 1: 17 rows (invalid), batch 2: 2 rows
    print(f"exact invalid length: Hq={Hq} Hkv={Hkv}", flush=True)
    o = _run(q, k, v, bad, Hq, Hkv, D).reshape(len(seqlens), Hq, D)
    assert np.isnan(oracle.f16_to_f32(o[1])).all()
    keep = [b for b in range(len(seqlens)) if b != 1]
    r, _ = oracle.decode(q, k, v, bad, Hq, Hkv, D, default_scale(D), p_mode=2, max_seqlen=17)
    assert np.array_equal(o[keep], r[keep])


def test_group_sizes_above_eight_are_rejected():
    """fmha_decode_fwd_exact takes at most 8 query heads per KV head; the
    default entry point runs a larger group on the matrix-core kernel."""
    import torch
    import fmha_amd
    seqlens = np.full(4, 8, np.int32)
    q, k, v, cu = make_inputs(4, 12, 1, 128, seqlens, seed=930)
    out = torch.full((4, 12, 128), 7.0, dtype=torch.float16, device="cuda")
    with pytest.raises(fmha_amd.FmhaDecodeError) as e:
        _run(q, k, v, cu, 12, 1, 128, out=out)
    assert "at most 8 query heads per KV head" in str(e.value)
    torch.cuda.synchronize()
    assert bool((out == 7.0).all())
    with pytest.raises(ValueError):
        fmha_amd.fmha_decode(to_dev(q), to_dev(k).view(4, 8, 1, 128), to_dev(v).view(4, 8, 1, 128), seqlen_kv=8,
                             exact=True)


def _gen(shape, seed, std, device):
    import torch
    g = torch.Generator(device=device).manual_seed(seed)
    x = torch.randn(*shape, generator=g, device=device, dtype=torch.bfloat16)
    return x * std if std != 1.0 else x


@pytest.mark.parametrize("cfg", [2, 3, 4, 5, "poisson"])
def test_full_size_sample_bit_exact(cfg):
    """Full-size workloads through fmha_decode_fwd_exact; a seeded sample of
    192 batches (plus the first and last) against the oracle, bit for bit."""
    import torch
    import fmha_amd
    if cfg == "poisson":  # the reference's own configuration 1 (fmha_host.cpp:58-82, :100)
        B, Hq, Hkv, D, std = 30720, 16, 16, 128, 1.0
        seqlens = oracle.generate_seqlens(B, 16)
    else:
        B, Hq, Hkv, S, D, std = CONFIGS[cfg]
        seqlens = np.full(B, S, np.int32)
    cu = cu_from_seqlens(seqlens)
    rows = int(cu[-1])
    seed = 0xE7A00000 + (16 * cfg if cfg != "poisson" else 0)
    print(f"exact full size: cfg={cfg} B={B} Hq={Hq} Hkv={Hkv} D={D} rows={rows}", flush=True)
    q = _gen((B, Hq, D), seed, std, "cuda")
    k = _gen((rows, Hkv, D), seed + 1, std, "cuda")
    v = _gen((rows, Hkv, D), seed + 2, std, "cuda")
    o = fmha_amd.fmha_decode(q, k, v, cu_seqlens_kv=torch.from_numpy(cu).cuda(), softmax_scale=default_scale(D),
                             exact=True)
    torch.cuda.synchronize()
    assert bool(torch.isfinite(o).all())
    rng = np.random.default_rng(17)
    sample = np.unique(np.concatenate([[0, B - 1], rng.choice(B, size=192, replace=False)]))
    idx = torch.from_numpy(sample).cuda()
    rows_sel = np.concatenate([np.arange(cu[b], cu[b + 1]) for b in sample]).astype(np.int64)
    ridx = torch.from_numpy(rows_sel).cuda()
    qs, ks, vs = _bits(q[idx]), _bits(k[ridx]), _bits(v[ridx])
    os_ = _bits(o[idx])
    cus = cu_from_seqlens(seqlens[sample])
    _assert_bit_exact(os_, qs, ks, vs, cus, Hq, Hkv, D, f"cfg {cfg} sample")
