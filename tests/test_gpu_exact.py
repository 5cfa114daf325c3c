"""GPU parity of the exact-arithmetic path (fmha_decode_fwd_exact): the
reference CPU loop's arithmetic step for step (fmha_host.cpp:179-244).

Its outputs must equal, bit for bit and with no gate or slack, the oracle's
bf16-weight loop with nearest-float exponentials (oracle.decode(p_mode=2));
the loop with the C library's expf (p_mode=0, the reference's own) then
differs from it only through the few exponentials that expf misrounds
(tests/test_oracle.py pins that).  Covered: every length 0..16, head dims
64/128/256, head counts below and above what one wave holds (the R-batch
kernel and the one-batch kernel), logit spreads, invalid lengths (NaN), the
rejected group sizes, and four BASELINE configurations at full size on a
seeded sample of batches.
"""
import numpy as np
import pytest

import oracle
from tests.common import CONFIGS, cu_from_seqlens, default_scale, make_inputs, to_dev

pytestmark = pytest.mark.gpu


def _bits(t):
    import torch
    return t.contiguous().view(torch.int16).cpu().numpy().view(np.uint16)


def _run(q, k, v, cu, H, D, out=None):
    import torch
    import fmha_amd
    o = fmha_amd.fmha_decode(to_dev(q), to_dev(k), to_dev(v), cu_seqlens_kv=torch.from_numpy(cu).cuda(),
                             softmax_scale=default_scale(D), out=out, exact=True)
    torch.cuda.synchronize()
    return _bits(o)


def _assert_bit_exact(o, q, k, v, cu, H, D, ctx):
    r, _ = oracle.decode(q, k, v, cu, H, H, D, default_scale(D), p_mode=2)
    o = o.reshape(r.shape)
    diff = int(np.count_nonzero(o != r))
    r0, _ = oracle.decode(q, k, v, cu, H, H, D, default_scale(D), p_mode=0)
    print(f"{ctx}: {o.size} outputs, {diff} differ from the nearest-exp loop, "
          f"{int(np.count_nonzero(o != r0))} from the expf loop", flush=True)
    assert diff == 0, f"{ctx}: {diff} outputs differ from the oracle (p_mode=2)"


@pytest.mark.parametrize("D", [64, 128, 256])
@pytest.mark.parametrize("H", [1, 2, 4, 16, 32])
def test_all_lengths_bit_exact(D, H):
    seqlens = np.array(list(range(17)) * 3, dtype=np.int32)
    np.random.default_rng(D + 7 * H).shuffle(seqlens)
    q, k, v, cu = make_inputs(len(seqlens), H, H, D, seqlens, seed=900 + D + H)
    print(f"exact: D={D} H={H} B={len(seqlens)}", flush=True)
    _assert_bit_exact(_run(q, k, v, cu, H, D), q, k, v, cu, H, D, f"D={D} H={H}")


@pytest.mark.parametrize("std", [0.25, 2.0, 4.0])
@pytest.mark.parametrize("D", [128, 256])
def test_logit_spread_bit_exact(std, D):
    seqlens = oracle.generate_seqlens(300, 16)
    q, k, v, cu = make_inputs(300, 16, 16, D, seqlens, seed=910, std=std)
    print(f"exact: std={std} D={D}", flush=True)
    _assert_bit_exact(_run(q, k, v, cu, 16, D), q, k, v, cu, 16, D, f"std={std} D={D}")


@pytest.mark.parametrize("H", [2, 16])
def test_invalid_lengths_give_nan(H):
    """A length outside [0, 16] turns that batch's outputs into NaN; the
    other batches stay exact."""
    D = 128
    seqlens = np.array([5, 16, 3, 9, 1, 0, 12, 7], np.int32)
    q, k, v, cu = make_inputs(len(seqlens), H, H, D, seqlens, seed=920)
    bad = cu.copy()
    bad[2] += 1  # batch 1: 17 rows (invalid), batch 2: 2 rows
    print(f"exact invalid length: H={H}", flush=True)
    o = _run(q, k, v, bad, H, D).reshape(len(seqlens), H, D)
    assert np.isnan(oracle.f16_to_f32(o[1])).all()
    keep = [b for b in range(len(seqlens)) if b != 1]
    r, _ = oracle.decode(q, k, v, bad, H, H, D, default_scale(D), p_mode=2, max_seqlen=17)
    assert np.array_equal(o[keep], r[keep])


def test_group_sizes_above_one_are_rejected():
    import torch
    import fmha_amd
    seqlens = np.full(4, 8, np.int32)
    q, k, v, cu = make_inputs(4, 8, 4, 128, seqlens, seed=930)
    out = torch.full((4, 8, 128), 7.0, dtype=torch.float16, device="cuda")
    with pytest.raises(fmha_amd.FmhaDecodeError) as e:
        _run(q, k, v, cu, 8, 128, out=out)
    assert "one query head per KV head" in str(e.value)
    torch.cuda.synchronize()
    assert bool((out == 7.0).all())


def _gen(shape, seed, std, device):
    import torch
    g = torch.Generator(device=device).manual_seed(seed)
    x = torch.randn(*shape, generator=g, device=device, dtype=torch.bfloat16)
    return x * std if std != 1.0 else x


@pytest.mark.parametrize("cfg", [2, 3, 5, "poisson"])
def test_full_size_sample_bit_exact(cfg):
    """Full-size workloads through the exact path; a seeded sample of 192
    batches (plus the first and last) against the oracle, bit for bit."""
    import torch
    import fmha_amd
    if cfg == "poisson":  # the reference's own configuration 1 (fmha_host.cpp:58-82, :100)
        B, H, D, std = 30720, 16, 128, 1.0
        seqlens = oracle.generate_seqlens(B, 16)
    else:
        B, Hq, Hkv, S, D, std = CONFIGS[cfg]
        assert Hq == Hkv
        H = Hq
        seqlens = np.full(B, S, np.int32)
    cu = cu_from_seqlens(seqlens)
    rows = int(cu[-1])
    seed = 0xE7A00000 + (16 * cfg if cfg != "poisson" else 0)
    print(f"exact full size: cfg={cfg} B={B} H={H} D={D} rows={rows}", flush=True)
    q = _gen((B, H, D), seed, std, "cuda")
    k = _gen((rows, H, D), seed + 1, std, "cuda")
    v = _gen((rows, H, D), seed + 2, std, "cuda")
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
    _assert_bit_exact(os_, qs, ks, vs, cus, H, D, f"cfg {cfg} sample")
