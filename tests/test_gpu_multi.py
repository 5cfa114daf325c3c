"""GPU parity of fmha_decode_multi_kernel: batches with fewer KV heads than
a wave holds (Hkv < 64 / (D/8), e.g. MQA), where each wave serves several
batches, one per lane group.  Reached through the ordinary entry points
(fmha_decode_fwd, _uniform, _strided, _fp32_weights); checked against the
oracle with the gate of tests/common.py, including wave tails (a batch
count that is not a multiple of the batches per wave), empty and invalid
lengths next to valid ones, and NaN in every row the kernel must not read."""
import numpy as np
import pytest

import oracle
from tests.common import (assert_pass, check, check_entry_points, cu_from_seqlens, default_scale, make_inputs,
                          run_gpu, to_dev)

pytestmark = pytest.mark.gpu

NAN_BITS = np.uint16(0x7FC0)

# (D, Hkv) with Hkv < heads per wave: the packed-units kernel runs.
SMALL_HKV = [(64, 1), (64, 2), (64, 4), (128, 1), (128, 2), (256, 1)]


def _batches_per_wave(D, Hkv):
    hpw = 64 // (D // 8)
    r = 1
    while Hkv * r * 2 <= hpw and hpw % (Hkv * r * 2) == 0:
        r *= 2
    return r


@pytest.mark.parametrize("D,Hkv", SMALL_HKV)
@pytest.mark.parametrize("G", [1, 2, 4, 8])
def test_varlen(D, Hkv, G):
    R = _batches_per_wave(D, Hkv)
    assert R > 1
    B = 8 * R + R - 1                        # last wave partly empty
    rng = np.random.default_rng(D * 10 + Hkv * 3 + G)
    seqlens = rng.integers(0, 17, size=B).astype(np.int32)
    seqlens[1] = 0
    seqlens[2] = 16
    q, k, v, cu = make_inputs(B, Hkv * G, Hkv, D, seqlens, seed=2000 + D + Hkv + G)
    check_entry_points(q, k, v, cu, Hkv * G, Hkv, D, ctx=f"multi varlen D={D} Hkv={Hkv} G={G}")


@pytest.mark.parametrize("D,Hkv", SMALL_HKV)
@pytest.mark.parametrize("S", [1, 5, 16])
def test_uniform(D, Hkv, S):
    B, G = 37, 4
    seqlens = np.full(B, S, np.int32)
    q, k, v, cu = make_inputs(B, Hkv * G, Hkv, D, seqlens, seed=2100 + D + S)
    check_entry_points(q, k, v, cu, Hkv * G, Hkv, D, uniform_s=S, ctx=f"multi uniform D={D} Hkv={Hkv} S={S}")


@pytest.mark.parametrize("D,Hkv", [(64, 1), (128, 2), (256, 1)])
def test_invalid_length_inside_a_wave(D, Hkv):
    """A broken length gives NaN for its batch only; the other batches of
    its wave are unaffected."""
    import torch
    import fmha_amd
    B, G = 3 * _batches_per_wave(D, Hkv), 2
    rng = np.random.default_rng(D)
    seqlens = rng.integers(1, 17, size=B).astype(np.int32)
    q, k, v, cu = make_inputs(B, Hkv * G, Hkv, D, seqlens, seed=2200 + D)
    bad = 1
    cu_bad = cu.copy()
    cu_bad[bad + 1:] += 20                    # batch `bad` gets length S+20 > 16
    k2 = np.concatenate([k[:cu[bad + 1]], np.zeros((20, Hkv, D), np.uint16), k[cu[bad + 1]:]])
    v2 = np.concatenate([v[:cu[bad + 1]], np.zeros((20, Hkv, D), np.uint16), v[cu[bad + 1]:]])
    o = fmha_amd.fmha_decode(to_dev(q), to_dev(k2), to_dev(v2), cu_seqlens_kv=torch.from_numpy(cu_bad).cuda())
    torch.cuda.synchronize()
    bits = o.view(torch.int16).cpu().numpy().view(np.uint16).reshape(B, Hkv * G, D)
    f = oracle.f16_to_f32(bits)
    assert np.all(np.isnan(f[bad]))
    keep = [b for b in range(B) if b != bad]
    assert np.all(np.isfinite(f[keep]))
    r, slack = oracle.decode(q, k, v, cu, Hkv * G, Hkv, D, default_scale(D), with_slack=True)
    st = oracle.compare(np.ascontiguousarray(bits[keep]).ravel(),
                        np.ascontiguousarray(r.reshape(B, Hkv * G, D)[keep]).ravel(),
                        np.ascontiguousarray(slack.reshape(B, Hkv * G, D)[keep]).ravel())
    assert_pass(st, f"neighbours of an invalid length D={D}")


@pytest.mark.parametrize("layout", ["bhsd", "bshd"])
@pytest.mark.parametrize("D,Hkv", [(64, 2), (128, 1), (256, 1)])
def test_strided(layout, D, Hkv):
    import torch
    import fmha_amd
    B, G, cap = 45, 4, 16
    rng = np.random.default_rng(D + Hkv)
    seqlens = rng.integers(0, cap + 1, size=B).astype(np.int32)
    q, k, v, cu = make_inputs(B, Hkv * G, Hkv, D, seqlens, seed=2300 + D)
    kc = np.full((B, cap, Hkv, D), NAN_BITS, np.uint16)
    vc = np.full((B, cap, Hkv, D), NAN_BITS, np.uint16)
    for b in range(B):
        kc[b, :seqlens[b]] = k[cu[b]:cu[b + 1]]
        vc[b, :seqlens[b]] = v[cu[b]:cu[b + 1]]
    if layout == "bhsd":
        kd = to_dev(np.ascontiguousarray(kc.transpose(0, 2, 1, 3))).transpose(1, 2)
        vd = to_dev(np.ascontiguousarray(vc.transpose(0, 2, 1, 3))).transpose(1, 2)
    else:
        kd, vd = to_dev(kc), to_dev(vc)
    o = fmha_amd.fmha_decode_strided(to_dev(q), kd, vd, seqlens_kv=torch.from_numpy(seqlens).cuda())
    torch.cuda.synchronize()
    bits = o.view(torch.int16).cpu().numpy().view(np.uint16)
    assert_pass(check(bits, q, k, v, cu, Hkv * G, Hkv, D), f"multi strided {layout} D={D} Hkv={Hkv}")


@pytest.mark.parametrize("D,Hkv", [(64, 1), (128, 2), (256, 1)])
def test_fp32_weights(D, Hkv):
    import torch
    import fmha_amd
    B, G = 41, 8
    rng = np.random.default_rng(D * 3 + Hkv)
    seqlens = rng.integers(0, 17, size=B).astype(np.int32)
    q, k, v, cu = make_inputs(B, Hkv * G, Hkv, D, seqlens, seed=2400 + D)
    o = fmha_amd.fmha_decode(to_dev(q), to_dev(k), to_dev(v), cu_seqlens_kv=torch.from_numpy(cu).cuda(),
                             fp32_weights=True)
    torch.cuda.synchronize()
    r, _ = oracle.decode(q, k, v, cu, Hkv * G, Hkv, D, default_scale(D), p_mode=1)
    bits = o.view(torch.int16).cpu().numpy().view(np.uint16)
    assert_pass(oracle.compare(bits.reshape(r.shape), r), f"multi fp32 weights D={D} Hkv={Hkv}")
