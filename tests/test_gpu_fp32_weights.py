"""GPU parity of the fp32-weight path (fmha_decode_fwd_fp32_weights): softmax
weights kept in fp32 and P.V as one fused multiply-add per row in row order,
the semantics of the reference's fmha_vectorized_fma
(fmha_vectorized_fma_kernel.hpp:243-296).  Checked against the oracle's
fp32-weight loop (oracle.decode(p_mode=1)) with the gate of tests/common.py
and no tie slack (there is no bf16 rounding of the weights to flip); the
comparison with the reference kernel itself is in
test_gpu_reference_kernels.py."""
import numpy as np
import pytest

import oracle
from tests.common import assert_pass, default_scale, make_inputs, to_dev

pytestmark = pytest.mark.gpu


def _run(q, k, v, cu, Hq, Hkv, D, fp32_weights=True):
    import torch
    import fmha_amd
    o = fmha_amd.fmha_decode(to_dev(q), to_dev(k), to_dev(v), cu_seqlens_kv=torch.from_numpy(cu).cuda(),
                             softmax_scale=default_scale(D), fp32_weights=fp32_weights)
    torch.cuda.synchronize()
    return o.view(torch.int16).cpu().numpy().view(np.uint16)


@pytest.mark.parametrize("D", [64, 128, 256])
@pytest.mark.parametrize("G", [1, 2, 4, 8])
def test_all_lengths_against_fp32_oracle(D, G):
    Hkv = 4
    seqlens = np.array(list(range(17)) * 2, dtype=np.int32)
    np.random.default_rng(D + 7 * G).shuffle(seqlens)
    q, k, v, cu = make_inputs(len(seqlens), Hkv * G, Hkv, D, seqlens, seed=700 + D + G)
    o = _run(q, k, v, cu, Hkv * G, Hkv, D)
    r, _ = oracle.decode(q, k, v, cu, Hkv * G, Hkv, D, default_scale(D), p_mode=1)
    st = oracle.compare(o.reshape(r.shape), r)
    print(f"D={D} G={G}: {st}", flush=True)
    assert_pass(st, f"fp32 weights D={D} G={G}")


@pytest.mark.parametrize("std", [0.25, 2.0, 4.0])
def test_logit_spread(std):
    seqlens = oracle.generate_seqlens(200, 16)
    q, k, v, cu = make_inputs(200, 16, 16, 128, seqlens, seed=710, std=std)
    o = _run(q, k, v, cu, 16, 16, 128)
    r, _ = oracle.decode(q, k, v, cu, 16, 16, 128, default_scale(128), p_mode=1)
    assert_pass(oracle.compare(o.reshape(r.shape), r), f"fp32 weights std={std}")


def test_s1_known_answer_bitexact():
    """One row: the weight is exactly 1, so O = fp16(V) bit for bit."""
    q, k, v, cu = make_inputs(64, 16, 8, 128, np.ones(64, np.int32), seed=711)
    o = _run(q, k, v, cu, 16, 8, 128).reshape(64, 16, 128)
    expect = oracle.f32_to_f16(oracle.bf16_to_f32(v.reshape(64, 8, 128)))
    assert np.array_equal(o, np.repeat(expect, 2, axis=1))


def test_closer_to_float64_than_bf16_weights():
    """fp32 weights drop the bf16 rounding of the weights, so over many heads
    the output sits closer to the float64 result than the bf16-weight path's
    (a dropped or mis-scaled fp32 path would not)."""
    seqlens = oracle.generate_seqlens(400, 16)
    q, k, v, cu = make_inputs(400, 16, 16, 128, seqlens, seed=712)
    o32 = oracle.f16_to_f32(_run(q, k, v, cu, 16, 16, 128)).ravel()
    o16 = oracle.f16_to_f32(_run(q, k, v, cu, 16, 16, 128, fp32_weights=False)).ravel()
    t = oracle.decode_f64(q, k, v, cu, 16, 16, 128, default_scale(128)).ravel()
    e32, e16 = np.abs(o32 - t).mean(), np.abs(o16 - t).mean()
    print(f"mean |error| vs float64: fp32 weights {e32:.3g}, bf16 weights {e16:.3g}", flush=True)
    assert e32 < 0.8 * e16


def test_poisoned_neighbours():
    """A batch's output does not depend on its neighbours' rows (NaN there)."""
    H, D = 16, 128
    seqlens = np.array([16, 7, 16], np.int32)
    q, k, v, cu = make_inputs(3, H, H, D, seqlens, seed=713)
    alone = _run(q[1:2], k[cu[1]:cu[2]], v[cu[1]:cu[2]], np.array([0, 7], np.int32), H, H, D)
    nan = np.uint16(0x7FC0)
    kp, vp = k.copy(), v.copy()
    for t in (kp, vp):
        t[: cu[1]] = nan
        t[cu[2]:] = nan
    o = _run(q, kp, vp, cu, H, H, D).reshape(3, H, D)
    assert np.array_equal(o[1], alone.reshape(H, D))


@pytest.mark.parametrize("Hq,Hkv", [(3, 3), (12, 3), (40, 5), (56, 7)])
@pytest.mark.parametrize("D", [64, 256])
def test_ragged_head_counts(Hq, Hkv, D):
    seqlens = np.random.default_rng(Hq + Hkv + D).integers(0, 17, size=19).astype(np.int32)
    q, k, v, cu = make_inputs(19, Hq, Hkv, D, seqlens, seed=714 + Hq + D)
    o = _run(q, k, v, cu, Hq, Hkv, D)
    r, _ = oracle.decode(q, k, v, cu, Hq, Hkv, D, default_scale(D), p_mode=1)
    assert_pass(oracle.compare(o.reshape(r.shape), r), f"fp32 weights Hq={Hq} Hkv={Hkv} D={D}")
