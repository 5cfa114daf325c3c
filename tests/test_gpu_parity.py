"""GPU parity: the HIP kernel against the CPU oracle on seeded inputs, at
sizes the oracle finishes in well under a second, through the C ABI.

Coverage follows the reference's only check (fmha_host.cpp:434-445, config 0
at fmha_host.cpp:512: B=10, H=16, D=128, Poisson lengths in [2, 16]) and
widens it: every head_dim the library takes, every GQA group size, every
length 0..16 and both length paths (cu_seqlens and uniform), ragged head
counts, NaN-poisoned neighbours and the S=1 known answer.
"""
import numpy as np
import pytest

import oracle
from tests.common import (assert_exact, assert_pass, check, check_entry_points, cu_from_seqlens, default_scale,
                          make_inputs, run_gpu)

pytestmark = pytest.mark.gpu


def _case(B, Hq, Hkv, D, seqlens, seed, std=1.0, uniform=False):
    """Default entry point bit for bit against the restated loop, _fast entry
    point through the gate (tests/common.py: check_entry_points)."""
    q, k, v, cu = make_inputs(B, Hq, Hkv, D, seqlens, seed, std)
    o = check_entry_points(q, k, v, cu, Hq, Hkv, D, uniform_s=(int(seqlens[0]) if uniform else None),
                           ctx=f"B={B} Hq={Hq} Hkv={Hkv} D={D} seed={seed}")
    return o, (q, k, v, cu)


def test_reference_smoke_config():
    """Config 0 of the reference (fmha_host.cpp:512) with its own length
    generator (fmha_host.cpp:58-72)."""
    seqlens = oracle.generate_seqlens(10, 16)
    _case(10, 16, 16, 128, seqlens, seed=1)


@pytest.mark.parametrize("D", [64, 128, 256])
@pytest.mark.parametrize("G", [1, 2, 4, 8])
def test_varlen_all_lengths(D, G):
    """Every length 0..16 appears (twice) in one varlen batch."""
    Hkv = 4
    seqlens = np.array(list(range(17)) * 2, dtype=np.int32)
    np.random.default_rng(D * 10 + G).shuffle(seqlens)
    _case(len(seqlens), Hkv * G, Hkv, D, seqlens, seed=100 + D + G)


@pytest.mark.parametrize("S", [0, 1, 2, 3, 4, 5, 7, 8, 9, 13, 16])
@pytest.mark.parametrize("D", [64, 128, 256])
def test_uniform_lengths(S, D):
    _case(37, 16, 16, D, np.full(37, S, np.int32), seed=200 + S + D, uniform=True)


@pytest.mark.parametrize("Hq,Hkv", [(1, 1), (3, 3), (5, 5), (6, 3), (12, 3), (40, 5), (56, 7), (64, 8)])
@pytest.mark.parametrize("D", [64, 128, 256])
def test_ragged_head_counts(Hq, Hkv, D):
    """Head counts that leave lanes of the last wave idle."""
    seqlens = np.random.default_rng(Hq * 7 + Hkv).integers(0, 17, size=19).astype(np.int32)
    _case(19, Hq, Hkv, D, seqlens, seed=300 + Hq + D)


@pytest.mark.parametrize("std", [0.25, 2.0, 4.0])
def test_logit_spread(std):
    """Wider inputs (config 5 uses std 2.0) sharpen the softmax."""
    seqlens = oracle.generate_seqlens(64, 16)
    _case(64, 16, 16, 256, seqlens, seed=400, std=std)


def test_s1_known_answer_bitexact():
    """S=1: P = 1 exactly, so O = fp16(V) bit for bit (config 1's answer)."""
    B, H, D = 33, 16, 128
    q, k, v, cu = make_inputs(B, H, H, D, np.ones(B, np.int32), seed=500)
    for uniform in (False, True):
        o = run_gpu(q, k, v, cu, H, H, D, uniform_s=1 if uniform else None)
        expect = oracle.f32_to_f16(oracle.bf16_to_f32(v)).reshape(B, H, D)
        assert np.array_equal(o.reshape(B, H, D), expect)


def test_poisoned_neighbours():
    """A batch's output does not depend on its neighbours' rows: the rows of
    batches 0 and 2 and rows past the end are NaN."""
    H, D = 16, 128
    seqlens = np.array([16, 5, 16], np.int32)
    q, k, v, cu = make_inputs(3, H, H, D, seqlens, seed=600)
    # reference run of batch 1 alone
    q1, k1, v1 = q[1:2], k[cu[1]:cu[2]], v[cu[1]:cu[2]]
    o_alone = run_gpu(q1, k1, v1, cu_from_seqlens([5]), H, H, D)
    nan_bf16 = np.uint16(0x7FC0)
    kp, vp = k.copy(), v.copy()
    kp[: cu[1]] = nan_bf16
    vp[: cu[1]] = nan_bf16
    kp[cu[2]:] = nan_bf16
    vp[cu[2]:] = nan_bf16
    extra = np.full((8, H, D), nan_bf16, np.uint16)  # rows past the last batch
    kp = np.concatenate([kp, extra])
    vp = np.concatenate([vp, extra])
    o = run_gpu(q, kp, vp, cu, H, H, D).reshape(3, H, D)
    assert np.array_equal(o[1], o_alone.reshape(H, D))


@pytest.mark.parametrize("G", [2, 3, 4, 8])
def test_gqa_equals_mha_on_repeated_kv(G):
    """Grouped heads give the MHA result on head-repeated K/V: bit for bit
    through fmha_decode_fwd_exact (its arithmetic does not depend on the
    group size; for G = 2 also through the default entry point, which takes
    those numerics there), within the gate through the _fast one (which
    reduces in a different order for the two group sizes)."""
    B, Hkv, D = 24, 16 if G <= 4 else 8, 128
    Hq = G * Hkv
    seqlens = oracle.generate_seqlens(B, 16)
    q, k, v, cu = make_inputs(B, Hq, Hkv, D, seqlens, seed=700 + G)
    kr, vr = np.repeat(k, G, axis=1), np.repeat(v, G, axis=1)
    o_mha = run_gpu(q, kr, vr, cu, Hq, Hq, D)
    assert np.array_equal(run_gpu(q, k, v, cu, Hq, Hkv, D, exact=True), o_mha)
    if G <= 2:
        assert np.array_equal(run_gpu(q, k, v, cu, Hq, Hkv, D), o_mha)
    o_gqa = run_gpu(q, k, v, cu, Hq, Hkv, D, fast=True)
    o_mha = run_gpu(q, kr, vr, cu, Hq, Hq, D, fast=True)
    r, slack = oracle.decode(q, kr, vr, cu, Hq, Hq, D, default_scale(D), with_slack=True)
    assert_pass(oracle.compare(o_gqa, o_mha, slack), "gqa vs mha")
    assert_pass(oracle.compare(o_gqa, r, slack), "gqa vs oracle")


def test_bad_lengths_give_nan():
    """A cu_seqlens span outside [0, 16] cannot be reported from the kernel;
    that batch's output is NaN and the other batches are unaffected."""
    H, D = 16, 128
    seqlens = np.array([4, 17, 3], np.int32)
    q, k, v, cu = make_inputs(3, H, H, D, seqlens, seed=800)
    o = run_gpu(q, k, v, cu, H, H, D).reshape(3, H, D)
    assert np.all(np.isnan(oracle.f16_to_f32(o[1])))
    for b in (0, 2):
        cb = cu_from_seqlens([seqlens[b]])
        r, slack = oracle.decode(q[b:b + 1], k[cu[b]:cu[b + 1]], v[cu[b]:cu[b + 1]], cb, H, H, D,
                                 default_scale(D), with_slack=True)
        assert_pass(oracle.compare(o[b:b + 1], r, slack), f"batch {b}")


def test_custom_scale():
    seqlens = oracle.generate_seqlens(16, 16)
    q, k, v, cu = make_inputs(16, 8, 8, 128, seqlens, seed=900)
    for scale in (0.0, 0.03125, 0.5):
        o = run_gpu(q, k, v, cu, 8, 8, 128, scale=scale)
        assert_exact(o, q, k, v, cu, 8, 8, 128, f"scale={scale}", scale=scale)
        o = run_gpu(q, k, v, cu, 8, 8, 128, scale=scale, fast=True)
        assert_pass(check(o, q, k, v, cu, 8, 8, 128, scale=scale), f"scale={scale} (fast)")
