"""Pins the CPU oracle (oracle/fmha_oracle.cpp) before anything is compared
with it.  Each check is chosen so that a plausible mistake in the oracle (a
dropped term, a wrong head mapping, a transposed index, a wrong rounding)
fails at least one of them:

  * bit-exact against the reference's own CPU loop: committed fixtures
    (tests/golden/mha_*.npz, written by the reference's do_validation) and,
    where the reference build exists, live random cases;
  * the reference's length generator (tests/golden/seqlens_ref.json);
  * float64 mode against torch's float64 scaled_dot_product_attention
    (committed GQA fixtures and live cases);
  * closed forms: S=1 gives fp16(V); Q=0 gives uniform bf16(1/S) weights; one
    dominant key gives fp16(V_j); S=0 gives 0;
  * invariants: GQA equals MHA on head-repeated K/V bit for bit; batch
    independence; permutation of the KV rows changes the result only within
    the gate;
  * rounding helpers against torch (bf16) and numpy (fp16) over every bf16
    bit pattern and random fp32 patterns.
"""
import glob
import json
import os

import numpy as np
import pytest

import oracle
from tests.common import ATOL, RTOL, cu_from_seqlens, default_scale, make_inputs

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
needs_ref = pytest.mark.skipif(not oracle.ref_available(),
                               reason="oracle/_ref not built (the reference is not mounted here)")


def _f32(bits):
    return oracle.bf16_to_f32(bits)


# ---------------------------------------------------------------- rounding
def test_f32_to_bf16_matches_torch():
    import torch
    rng = np.random.default_rng(0)
    bits = np.concatenate([rng.integers(0, 2 ** 32, 200000, dtype=np.uint64).astype(np.uint32),
                           # exact ties and near-ties around every rounding step
                           (np.arange(0, 2 ** 16, dtype=np.uint32) << 16) | 0x8000,
                           (np.arange(0, 2 ** 16, dtype=np.uint32) << 16) | 0x7fff,
                           (np.arange(0, 2 ** 16, dtype=np.uint32) << 16) | 0x8001]).astype(np.uint32)
    x = bits.view(np.float32)
    finite = np.isfinite(x)
    got = oracle.f32_to_bf16(x[finite])
    want = torch.from_numpy(x[finite].copy()).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(got, want)


def test_f32_to_f16_matches_numpy():
    rng = np.random.default_rng(1)
    # every bf16 value (the shape of the kernel's S=1 output path) plus random
    # fp32 patterns concentrated on the fp16 range, ties included
    allbf = (np.arange(0, 2 ** 16, dtype=np.uint32) << 16).view(np.float32)
    rnd = rng.integers(0, 2 ** 32, 300000, dtype=np.uint64).astype(np.uint32).view(np.float32)
    small = (rng.standard_normal(300000) * np.exp(rng.uniform(-20, 12, 300000))).astype(np.float32)
    f16 = np.arange(0, 2 ** 16, dtype=np.uint16).view(np.float16).astype(np.float32)
    with np.errstate(invalid="ignore"):
        ties = ((f16[:-1].astype(np.float64) + f16[1:].astype(np.float64)) / 2).astype(np.float32)
    x = np.concatenate([allbf, rnd, small, ties])
    x = x[~np.isnan(x)]
    got = oracle.f32_to_f16(x)
    with np.errstate(over="ignore"):
        want = x.astype(np.float16).view(np.uint16)
    assert np.array_equal(got, want)


# ---------------------------------------------------------------- reference
def test_seqlens_match_reference_fixture():
    fx = json.load(open(os.path.join(GOLDEN, "seqlens_ref.json")))
    got = oracle.generate_seqlens(len(fx["seqlens"]), 16)
    assert got.tolist() == fx["seqlens"]
    assert all(2 <= s <= 16 for s in got)


@needs_ref
def test_seqlens_match_reference_live():
    for b, m in [(1000, 16), (10, 16), (257, 8), (64, 4)]:
        assert np.array_equal(oracle.generate_seqlens(b, m), oracle.ref_generate_seqlens(b, m))


@pytest.mark.parametrize("path", sorted(glob.glob(os.path.join(GOLDEN, "mha_*.npz"))))
def test_bitexact_reference_fixtures(path):
    z = np.load(path, allow_pickle=False)
    B, Hq, Hkv, D = z["meta"].tolist()
    o, _ = oracle.decode(z["q"], z["k"], z["v"], z["cu"], Hq, Hkv, D, default_scale(D))
    assert np.array_equal(o, z["o"])


@needs_ref
@pytest.mark.parametrize("D", [128, 256])
@pytest.mark.parametrize("H", [1, 4, 16])
def test_bitexact_reference_live(D, H, capfd):
    seqlens = oracle.generate_seqlens(48, 16)
    seqlens[:3] = [1, 16, 5]
    q, k, v, cu = make_inputs(48, H, H, D, seqlens, seed=D + H, std=2.0 if D == 256 else 1.0)
    o, _ = oracle.decode(q, k, v, cu, H, H, D, default_scale(D))
    r, ok = oracle.ref_do_validation(q, k, v, cu, H, H, D, gpu_o=o)
    capfd.readouterr()  # the reference prints while it validates
    assert ok and np.array_equal(o, r)


# ---------------------------------------------------------------- float64
@pytest.mark.parametrize("path", sorted(glob.glob(os.path.join(GOLDEN, "gqa_sdpa_*.npz"))))
def test_f64_against_sdpa_fixtures(path):
    z = np.load(path, allow_pickle=False)
    B, Hq, Hkv, D = z["meta"].tolist()
    o = oracle.decode_f64(z["q"], z["k"], z["v"], z["cu"], Hq, Hkv, D, 1.0 / np.sqrt(D))
    assert np.max(np.abs(o - z["o"])) < 1e-12


@pytest.mark.parametrize("Hq,Hkv,D", [(4, 4, 64), (8, 2, 128), (4, 1, 256), (15, 5, 128), (12, 2, 64),
                                      (7, 1, 256), (40, 8, 128)])
def test_f64_against_sdpa_live(Hq, Hkv, D):
    import torch
    seqlens = [1, 2, 9, 16]
    q, k, v, cu = make_inputs(len(seqlens), Hq, Hkv, D, seqlens, seed=Hq * D)
    o = oracle.decode_f64(q, k, v, cu, Hq, Hkv, D, 1.0 / np.sqrt(D))
    t = lambda a: torch.from_numpy(_f32(a)).double()
    for b in range(len(seqlens)):
        kb = t(k[cu[b]:cu[b + 1]]).repeat_interleave(Hq // Hkv, 1).transpose(0, 1)
        vb = t(v[cu[b]:cu[b + 1]]).repeat_interleave(Hq // Hkv, 1).transpose(0, 1)
        ref = torch.nn.functional.scaled_dot_product_attention(t(q[b]).unsqueeze(1), kb, vb,
                                                               scale=1.0 / np.sqrt(D))[:, 0]
        assert np.max(np.abs(o[b] - ref.numpy())) < 1e-12


def test_bf16_weights_within_rounding_bound_of_f64():
    """The bf16-P output differs from the float64 truth by at most the weight
    rounding (unit roundoff 2^-8 per weight, so sum_j 2^-8 p_j |V_jd| <=
    2^-8 max_j |V_jd|), fp32 sums and one fp16 rounding (2^-11, doubled)."""
    seqlens = oracle.generate_seqlens(64, 16)
    q, k, v, cu = make_inputs(64, 8, 4, 128, seqlens, seed=5)
    o, _ = oracle.decode(q, k, v, cu, 8, 4, 128, default_scale(128))
    t = oracle.decode_f64(q, k, v, cu, 8, 4, 128, default_scale(128))
    vabs = np.abs(_f32(v)).astype(np.float64)
    of = oracle.f16_to_f32(o).astype(np.float64)
    for b in range(64):
        bound = 2.0 ** -8 * vabs[cu[b]:cu[b + 1]].max(axis=0).repeat(2, axis=0) + 1e-4
        bound = bound + np.abs(t[b]) * 2.0 ** -10
        assert np.all(np.abs(of[b] - t[b]) <= bound)


# ---------------------------------------------------------------- closed forms
def test_s1_is_fp16_of_v():
    q, k, v, cu = make_inputs(9, 4, 2, 128, [1] * 9, seed=7)
    o, _ = oracle.decode(q, k, v, cu, 4, 2, 128, default_scale(128))
    want = oracle.f32_to_f16(np.repeat(_f32(v), 2, axis=1))
    assert np.array_equal(o, want)


def test_s0_is_zero():
    q, k, v, cu = make_inputs(3, 4, 4, 64, [0, 3, 0], seed=8)
    o, _ = oracle.decode(q, k, v, cu, 4, 4, 64, default_scale(64))
    assert not o[0].any() and not o[2].any() and o[1].any()


@pytest.mark.parametrize("S", [2, 3, 5, 16])
def test_zero_query_gives_uniform_bf16_weights(S):
    q, k, v, cu = make_inputs(2, 4, 4, 128, [S, S], seed=S)
    q[:] = 0
    o, _ = oracle.decode(q, k, v, cu, 4, 4, 128, default_scale(128))
    w = _f32(oracle.f32_to_bf16(np.float32(1.0) / np.float32(S)))  # bf16(1/S)
    for b in range(2):
        acc = np.zeros((4, 128), np.float32)
        for j in range(S):                       # fp32, in row order
            acc = acc + w * _f32(v[cu[b] + j])
        assert np.array_equal(o[b], oracle.f32_to_f16(acc))


def test_dominant_key_is_one_hot():
    D, S = 128, 16
    q, k, v, cu = make_inputs(1, 2, 2, D, [S], seed=11)
    q[:] = oracle.f32_to_bf16(np.ones((1, 2, D), np.float32))
    k[:] = oracle.f32_to_bf16(np.full((S, 2, D), -1.0, np.float32))
    k[6] = oracle.f32_to_bf16(np.full((2, D), 16.0, np.float32))  # logit gap 17*128*scale > 200
    o, _ = oracle.decode(q, k, v, cu, 2, 2, D, default_scale(D))
    assert np.array_equal(o[0], oracle.f32_to_f16(_f32(v[6])))


# ------------------------------- nearest-float exponentials (p_mode=2): pins
# The loop the library's exact path (fmha_decode_fwd_exact) restates:
# p_mode 0 with exp_nearest, the float nearest exp(x), in place of the C
# library's expf.
def _exp_args(seed):
    rng = np.random.default_rng(seed)
    return np.concatenate([-rng.exponential(4.0, 200000), rng.uniform(-103.0, 88.0, 20000),
                           [0.0, -0.0, -1e-30, 1e-30]]).astype(np.float32)


def test_exp_nearest_is_the_nearest_float():
    x = _exp_args(50)
    e = oracle.exp_nearest(x)
    t = np.exp(x.astype(np.float64))
    assert np.array_equal(e, t.astype(np.float32))
    err = np.abs(e.astype(np.float64) - t)
    for side in (np.inf, -np.inf):
        nb = np.nextafter(e, np.float32(side)).astype(np.float64)
        assert np.all(err <= np.abs(nb - t))
    assert oracle.exp_nearest(np.float32([0.0]))[0] == 1.0


def test_c_library_expf_is_the_one_that_misses():
    """Where the C library's expf and exp_nearest disagree, expf's float is
    the farther one from exp(x) (glibc 2.35: about 7 arguments in 10 000)."""
    import ctypes
    import ctypes.util
    libm = ctypes.CDLL(ctypes.util.find_library("m") or "libm.so.6")
    libm.expf.restype = ctypes.c_float
    libm.expf.argtypes = [ctypes.c_float]
    x = _exp_args(51)[:60000]
    g = np.array([libm.expf(float(a)) for a in x], dtype=np.float32)
    e = oracle.exp_nearest(x)
    t = np.exp(x.astype(np.float64))
    miss = np.nonzero(g != e)[0]
    print(f"expf differs from the nearest float on {len(miss)} of {len(x)} arguments")
    assert len(miss) < len(x) // 200
    assert np.all(np.abs(g[miss].astype(np.float64) - t[miss]) > np.abs(e[miss].astype(np.float64) - t[miss]))


def test_nearest_exp_loop_equals_expf_loop_on_random_heads():
    """Apart from the exponential, p_mode 2 is p_mode 0: a misrounded expf
    changes an output only where it also flips a bf16 weight (none in ten
    million random heads measured), so on random heads both give the same
    bits, and so does any other change to p_mode 2 fail here."""
    seqlens = oracle.generate_seqlens(3000, 16)
    q, k, v, cu = make_inputs(3000, 8, 8, 128, seqlens, seed=52, std=2.0)
    r0, _ = oracle.decode(q, k, v, cu, 8, 8, 128, default_scale(128), p_mode=0)
    r2, _ = oracle.decode(q, k, v, cu, 8, 8, 128, default_scale(128), p_mode=2)
    assert np.array_equal(r0, r2)


@pytest.mark.parametrize("S", [1, 3, 16])
def test_nearest_exp_known_answers(S):
    """One row: fp16(V); zero query: the uniform bf16 weights bf16(1/S)."""
    q, k, v, cu = make_inputs(2, 4, 4, 128, [S, S], seed=53 + S)
    q[:] = 0
    o, _ = oracle.decode(q, k, v, cu, 4, 4, 128, default_scale(128), p_mode=2)
    w = _f32(oracle.f32_to_bf16(np.float32(1.0) / np.float32(S)))
    for b in range(2):
        acc = np.zeros((4, 128), np.float32)
        for j in range(S):
            acc = acc + w * _f32(v[cu[b] + j])
        assert np.array_equal(o[b], oracle.f32_to_f16(acc))


def test_unknown_p_mode_is_rejected():
    q, k, v, cu = make_inputs(2, 4, 4, 64, [3, 3], seed=60)
    with pytest.raises(ValueError):
        oracle.decode(q, k, v, cu, 4, 4, 64, default_scale(64), p_mode=3)


# ------------------------------------------- fp32 weights (p_mode=1): pins
# The fp32-weight loop (the numerics of fmha_vectorized_fma_kernel.hpp:243-296)
# keeps the weights unrounded; these checks would catch a stray bf16 rounding,
# a dropped normalisation or a wrong accumulation order.
@pytest.mark.parametrize("S", [2, 3, 5, 7, 16])
def test_fp32_weights_zero_query_is_exact_uniform(S):
    q, k, v, cu = make_inputs(2, 4, 4, 128, [S, S], seed=40 + S)
    q[:] = 0
    o, _ = oracle.decode(q, k, v, cu, 4, 4, 128, default_scale(128), p_mode=1)
    w = np.float32(1.0) / np.float32(S)          # exp(0) / S, not rounded to bf16
    for b in range(2):
        acc = np.zeros((4, 128), np.float32)
        for j in range(S):                       # fp32, in row order
            acc = acc + w * _f32(v[cu[b] + j])
        assert np.array_equal(o[b], oracle.f32_to_f16(acc))


def test_fp32_weights_one_row_and_dominant_key():
    q, k, v, cu = make_inputs(5, 4, 2, 128, [1] * 5, seed=44)
    o, _ = oracle.decode(q, k, v, cu, 4, 2, 128, default_scale(128), p_mode=1)
    assert np.array_equal(o, oracle.f32_to_f16(np.repeat(_f32(v), 2, axis=1)))
    D, S = 128, 16
    q, k, v, cu = make_inputs(1, 2, 2, D, [S], seed=45)
    q[:] = oracle.f32_to_bf16(np.ones((1, 2, D), np.float32))
    k[:] = oracle.f32_to_bf16(np.full((S, 2, D), -1.0, np.float32))
    k[9] = oracle.f32_to_bf16(np.full((2, D), 16.0, np.float32))
    o, _ = oracle.decode(q, k, v, cu, 2, 2, D, default_scale(D), p_mode=1)
    assert np.array_equal(o[0], oracle.f32_to_f16(_f32(v[9])))


def test_fp32_weights_within_fp16_rounding_of_f64():
    """Without the bf16 rounding of the weights the only sizeable error left
    is the final fp16 rounding (2^-11 relative) plus fp32 noise."""
    seqlens = oracle.generate_seqlens(64, 16)
    q, k, v, cu = make_inputs(64, 8, 4, 128, seqlens, seed=46)
    o, _ = oracle.decode(q, k, v, cu, 8, 4, 128, default_scale(128), p_mode=1)
    t = oracle.decode_f64(q, k, v, cu, 8, 4, 128, default_scale(128))
    of = oracle.f16_to_f32(o).astype(np.float64)
    assert np.all(np.abs(of - t) <= 2.0 ** -11 * np.abs(t) + 1e-5)
    ob, _ = oracle.decode(q, k, v, cu, 8, 4, 128, default_scale(128), p_mode=0)
    e32 = np.abs(of - t).mean()
    e16 = np.abs(oracle.f16_to_f32(ob).astype(np.float64) - t).mean()
    assert e32 < 0.5 * e16


# ---------------------------------------------------------------- invariants
def test_gqa_equals_mha_on_repeated_kv():
    seqlens = oracle.generate_seqlens(20, 16)
    for g in (2, 3, 4, 5, 7, 8, 12):
        q, k, v, cu = make_inputs(20, 2 * g, 2, 128, seqlens, seed=g)
        o_g, _ = oracle.decode(q, k, v, cu, 2 * g, 2, 128, default_scale(128))
        o_m, _ = oracle.decode(q, np.repeat(k, g, 1), np.repeat(v, g, 1), cu, 2 * g, 2 * g, 128,
                               default_scale(128))
        assert np.array_equal(o_g, o_m)
        # an interleaved mapping (KV head = h % Hkv) reads other rows; the
        # check above tells it apart from the grouped one
        o_wrong, _ = oracle.decode(q, np.tile(k, (1, g, 1)), np.tile(v, (1, g, 1)), cu, 2 * g, 2 * g,
                                   128, default_scale(128))
        assert not np.array_equal(o_g, o_wrong)


def test_batch_independence():
    seqlens = [4, 16, 9]
    q, k, v, cu = make_inputs(3, 4, 4, 128, seqlens, seed=12)
    o, _ = oracle.decode(q, k, v, cu, 4, 4, 128, default_scale(128))
    o1, _ = oracle.decode(q[1:2], k[cu[1]:cu[2]], v[cu[1]:cu[2]], cu_from_seqlens([16]), 4, 4, 128,
                          default_scale(128))
    assert np.array_equal(o[1], o1[0])


def test_row_permutation_within_gate():
    seqlens = [16] * 8
    q, k, v, cu = make_inputs(8, 4, 4, 128, seqlens, seed=13)
    perm = np.random.default_rng(0).permutation(16)
    kp = k.reshape(8, 16, 4, 128)[:, perm].reshape(k.shape)
    vp = v.reshape(8, 16, 4, 128)[:, perm].reshape(v.shape)
    o, slack = oracle.decode(q, k, v, cu, 4, 4, 128, default_scale(128), with_slack=True)
    op, _ = oracle.decode(q, kp, vp, cu, 4, 4, 128, default_scale(128))
    st = oracle.compare(op, o, slack, ATOL, RTOL)
    assert st["fails"] == 0 and st["ref_rule_fails"] == 0


def test_gate_rejects_planted_error():
    """The comparison flags a one-element error of 4 fp16 ulps at |r| ~ 1 and
    a NaN, and accepts identical outputs."""
    q, k, v, cu = make_inputs(4, 4, 4, 128, [16] * 4, seed=14)
    o, slack = oracle.decode(q, k, v, cu, 4, 4, 128, default_scale(128), with_slack=True)
    assert oracle.compare(o, o, slack)["fails"] == 0
    bad = o.copy().ravel()
    i = int(np.argmax(np.abs(oracle.f16_to_f32(bad)) > 0.5))
    val = oracle.f16_to_f32(bad[i:i + 1])[0]
    bad[i] = oracle.f32_to_f16(np.array([val * 1.03], np.float32))[0]
    st = oracle.compare(bad, o.ravel(), None)
    assert st["fails"] == 1 and st["first_fail"] == i
    bad[i] = 0x7e00
    st = oracle.compare(bad, o.ravel(), slack)
    assert st["fails"] == 1 and st["nonfinite"] == 1


def test_rejects_bad_lengths():
    q, k, v, cu = make_inputs(2, 1, 1, 64, [3, 3], seed=15)
    with pytest.raises(ValueError):
        oracle.decode(q, k, v, np.array([0, 17, 6], np.int32), 1, 1, 64, 0.125)
    with pytest.raises(ValueError):
        oracle.decode(q, k, v, np.array([0, 4, 3], np.int32), 1, 1, 64, 0.125)


# ------------------------------------------- rows longer than 16: pins
# The reference stops at 16 rows (fmha_mfma_4x4x4_kernel.hpp:179, README.md:
# 233); the oracle runs the same loop over longer rows for the split-KV,
# single-pass and paged kernels.  These checks pin that extension through
# closed forms and through float64 (itself checked against torch's SDPA at
# long rows), and test_long_row_checks_reject_planted_mistakes shows that each
# of four plausible mistakes in the long-row loop fails at least one of them.
LONG_S = (17, 100, 2048, 40000)


def _uniform_expected(v, cu, b, S, w, hq, hkv):
    """fp16(sum_j w * V_j) with the fp32 sum in row order (np.cumsum is
    sequential), query head h reading KV head h // (hq // hkv)."""
    rows = _f32(v[cu[b]:cu[b] + S]) * np.float32(w)
    acc = np.cumsum(rows, axis=0, dtype=np.float32)[-1]        # [Hkv, D]
    return oracle.f32_to_f16(np.repeat(acc, hq // hkv, axis=0))


def _long_row_failures():
    """Runs the long-row checks with whatever oracle library is loaded;
    returns the names of the checks that fail."""
    failed = []
    # Q = 0: every weight is exp(0)/S; bf16 and fp32 weight modes
    for S in LONG_S:
        D, hq, hkv = (64, 2, 1) if S > 2048 else (128, 4, 2)
        q, k, v, cu = make_inputs(2, hq, hkv, D, [S, 3], seed=S)
        q[:] = 0
        o, _ = oracle.decode(q, k, v, cu, hq, hkv, D, default_scale(D), max_seqlen=S)
        w = _f32(oracle.f32_to_bf16(np.float32(1.0) / np.float32(S)))
        if not np.array_equal(o[0], _uniform_expected(v, cu, 0, S, w, hq, hkv)):
            failed.append(f"zero-query S={S}")
        o1, _ = oracle.decode(q, k, v, cu, hq, hkv, D, default_scale(D), p_mode=1, max_seqlen=S)
        if not np.array_equal(o1[0], _uniform_expected(v, cu, 0, S, np.float32(1.0) / np.float32(S), hq, hkv)):
            failed.append(f"zero-query fp32 weights S={S}")
    # one dominant key (logit gap > 104): one-hot weights, O = fp16(V_j)
    for S in LONG_S[:3]:
        for j in sorted({16, S // 2, S - 1}):
            D = 128
            q, k, v, cu = make_inputs(1, 2, 2, D, [S], seed=S + j)
            q[:] = oracle.f32_to_bf16(np.ones((1, 2, D), np.float32))
            k[:] = oracle.f32_to_bf16(np.full((S, 2, D), -1.0, np.float32))
            k[j] = oracle.f32_to_bf16(np.full((2, D), 16.0, np.float32))
            for pm in (0, 1):
                o, _ = oracle.decode(q, k, v, cu, 2, 2, D, default_scale(D), p_mode=pm, max_seqlen=S)
                if not np.array_equal(o[0], oracle.f32_to_f16(_f32(v[j]))):
                    failed.append(f"dominant key S={S} j={j} p_mode={pm}")
    # random rows against float64 within the bf16-weight bound (no slack)
    from tests.common import f64_bound, f64_check
    for S, std in ((17, 1.0), (100, 2.0), (2048, 1.0)):
        seqlens = [S, 5, S - 1]
        q, k, v, cu = make_inputs(3, 4, 2, 128, seqlens, seed=3 * S, std=std)
        o, _ = oracle.decode(q, k, v, cu, 4, 2, 128, default_scale(128), max_seqlen=S)
        t, bound = f64_bound(q, k, v, cu, 4, 2, 128)
        if f64_check(o, t, bound)["f64_violations"]:
            failed.append(f"f64 bound S={S}")
    return failed


def test_long_rows_closed_forms_and_f64_bound():
    assert _long_row_failures() == []


@pytest.mark.parametrize("Hq,Hkv,D,seqlens", [(4, 2, 128, [17, 100, 2048]), (8, 1, 64, [40000, 33]),
                                              (6, 3, 256, [1000, 16, 17])])
def test_f64_against_sdpa_long_rows(Hq, Hkv, D, seqlens):
    import torch
    q, k, v, cu = make_inputs(len(seqlens), Hq, Hkv, D, seqlens, seed=Hq * D + len(seqlens))
    o = oracle.decode_f64(q, k, v, cu, Hq, Hkv, D, 1.0 / np.sqrt(D), max_seqlen=max(seqlens))
    t = lambda a: torch.from_numpy(_f32(a)).double()
    for b in range(len(seqlens)):
        kb = t(k[cu[b]:cu[b + 1]]).repeat_interleave(Hq // Hkv, 1).transpose(0, 1)
        vb = t(v[cu[b]:cu[b + 1]]).repeat_interleave(Hq // Hkv, 1).transpose(0, 1)
        ref = torch.nn.functional.scaled_dot_product_attention(t(q[b]).unsqueeze(1), kb, vb,
                                                               scale=1.0 / np.sqrt(D))[:, 0]
        assert np.max(np.abs(o[b] - ref.numpy())) < 1e-12


def test_f64_bound_is_tight_enough_to_catch_mistakes():
    """The bound passes the oracle's bf16 and fp32 weights, and rejects the
    output with one row left out, or with every weight moved by 2^-7."""
    from tests.common import f64_bound, f64_check
    seqlens = [16, 40, 300]
    q, k, v, cu = make_inputs(3, 4, 4, 128, seqlens, seed=77, std=2.0)
    t, bound = f64_bound(q, k, v, cu, 4, 4, 128)
    for pm in (0, 1):
        o, _ = oracle.decode(q, k, v, cu, 4, 4, 128, default_scale(128), p_mode=pm, max_seqlen=300)
        assert f64_check(o, t, bound)["f64_violations"] == 0
    # drop the last row of each batch: the truth of the shorter rows
    cu_short = cu.copy()
    ks = np.concatenate([k[cu[b]:cu[b + 1] - 1] for b in range(3)])
    vs = np.concatenate([v[cu[b]:cu[b + 1] - 1] for b in range(3)])
    cu_short = cu_from_seqlens([s - 1 for s in seqlens])
    o_drop, _ = oracle.decode(q, ks, vs, cu_short, 4, 4, 128, default_scale(128), max_seqlen=300)
    assert f64_check(o_drop, t, bound)["f64_violations"] > 0
    o_scaled = oracle.f32_to_f16(t.astype(np.float32) * np.float32(1 + 2.0 ** -6))
    assert f64_check(o_scaled, t, bound)["f64_violations"] > 0


def _build_mutant(tmp_path, n):
    import subprocess
    src = os.path.join(oracle.HERE, "fmha_oracle.cpp")
    out = os.path.join(str(tmp_path), f"liboracle_mutant{n}.so")
    subprocess.run(["g++", "-O2", "-std=c++17", "-fopenmp", "-fPIC", "-shared", f"-DORACLE_MUTANT={n}", "-o", out,
                    src], check=True)
    return out


@pytest.mark.parametrize("mutant", [1, 2, 3, 4])
def test_long_row_checks_reject_planted_mistakes(mutant, tmp_path, monkeypatch):
    """Each planted mistake (ORACLE_MUTANT in fmha_oracle.cpp) in the loop over
    rows past 16 makes at least one long-row check fail; the short-row
    fixtures still pass, so only the long-row checks see these mistakes."""
    import ctypes
    path = _build_mutant(tmp_path, mutant)
    monkeypatch.setattr(oracle, "_lib", None)
    monkeypatch.setattr(oracle, "LIB_PATH", path)
    oracle.lib()
    assert isinstance(oracle._lib, ctypes.CDLL)
    failed = _long_row_failures()
    assert failed, f"mutant {mutant} passed every long-row check"
    for path_fx in sorted(glob.glob(os.path.join(GOLDEN, "mha_*.npz"))):
        z = np.load(path_fx, allow_pickle=False)
        B, Hq, Hkv, D = z["meta"].tolist()
        o, _ = oracle.decode(z["q"], z["k"], z["v"], z["cu"], Hq, Hkv, D, default_scale(D))
        assert np.array_equal(o, z["o"])
