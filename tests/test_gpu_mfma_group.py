"""GPU parity of the matrix-core kernel (fmha_decode_group_kernel) against the
CPU oracle, through the packed-layout and strided entry points.

The library runs the kernel for every group size G = Hq / Hkv above 8 and
for the G <= 8 shapes where it measures faster than the VALU kernel; here
every test but the last ones forces it (FMHA_DECODE_GQA_KERNEL=mfma) so that
it meets every G, and the last ones cover the VALU kernel on G = 3, 5, 6, 7
and the library's own choice.  The
reference has no GQA (its kernels index K/V with the query head,
fmha_mfma_4x4x4_kernel.hpp:195-196); the oracle's mapping is KV head h / G
(fmha_host.cpp:169-245 otherwise).  Coverage: non-power-of-two and large G,
every length 0..16 in one varlen batch, uniform lengths, KV-head counts below
and not dividing a wave's 64 / (D/8) streams (waves spanning batches),
several waves per stream group (G * streams per wave > 64 query rows),
the S = 1 known answer, NaN-poisoned neighbour streams and batches,
invalid lengths, and strided caches (BHSD, padded BSHD with NaN padding).
"""
import numpy as np
import pytest

import oracle
import functools

from tests import common
from tests.common import assert_pass, check, cu_from_seqlens, default_scale, make_inputs

# FMHA_DECODE_GQA_KERNEL selects the kernel of the tree-order entry points
# (fmha_decode_fwd_fast, fmha_decode_fwd_uniform_fast, fmha_decode_fwd_strided);
# every call here goes through them.
run_gpu = functools.partial(common.run_gpu, fast=True)

pytestmark = pytest.mark.gpu


@pytest.fixture(autouse=True)
def mfma(monkeypatch):
    """Every test here runs the matrix-core kernel unless it asks otherwise
    (the valu and default_policy fixtures, requested after this one)."""
    monkeypatch.setenv("FMHA_DECODE_GQA_KERNEL", "mfma")


def _case(B, Hq, Hkv, D, seqlens, seed, std=1.0, uniform=False):
    q, k, v, cu = make_inputs(B, Hq, Hkv, D, seqlens, seed, std)
    o = run_gpu(q, k, v, cu, Hq, Hkv, D, uniform_s=(int(seqlens[0]) if uniform else None))
    st = check(o, q, k, v, cu, Hq, Hkv, D)
    assert_pass(st, f"B={B} Hq={Hq} Hkv={Hkv} D={D} seed={seed} uniform={uniform}")
    return o, (q, k, v, cu)


def _all_lengths(seed, reps=2):
    seqlens = np.array(list(range(17)) * reps, dtype=np.int32)
    np.random.default_rng(seed).shuffle(seqlens)
    return seqlens


@pytest.mark.parametrize("D", [64, 128, 256])
@pytest.mark.parametrize("G", [3, 5, 6, 7, 12, 16])
def test_group_sizes_varlen(D, G):
    """Group sizes the VALU kernel does not take, every length 0..16."""
    Hkv = 4
    seqlens = _all_lengths(D * 31 + G)
    _case(len(seqlens), Hkv * G, Hkv, D, seqlens, seed=1000 + D + G)


@pytest.mark.parametrize("D", [64, 128, 256])
@pytest.mark.parametrize("G", [24, 32, 64])
def test_large_groups(D, G):
    """More query rows per stream group than one wave takes: several waves
    per stream group (query chunks), MQA-like shapes."""
    for Hkv in (1, 2):
        seqlens = np.random.default_rng(G + Hkv).integers(0, 17, size=21).astype(np.int32)
        _case(len(seqlens), Hkv * G, Hkv, D, seqlens, seed=1100 + D + G + Hkv)


@pytest.mark.parametrize("D", [64, 128, 256])
@pytest.mark.parametrize("Hkv", [1, 2, 3, 5, 6, 7, 9])
def test_kv_heads_across_waves(D, Hkv):
    """KV-head counts below a wave's streams, or not dividing them: one wave
    reads several batches, or ends inside a batch."""
    G = 5
    seqlens = np.random.default_rng(Hkv * 13 + D).integers(0, 17, size=23).astype(np.int32)
    _case(len(seqlens), Hkv * G, Hkv, D, seqlens, seed=1200 + D + Hkv)


@pytest.mark.parametrize("S", [0, 1, 2, 3, 5, 8, 9, 16])
@pytest.mark.parametrize("D", [64, 128, 256])
def test_uniform_lengths(S, D):
    _case(29, 24, 8, D, np.full(29, S, np.int32), seed=1300 + S + D, uniform=True)


@pytest.mark.parametrize("D", [64, 128, 256])
@pytest.mark.parametrize("G", [1, 2, 4, 8])
def test_forced_on_valu_group_sizes(mfma, D, G):
    """The matrix-core kernel on the group sizes the VALU kernel also serves,
    including the reference's own Poisson-length workload shape."""
    Hkv = 4 if G > 1 else 16
    seqlens = _all_lengths(D + G)
    _case(len(seqlens), Hkv * G, Hkv, D, seqlens, seed=1400 + D + G)
    ref = oracle.generate_seqlens(10, 16)
    _case(10, 16, 16, 128, ref, seed=1450 + G)


@pytest.mark.parametrize("std", [0.25, 2.0, 4.0])
def test_logit_spread(std):
    seqlens = oracle.generate_seqlens(48, 16)
    _case(48, 40, 8, 128, seqlens, seed=1500, std=std)
    _case(48, 48, 8, 256, seqlens, seed=1501, std=std)


def test_s1_known_answer_bitexact():
    """S = 1: the weight is exactly 1, so O = fp16(V of the query's KV head)."""
    B, Hq, Hkv, D = 17, 20, 4, 128
    q, k, v, cu = make_inputs(B, Hq, Hkv, D, np.ones(B, np.int32), seed=1600)
    vf = oracle.f32_to_f16(oracle.bf16_to_f32(v)).reshape(B, Hkv, D)
    expect = np.repeat(vf, Hq // Hkv, axis=1)
    for uniform in (False, True):
        o = run_gpu(q, k, v, cu, Hq, Hkv, D, uniform_s=1 if uniform else None)
        assert np.array_equal(o.reshape(B, Hq, D), expect)


@pytest.mark.parametrize("D", [64, 128, 256])
def test_poisoned_neighbour_streams(D):
    """No product mixes two streams: NaN in every other (batch, KV head) --
    including streams that share a wave with the one checked -- leaves the
    checked stream's outputs equal to running it alone."""
    nan = np.uint16(0x7FC0)
    for Hkv, G in ((3, 5), (1, 6), (8, 3)):
        Hq = Hkv * G
        seqlens = np.array([16, 7, 16, 9], np.int32)
        q, k, v, cu = make_inputs(4, Hq, Hkv, D, seqlens, seed=1700 + Hkv + D)
        b, h = 1, Hkv - 1
        kp = np.full_like(k, nan)
        vp = np.full_like(v, nan)
        kp[cu[b]:cu[b + 1], h] = k[cu[b]:cu[b + 1], h]
        vp[cu[b]:cu[b + 1], h] = v[cu[b]:cu[b + 1], h]
        o = run_gpu(q, kp, vp, cu, Hq, Hkv, D).reshape(4, Hq, D)
        got = o[b, h * G:(h + 1) * G]
        cb = cu_from_seqlens([seqlens[b]])
        ks = k[cu[b]:cu[b + 1], h:h + 1]
        vs = v[cu[b]:cu[b + 1], h:h + 1]
        qs = q[b:b + 1, h * G:(h + 1) * G]
        r, slack = oracle.decode(qs, ks, vs, cb, G, 1, D, default_scale(D), with_slack=True)
        assert_pass(oracle.compare(got.reshape(r.shape), r, slack), f"Hkv={Hkv} G={G} D={D}")


def test_bad_lengths_give_nan():
    """A cu_seqlens span outside [0, 16]: that batch's rows are NaN, the
    batches that share its waves are unaffected."""
    Hkv, G, D = 1, 6, 128
    seqlens = np.array([4, 17, 3, 16, 2], np.int32)
    q, k, v, cu = make_inputs(5, Hkv * G, Hkv, D, seqlens, seed=1800)
    o = run_gpu(q, k, v, cu, Hkv * G, Hkv, D).reshape(5, Hkv * G, D)
    assert np.all(np.isnan(oracle.f16_to_f32(o[1])))
    for b in (0, 2, 3, 4):
        cb = cu_from_seqlens([seqlens[b]])
        r, slack = oracle.decode(q[b:b + 1], k[cu[b]:cu[b + 1]], v[cu[b]:cu[b + 1]], cb, Hkv * G, Hkv, D,
                                 default_scale(D), with_slack=True)
        assert_pass(oracle.compare(o[b:b + 1], r, slack), f"batch {b}")


def test_mfma_matches_valu_within_gate(mfma, monkeypatch):
    """Same inputs through both kernels (G = 4): each passes the oracle gate
    and they agree within it."""
    B, Hq, Hkv, D = 64, 32, 8, 128
    seqlens = oracle.generate_seqlens(B, 16)
    q, k, v, cu = make_inputs(B, Hq, Hkv, D, seqlens, seed=1900)
    o_mfma = run_gpu(q, k, v, cu, Hq, Hkv, D)
    monkeypatch.setenv("FMHA_DECODE_GQA_KERNEL", "valu")
    o_valu = run_gpu(q, k, v, cu, Hq, Hkv, D)
    r, slack = oracle.decode(q, k, v, cu, Hq, Hkv, D, default_scale(D), with_slack=True)
    assert_pass(oracle.compare(o_mfma, r, slack), "mfma")
    assert_pass(oracle.compare(o_valu, r, slack), "valu")
    assert_pass(oracle.compare(o_mfma, o_valu, slack), "mfma vs valu")


def _bf16_dev(gen, shape, dev):
    import torch
    return torch.randn(*shape, generator=gen, device=dev, dtype=torch.bfloat16)


def _bits(t):
    import torch
    return t.contiguous().view(torch.int16).cpu().numpy().view(np.uint16)


@pytest.mark.parametrize("layout", ["bhsd", "bshd"])
@pytest.mark.parametrize("D,Hq,Hkv", [(128, 15, 5), (64, 24, 8), (256, 12, 2), (128, 6, 1), (128, 40, 2)])
def test_strided_layouts(layout, D, Hq, Hkv):
    """Strided caches (BHSD through a transposed view, padded BSHD) with
    per-batch lengths below the padding; padding rows hold NaN and must not
    be read."""
    import torch
    import fmha_amd
    dev = torch.device("cuda", 0)
    gen = torch.Generator(device=dev).manual_seed(D * 100 + Hq + Hkv)
    B, cap = 23, 12
    seqlens = np.random.default_rng(Hq + Hkv).integers(0, cap + 1, size=B).astype(np.int32)
    q = _bf16_dev(gen, (B, Hq, 1, D), dev)
    if layout == "bhsd":
        kc = _bf16_dev(gen, (B, Hkv, cap, D), dev)
        vc = _bf16_dev(gen, (B, Hkv, cap, D), dev)
        for b in range(B):
            kc[b, :, seqlens[b]:] = float("nan")
            vc[b, :, seqlens[b]:] = float("nan")
        k, v = kc.transpose(1, 2), vc.transpose(1, 2)
    else:
        k = _bf16_dev(gen, (B, cap, Hkv, D), dev)
        v = _bf16_dev(gen, (B, cap, Hkv, D), dev)
        for b in range(B):
            k[b, seqlens[b]:] = float("nan")
            v[b, seqlens[b]:] = float("nan")
    o = fmha_amd.fmha_decode_strided(q, k, v, seqlens_kv=torch.from_numpy(seqlens).to(dev))
    torch.cuda.synchronize()
    pk = np.concatenate([_bits(k[b, :seqlens[b]]).reshape(-1, Hkv, D) for b in range(B)])
    pv = np.concatenate([_bits(v[b, :seqlens[b]]).reshape(-1, Hkv, D) for b in range(B)])
    r, slack = oracle.decode(_bits(q).reshape(B, Hq, D), pk, pv, cu_from_seqlens(seqlens), Hq, Hkv, D,
                             default_scale(D), with_slack=True)
    assert_pass(oracle.compare(_bits(o).reshape(r.shape), r, slack), f"{layout} D={D} Hq={Hq} Hkv={Hkv}")


@pytest.mark.parametrize("S", [1, 7, 16])
def test_strided_uniform_and_bad_length(S):
    """Uniform strided lengths; a per-batch length above the cache's rows gives
    NaN for that batch only."""
    import torch
    import fmha_amd
    dev = torch.device("cuda", 0)
    gen = torch.Generator(device=dev).manual_seed(S)
    B, Hq, Hkv, D = 19, 21, 3, 128
    q = _bf16_dev(gen, (B, Hq, 1, D), dev)
    k = _bf16_dev(gen, (B, S, Hkv, D), dev)
    v = _bf16_dev(gen, (B, S, Hkv, D), dev)
    o = fmha_amd.fmha_decode_strided(q, k, v)
    torch.cuda.synchronize()
    seqlens = np.full(B, S, np.int32)
    r, slack = oracle.decode(_bits(q).reshape(B, Hq, D), _bits(k).reshape(-1, Hkv, D), _bits(v).reshape(-1, Hkv, D),
                             cu_from_seqlens(seqlens), Hq, Hkv, D, default_scale(D), with_slack=True)
    assert_pass(oracle.compare(_bits(o).reshape(r.shape), r, slack), f"uniform S={S}")
    lens = np.full(B, S, np.int32)
    lens[4] = S + 1
    o2 = fmha_amd.fmha_decode_strided(q, k, v, seqlens_kv=torch.from_numpy(lens).to(dev))
    torch.cuda.synchronize()
    o2b = oracle.f16_to_f32(_bits(o2).reshape(B, Hq, D))
    assert np.all(np.isnan(o2b[4]))
    keep = [b for b in range(B) if b != 4]
    assert np.array_equal(_bits(o2).reshape(B, Hq, D)[keep], _bits(o).reshape(B, Hq, D)[keep])


@pytest.fixture
def valu(monkeypatch):
    monkeypatch.setenv("FMHA_DECODE_GQA_KERNEL", "valu")


@pytest.mark.parametrize("D", [64, 128, 256])
@pytest.mark.parametrize("G", [3, 5, 6, 7])
def test_valu_padded_group_sizes(valu, D, G):
    """G = 3, 5, 6, 7 on the VALU kernel's 4- and 8-head instantiations (the
    extra query heads of each KV head load and store nothing): every length
    0..16, a wave spanning several batches (Hkv = 1), and neighbouring rows
    of Q and O left untouched."""
    for Hkv in (4, 1):
        seqlens = _all_lengths(D * 7 + G + Hkv)
        o, _ = _case(len(seqlens), Hkv * G, Hkv, D, seqlens, seed=2000 + D + G + Hkv)


def test_valu_padded_fp32_weights_and_paged():
    """The fp32-weight and workspace-less paged entries (VALU kernel only)
    with G = 5 and 3: oracle parity (fp32 weights against the oracle's
    fp32-weight mode)."""
    import torch
    import fmha_amd
    seqlens = oracle.generate_seqlens(40, 16)
    q, k, v, cu = make_inputs(40, 20, 4, 128, seqlens, seed=2100)
    qd = torch.from_numpy(q.view(np.int16)).cuda().view(torch.bfloat16)
    kd = torch.from_numpy(k.view(np.int16)).cuda().view(torch.bfloat16)
    vd = torch.from_numpy(v.view(np.int16)).cuda().view(torch.bfloat16)
    cud = torch.from_numpy(cu).cuda()
    o32 = fmha_amd.fmha_decode(qd, kd, vd, cu_seqlens_kv=cud, fp32_weights=True)
    torch.cuda.synchronize()
    r32, _ = oracle.decode(q, k, v, cu, 20, 4, 128, default_scale(128), p_mode=1)
    assert_pass(oracle.compare(o32.view(torch.int16).cpu().numpy().view(np.uint16).reshape(r32.shape), r32),
                "fp32 weights G=5")
    # paged, 4-row pages, G = 3
    Hq, Hkv, D, ps = 12, 4, 128, 4
    q2, k2, v2, cu2 = make_inputs(40, Hq, Hkv, D, seqlens, seed=2101)
    need = [(int(s) + ps - 1) // ps for s in seqlens]
    bt = np.zeros((40, max(need)), np.int32)
    kc = np.zeros((sum(need), ps, Hkv, D), np.uint16)
    vc = np.zeros_like(kc)
    page = 0
    for b in range(40):
        for p in range(need[b]):
            r0, r1 = cu2[b] + p * ps, min(cu2[b] + (p + 1) * ps, cu2[b + 1])
            kc[page, :r1 - r0] = k2[r0:r1]
            vc[page, :r1 - r0] = v2[r0:r1]
            bt[b, p] = page
            page += 1
    to = lambda a: torch.from_numpy(np.ascontiguousarray(a).view(np.int16)).cuda().view(torch.bfloat16)
    o2 = fmha_amd.fmha_decode_paged(to(q2), to(kc), to(vc), torch.from_numpy(bt).cuda(),
                                    torch.from_numpy(seqlens).cuda())
    torch.cuda.synchronize()
    r2, slack = oracle.decode(q2, k2, v2, cu2, Hq, Hkv, D, default_scale(D), with_slack=True)
    assert_pass(oracle.compare(o2.view(torch.int16).cpu().numpy().view(np.uint16).reshape(r2.shape), r2, slack),
                "paged G=3")


@pytest.fixture
def default_policy(monkeypatch):
    monkeypatch.delenv("FMHA_DECODE_GQA_KERNEL", raising=False)


@pytest.mark.parametrize("D", [64, 128, 256])
@pytest.mark.parametrize("G", [3, 5, 7, 12])
def test_default_kernel_choice(default_policy, D, G):
    """The library's own kernel choice (no override): varlen lengths 0..16
    and uniform lengths 4 and 16, which take different kernels for some
    (G, D)."""
    Hkv = 4
    seqlens = _all_lengths(D * 13 + G)
    _case(len(seqlens), Hkv * G, Hkv, D, seqlens, seed=2200 + D + G)
    for S in (4, 16):
        seqlens = np.full(24, S, np.int32)
        _case(24, Hkv * G, Hkv, D, seqlens, seed=2300 + D + G + S, uniform=True)
