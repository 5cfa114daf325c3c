"""GPU parity of the split-KV path (fmha_decode_fwd_splitkv), lengths beyond
the reference's 16: the oracle runs the reference loop over the longer rows
(oracle.decode(max_seqlen=...)), gate as in tests/common.py."""
import numpy as np
import pytest

import oracle
from tests.common import assert_pass, cu_from_seqlens, default_scale, last_plan, make_inputs, to_dev
from tests.common import plan_kinds as _kinds, plan_launch as _launch

pytestmark = pytest.mark.gpu


def _run(q, k, v, cu, Hq, Hkv, D, max_len):
    import torch
    import fmha_amd
    o = fmha_amd.fmha_decode_splitkv(to_dev(q), to_dev(k), to_dev(v), torch.from_numpy(cu).cuda(), max_len,
                                     softmax_scale=default_scale(D))
    torch.cuda.synchronize()
    return o.view(torch.int16).cpu().numpy().view(np.uint16)


def _case(B, Hq, Hkv, D, seqlens, max_len, seed, std=1.0):
    """Oracle parity of one call; returns the call's plan (last_plan)."""
    q, k, v, cu = make_inputs(B, Hq, Hkv, D, seqlens, seed, std)
    o = _run(q, k, v, cu, Hq, Hkv, D, max_len)
    plan = last_plan()
    r, slack = oracle.decode(q, k, v, cu, Hq, Hkv, D, default_scale(D), with_slack=True, max_seqlen=max_len)
    st = oracle.compare(o.reshape(r.shape), r, slack)
    print(f"B={B} Hq={Hq} Hkv={Hkv} D={D} max={max_len}: {st} plan={plan}", flush=True)
    assert_pass(st, f"splitkv B={B} D={D} max={max_len}")
    return plan


@pytest.mark.parametrize("D,Hq,Hkv", [(128, 16, 16), (64, 32, 4), (256, 16, 8), (128, 8, 1), (128, 32, 8),
                                     (256, 16, 4)])
@pytest.mark.parametrize("max_len", [17, 100, 700, 2048])
def test_varlen_long(D, Hq, Hkv, max_len):
    rng = np.random.default_rng(max_len + D)
    B = 6
    seqlens = rng.integers(0, max_len + 1, size=B).astype(np.int32)
    seqlens[0] = max_len
    _case(B, Hq, Hkv, D, seqlens, max_len, seed=max_len * 3 + D)


@pytest.mark.parametrize("D,Hq,Hkv", [(128, 32, 8), (64, 16, 2), (256, 8, 8)])
def test_block_boundaries(D, Hq, Hkv):
    """Lengths on and next to the 16-row block edges: scores waves whose
    block is partly past the row's end, P.V sub-blocks likewise."""
    seqlens = np.array([16, 32, 48, 31, 33, 47, 15, 17, 1, 64], np.int32)
    _case(len(seqlens), Hq, Hkv, D, seqlens, 64, seed=11 + D)


def test_mid_chunk_count():
    """16 < chunks <= 256 with four query heads per KV head: rows of more
    P.V waves than one combine group (16), summed in two levels."""
    rng = np.random.default_rng(12)
    seqlens = rng.integers(6000, 8193, size=4).astype(np.int32)
    seqlens[0] = 8192
    _case(4, 32, 8, 128, seqlens, 8192, seed=12, std=0.5)
    assert 16 < _launch("split")["chunks"] <= 256


def test_mid_block_count():
    """512 < blocks <= 2048 on one long row: the 256-thread statistics pass."""
    _case(1, 32, 8, 128, np.array([20000], np.int32), 20000, seed=13, std=0.5)
    split = _launch("split")
    assert 512 < split["blocks"] <= 2048 and split["passes"] == 4


# (B, Hq, Hkv, D, max_len, kind, passes): rows of up to 64 blocks, whose P.V
# waves reduce the block statistics themselves (no statistics pass), and one
# block more; one chunk per row (O from the P.V pass) or several (combine).
STAT_CASES = [
    (6, 32, 8, 128, 1024, "split", 3),
    (6, 32, 8, 128, 1040, "split", 4),
    (256, 32, 8, 128, 1024, "split", 2),
    (256, 32, 8, 128, 1040, "split", 4),
    (8, 8, 2, 64, 1000, "split", 3),               # lane groups on several chunks
    (8, 64, 4, 128, 1024, "split_matrix_core", 3),
    (8, 64, 4, 128, 1040, "split_matrix_core", 4),
    (512, 64, 4, 256, 700, "split_matrix_core", 2),
]


@pytest.mark.parametrize("B,Hq,Hkv,D,max_len,kind,passes", STAT_CASES)
def test_block_statistics_in_pv(monkeypatch, B, Hq, Hkv, D, max_len, kind, passes):
    """The P.V waves' own reduction of the block statistics, at and past its
    64-block limit, with ragged lengths (0, 1, one block, the maximum); the
    matrix-core single passes off (FMHA_DECODE_ONEPASS_MFMA=0,
    FMHA_DECODE_ONEPASS_REG=0)."""
    monkeypatch.setenv("FMHA_DECODE_ONEPASS_MFMA", "0")
    monkeypatch.setenv("FMHA_DECODE_ONEPASS_REG", "0")
    rng = np.random.default_rng(B + max_len + Hq)
    seqlens = rng.integers(0, max_len + 1, size=B).astype(np.int32)
    seqlens[:4] = [max_len, 0, 1, 16]
    _case(B, Hq, Hkv, D, seqlens, max_len, seed=B * 7 + D + Hq, std=0.5)
    assert _launch(kind)["passes"] == passes


@pytest.mark.parametrize("max_len", [16, 5])
def test_short_lengths_match_short_path(max_len):
    """max_seqlen_kv <= 16 through the split-KV entry (the short kernel runs
    it): oracle parity, and NaN for a batch longer than max_seqlen_kv."""
    seqlens = np.minimum(oracle.generate_seqlens(300, 16), max_len).astype(np.int32)
    _case(300, 16, 16, 128, seqlens, max_len, seed=5)
    assert _launch("short")["numerics"] == "exact"
    if max_len < 16:
        bad = seqlens.copy()
        bad[7] = max_len + 1
        q, k, v, cu = make_inputs(300, 16, 16, 128, bad, seed=6)
        o = oracle.f16_to_f32(_run(q, k, v, cu, 16, 16, 128, max_len).reshape(300, 16, 128))
        assert np.all(np.isnan(o[7])) and np.all(np.isfinite(np.delete(o, 7, axis=0)))


def test_many_batches_direct_path():
    """max length fits one chunk: the PV kernel writes O directly."""
    seqlens = np.random.default_rng(3).integers(0, 41, size=200).astype(np.int32)
    _case(200, 8, 8, 128, seqlens, 40, seed=6)
    split = _launch("split")
    assert split["chunks"] == 1 and split["passes"] == 2


def test_one_long_sequence():
    """More than 256 chunks (the 1024-thread combine), more than 2048 blocks
    (the 1024-thread statistics)."""
    _case(1, 32, 8, 128, np.array([40000], np.int32), 40000, seed=7, std=0.5)
    split = _launch("split")
    assert split["chunks"] > 256 and split["blocks"] > 2048 and split["passes"] == 4


# (B, Hq, Hkv, D, max_len): fewer (batch, KV-head group) units than the
# one-wave single pass needs, but enough for two waves per row, rows that fit
# a workgroup's LDS.
GROUP_CASES = [
    (64, 16, 16, 128, 256),
    (200, 32, 8, 128, 96),
    (100, 16, 16, 128, 512),
    (64, 32, 32, 64, 256),
    (60, 16, 8, 256, 160),
    (96, 8, 8, 128, 64),     # two blocks per wave
]


@pytest.mark.parametrize("B,Hq,Hkv,D,max_len", GROUP_CASES)
def test_onepass_group(monkeypatch, B, Hq, Hkv, D, max_len):
    """The single pass with two waves per row: ragged lengths (0, 1, one
    block, the maximum, one past a wave's rows) and an invalid one (NaN);
    the register single pass off (it takes groups of 2 and 4 at D = 128
    first)."""
    monkeypatch.setenv("FMHA_DECODE_ONEPASS_REG", "0")
    rng = np.random.default_rng(B + max_len + D)
    seqlens = rng.integers(0, max_len + 1, size=B).astype(np.int32)
    seqlens[:5] = [max_len, 0, 1, 16, min(max_len, 33)]
    _case(B, Hq, Hkv, D, seqlens, max_len, seed=B + D + 5, std=0.5)
    assert _launch("onepass_group")["waves_per_row"] == 2
    bad = seqlens.copy()
    bad[3] = max_len + 1
    q, k, v, cu = make_inputs(B, Hq, Hkv, D, bad, seed=B + 3)
    o = oracle.f16_to_f32(_run(q, k, v, cu, Hq, Hkv, D, max_len).reshape(B, Hq, D))
    assert np.all(np.isnan(o[3])) and np.all(np.isfinite(np.delete(o, 3, axis=0)))


def test_onepass_group_off(monkeypatch):
    """FMHA_DECODE_ONEPASS_WAVES=1 (and the register single pass off): the
    same rows through the split passes."""
    monkeypatch.setenv("FMHA_DECODE_ONEPASS_WAVES", "1")
    monkeypatch.setenv("FMHA_DECODE_ONEPASS_REG", "0")
    seqlens = np.random.default_rng(1).integers(0, 257, size=64).astype(np.int32)
    _case(64, 16, 16, 128, seqlens, 256, seed=41, std=0.5)
    assert _kinds() == ["split"]


# (B, Hq, Hkv, D, max_len, waves, force): the matrix-core single pass with
# the scores in LDS (8 to 16 query heads per KV head after padding, at least
# 512 (batch, KV head) units, a row's scores within a workgroup's LDS): the
# planner's one wave per row at D = 256 up to 40 blocks, and at D = 128 and
# 64, where the register single pass takes every row this one fits, the
# waves per row FMHA_DECODE_ONEPASS_MFMA forces; the register single pass
# off (FMHA_DECODE_ONEPASS_REG=0).
MFMA_ONEPASS_CASES = [
    (256, 64, 8, 128, 1024, 2, "2"),    # G = 8
    (512, 16, 1, 128, 600, 2, "2"),     # G = 16, one KV head
    (128, 40, 8, 128, 700, 2, "2"),     # G = 5 on a group padded to 8
    (64, 96, 8, 128, 300, 2, "2"),      # G = 12 on a group padded to 16
    (600, 16, 2, 128, 150, 1, "1"),     # 10 blocks, one wave
    (512, 8, 1, 128, 1600, 4, "4"),     # 100 blocks, four waves
    (256, 32, 4, 256, 500, 1, None),    # D = 256, the planner's
    (600, 8, 1, 64, 1200, 2, "2"),      # D = 64
    (300, 16, 2, 128, 200, 4, "4"),     # four waves on a short row
]


def _nan_row_check(B, Hq, Hkv, D, seqlens, max_len):
    """A length above max_seqlen_kv: NaN for that batch only."""
    bad = seqlens.copy()
    bad[3] = max_len + 1
    q, k, v, cu = make_inputs(B, Hq, Hkv, D, bad, seed=B + 9)
    o = oracle.f16_to_f32(_run(q, k, v, cu, Hq, Hkv, D, max_len).reshape(B, Hq, D))
    assert np.all(np.isnan(o[3])) and np.all(np.isfinite(np.delete(o, 3, axis=0)))


@pytest.mark.parametrize("B,Hq,Hkv,D,max_len,waves,force", MFMA_ONEPASS_CASES)
def test_onepass_matrix_core(monkeypatch, B, Hq, Hkv, D, max_len, waves, force):
    """Groups of 8-16 query heads on the matrix-core single pass with the
    scores in LDS (1, 2 or 4 waves per (batch, KV head)): ragged lengths (0,
    1, one block, a round's rows and one past them, the maximum) and an
    invalid one (NaN)."""
    if force:
        monkeypatch.setenv("FMHA_DECODE_ONEPASS_MFMA", force)
    else:
        monkeypatch.delenv("FMHA_DECODE_ONEPASS_MFMA", raising=False)
    monkeypatch.setenv("FMHA_DECODE_ONEPASS_REG", "0")
    rng = np.random.default_rng(B + max_len + D + Hq)
    seqlens = rng.integers(0, max_len + 1, size=B).astype(np.int32)
    seqlens[:6] = [max_len, 0, 1, 16, min(max_len, 64), min(max_len, 65)]
    _case(B, Hq, Hkv, D, seqlens, max_len, seed=B + D + Hq, std=0.5)
    assert _launch("onepass_matrix_core")["waves_per_row"] == waves
    _nan_row_check(B, Hq, Hkv, D, seqlens, max_len)


def test_onepass_matrix_core_off(monkeypatch):
    """FMHA_DECODE_ONEPASS_MFMA=0 and FMHA_DECODE_ONEPASS_REG=0: the same
    rows through the matrix-core split passes."""
    monkeypatch.setenv("FMHA_DECODE_ONEPASS_MFMA", "0")
    monkeypatch.setenv("FMHA_DECODE_ONEPASS_REG", "0")
    seqlens = np.random.default_rng(2).integers(0, 1025, size=256).astype(np.int32)
    _case(256, 64, 8, 128, seqlens, 1024, seed=42, std=0.5)
    assert _kinds() == ["split_matrix_core"]


# (B, Hq, Hkv, D, max_len, waves, tiles, force): the matrix-core single pass
# with the scores in registers (at least 128-256 (batch, KV head) units by
# head dim and group, and 4 blocks,
# ceil(blocks / tiles) <= 8 waves per row), groups of 8-16 through
# the matrix-core launcher and of 2 and 4 through the VALU one where the
# one-wave single pass does not hold the row: 8 tiles per wave up to 32
# blocks, 16 up to 128, else 32, or what FMHA_DECODE_ONEPASS_REG forces.
REG_ONEPASS_CASES = [
    (256, 64, 8, 128, 1024, 4, 16, None),   # G = 8
    (512, 16, 1, 128, 600, 3, 16, None),    # G = 16, one KV head
    (128, 40, 8, 128, 700, 3, 16, None),    # G = 5 on a group padded to 8
    (64, 96, 8, 128, 300, 3, 8, None),      # G = 12 on a group padded to 16
    (600, 16, 2, 128, 150, 2, 8, None),     # 10 blocks
    (70, 128, 8, 128, 2000, 8, 16, None),   # eight waves, G = 16
    (128, 32, 8, 128, 256, 2, 8, None),     # G = 4 (the VALU launcher)
    (512, 8, 2, 128, 128, 1, 8, None),      # G = 4, one wave
    (64, 32, 16, 128, 256, 2, 8, None),     # G = 2
    (600, 8, 1, 64, 1200, 5, 16, None),     # D = 64
    (1024, 32, 4, 64, 128, 1, 8, None),     # D = 64, one wave
    (256, 32, 4, 256, 500, 2, 16, "16"),    # D = 256, forced
    (256, 32, 4, 256, 1000, 4, 16, None),   # D = 256 beyond 40 blocks
    (300, 16, 2, 128, 200, 1, 16, "16"),    # 16 tiles on a short row, forced
    (64, 32, 8, 128, 4096, 8, 32, None),    # 32 tiles, G = 4, rows of 4096
    (256, 16, 2, 128, 2100, 5, 32, None),   # 32 tiles, G = 8
    (512, 16, 1, 64, 2500, 5, 32, None),    # 32 tiles, D = 64, G = 16
    (256, 16, 4, 64, 1000, 4, 16, None),    # D = 64, G = 4 (the VALU launcher)
    (128, 16, 2, 128, 1024, 4, 16, None),   # 256 units, G = 8
    (16, 64, 8, 128, 1024, 4, 16, None),    # 128 units, G = 8
    (64, 16, 4, 128, 512, 4, 8, None),      # 256 units, G = 4
    (16, 64, 8, 64, 2048, 8, 16, None),     # 128 units, D = 64
    (32, 64, 8, 256, 1024, 4, 16, None),    # 256 units, D = 256
    (4200, 4, 1, 64, 160, 2, 8, None),      # D = 64, G = 4, one KV head (the VALU launcher's several batches per wave)
]


@pytest.mark.parametrize("B,Hq,Hkv,D,max_len,waves,tiles,force", REG_ONEPASS_CASES)
def test_onepass_registers(monkeypatch, B, Hq, Hkv, D, max_len, waves, tiles, force):
    """The matrix-core single pass with each wave's scores in registers:
    ragged lengths (0, 1, one block, four blocks and one row past them, the
    maximum), waves with no rows, and an invalid length (NaN)."""
    if force:
        monkeypatch.setenv("FMHA_DECODE_ONEPASS_REG", force)
    else:
        monkeypatch.delenv("FMHA_DECODE_ONEPASS_REG", raising=False)
    rng = np.random.default_rng(B + max_len + D + Hq + 1)
    seqlens = rng.integers(0, max_len + 1, size=B).astype(np.int32)
    seqlens[:6] = [max_len, 0, 1, 16, min(max_len, 64), min(max_len, 65)]
    _case(B, Hq, Hkv, D, seqlens, max_len, seed=B + D + Hq + 1, std=0.5)
    launch = _launch("onepass_matrix_core_regs")
    assert launch["waves_per_row"] == waves and launch["tiles_per_wave"] == tiles, launch
    _nan_row_check(B, Hq, Hkv, D, seqlens, max_len)


def test_onepass_registers_off(monkeypatch):
    """FMHA_DECODE_ONEPASS_REG=0: a group of 4 on the split passes."""
    monkeypatch.setenv("FMHA_DECODE_ONEPASS_REG", "0")
    seqlens = np.random.default_rng(3).integers(0, 257, size=128).astype(np.int32)
    _case(128, 32, 8, 128, seqlens, 256, seed=43, std=0.5)
    assert _kinds() == ["split"]


def test_wide_logits():
    seqlens = np.array([513, 1, 0, 257], np.int32)
    _case(4, 16, 16, 256, seqlens, 600, seed=8, std=2.0)


def test_bad_and_empty_lengths():
    import torch
    H, D = 4, 128
    seqlens = [20, 0, 30]
    q, k, v, cu = make_inputs(3, H, H, D, seqlens, seed=9)
    o = _run(q, k, v, cu, H, H, D, 25).reshape(3, H, D)   # batch 2 is longer than max
    f = oracle.f16_to_f32(o)
    assert np.all(np.isnan(f[2])) and np.all(f[1] == 0) and np.all(np.isfinite(f[0]))
    r, slack = oracle.decode(q[:1], k[:20], v[:20], cu_from_seqlens([20]), H, H, D, default_scale(D),
                             with_slack=True, max_seqlen=25)
    assert_pass(oracle.compare(o[:1], r, slack), "batch 0")


# Single-pass path (onepass_decode_kernel): taken by fmha_decode_fwd_splitkv
# for many rows of a few 16-row blocks (the planner's rules in
# fmha_decode_launch.hpp: launch_split_dg); the tests below assert the plan
# the library reports for each call.


@pytest.mark.parametrize("D,Hq,Hkv,max_len,kind", [(128, 16, 16, 2048, "split"), (128, 32, 8, 8192, "split"),
                                                   (256, 16, 16, 6000, "split"), (64, 16, 2, 64, "split_matrix_core"),
                                                   (128, 32, 8, 64, "split")])
def test_split_path_still_covered(D, Hq, Hkv, max_len, kind):
    """Few batches: the split-KV launches (VALU, or matrix cores for groups
    of 8), not the single pass."""
    B = 10
    seqlens = np.random.default_rng(D + max_len).integers(0, max_len + 1, size=B).astype(np.int32)
    seqlens[0] = max_len
    _case(B, Hq, Hkv, D, seqlens, max_len, seed=D + max_len + Hq)
    assert _kinds() == [kind]


@pytest.mark.parametrize("D,B", [(64, 1024), (128, 512), (256, 256)])
@pytest.mark.parametrize("G", [1, 2, 4, 8])
def test_onepass_all_shapes(D, B, G):
    Hkv, max_len = 16, 96
    seqlens = np.random.default_rng(D + G).integers(0, max_len + 1, size=B).astype(np.int32)
    seqlens[0] = max_len
    _case(B, Hkv * G, Hkv, D, seqlens, max_len, seed=900 + D + G)
    assert _kinds() == ["onepass"]


@pytest.mark.parametrize("D,Hkv,B,max_len", [(64, 16, 1024, 96), (64, 1, 4100, 64), (128, 8, 1100, 96),
                                             (128, 2, 2050, 96), (256, 8, 600, 128), (256, 1, 1030, 128)])
def test_onepass_group_of_eight(D, Hkv, B, max_len):
    """G = 8 on the single pass at the longest rows it takes there for each
    head dim (one batch per wave, and several: Hkv = 1, 2), with the 16-row
    edges, empty rows and a last wave partly empty."""
    Hq = 8 * Hkv
    rng = np.random.default_rng(D * 3 + Hkv + B)
    seqlens = rng.integers(0, max_len + 1, size=B).astype(np.int32)
    seqlens[:7] = np.minimum([max_len, 0, 1, 15, 16, 17, 31], max_len)
    seqlens[-1] = max_len
    _case(B, Hq, Hkv, D, seqlens, max_len, seed=2000 + D + Hkv)
    assert _kinds() == ["onepass"]
    # one row more and the same lengths leave the single pass
    q, k, v, cu = make_inputs(B, Hq, Hkv, D, seqlens, seed=2000 + D + Hkv)
    _run(q, k, v, cu, Hq, Hkv, D, max_len + 1)
    assert "onepass" not in _kinds()


def test_onepass_edge_lengths():
    """Rows shorter than a head's lanes, on and next to the 16-row edges, the
    row bound itself and an empty row, in one batch that takes the single
    pass; an invalid length gives NaN for its batch only."""
    import torch
    B, Hq, Hkv, D, max_len = 2048, 32, 8, 128, 256
    edge = np.array([0, 1, 2, 3, 15, 16, 17, 31, 32, 33, 47, 48, 49, 255, 256], np.int32)
    seqlens = np.random.default_rng(31).integers(1, 64, size=B).astype(np.int32)
    seqlens[: len(edge)] = edge
    _case(B, Hq, Hkv, D, seqlens, max_len, seed=931)
    assert _kinds() == ["onepass"]
    bad = seqlens.copy()
    bad[5] = max_len + 1
    q, k, v, cu = make_inputs(B, Hq, Hkv, D, bad, seed=932)
    o = oracle.f16_to_f32(_run(q, k, v, cu, Hq, Hkv, D, max_len).reshape(B, Hq, D))
    assert np.all(np.isnan(o[5])) and np.all(np.isfinite(np.delete(o, 5, axis=0)))
    assert np.all(o[0] == 0)


# Fewer KV heads than a wave holds (64 / (D/8)): the split kernels give each
# lane group its own block (scores) or chunk (P.V), 2^shift per wave.
def _sub_units(Hkv, D):
    hpw = 64 // (D // 8)
    r = 1
    while Hkv * r * 2 <= hpw and hpw % (Hkv * r * 2) == 0:
        r *= 2
    return r


@pytest.mark.parametrize("D,Hq,Hkv,force_valu", [(64, 4, 1, False), (64, 8, 2, False), (64, 16, 4, False),
                                                (128, 4, 1, False), (128, 8, 2, False), (256, 4, 1, False),
                                                (128, 4, 2, False), (64, 8, 1, True), (64, 32, 4, True),
                                                (128, 16, 2, True), (256, 8, 1, True)])
@pytest.mark.parametrize("max_len", [300, 2050])
def test_sub_units(monkeypatch, D, Hq, Hkv, force_valu, max_len):
    """Lane groups of the VALU split passes serving different blocks and
    chunks: block and chunk counts that are not multiples of the groups per
    wave, empty and short rows next to long ones.  Groups of up to 4 take
    these passes by default; groups of 8 take the matrix-core split unless
    FMHA_DECODE_GQA_KERNEL=valu keeps them here."""
    if force_valu:
        monkeypatch.setenv("FMHA_DECODE_GQA_KERNEL", "valu")
    else:
        monkeypatch.delenv("FMHA_DECODE_GQA_KERNEL", raising=False)
    assert _sub_units(Hkv, D) > 1
    B = 5
    seqlens = np.array([max_len, 1, 0, max_len - 17, 33], np.int32)
    _case(B, Hq, Hkv, D, seqlens, max_len, seed=1300 + D + Hkv + max_len)
    assert _launch("split")["sub_units"] == _sub_units(Hkv, D)


@pytest.mark.parametrize("D,Hq,Hkv,B,max_len", [(128, 8, 1, 2047, 32), (128, 4, 1, 2047, 96), (64, 8, 2, 2050, 64),
                                                 (256, 8, 1, 1030, 32), (256, 4, 1, 1030, 96), (128, 8, 2, 1100, 96)])
def test_onepass_batches_per_wave(D, Hq, Hkv, B, max_len):
    """Single pass with several batches per wave (fewer KV heads than a wave
    holds): mixed lengths in one wave, empty rows, a last wave partly empty."""
    assert _sub_units(Hkv, D) > 1
    rng = np.random.default_rng(D + Hkv + B)
    seqlens = rng.integers(0, max_len + 1, size=B).astype(np.int32)
    seqlens[:6] = np.minimum([max_len, 0, 1, 17, 33, 95], max_len)
    _case(B, Hq, Hkv, D, seqlens, max_len, seed=1500 + D + Hkv)
    assert _launch("onepass")["batches_per_wave"] == _sub_units(Hkv, D)


def test_onepass_batches_per_wave_invalid_length():
    """An invalid length gives NaN for its batch only, the other batches of
    its wave stay exact."""
    import torch
    B, Hq, Hkv, D, max_len = 2048, 8, 1, 128, 32
    rng = np.random.default_rng(77)
    seqlens = rng.integers(1, max_len + 1, size=B).astype(np.int32)
    bad = 5
    q, k, v, cu = make_inputs(B, Hq, Hkv, D, seqlens, seed=1600)
    lens_bad = seqlens.copy()
    lens_bad[bad] = max_len + 3
    cu_bad = cu_from_seqlens(lens_bad)
    k2 = np.concatenate([k[:cu[bad + 1]], np.zeros((max_len + 3 - seqlens[bad], Hkv, D), np.uint16), k[cu[bad + 1]:]])
    v2 = np.concatenate([v[:cu[bad + 1]], np.zeros((max_len + 3 - seqlens[bad], Hkv, D), np.uint16), v[cu[bad + 1]:]])
    bits = _run(q, k2, v2, cu_bad, Hq, Hkv, D, max_len).reshape(B, Hq, D)
    assert _launch("onepass")["batches_per_wave"] > 1
    f = oracle.f16_to_f32(bits)
    assert np.all(np.isnan(f[bad]))
    keep = np.array([b for b in range(B) if b != bad])
    assert np.all(np.isfinite(f[keep]))
    r, slack = oracle.decode(q, k, v, cu, Hq, Hkv, D, default_scale(D), with_slack=True, max_seqlen=max_len)
    st = oracle.compare(np.ascontiguousarray(bits[keep]).ravel(),
                        np.ascontiguousarray(r.reshape(B, Hq, D)[keep]).ravel(),
                        np.ascontiguousarray(slack.reshape(B, Hq, D)[keep]).ravel())
    assert_pass(st, "neighbours of an invalid length, single pass")


@pytest.mark.parametrize("D,Hq,Hkv", [(128, 24, 8), (64, 20, 4), (256, 14, 2), (128, 7, 1), (128, 12, 2)])
@pytest.mark.parametrize("B,max_len", [(5, 700), (600, 48), (3, 17)])
def test_padded_query_group(D, Hq, Hkv, B, max_len):
    """Group sizes 3, 5, 6, 7 beyond 16 rows: the split-KV launches (few
    batches) and the single pass (many) run on copies of Q and O padded to 4
    or 8 query heads per KV head in the workspace."""
    rng = np.random.default_rng(B + max_len + D + Hq)
    seqlens = rng.integers(0, max_len + 1, size=B).astype(np.int32)
    seqlens[0] = max_len
    _case(B, Hq, Hkv, D, seqlens, max_len, seed=B + max_len + Hq)
    assert _kinds()[0] == "pad_query_group"


@pytest.mark.parametrize("Hq,Hkv", [(24, 8), (48, 4), (32, 1)])
def test_any_group_short_rows_through_split_entry(Hq, Hkv):
    """max_seqlen_kv <= 16 with a group size outside {1, 2, 4, 8}: the split
    entry runs the short-row kernels directly (G = 3 on the VALU kernel's
    4-head instantiation, G = 12 and 32 on the matrix-core kernel)."""
    rng = np.random.default_rng(Hq)
    seqlens = rng.integers(0, 11, size=33).astype(np.int32)
    _case(33, Hq, Hkv, 128, seqlens, 10, seed=Hq + 7)
    assert _kinds() == (["short_matrix_core"] if Hq // Hkv > 8 else ["short"])
    q, k, v, cu = make_inputs(3, Hq, Hkv, 128, np.array([4, 12, 9], np.int32), seed=Hq + 8)
    o = _run(q, k, v, cu, Hq, Hkv, 128, 10).reshape(3, Hq, 128)
    assert np.all(np.isnan(oracle.f16_to_f32(o[1])))      # 12 > max_seqlen_kv
    assert np.all(np.isfinite(oracle.f16_to_f32(o[[0, 2]])))


@pytest.fixture(params=["mfma", "valu"])
def long_group_kernel(request, monkeypatch):
    """The two paths of a query group above 8 beyond 16 rows: the
    matrix-core split passes (the default) and the VALU passes on ceil(G / 8)
    launch KV heads of 8 query heads (FMHA_DECODE_GQA_KERNEL=valu)."""
    if request.param == "valu":
        monkeypatch.setenv("FMHA_DECODE_GQA_KERNEL", "valu")
    else:
        monkeypatch.delenv("FMHA_DECODE_GQA_KERNEL", raising=False)
    return request.param


@pytest.mark.parametrize("D,Hq,Hkv", [(128, 24, 2), (128, 32, 1), (64, 48, 4), (256, 20, 2)])
@pytest.mark.parametrize("B,max_len", [(4, 500), (700, 40)])
def test_group_slices_beyond_eight(long_group_kernel, D, Hq, Hkv, B, max_len):
    """G = 12, 32, 10 beyond 16 rows, on copies of Q and O padded to a
    multiple of 8 query heads per KV head (G = 12, 10) or on Q and O
    themselves (G = 32): the matrix-core passes over each KV head's padded
    group, or ceil(G / 8) launch KV heads of 8 (launch head h reading KV head
    h / ceil(G / 8))."""
    rng = np.random.default_rng(B + max_len + Hq + D)
    seqlens = rng.integers(0, max_len + 1, size=B).astype(np.int32)
    seqlens[0] = max_len
    _case(B, Hq, Hkv, D, seqlens, max_len, seed=B + max_len + Hq + 1)
    kinds = _kinds()
    # On the matrix cores: the split passes, or with enough (batch, KV head)
    # units the register single pass (from two blocks above 8 query heads).
    mc = any(k in ("split_matrix_core", "onepass_matrix_core_regs") for k in kinds)
    assert mc == (long_group_kernel == "mfma"), kinds


@pytest.mark.parametrize("D,Hq,Hkv", [(128, 16, 1), (128, 24, 1), (64, 32, 2), (256, 16, 1), (128, 48, 2)])
@pytest.mark.parametrize("B,max_len", [(3, 900), (600, 33), (9, 17)])
def test_grouped_launch_kv_heads(long_group_kernel, D, Hq, Hkv, B, max_len):
    """G = 16, 24, 16, 16, 24 beyond 16 rows, multiples of 8 (no copies of Q
    and O).  Matrix cores: one or two 16-column tiles per KV head (24: the
    second half padding).  VALU: launch KV heads = Hkv * G / 8, which the
    lane groups of a wave share as sub-units (Hkv * G / 8 = 2 at D = 128:
    blocks, chunks or batches per lane group) or leave partly idle (3 launch
    heads)."""
    rng = np.random.default_rng(B * 3 + max_len + Hq + D)
    seqlens = rng.integers(0, max_len + 1, size=B).astype(np.int32)
    seqlens[0] = max_len
    _case(B, Hq, Hkv, D, seqlens, max_len, seed=B + max_len + Hq + 2)
    kinds = _kinds()
    mc = any(k in ("split_matrix_core", "onepass_matrix_core_regs") for k in kinds)
    assert mc == (long_group_kernel == "mfma") and "pad_query_group" not in kinds, kinds


@pytest.mark.parametrize("B,max_len", [(4, 300), (700, 40)])
def test_grouped_launch_kv_heads_bad_lengths(long_group_kernel, B, max_len):
    """A length above max_seqlen_kv with G = 16 (split and single pass): NaN
    for that batch only, oracle parity for the rest."""
    import fmha_amd
    import torch
    D, Hq, Hkv = 128, 32, 2
    rng = np.random.default_rng(B + 77)
    seqlens = rng.integers(1, max_len + 1, size=B).astype(np.int32)
    seqlens[0] = max_len
    bad = B // 2
    seqlens_big = seqlens.copy()
    seqlens_big[bad] = max_len + 5
    q, k, v, cu = make_inputs(B, Hq, Hkv, D, seqlens_big, seed=B + 78)
    o = fmha_amd.fmha_decode_splitkv(to_dev(q), to_dev(k), to_dev(v), torch.from_numpy(cu).cuda(), max_len,
                                     softmax_scale=default_scale(D))
    torch.cuda.synchronize()
    bits = o.view(torch.int16).cpu().numpy().view(np.uint16).reshape(B, Hq, D)
    f = oracle.f16_to_f32(bits)
    assert np.all(np.isnan(f[bad]))
    keep = np.array([b for b in range(B) if b != bad])
    r, slack = oracle.decode(q, k, v, cu, Hq, Hkv, D, default_scale(D), with_slack=True,
                             max_seqlen=max_len + 5)
    st = oracle.compare(np.ascontiguousarray(bits[keep]).ravel(),
                        np.ascontiguousarray(r.reshape(B, Hq, D)[keep]).ravel(),
                        np.ascontiguousarray(slack.reshape(B, Hq, D)[keep]).ravel())
    assert_pass(st, f"G=16 neighbours of an invalid length B={B}")


@pytest.mark.parametrize("D,Hq,Hkv,B,max_len", [(128, 64, 1, 2, 3000), (64, 128, 1, 3, 700), (256, 48, 2, 5, 300),
                                               (128, 40, 1, 3, 1100), (128, 96, 3, 9, 77)])
def test_matrix_core_split_many_tiles(D, Hq, Hkv, B, max_len):
    """The matrix-core split passes with more tiles than a P.V wave holds
    (G = 64, 128, 24 at D = 256, 40, 32): several tile chunks
    per (batch, KV head, chunk), every length 0..max_len region covered."""
    rng = np.random.default_rng(B * 11 + max_len + Hq + D)
    seqlens = rng.integers(0, max_len + 1, size=B).astype(np.int32)
    seqlens[0] = max_len
    _case(B, Hq, Hkv, D, seqlens, max_len, seed=B + max_len + Hq + 3)
    assert "split_matrix_core" in _kinds()


@pytest.mark.parametrize("D,Hq,Hkv", [(128, 8, 8), (128, 32, 8), (64, 8, 2), (256, 12, 4), (128, 20, 4)])
@pytest.mark.parametrize("B,max_len", [(4, 600), (300, 40)])
def test_matrix_core_split_small_groups(monkeypatch, D, Hq, Hkv, B, max_len):
    """FMHA_DECODE_GQA_KERNEL=mfma puts every group size on the matrix-core
    split passes: G = 1, 4, 4, 3 (padded to 4), 5 (padded to 8), one tile
    whose columns past G are padding (never stored, zero weights)."""
    monkeypatch.setenv("FMHA_DECODE_GQA_KERNEL", "mfma")
    rng = np.random.default_rng(B * 13 + max_len + Hq + D)
    seqlens = rng.integers(0, max_len + 1, size=B).astype(np.int32)
    seqlens[0] = max_len
    _case(B, Hq, Hkv, D, seqlens, max_len, seed=B + max_len + Hq + 4)
    assert "split_matrix_core" in _kinds()
