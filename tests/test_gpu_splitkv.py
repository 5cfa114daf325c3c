"""GPU parity of the split-KV path (fmha_decode_fwd_splitkv), lengths beyond
the reference's 16: the oracle runs the reference loop over the longer rows
(oracle.decode(max_seqlen=...)), gate as in tests/common.py."""
import numpy as np
import pytest

import oracle
from tests.common import assert_pass, cu_from_seqlens, default_scale, make_inputs, to_dev

pytestmark = pytest.mark.gpu


def _run(q, k, v, cu, Hq, Hkv, D, max_len):
    import torch
    import fmha_amd
    o = fmha_amd.fmha_decode_splitkv(to_dev(q), to_dev(k), to_dev(v), torch.from_numpy(cu).cuda(), max_len,
                                     softmax_scale=default_scale(D))
    torch.cuda.synchronize()
    return o.view(torch.int16).cpu().numpy().view(np.uint16)


def _case(B, Hq, Hkv, D, seqlens, max_len, seed, std=1.0):
    q, k, v, cu = make_inputs(B, Hq, Hkv, D, seqlens, seed, std)
    o = _run(q, k, v, cu, Hq, Hkv, D, max_len)
    r, slack = oracle.decode(q, k, v, cu, Hq, Hkv, D, default_scale(D), with_slack=True, max_seqlen=max_len)
    st = oracle.compare(o.reshape(r.shape), r, slack)
    print(f"B={B} Hq={Hq} Hkv={Hkv} D={D} max={max_len}: {st}", flush=True)
    assert_pass(st, f"splitkv B={B} D={D} max={max_len}")


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
    """Lengths on and next to the 16-row block edges: a scores wave whose
    second block is partly or wholly past the row's end."""
    seqlens = np.array([16, 32, 48, 31, 33, 47, 15, 17, 1, 64], np.int32)
    _case(len(seqlens), Hq, Hkv, D, seqlens, 64, seed=11 + D)


def test_mid_chunk_count():
    """16 < chunks <= 256 (the 256-thread combine) with two heads per KV head."""
    rng = np.random.default_rng(12)
    seqlens = rng.integers(6000, 8193, size=16).astype(np.int32)
    seqlens[0] = 8192
    _case(16, 32, 8, 128, seqlens, 8192, seed=12, std=0.5)


def test_mid_block_count():
    """512 < blocks <= 2048 (the 256-thread statistics) on one long row."""
    _case(1, 32, 8, 128, np.array([20000], np.int32), 20000, seed=13, std=0.5)


def test_short_lengths_match_short_path():
    """Lengths <= 16 through split-KV agree with the oracle as the short path does."""
    seqlens = oracle.generate_seqlens(300, 16)
    _case(300, 16, 16, 128, seqlens, 16, seed=5)


def test_many_batches_direct_path():
    """max length fits one chunk: the PV kernel writes O directly."""
    seqlens = np.random.default_rng(3).integers(0, 41, size=2000).astype(np.int32)
    _case(2000, 8, 8, 128, seqlens, 40, seed=6)


def test_one_long_sequence():
    _case(1, 32, 8, 128, np.array([40000], np.int32), 40000, seed=7, std=0.5)


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
