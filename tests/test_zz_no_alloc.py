"""fmha_decode_fwd_splitkv_noalloc, the split-KV entry point that allocates
nothing (its workspace is a device array inside the library), called through
the C ABI: its output must equal fmha_decode_fwd_splitkv's (same kernels,
caller workspace) bit for bit and pass the oracle gate, on two calls in a
row, the second with a smaller input; a call that needs more scratch than
the array holds is rejected before anything is launched."""
import ctypes

import numpy as np
import pytest

import oracle
from tests.common import assert_pass, default_scale, make_inputs, to_dev

pytestmark = pytest.mark.gpu


def _call_pair(B, Hq, Hkv, D, seqlens, max_len, seed):
    import torch
    import fmha_amd
    from fmha_amd import _lib
    lib = _lib.load()
    q, k, v, cu = make_inputs(B, Hq, Hkv, D, seqlens, seed)
    qd, kd, vd = to_dev(q), to_dev(k), to_dev(v)
    cud = torch.from_numpy(cu).cuda()
    scale = default_scale(D)
    stream = torch.cuda.current_stream().cuda_stream
    need = fmha_amd.splitkv_workspace_size(B, Hq, Hkv, max_len, D)
    assert 0 < need <= fmha_amd.NOALLOC_SCRATCH_BYTES
    ws = torch.empty(need, dtype=torch.uint8, device="cuda")
    o_ws = torch.full((B, Hq, D), float("nan"), dtype=torch.float16, device="cuda")
    o_na = torch.full((B, Hq, D), float("nan"), dtype=torch.float16, device="cuda")
    rc = lib.fmha_decode_fwd_splitkv(stream, qd.data_ptr(), kd.data_ptr(), vd.data_ptr(), o_ws.data_ptr(),
                                     cud.data_ptr(), max_len, B, Hq, Hkv, 1, D, D, scale, ws.data_ptr(), need)
    assert rc == 0, lib.fmha_decode_last_error_detail()
    rc = lib.fmha_decode_fwd_splitkv_noalloc(stream, qd.data_ptr(), kd.data_ptr(), vd.data_ptr(), o_na.data_ptr(),
                                             cud.data_ptr(), max_len, B, Hq, Hkv, 1, D, D, scale)
    assert rc == 0, lib.fmha_decode_last_error_detail()
    torch.cuda.synchronize()
    assert torch.equal(o_na.view(torch.int16), o_ws.view(torch.int16))
    bits = o_na.view(torch.int16).cpu().numpy().view(np.uint16)
    r, slack = oracle.decode(q, k, v, cu, Hq, Hkv, D, scale, with_slack=True, max_seqlen=max_len)
    st = oracle.compare(bits.reshape(r.shape), r, slack)
    print(f"noalloc B={B} Hq={Hq} Hkv={Hkv} D={D} max={max_len}: {st}", flush=True)
    assert_pass(st, f"noalloc B={B} D={D}")


def test_noalloc_matches_workspace_entry_two_calls():
    """A long call (several P.V chunks per row: partial outputs in the
    scratch) with a padded query group (G = 6: Q and O copies in the
    scratch too), then a smaller one that reuses the same scratch."""
    rng = np.random.default_rng(11)
    seqlens = rng.integers(0, 1501, size=9).astype(np.int32)
    seqlens[0] = 1500
    _call_pair(9, 24, 4, 128, seqlens, 1500, seed=1)
    _call_pair(3, 16, 16, 64, np.array([40, 7, 100], np.int32), 100, seed=2)


def test_noalloc_short_rows_and_rejects_oversize():
    import torch
    import fmha_amd
    from fmha_amd import _lib
    lib = _lib.load()
    _call_pair(5, 8, 8, 128, np.array([16, 3, 0, 9, 1], np.int32), 16, seed=3)
    # a call needing more scratch than the array holds: rejected, nothing launched
    B, Hq, Hkv, D, max_len = 4096, 32, 8, 128, 4096
    need = fmha_amd.splitkv_workspace_size(B, Hq, Hkv, max_len, D)
    assert need > fmha_amd.NOALLOC_SCRATCH_BYTES
    t = torch.zeros(64, dtype=torch.bfloat16, device="cuda")
    cu = torch.zeros(B + 1, dtype=torch.int32, device="cuda")
    rc = lib.fmha_decode_fwd_splitkv_noalloc(torch.cuda.current_stream().cuda_stream, t.data_ptr(), t.data_ptr(),
                                             t.data_ptr(), t.data_ptr(), cu.data_ptr(), max_len, B, Hq, Hkv, 1, D, D,
                                             default_scale(D))
    assert rc == 1 and b"scratch" in lib.fmha_decode_last_error_detail()
    torch.cuda.synchronize()
