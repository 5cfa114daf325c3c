"""The library's one piece of state cannot change a result.

The entry points that read lengths from a device cu_seqlens_kv array size
their launch (waves per CU) from the mean length the previous call on the
device reported through a word of pinned host memory, and
FMHA_DECODE_WAVE_CAP overrides that cap for sweeps.  Neither may change a
single output bit: every entry point here runs under caps of 3 to 16 waves
per CU, under the default cap, and right after calls whose lengths were very
different (the feedback word then holds a stale mean), and each must give
the same bits every time; the default and exact entry points' bits are also
the restated reference loop's."""
import numpy as np
import pytest

import oracle
from tests.common import assert_exact, last_plan, make_inputs, to_dev

pytestmark = pytest.mark.gpu

ENTRIES = ("default", "fast", "exact", "fp32_weights")


def _call(entry, qd, kd, vd, cud):
    import torch
    import fmha_amd
    o = fmha_amd.fmha_decode(qd, kd, vd, cu_seqlens_kv=cud, fast=entry == "fast", exact=entry == "exact",
                             fp32_weights=entry == "fp32_weights")
    torch.cuda.synchronize()
    return o.view(torch.int16).cpu().numpy().view(np.uint16)


@pytest.mark.parametrize("Hq,Hkv,D", [(16, 16, 128), (32, 16, 128), (32, 32, 256), (8, 1, 128)])
def test_results_do_not_depend_on_wave_cap_or_feedback(monkeypatch, Hq, Hkv, D):
    import torch
    B = 600
    seqlens = oracle.generate_seqlens(B, 16)
    q, k, v, cu = make_inputs(B, Hq, Hkv, D, seqlens, seed=4400 + Hq + D)
    qd, kd, vd, cud = to_dev(q), to_dev(k), to_dev(v), torch.from_numpy(cu).cuda()
    # a call whose lengths are all 16 and one whose lengths are all 1: the
    # feedback word then holds a mean far from this batch's
    long_lens = np.full(B, 16, np.int32)
    ql, kl, vl, cul = make_inputs(B, Hq, Hkv, D, long_lens, seed=4500)
    qs, ks, vs, cus = make_inputs(B, Hq, Hkv, D, np.ones(B, np.int32), seed=4501)
    stale = [(to_dev(ql), to_dev(kl), to_dev(vl), torch.from_numpy(cul).cuda()),
             (to_dev(qs), to_dev(ks), to_dev(vs), torch.from_numpy(cus).cuda())]
    monkeypatch.delenv("FMHA_DECODE_WAVE_CAP", raising=False)
    ref = {e: _call(e, qd, kd, vd, cud) for e in ENTRIES}
    if Hq // Hkv <= 2:
        assert_exact(ref["default"], q, k, v, cu, Hq, Hkv, D, "default entry")
    assert_exact(ref["exact"], q, k, v, cu, Hq, Hkv, D, "exact entry")
    caps_seen = set()
    for cap in (3, 4, 6, 8, 12, 16, None):
        if cap is None:
            monkeypatch.delenv("FMHA_DECODE_WAVE_CAP", raising=False)
        else:
            monkeypatch.setenv("FMHA_DECODE_WAVE_CAP", str(cap))
        for before in stale:
            for e in ENTRIES:
                _call(e, *before)                  # leaves its own mean in the feedback word
                o = _call(e, qd, kd, vd, cud)
                _, fields = last_plan()[-1]        # short or short_multi: this call's cap
                caps_seen.add(fields["waves_per_cu"])
                assert np.array_equal(o, ref[e]), f"{e}: bits changed under cap {cap} after a stale mean"
    print(f"Hq={Hq} Hkv={Hkv} D={D}: waves per CU seen {sorted(caps_seen)}", flush=True)
    assert len(caps_seen) >= 4
