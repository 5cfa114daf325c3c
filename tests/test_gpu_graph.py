"""The decode kernels inside a captured HIP graph (torch.cuda.CUDAGraph):
the launch path allocates nothing and records no memset, so a graph of
several decode calls replays to the eager result every time.  Each replay is
checked against the eager output, with eager work and synchronisations
between replays."""
import numpy as np
import pytest

import oracle
from tests.common import make_inputs, to_dev

pytestmark = pytest.mark.gpu


def test_graph_replays_match_eager():
    import torch
    import fmha_amd
    seqlens = oracle.generate_seqlens(64, 16)
    q, k, v, cu = make_inputs(64, 16, 8, 128, seqlens, seed=77)
    qd, kd, vd = to_dev(q), to_dev(k), to_dev(v)
    cud = torch.from_numpy(cu).cuda()
    _, ku, vu, _ = make_inputs(64, 16, 8, 128, [5] * 64, seed=78)
    kb = to_dev(ku).reshape(64, 5, 8, 128)
    vb = to_dev(vu).reshape(64, 5, 8, 128)
    ws = torch.empty(fmha_amd.splitkv_workspace_size(64, 16, 8, 16, 128), dtype=torch.uint8, device="cuda")
    outs = [torch.empty(64, 16, 128, dtype=torch.float16, device="cuda") for _ in range(4)]

    def calls():
        fmha_amd.fmha_decode(qd, kd, vd, cu_seqlens_kv=cud, out=outs[0])
        fmha_amd.fmha_decode(qd, kb, vb, out=outs[1])
        fmha_amd.fmha_decode_strided(qd, kb, vb, out=outs[2])
        fmha_amd.fmha_decode_splitkv(qd, kd, vd, cud, 16, out=outs[3], workspace=ws)

    calls()
    torch.cuda.synchronize()
    eager = [o.clone() for o in outs]
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        calls()  # warm-up on the capture stream
    torch.cuda.current_stream().wait_stream(s)
    g = torch.cuda.CUDAGraph()
    for o in outs:
        o.fill_(0)
    torch.cuda.synchronize()
    with torch.cuda.graph(g):
        calls()
    for rep in range(5):
        for o in outs:
            o.fill_(float("nan"))
        g.replay()
        torch.cuda.synchronize()
        for i, (o, e) in enumerate(zip(outs, eager)):
            assert torch.equal(o.view(torch.int16), e.view(torch.int16)), f"replay {rep}, call {i}"
        # eager work between replays
        fmha_amd.fmha_decode(qd, kd, vd, cu_seqlens_kv=cud)
        torch.cuda.synchronize()
