"""The decode kernels inside a captured HIP graph (torch.cuda.CUDAGraph):
the launch path allocates nothing and records no memset, so a graph of
several decode calls replays to the eager result every time.  Each replay is
checked against the eager output, with eager work and synchronisations
between replays."""
import numpy as np
import pytest

import oracle
from tests.common import assert_pass, default_scale, last_plan, make_inputs, to_dev

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


def test_graph_long_rows_replay_match_eager():
    """Lengths beyond 16 in a graph: the four split-KV launches (few
    batches), the single pass (many), and the strided and paged variants,
    each replay checked bit for bit against the eager result."""
    import torch
    import fmha_amd
    rng = np.random.default_rng(90)
    outs = []
    calls = []
    # split-KV launches: 3 batches, rows up to 700
    s1 = np.array([700, 1, 333], np.int32)
    q1, k1, v1, cu1 = make_inputs(3, 16, 4, 128, s1, seed=91)
    q1d, k1d, v1d, cu1d = to_dev(q1), to_dev(k1), to_dev(v1), torch.from_numpy(cu1).cuda()
    ws1 = torch.empty(fmha_amd.splitkv_workspace_size(3, 16, 4, 700, 128), dtype=torch.uint8, device="cuda")
    # single pass: 600 batches, rows up to 64
    s2 = rng.integers(0, 65, size=600).astype(np.int32)
    q2, k2, v2, cu2 = make_inputs(600, 32, 8, 128, s2, seed=92)
    q2d, k2d, v2d, cu2d = to_dev(q2), to_dev(k2), to_dev(v2), torch.from_numpy(cu2).cuda()
    ws2 = torch.empty(fmha_amd.splitkv_workspace_size(600, 32, 8, 64, 128), dtype=torch.uint8, device="cuda")
    # strided (BHSD view) and paged copies of the first case
    kb = torch.zeros(3, 4, 700, 128, dtype=torch.bfloat16, device="cuda")
    vb = torch.zeros_like(kb)
    kc = torch.zeros(3 * 44, 16, 4, 128, dtype=torch.bfloat16, device="cuda")
    vc = torch.zeros_like(kc)
    bt = torch.arange(3 * 44, dtype=torch.int32, device="cuda").view(3, 44)
    for b in range(3):
        n, r0 = int(s1[b]), int(cu1[b])
        kb[b, :, :n] = k1d[r0:r0 + n].transpose(0, 1)
        vb[b, :, :n] = v1d[r0:r0 + n].transpose(0, 1)
        for j in range(0, n, 16):
            m = min(16, n - j)
            kc[bt[b, j // 16], :m] = k1d[r0 + j:r0 + j + m]
            vc[bt[b, j // 16], :m] = v1d[r0 + j:r0 + j + m]
    lens1 = torch.from_numpy(s1).cuda()
    ws3 = torch.empty_like(ws1)
    ws4 = torch.empty_like(ws1)
    outs = [torch.empty(3, 16, 128, dtype=torch.float16, device="cuda"),
            torch.empty(600, 32, 128, dtype=torch.float16, device="cuda"),
            torch.empty(3, 16, 128, dtype=torch.float16, device="cuda"),
            torch.empty(3, 16, 128, dtype=torch.float16, device="cuda")]

    def calls():
        fmha_amd.fmha_decode_splitkv(q1d, k1d, v1d, cu1d, 700, out=outs[0], workspace=ws1)
        fmha_amd.fmha_decode_splitkv(q2d, k2d, v2d, cu2d, 64, out=outs[1], workspace=ws2)
        fmha_amd.fmha_decode_strided(q1d, kb.transpose(1, 2), vb.transpose(1, 2), seqlens_kv=lens1, out=outs[2],
                                     workspace=ws3)
        fmha_amd.fmha_decode_paged(q1d, kc, vc, bt, lens1, out=outs[3], max_seqlen_kv=700, workspace=ws4)

    calls()
    torch.cuda.synchronize()
    eager = [o.clone() for o in outs]
    assert torch.equal(eager[0].view(torch.int16), eager[2].view(torch.int16))
    assert torch.equal(eager[0].view(torch.int16), eager[3].view(torch.int16))
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        calls()
    torch.cuda.current_stream().wait_stream(s)
    g = torch.cuda.CUDAGraph()
    torch.cuda.synchronize()
    with torch.cuda.graph(g):
        calls()
    for rep in range(4):
        for o in outs:
            o.fill_(float("nan"))
        ws1.fill_(255)
        g.replay()
        torch.cuda.synchronize()
        for i, (o, e) in enumerate(zip(outs, eager)):
            assert torch.equal(o.view(torch.int16), e.view(torch.int16)), f"replay {rep}, call {i}"
        fmha_amd.fmha_decode_splitkv(q2d, k2d, v2d, cu2d, 64)
        torch.cuda.synchronize()


def test_graph_register_single_pass_replays_match_eager():
    """The matrix-core register single pass (no workspace, one launch) in a
    graph: a packed call (G = 4, two waves per row) and the same rows over
    16-row pages, each replay checked bit for bit against the eager result
    and the eager result against the oracle."""
    import torch
    import fmha_amd
    rng = np.random.default_rng(95)
    B, Hq, Hkv, D, cap = 128, 32, 8, 128, 256
    lens = rng.integers(0, cap + 1, size=B).astype(np.int32)
    lens[:3] = [cap, 0, 17]
    q, k, v, cu = make_inputs(B, Hq, Hkv, D, lens, seed=96)
    qd, kd, vd, cud = to_dev(q), to_dev(k), to_dev(v), torch.from_numpy(cu).cuda()
    npg = B * (cap // 16)
    bt = torch.from_numpy(rng.permutation(npg).astype(np.int32).reshape(B, cap // 16)).cuda()
    kc = torch.zeros(npg, 16, Hkv, D, dtype=torch.bfloat16, device="cuda")
    vc = torch.zeros_like(kc)
    for b in range(B):
        n, r0 = int(lens[b]), int(cu[b])
        for j in range(0, n, 16):
            m = min(16, n - j)
            kc[int(bt[b, j // 16]), :m] = kd[r0 + j:r0 + j + m]
            vc[int(bt[b, j // 16]), :m] = vd[r0 + j:r0 + j + m]
    lensd = torch.from_numpy(lens).cuda()
    outs = [torch.empty(B, Hq, D, dtype=torch.float16, device="cuda") for _ in range(2)]
    kinds = []

    def calls():
        fmha_amd.fmha_decode_splitkv(qd, kd, vd, cud, cap, out=outs[0])
        kinds.append(last_plan()[-1][0])
        fmha_amd.fmha_decode_paged(qd, kc, vc, bt, lensd, out=outs[1], max_seqlen_kv=cap)
        kinds.append(last_plan()[-1][0])

    calls()
    torch.cuda.synchronize()
    assert kinds == ["onepass_matrix_core_regs"] * 2, kinds
    eager = [o.clone() for o in outs]
    assert torch.equal(eager[0].view(torch.int16), eager[1].view(torch.int16))
    r, slack = oracle.decode(q, k, v, cu, Hq, Hkv, D, default_scale(D), with_slack=True, max_seqlen=cap)
    assert_pass(oracle.compare(eager[0].view(torch.int16).cpu().numpy().view(np.uint16).reshape(r.shape), r, slack),
                "register single pass")
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        calls()
    torch.cuda.current_stream().wait_stream(s)
    g = torch.cuda.CUDAGraph()
    torch.cuda.synchronize()
    with torch.cuda.graph(g):
        calls()
    for rep in range(4):
        for o in outs:
            o.fill_(float("nan"))
        g.replay()
        torch.cuda.synchronize()
        for i, (o, e) in enumerate(zip(outs, eager)):
            assert torch.equal(o.view(torch.int16), e.view(torch.int16)), f"replay {rep}, call {i}"
        fmha_amd.fmha_decode_splitkv(qd, kd, vd, cud, cap)
        torch.cuda.synchronize()


@pytest.mark.parametrize("kernel", ["mfma", "default"])
def test_graph_matrix_core_kernel_replays_match_eager(monkeypatch, kernel):
    """Group sizes outside {1, 2, 4, 8} in a graph: varlen, uniform and
    strided calls with G = 5, an MQA shape with two waves per stream group,
    every replay bit-equal to the eager result; once with the matrix-core
    kernel forced for all of them, once with the library's choice (the VALU
    kernel's 8-head instantiation for G = 5)."""
    if kernel == "mfma":
        monkeypatch.setenv("FMHA_DECODE_GQA_KERNEL", "mfma")
    else:
        monkeypatch.delenv("FMHA_DECODE_GQA_KERNEL", raising=False)
    import torch
    import fmha_amd
    seqlens = oracle.generate_seqlens(48, 16)
    q, k, v, cu = make_inputs(48, 20, 4, 128, seqlens, seed=95)
    qd, kd, vd = to_dev(q), to_dev(k), to_dev(v)
    cud = torch.from_numpy(cu).cuda()
    _, ku, vu, _ = make_inputs(48, 20, 4, 128, [7] * 48, seed=96)
    kb = to_dev(ku).reshape(48, 7, 4, 128)
    vb = to_dev(vu).reshape(48, 7, 4, 128)
    qm, km, vm, cum = make_inputs(40, 32, 1, 64, seqlens[:40], seed=97)
    qmd, kmd, vmd, cumd = to_dev(qm), to_dev(km), to_dev(vm), torch.from_numpy(cum).cuda()
    outs = [torch.empty(48, 20, 128, dtype=torch.float16, device="cuda") for _ in range(3)]
    outs.append(torch.empty(40, 32, 64, dtype=torch.float16, device="cuda"))

    # the tree-order entry points, whose kernel FMHA_DECODE_GQA_KERNEL selects
    def calls():
        fmha_amd.fmha_decode(qd, kd, vd, cu_seqlens_kv=cud, out=outs[0], fast=True)
        fmha_amd.fmha_decode(qd, kb, vb, out=outs[1], fast=True)
        fmha_amd.fmha_decode_strided(qd, kb, vb, out=outs[2])
        fmha_amd.fmha_decode(qmd, kmd, vmd, cu_seqlens_kv=cumd, out=outs[3], fast=True)

    calls()
    torch.cuda.synchronize()
    eager = [o.clone() for o in outs]
    assert torch.equal(eager[1].view(torch.int16), eager[2].view(torch.int16))
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        calls()
    torch.cuda.current_stream().wait_stream(s)
    g = torch.cuda.CUDAGraph()
    torch.cuda.synchronize()
    with torch.cuda.graph(g):
        calls()
    for rep in range(4):
        for o in outs:
            o.fill_(float("nan"))
        g.replay()
        torch.cuda.synchronize()
        for i, (o, e) in enumerate(zip(outs, eager)):
            assert torch.equal(o.view(torch.int16), e.view(torch.int16)), f"replay {rep}, call {i}"
        fmha_amd.fmha_decode(qd, kd, vd, cu_seqlens_kv=cud)
        torch.cuda.synchronize()


def test_graph_long_rows_large_group_replays_match_eager():
    """Lengths beyond 16 with G > 8 in a graph: the matrix-core split passes
    (G = 16 on Q and O themselves, several chunks; G = 12 on the padded
    copies, one chunk per row) and the paged route (launch KV heads of 8
    query heads), each replay bit-equal to the eager result."""
    import torch
    import fmha_amd
    s1 = np.array([900, 3, 517, 0], np.int32)
    q1, k1, v1, cu1 = make_inputs(4, 32, 2, 128, s1, seed=101)
    q1d, k1d, v1d, cu1d = to_dev(q1), to_dev(k1), to_dev(v1), torch.from_numpy(cu1).cuda()
    ws1 = torch.empty(fmha_amd.splitkv_workspace_size(4, 32, 2, 900, 128), dtype=torch.uint8, device="cuda")
    s2 = np.random.default_rng(102).integers(0, 41, size=300).astype(np.int32)
    q2, k2, v2, cu2 = make_inputs(300, 24, 2, 64, s2, seed=103)
    q2d, k2d, v2d, cu2d = to_dev(q2), to_dev(k2), to_dev(v2), torch.from_numpy(cu2).cuda()
    ws2 = torch.empty(fmha_amd.splitkv_workspace_size(300, 24, 2, 40, 64), dtype=torch.uint8, device="cuda")
    # the first case over 16-row pages
    kc = torch.zeros(4 * 57, 16, 2, 128, dtype=torch.bfloat16, device="cuda")
    vc = torch.zeros_like(kc)
    bt = torch.arange(4 * 57, dtype=torch.int32, device="cuda").view(4, 57)
    for b in range(4):
        n, r0 = int(s1[b]), int(cu1[b])
        for j in range(0, n, 16):
            m = min(16, n - j)
            kc[bt[b, j // 16], :m] = k1d[r0 + j:r0 + j + m]
            vc[bt[b, j // 16], :m] = v1d[r0 + j:r0 + j + m]
    lens1 = torch.from_numpy(s1).cuda()
    ws3 = torch.empty_like(ws1)
    outs = [torch.empty(4, 32, 128, dtype=torch.float16, device="cuda"),
            torch.empty(300, 24, 64, dtype=torch.float16, device="cuda"),
            torch.empty(4, 32, 128, dtype=torch.float16, device="cuda")]

    def calls():
        fmha_amd.fmha_decode_splitkv(q1d, k1d, v1d, cu1d, 900, out=outs[0], workspace=ws1)
        fmha_amd.fmha_decode_splitkv(q2d, k2d, v2d, cu2d, 40, out=outs[1], workspace=ws2)
        fmha_amd.fmha_decode_paged(q1d, kc, vc, bt, lens1, out=outs[2], max_seqlen_kv=900, workspace=ws3)

    calls()
    torch.cuda.synchronize()
    eager = [o.clone() for o in outs]
    r1, slack1 = oracle.decode(q1, k1, v1, cu1, 32, 2, 128, default_scale(128), with_slack=True, max_seqlen=900)
    for i in (0, 2):
        assert_pass(oracle.compare(eager[i].view(torch.int16).cpu().numpy().view(np.uint16).reshape(r1.shape), r1,
                                   slack1), f"G=16 long rows, call {i}")
    r2, slack2 = oracle.decode(q2, k2, v2, cu2, 24, 2, 64, default_scale(64), with_slack=True, max_seqlen=40)
    assert_pass(oracle.compare(eager[1].view(torch.int16).cpu().numpy().view(np.uint16).reshape(r2.shape), r2,
                               slack2), "G=12 padded, one chunk")
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        calls()
    torch.cuda.current_stream().wait_stream(s)
    g = torch.cuda.CUDAGraph()
    torch.cuda.synchronize()
    with torch.cuda.graph(g):
        calls()
    for rep in range(4):
        for o in outs:
            o.fill_(float("nan"))
        ws1.fill_(255)
        ws2.fill_(255)
        g.replay()
        torch.cuda.synchronize()
        for i, (o, e) in enumerate(zip(outs, eager)):
            assert torch.equal(o.view(torch.int16), e.view(torch.int16)), f"replay {rep}, call {i}"
        fmha_amd.fmha_decode_splitkv(q2d, k2d, v2d, cu2d, 40)
        torch.cuda.synchronize()
