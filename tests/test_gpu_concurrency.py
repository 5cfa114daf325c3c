"""Calls from several host threads on their own streams are independent:
four threads, each with its own (default-priority) stream and its own
workload -- the varlen, uniform, paged and split-KV entry points -- repeat
their call and must reproduce, bit for bit, the output of the same call made
alone beforehand."""
import threading

import numpy as np
import pytest

import oracle
from tests.common import make_inputs, to_dev

pytestmark = pytest.mark.gpu


def test_threads_on_separate_streams_match_sequential():
    import torch
    import fmha_amd
    dev = "cuda"
    seqlens = oracle.generate_seqlens(512, 16)
    q, k, v, cu = make_inputs(512, 16, 8, 128, seqlens, seed=91)
    qd, kd, vd = to_dev(q), to_dev(k), to_dev(v)
    cud = torch.from_numpy(cu).to(dev)
    _, ku, vu, _ = make_inputs(512, 16, 8, 128, [11] * 512, seed=92)
    kb = to_dev(ku).reshape(512, 11, 8, 128)
    vb = to_dev(vu).reshape(512, 11, 8, 128)
    # paged: page size 4, pages of each batch scattered by a fixed permutation
    page, npages = 4, 512 * 4
    perm = np.random.default_rng(93).permutation(npages).astype(np.int32)
    bt = torch.from_numpy(perm.reshape(512, 4)).to(dev)
    kc = torch.randn(npages, page, 8, 128, device=dev, dtype=torch.bfloat16)
    vc = torch.randn(npages, page, 8, 128, device=dev, dtype=torch.bfloat16)
    lens = torch.from_numpy(seqlens.astype(np.int32)).to(dev)
    long_lens = np.random.default_rng(94).integers(1, 300, size=64).astype(np.int32)
    ql, kl, vl, cul = make_inputs(64, 16, 8, 128, long_lens, seed=95)
    qld, kld, vld = to_dev(ql), to_dev(kl), to_dev(vl)
    culd = torch.from_numpy(cul).to(dev)

    def job(i, out, ws):
        if i == 0:
            fmha_amd.fmha_decode(qd, kd, vd, cu_seqlens_kv=cud, out=out)
        elif i == 1:
            fmha_amd.fmha_decode(qd, kb, vb, out=out)
        elif i == 2:
            fmha_amd.fmha_decode_paged(qd, kc, vc, bt, lens, out=out)
        else:
            fmha_amd.fmha_decode_splitkv(qld, kld, vld, culd, 300, out=out, workspace=ws)

    shapes = [(512, 16, 128)] * 3 + [(64, 16, 128)]
    wss = [None] * 3 + [torch.empty(fmha_amd.splitkv_workspace_size(64, 16, 8, 300, 128), dtype=torch.uint8,
                                    device=dev)]
    expected = []
    for i in range(4):
        o = torch.empty(*shapes[i], dtype=torch.float16, device=dev)
        job(i, o, wss[i])
        torch.cuda.synchronize()
        expected.append(o.clone())

    outs = [torch.full(shapes[i], float("nan"), dtype=torch.float16, device=dev) for i in range(4)]
    torch.cuda.synchronize()
    errors = []
    start = threading.Barrier(4)

    def worker(i):
        try:
            s = torch.cuda.Stream()
            with torch.cuda.stream(s):
                start.wait()
                for rep in range(20):
                    job(i, outs[i], wss[i])
                s.synchronize()
            if not torch.equal(outs[i].view(torch.int16), expected[i].view(torch.int16)):
                errors.append(f"job {i} differs from its sequential result")
        except Exception as e:  # reported below, with the job that raised it
            errors.append(f"job {i}: {e!r}")

    threads = [threading.Thread(target=worker, args=(i,)) for i in range(4)]
    for t in threads:
        t.start()
    for t in threads:
        t.join()
    assert not errors, errors
