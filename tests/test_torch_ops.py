"""torch.library registration of the kernel (fmha_amd/torch_ops.py)."""
import numpy as np
import pytest

import oracle
from tests.common import default_scale, make_inputs, to_dev


def test_fake_impl_shapes_without_gpu():
    import torch
    import fmha_amd.torch_ops  # noqa: F401
    from torch._subclasses.fake_tensor import FakeTensorMode
    with FakeTensorMode():
        q = torch.empty(4, 8, 1, 128, dtype=torch.bfloat16, device="cuda")
        k = torch.empty(20, 2, 128, dtype=torch.bfloat16, device="cuda")
        cu = torch.empty(5, dtype=torch.int32, device="cuda")
        o = torch.ops.fmha_amd.decode(q, k, k, cu, -1, 0.0)
        assert o.shape == q.shape and o.dtype == torch.float16
        q3 = torch.empty(4, 8, 64, dtype=torch.bfloat16, device="cuda")
        ku = torch.empty(4, 3, 8, 64, dtype=torch.bfloat16, device="cuda")
        assert torch.ops.fmha_amd.decode(q3, ku, ku, None, 3, 0.125).shape == q3.shape
        ks = torch.empty(400, 2, 128, dtype=torch.bfloat16, device="cuda")
        assert torch.ops.fmha_amd.decode_splitkv(q, ks, ks, cu, 100, 0.0).shape == q.shape
        kb = torch.empty(4, 2, 300, 128, dtype=torch.bfloat16, device="cuda").transpose(1, 2)
        lens = torch.empty(4, dtype=torch.int32, device="cuda")
        assert torch.ops.fmha_amd.decode_strided(q, kb, kb, lens, 0.0).dtype == torch.float16
        kc = torch.empty(40, 16, 2, 128, dtype=torch.bfloat16, device="cuda")
        bt = torch.empty(4, 10, dtype=torch.int32, device="cuda")
        assert torch.ops.fmha_amd.decode_paged(q, kc, kc, bt, lens, 0.0, 160).shape == q.shape


@pytest.mark.gpu
def test_op_matches_direct_call_and_oracle():
    import torch
    import fmha_amd
    import fmha_amd.torch_ops  # noqa: F401
    from tests.common import assert_pass
    seqlens = oracle.generate_seqlens(32, 16)
    q, k, v, cu = make_inputs(32, 8, 4, 128, seqlens, seed=1000)
    qd, kd, vd = to_dev(q), to_dev(k), to_dev(v)
    cud = torch.from_numpy(cu).cuda()
    o_op = torch.ops.fmha_amd.decode(qd, kd, vd, cud, -1, 0.0)
    o_dir = fmha_amd.fmha_decode(qd, kd, vd, cu_seqlens_kv=cud)
    out = torch.empty_like(o_dir)
    torch.ops.fmha_amd.decode_out(qd, kd, vd, cud, -1, 0.0, out)
    torch.cuda.synchronize()
    assert torch.equal(o_op.view(torch.int16), o_dir.view(torch.int16))
    assert torch.equal(out.view(torch.int16), o_dir.view(torch.int16))
    r, slack = oracle.decode(q, k, v, cu, 8, 4, 128, default_scale(128), with_slack=True)
    bits = o_op.view(torch.int16).cpu().numpy().view(np.uint16)
    assert_pass(oracle.compare(bits, r, slack), "torch op")
    # fp32 weights through the op
    o32_op = torch.ops.fmha_amd.decode(qd, kd, vd, cud, -1, 0.0, True)
    o32_dir = fmha_amd.fmha_decode(qd, kd, vd, cu_seqlens_kv=cud, fp32_weights=True)
    torch.cuda.synchronize()
    assert torch.equal(o32_op.view(torch.int16), o32_dir.view(torch.int16))
    r32, _ = oracle.decode(q, k, v, cu, 8, 4, 128, default_scale(128), p_mode=1)
    assert_pass(oracle.compare(o32_op.view(torch.int16).cpu().numpy().view(np.uint16), r32), "torch op fp32")


@pytest.mark.gpu
def test_op_exact():
    """torch.ops.fmha_amd.decode(..., exact=True) and decode_out: the bits of
    the direct exact call, which are the CPU loop's (oracle p_mode=2)."""
    import torch
    import fmha_amd
    import fmha_amd.torch_ops  # noqa: F401
    seqlens = oracle.generate_seqlens(40, 16)
    q, k, v, cu = make_inputs(40, 8, 8, 128, seqlens, seed=1002)
    qd, kd, vd = to_dev(q), to_dev(k), to_dev(v)
    cud = torch.from_numpy(cu).cuda()
    o_op = torch.ops.fmha_amd.decode(qd, kd, vd, cud, -1, 0.0, False, True)
    o_dir = fmha_amd.fmha_decode(qd, kd, vd, cu_seqlens_kv=cud, exact=True)
    out = torch.empty_like(o_dir)
    torch.ops.fmha_amd.decode_out(qd, kd, vd, cud, -1, 0.0, out, exact=True)
    torch.cuda.synchronize()
    assert torch.equal(o_op.view(torch.int16), o_dir.view(torch.int16))
    assert torch.equal(out.view(torch.int16), o_dir.view(torch.int16))
    r, _ = oracle.decode(q, k, v, cu, 8, 8, 128, default_scale(128), p_mode=2)
    assert np.array_equal(o_op.view(torch.int16).cpu().numpy().view(np.uint16), r)


@pytest.mark.gpu
def test_op_any_group_size():
    """torch.ops.fmha_amd.decode with a group size outside {1, 2, 4, 8}
    (G = 7): same bits as the direct call, oracle parity."""
    import torch
    import fmha_amd
    import fmha_amd.torch_ops  # noqa: F401
    from tests.common import assert_pass
    seqlens = oracle.generate_seqlens(24, 16)
    q, k, v, cu = make_inputs(24, 21, 3, 128, seqlens, seed=1001)
    qd, kd, vd = to_dev(q), to_dev(k), to_dev(v)
    cud = torch.from_numpy(cu).cuda()
    o_op = torch.ops.fmha_amd.decode(qd, kd, vd, cud, -1, 0.0)
    o_dir = fmha_amd.fmha_decode(qd, kd, vd, cu_seqlens_kv=cud)
    torch.cuda.synchronize()
    assert torch.equal(o_op.view(torch.int16), o_dir.view(torch.int16))
    r, slack = oracle.decode(q, k, v, cu, 21, 3, 128, default_scale(128), with_slack=True)
    assert_pass(oracle.compare(o_op.view(torch.int16).cpu().numpy().view(np.uint16), r, slack), "torch op G=7")


@pytest.mark.gpu
def test_opcheck_and_compile():
    import torch
    import fmha_amd.torch_ops  # noqa: F401
    seqlens = [3, 16, 0, 7]
    q, k, v, cu = make_inputs(4, 4, 4, 64, seqlens, seed=1001)
    args = (to_dev(q), to_dev(k), to_dev(v), torch.from_numpy(cu).cuda(), -1, 0.0)
    torch.library.opcheck(torch.ops.fmha_amd.decode.default, args,
                          test_utils=("test_schema", "test_faketensor", "test_aot_dispatch_static"))

    def f(q_, k_, v_, cu_):
        return torch.ops.fmha_amd.decode(q_, k_, v_, cu_, -1, 0.0) * 2

    g = torch.compile(f, backend="aot_eager", fullgraph=True)
    o1 = g(*args[:4])
    o2 = f(*args[:4])
    torch.cuda.synchronize()
    assert torch.equal(o1, o2)


@pytest.mark.gpu
def test_layout_ops_match_direct_calls():
    """decode_splitkv / decode_strided / decode_paged give the bits of the
    direct calls, pass opcheck, and run under torch.compile."""
    import torch
    import fmha_amd
    import fmha_amd.torch_ops  # noqa: F401
    B, Hq, Hkv, D, S = 6, 16, 4, 128, 200
    seqlens = np.array([200, 17, 0, 150, 3, 99], np.int32)
    q, k, v, cu = make_inputs(B, Hq, Hkv, D, seqlens, seed=1002)
    qd, kd, vd, cud = to_dev(q), to_dev(k), to_dev(v), torch.from_numpy(cu).cuda()
    lens = torch.from_numpy(seqlens).cuda()
    o_sk = torch.ops.fmha_amd.decode_splitkv(qd, kd, vd, cud, S, 0.0)
    # the same rows as a BHSD cache and as a paged cache of 16-row pages
    kb = torch.zeros(B, Hkv, S, D, dtype=torch.bfloat16, device="cuda")
    vb = torch.zeros_like(kb)
    pages_per = (S + 15) // 16
    kc = torch.zeros(B * pages_per, 16, Hkv, D, dtype=torch.bfloat16, device="cuda")
    vc = torch.zeros_like(kc)
    bt = torch.arange(B * pages_per, dtype=torch.int32, device="cuda").flip(0).view(B, pages_per).contiguous()
    for b in range(B):
        rows = slice(int(cu[b]), int(cu[b + 1]))
        n = int(seqlens[b])
        kb[b, :, :n] = kd[rows].transpose(0, 1)
        vb[b, :, :n] = vd[rows].transpose(0, 1)
        for j in range(0, n, 16):
            m = min(16, n - j)
            kc[bt[b, j // 16], :m] = kd[int(cu[b]) + j:int(cu[b]) + j + m]
            vc[bt[b, j // 16], :m] = vd[int(cu[b]) + j:int(cu[b]) + j + m]
    o_st = torch.ops.fmha_amd.decode_strided(qd, kb.transpose(1, 2), vb.transpose(1, 2), lens, 0.0)
    o_pg = torch.ops.fmha_amd.decode_paged(qd, kc, vc, bt, lens, 0.0, S)
    torch.cuda.synchronize()
    assert torch.equal(o_sk.view(torch.int16),
                       fmha_amd.fmha_decode_splitkv(qd, kd, vd, cud, S).view(torch.int16))
    assert torch.equal(o_st.view(torch.int16),
                       fmha_amd.fmha_decode_strided(qd, kb.transpose(1, 2), vb.transpose(1, 2),
                                                    seqlens_kv=lens).view(torch.int16))
    assert torch.equal(o_pg.view(torch.int16),
                       fmha_amd.fmha_decode_paged(qd, kc, vc, bt, lens, max_seqlen_kv=S).view(torch.int16))
    from tests.common import assert_pass
    r, slack = oracle.decode(q, k, v, cu, Hq, Hkv, D, default_scale(D), with_slack=True, max_seqlen=S)
    for name, o in (("splitkv", o_sk), ("strided", o_st), ("paged", o_pg)):
        assert_pass(oracle.compare(o.view(torch.int16).cpu().numpy().view(np.uint16), r, slack), f"op {name}")
    tests = ("test_schema", "test_faketensor", "test_aot_dispatch_static")
    torch.library.opcheck(torch.ops.fmha_amd.decode_splitkv.default, (qd, kd, vd, cud, S, 0.0), test_utils=tests)
    torch.library.opcheck(torch.ops.fmha_amd.decode_paged.default, (qd, kc, vc, bt, lens, 0.0, S),
                          test_utils=tests)

    def f(q_, kc_, vc_, bt_, lens_):
        return torch.ops.fmha_amd.decode_paged(q_, kc_, vc_, bt_, lens_, 0.0, S).float().sum(dim=-1)

    g = torch.compile(f, backend="aot_eager", fullgraph=True)
    assert torch.equal(g(qd, kc, vc, bt, lens), f(qd, kc, vc, bt, lens))
