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
