"""GPU parity of lengths beyond 16 over strided and paged caches
(fmha_decode_fwd_splitkv_strided / fmha_decode_fwd_splitkv_paged, reached
through fmha_amd.fmha_decode_strided and fmha_amd.fmha_decode_paged).

Each case builds the cache on the host from packed rows (tests.common
make_inputs), with every row, slot and page the kernels must not read set to
NaN, and checks the output against the oracle run over the packed rows past
16 (oracle.decode(max_seqlen=...)), gate as in tests/common.py.  Small
batches take the split-KV launches, large ones the single pass (batch * KV
head groups >= 512); page sizes below 16 look pages up per row, 16 and above
per 16-row sub-block."""
import numpy as np
import pytest

import oracle
from tests.common import assert_pass, cu_from_seqlens, default_scale, last_plan, make_inputs, to_dev

pytestmark = pytest.mark.gpu

NAN_BITS = np.uint16(0x7FC0)


def _units(B, Hkv, D):
    hpw = 64 // (D // 8)
    return B * ((Hkv + hpw - 1) // hpw)


def _check(o, q, kp, vp, seqlens, Hq, Hkv, D, max_len, ctx):
    import torch
    bits = o.view(torch.int16).cpu().numpy().view(np.uint16)
    r, slack = oracle.decode(q, kp, vp, cu_from_seqlens(seqlens), Hq, Hkv, D, default_scale(D), with_slack=True,
                             max_seqlen=max_len)
    st = oracle.compare(bits.reshape(r.shape), r, slack)
    print(f"{ctx}: {st}", flush=True)
    assert_pass(st, ctx)


def _strided_cache(kp, seqlens, cap, Hkv, D, layout):
    """Host cache [B, cap, Hkv, D] (bshd) or [B, Hkv, cap, D] (bhsd) with NaN padding."""
    B = len(seqlens)
    cu = cu_from_seqlens(seqlens)
    c = np.full((B, cap, Hkv, D), NAN_BITS, np.uint16)
    for b in range(B):
        c[b, :seqlens[b]] = kp[cu[b]:cu[b + 1]]
    if layout == "bhsd":
        c = np.ascontiguousarray(c.transpose(0, 2, 1, 3))
    return c


def _strided_view(c, layout):
    t = to_dev(c)
    return t.transpose(1, 2) if layout == "bhsd" else t


@pytest.mark.parametrize("layout", ["bhsd", "bshd"])
@pytest.mark.parametrize("B,cap", [(5, 700), (600, 72)])
@pytest.mark.parametrize("D,Hq,Hkv", [(128, 32, 8), (64, 16, 2), (256, 16, 4)])
def test_strided_long(layout, B, cap, D, Hq, Hkv):
    import fmha_amd
    import torch
    rng = np.random.default_rng(B + cap + D)
    seqlens = rng.integers(0, cap + 1, size=B).astype(np.int32)
    seqlens[0] = cap
    seqlens[1] = 0
    q, kp, vp, cu = make_inputs(B, Hq, Hkv, D, seqlens, seed=B * 7 + D)
    kc = _strided_view(_strided_cache(kp, seqlens, cap, Hkv, D, layout), layout)
    vc = _strided_view(_strided_cache(vp, seqlens, cap, Hkv, D, layout), layout)
    o = fmha_amd.fmha_decode_strided(to_dev(q), kc, vc, seqlens_kv=torch.from_numpy(seqlens).cuda())
    torch.cuda.synchronize()
    path = "single pass" if _units(B, Hkv, D) >= 512 else "split"
    _check(o, q, kp, vp, seqlens, Hq, Hkv, D, cap, f"{layout} B={B} cap={cap} D={D} Hq={Hq} Hkv={Hkv} ({path})")


@pytest.mark.parametrize("layout", ["bhsd", "bshd"])
@pytest.mark.parametrize("D,Hq,Hkv,B,cap", [(128, 16, 16, 64, 256), (128, 32, 8, 200, 96), (256, 16, 8, 60, 160)])
def test_strided_onepass_group(monkeypatch, layout, D, Hq, Hkv, B, cap):
    """Strided caches with too few units for one wave each: the single pass
    with two waves per row (plan onepass_group; the register single pass,
    which takes groups of 2 and 4 at D = 128 first, off), NaN padding past
    each length never read."""
    import fmha_amd
    import torch
    monkeypatch.setenv("FMHA_DECODE_ONEPASS_REG", "0")
    rng = np.random.default_rng(B + cap + D + 1)
    seqlens = rng.integers(0, cap + 1, size=B).astype(np.int32)
    seqlens[:4] = [cap, 0, 1, 33]
    q, kp, vp, cu = make_inputs(B, Hq, Hkv, D, seqlens, seed=B * 5 + D)
    kc = _strided_view(_strided_cache(kp, seqlens, cap, Hkv, D, layout), layout)
    vc = _strided_view(_strided_cache(vp, seqlens, cap, Hkv, D, layout), layout)
    o = fmha_amd.fmha_decode_strided(to_dev(q), kc, vc, seqlens_kv=torch.from_numpy(seqlens).cuda())
    torch.cuda.synchronize()
    assert [k for k, _ in last_plan()] == ["onepass_group"], last_plan()
    _check(o, q, kp, vp, seqlens, Hq, Hkv, D, cap, f"{layout} group B={B} cap={cap} D={D} Hq={Hq} Hkv={Hkv}")


@pytest.mark.parametrize("layout", ["bhsd", "bshd"])
@pytest.mark.parametrize("D,kind", [(128, "onepass_matrix_core_regs"), (256, "onepass_matrix_core")])
def test_strided_onepass_matrix_core(layout, D, kind):
    """Strided caches, 8 query heads per KV head, 512 (batch, KV head)
    units: the matrix-core single pass, the scores in registers at D = 128
    and in LDS at D = 256."""
    import fmha_amd
    import torch
    B, Hq, Hkv, cap = 128, 32, 4, 400
    rng = np.random.default_rng(77)
    seqlens = rng.integers(0, cap + 1, size=B).astype(np.int32)
    seqlens[:4] = [cap, 0, 1, 65]
    q, kp, vp, cu = make_inputs(B, Hq, Hkv, D, seqlens, seed=78)
    kc = _strided_view(_strided_cache(kp, seqlens, cap, Hkv, D, layout), layout)
    vc = _strided_view(_strided_cache(vp, seqlens, cap, Hkv, D, layout), layout)
    o = fmha_amd.fmha_decode_strided(to_dev(q), kc, vc, seqlens_kv=torch.from_numpy(seqlens).cuda())
    torch.cuda.synchronize()
    assert [k for k, _ in last_plan()] == [kind], last_plan()
    _check(o, q, kp, vp, seqlens, Hq, Hkv, D, cap, f"{layout} {kind}")


def test_strided_uniform_long_bhsd():
    """No lengths array: every batch has all cap rows."""
    import fmha_amd
    import torch
    B, Hq, Hkv, D, cap = 3, 16, 16, 128, 300
    seqlens = np.full(B, cap, np.int32)
    q, kp, vp, cu = make_inputs(B, Hq, Hkv, D, seqlens, seed=77)
    kc = _strided_view(_strided_cache(kp, seqlens, cap, Hkv, D, "bhsd"), "bhsd")
    vc = _strided_view(_strided_cache(vp, seqlens, cap, Hkv, D, "bhsd"), "bhsd")
    o = fmha_amd.fmha_decode_strided(to_dev(q), kc, vc)
    torch.cuda.synchronize()
    _check(o, q, kp, vp, seqlens, Hq, Hkv, D, cap, "bhsd uniform S=300")


def test_strided_long_length_beyond_capacity_is_nan():
    import fmha_amd
    import torch
    B, H, D, cap = 3, 4, 128, 40
    seqlens = np.array([40, 30, 2], np.int32)
    q, kp, vp, cu = make_inputs(B, H, H, D, seqlens, seed=78)
    kc = to_dev(_strided_cache(kp, seqlens, cap, H, D, "bshd"))
    vc = to_dev(_strided_cache(vp, seqlens, cap, H, D, "bshd"))
    lens = torch.tensor([40, 41, 2], dtype=torch.int32, device="cuda")
    o = fmha_amd.fmha_decode_strided(to_dev(q), kc, vc, seqlens_kv=lens).float()
    torch.cuda.synchronize()
    assert torch.isnan(o[1]).all() and torch.isfinite(o[0]).all() and torch.isfinite(o[2]).all()


def _paged_cache(kp, vp, seqlens, page_size, Hkv, D, rng, extra_pages=5, spare_entries=1):
    """Host page caches with pages handed out in random order, NaN in every
    slot no batch owns, -1 in every block-table entry past a batch's pages."""
    B = len(seqlens)
    cu = cu_from_seqlens(seqlens)
    need = [(int(s) + page_size - 1) // page_size for s in seqlens]
    max_pages = max(max(need), 1) + spare_entries
    num_pages = sum(need) + extra_pages
    perm = rng.permutation(num_pages).astype(np.int32)
    bt = np.full((B, max_pages), -1, np.int32)
    kc = np.full((num_pages, page_size, Hkv, D), NAN_BITS, np.uint16)
    vc = np.full((num_pages, page_size, Hkv, D), NAN_BITS, np.uint16)
    i = 0
    for b in range(B):
        for p in range(need[b]):
            page = perm[i]
            i += 1
            bt[b, p] = page
            r0, r1 = cu[b] + p * page_size, min(cu[b] + (p + 1) * page_size, cu[b + 1])
            kc[page, :r1 - r0] = kp[r0:r1]
            vc[page, :r1 - r0] = vp[r0:r1]
    return kc, vc, bt


@pytest.mark.parametrize("page_size", [1, 4, 16, 64])
@pytest.mark.parametrize("B,max_len", [(4, 600), (700, 40)])
@pytest.mark.parametrize("D,Hq,Hkv", [(128, 32, 8), (64, 8, 1), (256, 16, 8)])
def test_paged_long(page_size, B, max_len, D, Hq, Hkv):
    import fmha_amd
    import torch
    rng = np.random.default_rng(page_size * 1000 + B + D)
    seqlens = rng.integers(0, max_len + 1, size=B).astype(np.int32)
    seqlens[0] = max_len
    seqlens[-1] = 0
    q, kp, vp, cu = make_inputs(B, Hq, Hkv, D, seqlens, seed=page_size + B + D)
    kc, vc, bt = _paged_cache(kp, vp, seqlens, page_size, Hkv, D, rng)
    o = fmha_amd.fmha_decode_paged(to_dev(q), to_dev(kc), to_dev(vc), torch.from_numpy(bt).cuda(),
                                   torch.from_numpy(seqlens).cuda(), max_seqlen_kv=max_len)
    torch.cuda.synchronize()
    path = "single pass" if _units(B, Hkv, D) >= 512 else "split"
    _check(o, q, kp, vp, seqlens, Hq, Hkv, D, max_len,
           f"paged ps={page_size} B={B} max={max_len} D={D} Hq={Hq} Hkv={Hkv} ({path})")


@pytest.mark.parametrize("page_size", [2, 32])
def test_paged_long_bounds_are_nan(page_size):
    """A length above max_seqlen_kv, and one above what the block-table row
    maps (block_table_stride * page_size), give NaN for that batch only."""
    import fmha_amd
    import torch
    B, H, D, max_len = 4, 8, 128, 100
    rng = np.random.default_rng(page_size)
    seqlens = np.array([100, 60, 7, 33], np.int32)
    q, kp, vp, cu = make_inputs(B, H, H, D, seqlens, seed=79)
    kc, vc, bt = _paged_cache(kp, vp, seqlens, page_size, H, D, rng, spare_entries=0)
    lens = torch.from_numpy(seqlens).cuda()
    lens[2] = max_len + 1
    o = fmha_amd.fmha_decode_paged(to_dev(q), to_dev(kc), to_dev(vc), torch.from_numpy(bt).cuda(), lens,
                                   max_seqlen_kv=max_len).float()
    torch.cuda.synchronize()
    assert torch.isnan(o[2]).all()
    assert torch.isfinite(o[[0, 1, 3]]).all()
    # The table rows end at the longest batch's pages: a bound above them is
    # cut to the row's capacity, so a length past it is NaN as well.
    cap = bt.shape[1] * page_size
    lens2 = torch.from_numpy(seqlens).cuda()
    lens2[3] = cap + 1
    o2 = fmha_amd.fmha_decode_paged(to_dev(q), to_dev(kc), to_dev(vc), torch.from_numpy(bt).cuda(), lens2,
                                    max_seqlen_kv=10 * cap).float()
    torch.cuda.synchronize()
    assert torch.isnan(o2[3]).all() and torch.isfinite(o2[[0, 1, 2]]).all()


def test_paged_short_bound_through_long_entry():
    """max_seqlen_kv <= 16 runs the short kernel with that bound."""
    import fmha_amd
    import torch
    B, Hq, Hkv, D, page_size = 40, 16, 4, 128, 4
    rng = np.random.default_rng(5)
    seqlens = rng.integers(0, 11, size=B).astype(np.int32)
    q, kp, vp, cu = make_inputs(B, Hq, Hkv, D, seqlens, seed=80)
    kc, vc, bt = _paged_cache(kp, vp, seqlens, page_size, Hkv, D, rng)
    o = fmha_amd.fmha_decode_paged(to_dev(q), to_dev(kc), to_dev(vc), torch.from_numpy(bt).cuda(),
                                   torch.from_numpy(seqlens).cuda(), max_seqlen_kv=10)
    torch.cuda.synchronize()
    _check(o, q, kp, vp, seqlens, Hq, Hkv, D, 16, "paged short bound 10")
    lens = torch.from_numpy(seqlens).cuda()
    lens[3] = 11
    o2 = fmha_amd.fmha_decode_paged(to_dev(q), to_dev(kc), to_dev(vc), torch.from_numpy(bt).cuda(), lens,
                                    max_seqlen_kv=10).float()
    torch.cuda.synchronize()
    assert torch.isnan(o2[3]).all()


@pytest.mark.parametrize("D,Hq,Hkv", [(128, 8, 1), (64, 16, 2), (256, 8, 1)])
def test_strided_long_sub_units(D, Hq, Hkv):
    """BHSD with fewer KV heads than a wave holds (lane groups on different
    blocks and chunks), NaN padding between the heads' rows."""
    import fmha_amd
    import torch
    B, cap = 4, 1000
    seqlens = np.array([1000, 999, 15, 400], np.int32)
    q, kp, vp, cu = make_inputs(B, Hq, Hkv, D, seqlens, seed=1400 + D)
    kc = _strided_view(_strided_cache(kp, seqlens, cap, Hkv, D, "bhsd"), "bhsd")
    vc = _strided_view(_strided_cache(vp, seqlens, cap, Hkv, D, "bhsd"), "bhsd")
    o = fmha_amd.fmha_decode_strided(to_dev(q), kc, vc, seqlens_kv=torch.from_numpy(seqlens).cuda())
    torch.cuda.synchronize()
    _check(o, q, kp, vp, seqlens, Hq, Hkv, D, cap, f"bhsd sub-units D={D} Hq={Hq} Hkv={Hkv}")


@pytest.mark.parametrize("D,Hq,Hkv,B,cap", [(64, 8, 1, 4100, 64), (128, 8, 1, 2049, 96), (128, 4, 1, 2049, 80),
                                             (64, 8, 2, 2100, 80)])
def test_strided_single_pass_batches_per_wave(D, Hq, Hkv, B, cap):
    """Single pass, several batches per wave through one strided descriptor,
    BHSD with NaN padding (G = 8 takes it on rows of up to 64 at D = 64 and
    96 at D = 128)."""
    import fmha_amd
    import torch
    rng = np.random.default_rng(D + B)
    seqlens = rng.integers(0, cap + 1, size=B).astype(np.int32)
    seqlens[:4] = [cap, 0, 1, 17]
    q, kp, vp, cu = make_inputs(B, Hq, Hkv, D, seqlens, seed=1700 + D)
    kc = _strided_view(_strided_cache(kp, seqlens, cap, Hkv, D, "bhsd"), "bhsd")
    vc = _strided_view(_strided_cache(vp, seqlens, cap, Hkv, D, "bhsd"), "bhsd")
    o = fmha_amd.fmha_decode_strided(to_dev(q), kc, vc, seqlens_kv=torch.from_numpy(seqlens).cuda())
    torch.cuda.synchronize()
    _check(o, q, kp, vp, seqlens, Hq, Hkv, D, cap, f"bhsd single pass per-wave batches D={D} Hkv={Hkv}")


@pytest.mark.parametrize("layout", ["bhsd", "bshd"])
@pytest.mark.parametrize("B,cap", [(5, 300), (600, 40)])
def test_strided_long_padded_group(layout, B, cap):
    """G = 5 beyond 16 rows over a strided cache (padded query group)."""
    import fmha_amd
    import torch
    D, Hq, Hkv = 128, 20, 4
    rng = np.random.default_rng(B + cap)
    seqlens = rng.integers(0, cap + 1, size=B).astype(np.int32)
    seqlens[0] = cap
    q, kp, vp, cu = make_inputs(B, Hq, Hkv, D, seqlens, seed=B + cap + 3)
    kc = _strided_cache(kp, seqlens, cap, Hkv, D, layout)
    vc = _strided_cache(vp, seqlens, cap, Hkv, D, layout)
    o = fmha_amd.fmha_decode_strided(to_dev(q), _strided_view(kc, layout), _strided_view(vc, layout),
                                     seqlens_kv=torch.from_numpy(seqlens).cuda())
    torch.cuda.synchronize()
    _check(o, q, kp, vp, seqlens, Hq, Hkv, D, cap, f"strided {layout} G=5 B={B} cap={cap}")


@pytest.mark.parametrize("page_size", [1, 16])
@pytest.mark.parametrize("B,max_len", [(4, 300), (700, 40), (40, 10)])
def test_paged_padded_group(page_size, B, max_len):
    """G = 7 over a paged cache through the workspace entry: split, single
    pass and (max_seqlen_kv <= 16) the short paged kernel, all on the padded
    query group."""
    import fmha_amd
    import torch
    D, Hq, Hkv = 128, 14, 2
    rng = np.random.default_rng(page_size * 7 + B + max_len)
    seqlens = rng.integers(0, max_len + 1, size=B).astype(np.int32)
    seqlens[0] = max_len
    q, kp, vp, cu = make_inputs(B, Hq, Hkv, D, seqlens, seed=page_size + B + max_len + 5)
    kc, vc, bt = _paged_cache(kp, vp, seqlens, page_size, Hkv, D, rng)
    o = fmha_amd.fmha_decode_paged(to_dev(q), to_dev(kc), to_dev(vc), torch.from_numpy(bt).cuda(),
                                   torch.from_numpy(seqlens).cuda(), max_seqlen_kv=max_len)
    torch.cuda.synchronize()
    _check(o, q, kp, vp, seqlens, Hq, Hkv, D, max(max_len, 16), f"paged G=7 ps={page_size} B={B} max={max_len}")


def test_long_layouts_group_slices():
    """G = 12 beyond 16 rows over BHSD and 16-row pages (two groups of 8 on
    one launch, padded to 16 query heads per KV head), and G = 12 with at
    most 16 rows through the paged workspace entry (the split kernels, one
    block)."""
    import fmha_amd
    import torch
    D, Hq, Hkv, B = 128, 24, 2, 5
    rng = np.random.default_rng(31)
    for cap in (200, 12):
        seqlens = rng.integers(0, cap + 1, size=B).astype(np.int32)
        seqlens[0] = cap
        q, kp, vp, cu = make_inputs(B, Hq, Hkv, D, seqlens, seed=cap + 32)
        kc = _strided_cache(kp, seqlens, cap, Hkv, D, "bhsd")
        vc = _strided_cache(vp, seqlens, cap, Hkv, D, "bhsd")
        o = fmha_amd.fmha_decode_strided(to_dev(q), _strided_view(kc, "bhsd"), _strided_view(vc, "bhsd"),
                                         seqlens_kv=torch.from_numpy(seqlens).cuda())
        torch.cuda.synchronize()
        _check(o, q, kp, vp, seqlens, Hq, Hkv, D, max(cap, 16), f"bhsd G=12 cap={cap}")
        kc2, vc2, bt = _paged_cache(kp, vp, seqlens, 16, Hkv, D, rng)
        o2 = fmha_amd.fmha_decode_paged(to_dev(q), to_dev(kc2), to_dev(vc2), torch.from_numpy(bt).cuda(),
                                        torch.from_numpy(seqlens).cuda(), max_seqlen_kv=cap)
        torch.cuda.synchronize()
        _check(o2, q, kp, vp, seqlens, Hq, Hkv, D, max(cap, 16), f"paged G=12 cap={cap}")


@pytest.mark.parametrize("kernel", ["mfma", "valu"])
@pytest.mark.parametrize("B,cap", [(3, 400), (600, 40), (7, 9)])
def test_long_layouts_grouped_launch_kv_heads(monkeypatch, kernel, B, cap):
    """G = 16 with one KV head, no copies of Q and O, over BHSD (the
    matrix-core split passes, or two VALU launch KV heads reading the same
    cache head) and over 1- and 16-row pages (launch KV heads)."""
    import fmha_amd
    import torch
    if kernel == "valu":
        monkeypatch.setenv("FMHA_DECODE_GQA_KERNEL", "valu")
    else:
        monkeypatch.delenv("FMHA_DECODE_GQA_KERNEL", raising=False)
    D, Hq, Hkv = 128, 16, 1
    rng = np.random.default_rng(B * 5 + cap)
    seqlens = rng.integers(0, cap + 1, size=B).astype(np.int32)
    seqlens[0] = cap
    q, kp, vp, cu = make_inputs(B, Hq, Hkv, D, seqlens, seed=B + cap + 41)
    kc = _strided_cache(kp, seqlens, cap, Hkv, D, "bhsd")
    vc = _strided_cache(vp, seqlens, cap, Hkv, D, "bhsd")
    o = fmha_amd.fmha_decode_strided(to_dev(q), _strided_view(kc, "bhsd"), _strided_view(vc, "bhsd"),
                                     seqlens_kv=torch.from_numpy(seqlens).cuda())
    torch.cuda.synchronize()
    _check(o, q, kp, vp, seqlens, Hq, Hkv, D, max(cap, 16), f"bhsd G=16 B={B} cap={cap}")
    for ps in (1, 16):
        kc2, vc2, bt = _paged_cache(kp, vp, seqlens, ps, Hkv, D, rng)
        o2 = fmha_amd.fmha_decode_paged(to_dev(q), to_dev(kc2), to_dev(vc2), torch.from_numpy(bt).cuda(),
                                        torch.from_numpy(seqlens).cuda(), max_seqlen_kv=cap)
        torch.cuda.synchronize()
        _check(o2, q, kp, vp, seqlens, Hq, Hkv, D, max(cap, 16), f"paged G=16 ps={ps} B={B} cap={cap}")


@pytest.mark.parametrize("page_size", [1, 8, 16, 32])
@pytest.mark.parametrize("D,Hq,Hkv", [(128, 8, 1), (128, 8, 2), (256, 4, 1), (128, 2, 2), (64, 20, 4)])
@pytest.mark.parametrize("B,max_len", [(3, 2000), (9, 100)])
def test_paged_long_few_kv_heads(page_size, D, Hq, Hkv, B, max_len):
    """Paged caches with fewer KV heads than a wave holds (MQA, GQA after
    tensor-parallel sharding): the split passes read through per-lane
    addresses, each lane group taking its own blocks and chunks (sub-units),
    with several chunks per row (2000) or one (100, the P.V pass writing O);
    G = 8, 4, 4, 1 and 5 (padded to 8)."""
    import fmha_amd
    import torch
    rng = np.random.default_rng(page_size * 7 + D + Hq + Hkv + B)
    seqlens = rng.integers(0, max_len + 1, size=B).astype(np.int32)
    seqlens[0] = max_len
    q, kp, vp, cu = make_inputs(B, Hq, Hkv, D, seqlens, seed=page_size + D + Hq + B + 61)
    kc, vc, bt = _paged_cache(kp, vp, seqlens, page_size, Hkv, D, rng)
    o = fmha_amd.fmha_decode_paged(to_dev(q), to_dev(kc), to_dev(vc), torch.from_numpy(bt).cuda(),
                                   torch.from_numpy(seqlens).cuda(), max_seqlen_kv=max_len)
    torch.cuda.synchronize()
    _check(o, q, kp, vp, seqlens, Hq, Hkv, D, max_len, f"paged ps={page_size} D={D} {Hq}/{Hkv} B={B}")


@pytest.mark.parametrize("page_size", [1, 4, 8, 16, 32, 64])
@pytest.mark.parametrize("Hq,Hkv,B,max_len", [(64, 8, 128, 1000), (32, 8, 100, 700), (128, 8, 70, 2000)])
def test_paged_onepass_registers(page_size, Hq, Hkv, B, max_len):
    """Paged caches, rows of 4 blocks and more with >= 512 (batch, KV head)
    units: the matrix-core register single pass (groups of 8, 4 and 16),
    each 16-row tile read through its page (pages of 16 rows and more) or
    each row through its own (smaller pages), NaN in every slot no batch
    owns; ragged lengths, empty rows and 16-row edges."""
    import fmha_amd
    import torch
    D = 128
    rng = np.random.default_rng(page_size * 13 + Hq + B + max_len)
    seqlens = rng.integers(0, max_len + 1, size=B).astype(np.int32)
    seqlens[:5] = [max_len, 0, 1, 16, 257]
    q, kp, vp, cu = make_inputs(B, Hq, Hkv, D, seqlens, seed=page_size + Hq + B + 71)
    kc, vc, bt = _paged_cache(kp, vp, seqlens, page_size, Hkv, D, rng)
    print(f"paged register pass: ps={page_size} {Hq}/{Hkv} B={B} max={max_len}", flush=True)
    o = fmha_amd.fmha_decode_paged(to_dev(q), to_dev(kc), to_dev(vc), torch.from_numpy(bt).cuda(),
                                   torch.from_numpy(seqlens).cuda(), max_seqlen_kv=max_len)
    torch.cuda.synchronize()
    assert _route() == ("onepass_matrix_core_regs", "paged16" if page_size >= 16 else "paged"), last_plan()
    _check(o, q, kp, vp, seqlens, Hq, Hkv, D, max_len, f"paged register pass ps={page_size} {Hq}/{Hkv} B={B}")


def _route():
    """(kind, layout) of the last launch of the most recent call."""
    kind, fields = last_plan()[-1]
    return kind, fields["layout"]


# The route each paged single-pass case takes, by (D, Hq, Hkv, max_len):
# (pages under 16 rows, 16-row pages and larger).  "onepass" with a *_lanes
# layout is the single pass with per-lane page lookups (several batches per
# wave); rows of four blocks take the matrix-core register single pass
# where that is faster (the planner's rules in split_on_matrix_cores,
# launch_split_dg and onepass_reg_tiles, fmha_decode_api.hip /
# fmha_decode_launch.hpp).
_LANES = ("onepass", "paged_lanes")
_LANES16 = ("onepass", "paged16_lanes")
_REG16 = ("onepass_matrix_core_regs", "paged16")
_REG = ("onepass_matrix_core_regs", "paged")
PAGED_FEW_ROUTES = {
    (128, 8, 1, 17): (_LANES, _LANES16), (128, 8, 1, 32): (_LANES, _LANES16), (128, 8, 1, 64): (_LANES, _REG16),
    (128, 16, 2, 17): (_LANES, _LANES16), (128, 16, 2, 32): (_LANES, _LANES16), (128, 16, 2, 64): (_LANES, _REG16),
    (256, 4, 1, 17): (_LANES, _LANES16), (256, 4, 1, 32): (_LANES, _LANES16),
    (256, 4, 1, 64): (_LANES, _LANES16),
    (64, 8, 1, 17): (_LANES, _LANES16), (64, 8, 1, 32): (_LANES, _LANES16), (64, 8, 1, 64): (_LANES, _REG16),
    (128, 40, 8, 17): (("onepass", "paged"), ("onepass", "paged16")),
    (128, 40, 8, 32): (("onepass", "paged"), ("onepass", "paged16")),
    (128, 40, 8, 64): (("onepass", "paged"), ("onepass", "paged16")),
}
PAGED_LONGER_ROUTES = {
    (128, 4, 1, 48): (_LANES, _LANES16), (128, 4, 1, 128): (_LANES, _LANES16),
    (64, 2, 1, 48): (_LANES, _LANES16), (64, 2, 1, 128): (_LANES, _LANES16),
    (128, 8, 2, 48): (_LANES, _LANES16), (128, 8, 2, 128): (_LANES, _LANES16),
    (64, 1, 1, 48): (_LANES, _LANES16), (64, 1, 1, 128): (_LANES, _LANES16),
}


@pytest.mark.parametrize("page_size", [16, 32, 64])
@pytest.mark.parametrize("Hq,Hkv,B,cap", [(64, 8, 80, 400), (32, 4, 130, 300)])
def test_paged_onepass_matrix_core(page_size, Hq, Hkv, B, cap):
    """Pages of 16 rows or more at D = 256, groups of 8, at least 512
    (batch, KV head) units and rows of at most 40 blocks: the matrix-core
    single pass with the row's scores in LDS, every lane addressing its own
    rows; empty rows and 16-row edges."""
    import fmha_amd
    import torch
    D = 256
    rng = np.random.default_rng(page_size * 5 + Hq + B)
    seqlens = rng.integers(0, cap + 1, size=B).astype(np.int32)
    seqlens[:5] = [cap, 0, 1, 16, 129]
    q, kp, vp, cu = make_inputs(B, Hq, Hkv, D, seqlens, seed=page_size + Hq + B + 5)
    kc, vc, bt = _paged_cache(kp, vp, seqlens, page_size, Hkv, D, rng)
    print(f"paged matrix-core single pass: ps={page_size} {Hq}/{Hkv} B={B} cap={cap}", flush=True)
    o = fmha_amd.fmha_decode_paged(to_dev(q), to_dev(kc), to_dev(vc), torch.from_numpy(bt).cuda(),
                                   torch.from_numpy(seqlens).cuda(), max_seqlen_kv=cap)
    torch.cuda.synchronize()
    assert _route() == ("onepass_matrix_core", "paged16"), last_plan()
    _check(o, q, kp, vp, seqlens, Hq, Hkv, D, cap, f"paged matrix-core single pass ps={page_size} {Hq}/{Hkv}")


@pytest.mark.parametrize("page_size", [1, 4, 16, 32])
@pytest.mark.parametrize("D,Hq,Hkv,B", [(128, 8, 1, 2100), (128, 16, 2, 1100), (256, 4, 1, 1100), (64, 8, 1, 4200),
                                        (128, 40, 8, 700)])
@pytest.mark.parametrize("max_len", [17, 32, 64])
def test_paged_single_pass_few_kv_heads(page_size, D, Hq, Hkv, B, max_len):
    """Rows of one to four 16-row blocks over paged caches with fewer KV
    heads than a wave holds and >= 512 waves: the single pass with each lane
    group looking up its own batch's pages (several batches per wave), or
    the matrix-core split, as PAGED_FEW_ROUTES pins each case; the last
    shape fills a wave and runs one batch per wave."""
    import fmha_amd
    import torch
    rng = np.random.default_rng(page_size * 11 + D + Hq + Hkv + B + max_len)
    seqlens = rng.integers(0, max_len + 1, size=B).astype(np.int32)
    seqlens[0] = max_len
    seqlens[-1] = 0
    q, kp, vp, cu = make_inputs(B, Hq, Hkv, D, seqlens, seed=page_size + D + Hq + B + max_len)
    kc, vc, bt = _paged_cache(kp, vp, seqlens, page_size, Hkv, D, rng)
    print(f"paged single pass: ps={page_size} D={D} {Hq}/{Hkv} B={B} max={max_len}", flush=True)
    o = fmha_amd.fmha_decode_paged(to_dev(q), to_dev(kc), to_dev(vc), torch.from_numpy(bt).cuda(),
                                   torch.from_numpy(seqlens).cuda(), max_seqlen_kv=max_len)
    torch.cuda.synchronize()
    assert _route() == PAGED_FEW_ROUTES[(D, Hq, Hkv, max_len)][page_size >= 16], last_plan()
    _check(o, q, kp, vp, seqlens, Hq, Hkv, D, max_len, f"paged single pass ps={page_size} D={D} {Hq}/{Hkv} B={B}")



@pytest.mark.parametrize("page_size", [1, 4, 16])
@pytest.mark.parametrize("D,max_len", [(64, 64), (128, 96), (256, 128), (128, 48)])
def test_paged_single_pass_group_of_eight(page_size, D, max_len):
    """Eight query heads per KV head on the single pass (one batch per wave)
    over paged caches: pages under 16 rows (per-row page lookups) at the
    longest rows it takes there for each head dim, 16-row pages with rows of
    up to four blocks (the kernel scheduled for two waves per SIMD) and
    longer; empty rows and 16-row edges."""
    import fmha_amd
    import torch
    B, Hq, Hkv = 600, 64, 8
    rng = np.random.default_rng(page_size * 13 + D + max_len)
    seqlens = rng.integers(0, max_len + 1, size=B).astype(np.int32)
    seqlens[:6] = [max_len, 0, 1, 15, 16, 17]
    q, kp, vp, cu = make_inputs(B, Hq, Hkv, D, seqlens, seed=page_size + D + max_len + 71)
    kc, vc, bt = _paged_cache(kp, vp, seqlens, page_size, Hkv, D, rng)
    print(f"paged single pass G=8: ps={page_size} D={D} B={B} max={max_len}", flush=True)
    o = fmha_amd.fmha_decode_paged(to_dev(q), to_dev(kc), to_dev(vc), torch.from_numpy(bt).cuda(),
                                   torch.from_numpy(seqlens).cuda(), max_seqlen_kv=max_len)
    torch.cuda.synchronize()
    assert _route() == ("onepass", "paged16" if page_size >= 16 else "paged"), last_plan()
    _check(o, q, kp, vp, seqlens, Hq, Hkv, D, max_len, f"paged single pass G=8 ps={page_size} D={D}")


@pytest.mark.parametrize("page_size", [1, 4, 16, 32])
@pytest.mark.parametrize("D,Hq,Hkv,B", [(128, 4, 1, 2100), (64, 2, 1, 4200), (128, 8, 2, 1100), (64, 1, 1, 4200)])
@pytest.mark.parametrize("max_len", [48, 128])
def test_paged_single_pass_few_kv_heads_longer_rows(page_size, D, Hq, Hkv, B, max_len):
    """Rows of three to eight 16-row blocks over paged caches with fewer KV
    heads than a wave holds, up to 4 query heads per KV head, >= 512 waves:
    the single pass with per-lane page lookups, several batches per wave,
    empty rows, rows on and next to the 16-row edges."""
    import fmha_amd
    import torch
    rng = np.random.default_rng(page_size * 17 + D + Hq + Hkv + B + max_len)
    seqlens = rng.integers(0, max_len + 1, size=B).astype(np.int32)
    seqlens[:7] = [max_len, 0, 1, 15, 16, 17, 33]
    seqlens[-1] = max_len
    q, kp, vp, cu = make_inputs(B, Hq, Hkv, D, seqlens, seed=page_size + D + Hq + B + max_len + 3)
    kc, vc, bt = _paged_cache(kp, vp, seqlens, page_size, Hkv, D, rng)
    print(f"paged single pass longer rows: ps={page_size} D={D} {Hq}/{Hkv} B={B} max={max_len}", flush=True)
    o = fmha_amd.fmha_decode_paged(to_dev(q), to_dev(kc), to_dev(vc), torch.from_numpy(bt).cuda(),
                                   torch.from_numpy(seqlens).cuda(), max_seqlen_kv=max_len)
    torch.cuda.synchronize()
    assert _route() == PAGED_LONGER_ROUTES[(D, Hq, Hkv, max_len)][page_size >= 16], last_plan()
    _check(o, q, kp, vp, seqlens, Hq, Hkv, D, max_len,
           f"paged single pass longer rows ps={page_size} D={D} {Hq}/{Hkv} B={B} max={max_len}")


def _random_register_cases(n=12, seed=2026):
    """Seeded shapes inside the register single pass's domain: groups of
    2-16 query heads per KV head (after padding), D = 64 or 128, at least
    512 (batch, KV head) units, max_len from 4 blocks to 4096 rows, and the
    layout: packed, BHSD, or pages of 16 or 32 rows."""
    rng = np.random.default_rng(seed)
    cases = []
    while len(cases) < n:
        D = int(rng.choice([64, 128]))
        G = int(rng.choice([2, 3, 4, 5, 6, 8, 12, 16]))
        Hkv = int(rng.choice([1, 2, 4, 8]))
        max_len = int(rng.integers(64, 4097))
        units = int(rng.integers(512, 1400))
        B = -(-units // Hkv)
        layout = str(rng.choice(["packed", "bhsd", "paged16", "paged32"]))
        # bound the oracle's work (rows x query heads x D)
        if B * max_len * G * Hkv * D // 2 > 2.5e9:
            continue
        cases.append((D, G * Hkv, Hkv, B, max_len, layout))
    return cases


@pytest.mark.parametrize("D,Hq,Hkv,B,max_len,layout", _random_register_cases())
def test_register_single_pass_random_shapes(D, Hq, Hkv, B, max_len, layout):
    """Seeded random shapes that the planner sends to the matrix-core register
    single pass (where the VALU single pass does not hold the row first),
    against the oracle, with ragged lengths (0, 1, one block and the maximum
    among them); the plan is checked to be that pass for groups of 5 and
    more, whose routes it always takes here."""
    import fmha_amd
    import torch
    rng = np.random.default_rng(D + Hq * 7 + Hkv * 31 + B + max_len)
    seqlens = rng.integers(0, max_len + 1, size=B).astype(np.int32)
    seqlens[:4] = [max_len, 0, 1, 16]
    q, kp, vp, cu = make_inputs(B, Hq, Hkv, D, seqlens, seed=B + max_len + Hq)
    print(f"register pass random: {layout} D={D} {Hq}/{Hkv} B={B} max={max_len}", flush=True)
    if layout == "packed":
        o = fmha_amd.fmha_decode_splitkv(to_dev(q), to_dev(kp), to_dev(vp), torch.from_numpy(cu).cuda(), max_len)
    elif layout == "bhsd":
        kc = _strided_view(_strided_cache(kp, seqlens, max_len, Hkv, D, "bhsd"), "bhsd")
        vc = _strided_view(_strided_cache(vp, seqlens, max_len, Hkv, D, "bhsd"), "bhsd")
        o = fmha_amd.fmha_decode_strided(to_dev(q), kc, vc, seqlens_kv=torch.from_numpy(seqlens).cuda())
    else:
        kc, vc, bt = _paged_cache(kp, vp, seqlens, int(layout[5:]), Hkv, D, rng)
        o = fmha_amd.fmha_decode_paged(to_dev(q), to_dev(kc), to_dev(vc), torch.from_numpy(bt).cuda(),
                                       torch.from_numpy(seqlens).cuda(), max_seqlen_kv=max_len)
    torch.cuda.synchronize()
    kinds = [k for k, _ in last_plan()]
    if Hq // Hkv >= 5:
        assert kinds[-1] == "onepass_matrix_core_regs", last_plan()
    _check(o, q, kp, vp, seqlens, Hq, Hkv, D, max_len, f"register pass random {layout} D={D} {Hq}/{Hkv} B={B}")
