"""GPU parity for the strided (BSHD, BHSD, padded) and paged KV layouts
(fmha_decode_fwd_strided / fmha_decode_fwd_paged): each case gathers the
rows a batch owns into the packed layout and checks the kernel against the
oracle there, with every row the kernel must not read poisoned with NaN."""
import numpy as np
import pytest

import oracle
from tests.common import assert_pass, cu_from_seqlens, default_scale, last_plan

pytestmark = pytest.mark.gpu

NAN = np.uint16(0x7FC0)


def _bf16(gen, shape, device):
    import torch
    return torch.randn(*shape, generator=gen, device=device, dtype=torch.bfloat16)


def _bits(t):
    import torch
    return t.contiguous().view(torch.int16).cpu().numpy().view(np.uint16)


def _check(o, q, packed_k, packed_v, seqlens, Hq, Hkv, D, ctx):
    r, slack = oracle.decode(_bits(q).reshape(len(seqlens), Hq, D), packed_k, packed_v,
                             cu_from_seqlens(seqlens), Hq, Hkv, D, default_scale(D), with_slack=True)
    assert_pass(oracle.compare(_bits(o).reshape(r.shape), r, slack), ctx)


@pytest.mark.parametrize("layout", ["bhsd", "bshd"])
@pytest.mark.parametrize("cap", [5, 16, 24])
@pytest.mark.parametrize("D,Hq,Hkv", [(128, 16, 16), (256, 8, 4), (64, 16, 2)])
def test_strided_varlen(layout, cap, D, Hq, Hkv):
    import torch
    import fmha_amd
    dev = torch.device("cuda", 0)
    gen = torch.Generator(device=dev).manual_seed(cap * 1000 + D + Hq)
    B = 37
    rng = np.random.default_rng(cap + D)
    seqlens = rng.integers(0, min(cap, 16) + 1, size=B).astype(np.int32)
    q = _bf16(gen, (B, Hq, 1, D), dev)
    if layout == "bhsd":
        kc = _bf16(gen, (B, Hkv, cap, D), dev)
        vc = _bf16(gen, (B, Hkv, cap, D), dev)
        for b in range(B):                      # poison the padding rows
            kc[b, :, seqlens[b]:] = float("nan")
            vc[b, :, seqlens[b]:] = float("nan")
        k, v = kc.transpose(1, 2), vc.transpose(1, 2)
    else:
        k = _bf16(gen, (B, cap, Hkv, D), dev)
        v = _bf16(gen, (B, cap, Hkv, D), dev)
        for b in range(B):
            k[b, seqlens[b]:] = float("nan")
            v[b, seqlens[b]:] = float("nan")
    lens = torch.from_numpy(seqlens).to(dev)
    o = fmha_amd.fmha_decode_strided(q, k, v, seqlens_kv=lens)
    torch.cuda.synchronize()
    pk = np.concatenate([_bits(k[b, :seqlens[b]]) for b in range(B)])
    pv = np.concatenate([_bits(v[b, :seqlens[b]]) for b in range(B)])
    _check(o, q, pk, pv, seqlens, Hq, Hkv, D, f"{layout} cap={cap} D={D}")


@pytest.mark.parametrize("S", [1, 6, 16])
def test_strided_uniform_bhsd(S):
    import torch
    import fmha_amd
    dev = torch.device("cuda", 0)
    gen = torch.Generator(device=dev).manual_seed(S)
    B, Hq, Hkv, D = 29, 32, 16, 128
    q = _bf16(gen, (B, Hq, 1, D), dev)
    kc = _bf16(gen, (B, Hkv, S, D), dev)
    vc = _bf16(gen, (B, Hkv, S, D), dev)
    o = fmha_amd.fmha_decode_strided(q, kc.transpose(1, 2), vc.transpose(1, 2))
    torch.cuda.synchronize()
    seqlens = np.full(B, S, np.int32)
    _check(o, q, _bits(kc.transpose(1, 2)).reshape(-1, Hkv, D), _bits(vc.transpose(1, 2)).reshape(-1, Hkv, D),
           seqlens, Hq, Hkv, D, f"bhsd uniform S={S}")


def test_strided_length_beyond_capacity_is_nan():
    import torch
    import fmha_amd
    dev = torch.device("cuda", 0)
    gen = torch.Generator(device=dev).manual_seed(7)
    B, H, D, cap = 3, 4, 128, 6
    q = _bf16(gen, (B, H, 1, D), dev)
    k = _bf16(gen, (B, cap, H, D), dev)
    v = _bf16(gen, (B, cap, H, D), dev)
    lens = torch.tensor([6, 7, 2], dtype=torch.int32, device=dev)
    o = fmha_amd.fmha_decode_strided(q, k, v, seqlens_kv=lens).float()
    torch.cuda.synchronize()
    assert torch.isnan(o[1]).all() and torch.isfinite(o[0]).all() and torch.isfinite(o[2]).all()


@pytest.mark.parametrize("page_size", [1, 2, 4, 8, 16, 32])
@pytest.mark.parametrize("D,Hq,Hkv", [(128, 16, 16), (256, 16, 8), (64, 8, 1)])
def test_paged(page_size, D, Hq, Hkv):
    import torch
    import fmha_amd
    dev = torch.device("cuda", 0)
    gen = torch.Generator(device=dev).manual_seed(page_size * 100 + D)
    B = 41
    rng = np.random.default_rng(page_size + D)
    seqlens = rng.integers(0, 17, size=B).astype(np.int32)
    need = [(int(s) + page_size - 1) // page_size for s in seqlens]
    max_pages = max(max(need), 1) + 1
    num_pages = sum(need) + 7
    perm = rng.permutation(num_pages)
    bt = np.full((B, max_pages), -1, np.int32)   # unused entries hold garbage
    used, i = [], 0
    for b in range(B):
        for p in range(need[b]):
            bt[b, p] = perm[i]
            used.append(perm[i])
            i += 1
    kc = torch.full((num_pages, page_size, Hkv, D), float("nan"), dtype=torch.bfloat16, device=dev)
    vc = torch.full((num_pages, page_size, Hkv, D), float("nan"), dtype=torch.bfloat16, device=dev)
    q = _bf16(gen, (B, Hq, 1, D), dev)
    rows_k, rows_v = [], []
    for b in range(B):
        for j in range(seqlens[b]):
            page, slot = bt[b, j // page_size], j % page_size
            kr, vr = _bf16(gen, (Hkv, D), dev), _bf16(gen, (Hkv, D), dev)
            kc[page, slot], vc[page, slot] = kr, vr
            rows_k.append(_bits(kr))
            rows_v.append(_bits(vr))
    o = fmha_amd.fmha_decode_paged(q, kc, vc, torch.from_numpy(bt).to(dev), torch.from_numpy(seqlens).to(dev))
    torch.cuda.synchronize()
    pk = np.stack(rows_k) if rows_k else np.zeros((0, Hkv, D), np.uint16)
    pv = np.stack(rows_v) if rows_v else np.zeros((0, Hkv, D), np.uint16)
    _check(o, q, pk, pv, seqlens, Hq, Hkv, D, f"paged ps={page_size} D={D}")


def test_paged_bad_length_is_nan():
    import torch
    import fmha_amd
    dev = torch.device("cuda", 0)
    gen = torch.Generator(device=dev).manual_seed(9)
    q = _bf16(gen, (2, 4, 1, 64), dev)
    kc = _bf16(gen, (4, 16, 4, 64), dev)
    bt = torch.tensor([[0, 1], [2, 3]], dtype=torch.int32, device=dev)
    lens = torch.tensor([17, 3], dtype=torch.int32, device=dev)
    o = fmha_amd.fmha_decode_paged(q, kc, kc, bt, lens).float()
    torch.cuda.synchronize()
    assert torch.isnan(o[0]).all() and torch.isfinite(o[1]).all()


@pytest.mark.parametrize("page_size", [1, 4, 16])
@pytest.mark.parametrize("D,Hq,Hkv", [(128, 8, 1), (128, 16, 2), (256, 4, 1), (128, 2, 2), (64, 20, 4)])
def test_paged_few_kv_heads_batches_per_wave(page_size, D, Hq, Hkv):
    """Fewer KV heads than a wave holds on a paged cache: the lane groups of
    a wave serve different batches, each lane with its own page lookups and
    addresses.  Block tables of 12 rows (below the 16-row bucket the longest
    length picks), NaN in every slot no batch owns and -1 in unused
    entries, empty batches, and a length beyond what the table addresses
    (NaN for that batch only, its neighbours in the same wave exact); G = 8,
    8, 4, 1, 5."""
    import torch
    import fmha_amd
    dev = torch.device("cuda", 0)
    gen = torch.Generator(device=dev).manual_seed(page_size * 31 + D + Hq)
    B = 37
    cap = 12
    rng = np.random.default_rng(page_size * 5 + D + Hq + Hkv)
    seqlens = rng.integers(0, cap + 1, size=B).astype(np.int32)
    seqlens[0] = cap
    seqlens[5] = 0
    ps_pages = (cap + page_size - 1) // page_size
    need = [(int(s) + page_size - 1) // page_size for s in seqlens]
    num_pages = sum(need) + 3
    perm = rng.permutation(num_pages)
    bt = np.full((B, ps_pages), -1, np.int32)
    i = 0
    for b in range(B):
        for p in range(need[b]):
            bt[b, p] = perm[i]
            i += 1
    kc = torch.full((num_pages, page_size, Hkv, D), float("nan"), dtype=torch.bfloat16, device=dev)
    vc = torch.full((num_pages, page_size, Hkv, D), float("nan"), dtype=torch.bfloat16, device=dev)
    q = _bf16(gen, (B, Hq, 1, D), dev)
    rows_k, rows_v = [], []
    for b in range(B):
        for j in range(seqlens[b]):
            page, slot = bt[b, j // page_size], j % page_size
            kr, vr = _bf16(gen, (Hkv, D), dev), _bf16(gen, (Hkv, D), dev)
            kc[page, slot], vc[page, slot] = kr, vr
            rows_k.append(_bits(kr))
            rows_v.append(_bits(vr))
    bt_dev = torch.from_numpy(bt).to(dev)
    o = fmha_amd.fmha_decode_paged(q, kc, vc, bt_dev, torch.from_numpy(seqlens).to(dev))
    torch.cuda.synchronize()
    _check(o, q, np.stack(rows_k), np.stack(rows_v), seqlens, Hq, Hkv, D, f"paged few heads ps={page_size} D={D}")
    # A length beyond the rows the table addresses (its entries times the
    # page size, at most 16): NaN for that batch only, nothing read.  (A
    # length within them promises pages for its rows, which the kernels
    # follow: 13 with one 16-row page per batch would send an empty batch's
    # -1 entry to memory.)
    bad = seqlens.copy()
    bad[3] = min(16, ps_pages * page_size) + 1
    o2 = fmha_amd.fmha_decode_paged(q, kc, vc, bt_dev, torch.from_numpy(bad).to(dev))
    torch.cuda.synchronize()
    assert torch.isnan(o2[3].float()).all()
    keep = [b for b in range(B) if b != 3]
    assert torch.equal(o2[keep].view(torch.int16), o[keep].view(torch.int16))


# (entry, page size, lengths up to): the workspace-less entry accepts up to
# 16 rows, so its pages are of 16 rows or more.
@pytest.mark.parametrize("entry,page_size,cap", [("short", 16, 16), ("short", 64, 16), ("splitkv", 16, 16),
                                                 ("splitkv", 64, 16), ("splitkv", 8, 8)])
@pytest.mark.parametrize("D,Hq,Hkv,layout", [(128, 64, 4, "paged"), (64, 96, 8, "paged"), (256, 48, 2, "paged"),
                                              (128, 160, 4, "paged"), (128, 32, 1, "paged_lanes"),
                                              (128, 36, 2, "paged_lanes"), (64, 72, 6, "paged_lanes"),
                                              (256, 27, 1, "paged_lanes")])
def test_paged_groups_above_eight(entry, page_size, cap, D, Hq, Hkv, layout):
    """Short rows with more than 8 query heads per KV head on a paged cache,
    G = 16, 12, 24, 40, 32, 18, 12 and 27 (one to three 16-column query
    tiles per stream): the matrix-core short kernel with its descriptor based
    at each batch's page where a wave's streams share a batch, else with an
    address per lane, through the workspace-less entry (max_seqlen_kv None)
    and the split entry (max_seqlen_kv = cap).  NaN in every slot no batch
    owns, -1 in unused entries, empty batches; then a length beyond the
    capacity and an unmapped page give NaN for their batches only."""
    import torch
    import fmha_amd
    print(f"paged groups above 8: {entry} ps={page_size} cap={cap} D={D} Hq={Hq} Hkv={Hkv}", flush=True)
    dev = torch.device("cuda", 0)
    gen = torch.Generator(device=dev).manual_seed(page_size + D + Hq)
    rng = np.random.default_rng(page_size * 3 + D + Hq + Hkv)
    B = 45
    seqlens = rng.integers(0, cap + 1, size=B).astype(np.int32)
    seqlens[0], seqlens[7] = cap, 0
    num_pages = B + 5
    perm = rng.permutation(num_pages)
    bt = np.full((B, 2), -1, np.int32)
    for b in range(B):
        if seqlens[b] > 0:
            bt[b, 0] = perm[b]
    kc = torch.full((num_pages, page_size, Hkv, D), float("nan"), dtype=torch.bfloat16, device=dev)
    vc = torch.full((num_pages, page_size, Hkv, D), float("nan"), dtype=torch.bfloat16, device=dev)
    q = _bf16(gen, (B, Hq, 1, D), dev)
    rows_k, rows_v = [], []
    for b in range(B):
        for j in range(seqlens[b]):
            kr, vr = _bf16(gen, (Hkv, D), dev), _bf16(gen, (Hkv, D), dev)
            kc[bt[b, 0], j], vc[bt[b, 0], j] = kr, vr
            rows_k.append(_bits(kr))
            rows_v.append(_bits(vr))
    max_s = None if entry == "short" else cap

    def run(table, lens):
        o = fmha_amd.fmha_decode_paged(q, kc, vc, torch.from_numpy(table).to(dev), torch.from_numpy(lens).to(dev),
                                       max_seqlen_kv=max_s)
        torch.cuda.synchronize()
        return o

    o = run(bt, seqlens)
    kind, fields = last_plan()[-1]
    assert (kind, fields["layout"]) == ("short_matrix_core", layout), last_plan()
    _check(o, q, np.stack(rows_k), np.stack(rows_v), seqlens, Hq, Hkv, D,
           f"paged G={Hq // Hkv} {entry} ps={page_size} D={D}")
    bad_lens, bad_bt = seqlens.copy(), bt.copy()
    bad_lens[3] = cap + 1
    bad_bt[0, 0] = -1
    o2 = run(bad_bt, bad_lens)
    assert torch.isnan(o2[[0, 3]].float()).all()
    keep = [b for b in range(B) if b not in (0, 3)]
    assert torch.equal(o2[keep].view(torch.int16), o[keep].view(torch.int16))


def test_paged_groups_above_eight_rows_beyond_a_page():
    """Groups above 8 whose rows may reach past a batch's first page: the
    split entry runs them on the split passes (exact against the oracle);
    the workspace-less entry rejects them."""
    import torch
    import fmha_amd
    dev = torch.device("cuda", 0)
    gen = torch.Generator(device=dev).manual_seed(5)
    for page_size, Hq, Hkv in [(8, 32, 2), (4, 64, 4)]:
        D, B, cap = 128, 9, 16
        seqlens = np.array([16, 3, 0, 9, 16, 1, 12, 5, 7], np.int32)
        pages = (cap + page_size - 1) // page_size
        bt = np.arange(B * pages, dtype=np.int32).reshape(B, pages)
        kc = _bf16(gen, (B * pages, page_size, Hkv, D), dev)
        vc = _bf16(gen, (B * pages, page_size, Hkv, D), dev)
        q = _bf16(gen, (B, Hq, 1, D), dev)
        rows_k = [_bits(kc[bt[b, j // page_size], j % page_size]) for b in range(B) for j in range(seqlens[b])]
        rows_v = [_bits(vc[bt[b, j // page_size], j % page_size]) for b in range(B) for j in range(seqlens[b])]
        bt_dev, lens = torch.from_numpy(bt).to(dev), torch.from_numpy(seqlens).to(dev)
        o = fmha_amd.fmha_decode_paged(q, kc, vc, bt_dev, lens, max_seqlen_kv=cap)
        torch.cuda.synchronize()
        assert last_plan()[-1][0] == "split_matrix_core", last_plan()
        _check(o, q, np.stack(rows_k), np.stack(rows_v), seqlens, Hq, Hkv, D, f"paged G>8 split ps={page_size}")
        with pytest.raises(RuntimeError, match="above 8"):
            fmha_amd.fmha_decode_paged(q, kc, vc, bt_dev, lens)


def test_tensors_on_another_device_are_rejected_before_launch():
    """out, k, v, caches, block tables and lengths must be on q's device: a
    host tensor's pointer handed to the kernel would fault, so every wrapper
    raises ValueError before anything is launched."""
    import torch
    import fmha_amd
    dev = torch.device("cuda", 0)
    B, H, D = 4, 4, 128
    q = torch.zeros(B, H, 1, D, device=dev, dtype=torch.bfloat16)
    k = torch.zeros(B * 3, H, D, device=dev, dtype=torch.bfloat16)
    cu = torch.arange(0, 3 * (B + 1), 3, dtype=torch.int32, device=dev)
    cpu_out = torch.empty(B, H, 1, D, dtype=torch.float16)
    with pytest.raises(ValueError, match="device"):
        fmha_amd.fmha_decode(q, k, k, cu_seqlens_kv=cu, out=cpu_out)
    with pytest.raises(ValueError):
        fmha_amd.fmha_decode(q, k, k.cpu(), cu_seqlens_kv=cu)
    with pytest.raises(ValueError, match="device"):
        fmha_amd.fmha_decode_splitkv(q, k, k, cu, 3, out=cpu_out)
    k4 = k.view(B, 3, H, D)
    with pytest.raises(ValueError, match="device"):
        fmha_amd.fmha_decode_strided(q, k4, k4, out=cpu_out)
    pages = torch.zeros(B, 16, H, D, device=dev, dtype=torch.bfloat16)
    bt = torch.arange(B, dtype=torch.int32, device=dev).view(B, 1)
    lens = torch.full((B,), 3, dtype=torch.int32, device=dev)
    with pytest.raises(ValueError, match="device"):
        fmha_amd.fmha_decode_paged(q, pages, pages, bt, lens, out=cpu_out)
    with pytest.raises(ValueError):
        fmha_amd.fmha_decode_paged(q, pages, pages, bt.cpu(), lens)
    with pytest.raises(ValueError):
        fmha_amd.fmha_decode_paged(q, pages, pages, bt, lens.cpu())
    torch.cuda.synchronize()


# (max_seqlen_kv or None for the short kernel, page_size, D, Hq, Hkv, B,
# (kind, layout) of the call's last launch as the library reports it): the
# short kernel one batch per wave (16 KV heads) and several batches per wave
# (1 and 2 KV heads); beyond 16 rows the single pass (>= 512 waves), the
# split passes over one page per wave (page size 16) and per-lane pages
# (few KV heads, page sizes 4 and 16), the matrix-core split passes (G =
# 16, 12, and groups of 8 with too few waves for the single pass on pages
# under 16 rows), the per-lane single pass on short rows at D >= 128, and
# the matrix-core short kernel for groups above 8 (G = 16 and 12, both
# entries; G = 32 on one KV head, an address per lane).
NEG_CASES = [
    (None, 4, 128, 16, 16, 23, ("short", "paged")), (None, 1, 128, 8, 1, 37, ("short_multi", "paged")),
    (None, 16, 128, 64, 4, 40, ("short_matrix_core", "paged")), (16, 32, 64, 96, 8, 30, ("short_matrix_core", "paged")),
    (None, 16, 128, 32, 1, 41, ("short_matrix_core", "paged_lanes")),
    (None, 16, 128, 16, 2, 37, ("short_multi", "paged")), (None, 8, 256, 4, 1, 19, ("short_multi", "paged")),
    (40, 16, 128, 8, 4, 600, ("onepass", "paged16")), (70, 16, 128, 16, 16, 9, ("split", "paged16")),
    (70, 4, 128, 16, 2, 9, ("split_matrix_core", "paged")), (70, 16, 128, 8, 2, 9, ("split", "paged16_lanes")),
    (70, 4, 64, 16, 1, 9, ("split_matrix_core", "paged")),
    (100, 16, 128, 24, 2, 7, ("split_matrix_core", "paged16")), (100, 4, 256, 24, 2, 7, ("split_matrix_core", "paged")),
    (24, 4, 128, 16, 2, 1100, ("onepass", "paged_lanes")), (32, 8, 256, 4, 1, 1100, ("onepass", "paged_lanes")),
    # >= 512 waves with few KV heads: the single pass with per-lane page
    # lookups, several batches per wave: groups of 8 on rows of two blocks
    # (16-row pages at D = 128, one-row pages at D = 64) and of three (16-row
    # pages at D = 64), groups of up to 4 on rows of three to eight blocks
    (32, 16, 128, 8, 1, 2100, ("onepass", "paged16_lanes")), (32, 1, 64, 8, 1, 4200, ("onepass", "paged_lanes")),
    (48, 16, 64, 8, 1, 4200, ("onepass", "paged16_lanes")), (48, 16, 128, 4, 1, 2100, ("onepass", "paged16_lanes")),
    (128, 1, 64, 2, 1, 4200, ("onepass", "paged_lanes")), (128, 4, 128, 8, 2, 1100, ("onepass", "paged_lanes")),
    # rows of 4 blocks and more with >= 512 (batch, KV head) units: the
    # matrix-core register single pass (groups of 8 and 4, pages of 16 and
    # 32 rows, then of 1 and 4)
    (600, 16, 128, 64, 8, 128, ("onepass_matrix_core_regs", "paged16")),
    (300, 32, 128, 32, 8, 128, ("onepass_matrix_core_regs", "paged16")),
    (600, 1, 128, 64, 8, 128, ("onepass_matrix_core_regs", "paged")),
    (300, 4, 128, 32, 8, 128, ("onepass_matrix_core_regs", "paged")),
    # D = 256, rows of at most 40 blocks: the matrix-core single pass with
    # the scores in LDS (16-row pages)
    (300, 16, 256, 64, 8, 80, ("onepass_matrix_core", "paged16")),
]


@pytest.mark.parametrize("max_s,page_size,D,Hq,Hkv,B,route", NEG_CASES)
def test_paged_negative_entries_give_nan(max_s, page_size, D, Hq, Hkv, B, route):
    """A negative block-table entry (serving engines pad with -1) for a row a
    batch has: that batch's outputs are NaN and its unmapped pages are never
    read; every other batch keeps its exact bits.  -1 entries past a
    batch's rows are padding, as always."""
    import torch
    import fmha_amd
    print(f"paged negative entries: max_s={max_s} ps={page_size} D={D} Hq={Hq} Hkv={Hkv} B={B}", flush=True)
    dev = torch.device("cuda", 0)
    gen = torch.Generator(device=dev).manual_seed(page_size * 7 + D + Hq + B)
    rng = np.random.default_rng(page_size * 3 + D + Hq + Hkv + B)
    cap = 16 if max_s is None else max_s
    seqlens = rng.integers(1, cap + 1, size=B).astype(np.int32)
    seqlens[0] = cap
    need = [(int(s) + page_size - 1) // page_size for s in seqlens]
    max_pages = (cap + page_size - 1) // page_size
    num_pages = sum(need) + 2
    perm = rng.permutation(num_pages)
    bt = np.full((B, max_pages), -1, np.int32)
    i = 0
    for b in range(B):
        for p in range(need[b]):
            bt[b, p] = perm[i]
            i += 1
    kc = torch.randn(num_pages, page_size, Hkv, D, generator=gen, device=dev, dtype=torch.bfloat16)
    vc = torch.randn(num_pages, page_size, Hkv, D, generator=gen, device=dev, dtype=torch.bfloat16)
    q = _bf16(gen, (B, Hq, 1, D), dev)
    lens = torch.from_numpy(seqlens).to(dev)

    def run(table):
        o = fmha_amd.fmha_decode_paged(q, kc, vc, torch.from_numpy(table).to(dev), lens, max_seqlen_kv=max_s)
        torch.cuda.synchronize()
        return o

    o = run(bt)
    kind, fields = last_plan()[-1]
    assert (kind, fields["layout"]) == route, last_plan()
    assert bool(torch.isfinite(o.float()).all())
    poisoned = sorted(set(rng.choice(B, size=max(1, B // 4), replace=False).tolist()) | {0})
    bad = bt.copy()
    for n, b in enumerate(poisoned):
        e = int(rng.integers(0, need[b]))            # an entry the batch's rows use
        bad[b, e] = -1 if n % 2 == 0 else -(2 ** 31)
    o2 = run(bad)
    for b in range(B):
        if b in poisoned:
            assert bool(torch.isnan(o2[b].float()).all()), f"batch {b} with an unmapped page is not NaN"
        else:
            assert torch.equal(o2[b].view(torch.int16), o[b].view(torch.int16)), f"batch {b} changed"
