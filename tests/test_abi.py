"""CPU-side checks of the C ABI: the library loads, exports every function
include/fmha_decode.h declares, and rejects bad arguments before touching the
GPU (no call here reaches a kernel launch)."""
import ctypes
import os
import re

import pytest

from tests.conftest import ROOT

HEADER = os.path.join(ROOT, "include", "fmha_decode.h")
BAD = 1      # hipErrorInvalidValue
NOTSUP = 801  # hipErrorNotSupported

# Fake but 16-byte aligned device addresses: every call below is rejected (or
# is a batch-0 no-op) before anything dereferences them.
P = 0x10000
Q, K, V, O, CU = P, P * 2, P * 3, P * 4, P * 5


def header_functions():
    text = open(HEADER).read()
    return sorted(set(re.findall(r"^\s*(?:const\s+)?\w+\s*\*?\s*(fmha_decode_\w+)\s*\(", text, re.M)))


@pytest.fixture(scope="module")
def lib():
    from fmha_amd import _lib
    return _lib.load()


def test_exports_every_declared_function(lib):
    names = header_functions()
    assert set(names) == {"fmha_decode_fwd", "fmha_decode_fwd_fast", "fmha_decode_fwd_fp32_weights",
                          "fmha_decode_fwd_exact", "fmha_decode_fwd_uniform", "fmha_decode_fwd_uniform_fast",
                          "fmha_decode_fwd_strided",
                          "fmha_decode_fwd_paged", "fmha_decode_splitkv_workspace_size",
                          "fmha_decode_fwd_splitkv", "fmha_decode_fwd_splitkv_noalloc",
                          "fmha_decode_fwd_splitkv_strided",
                          "fmha_decode_fwd_splitkv_paged", "fmha_decode_error_string",
                          "fmha_decode_last_error_detail", "fmha_decode_last_plan", "fmha_decode_version"}
    from fmha_amd import _lib
    assert set(names) == set(_lib.EXPORTED)
    for n in names:
        assert hasattr(lib, n), n


def test_version_and_strings(lib):
    assert lib.fmha_decode_version() >= 100
    assert lib.fmha_decode_error_string(0) == b"success"
    assert lib.fmha_decode_error_string(BAD) == b"invalid argument"
    assert lib.fmha_decode_error_string(NOTSUP) == b"configuration not supported"


def fwd(lib, **kw):
    a = dict(stream=None, q=Q, k=K, v=V, o=O, cu=CU, batch=4, hq=16, hkv=16, sq=1, dq=128, dkv=128,
             scale=0.088)
    a.update(kw)
    return lib.fmha_decode_fwd(a["stream"], a["q"], a["k"], a["v"], a["o"], a["cu"], a["batch"], a["hq"],
                               a["hkv"], a["sq"], a["dq"], a["dkv"], a["scale"])


def fwd_fast(lib, **kw):
    a = dict(stream=None, q=Q, k=K, v=V, o=O, cu=CU, batch=4, hq=16, hkv=16, sq=1, dq=128, dkv=128,
             scale=0.088)
    a.update(kw)
    return lib.fmha_decode_fwd_fast(a["stream"], a["q"], a["k"], a["v"], a["o"], a["cu"], a["batch"], a["hq"],
                                    a["hkv"], a["sq"], a["dq"], a["dkv"], a["scale"])


def fwd32(lib, **kw):
    a = dict(stream=None, q=Q, k=K, v=V, o=O, cu=CU, batch=4, hq=16, hkv=16, sq=1, dq=128, dkv=128,
             scale=0.088)
    a.update(kw)
    return lib.fmha_decode_fwd_fp32_weights(a["stream"], a["q"], a["k"], a["v"], a["o"], a["cu"], a["batch"],
                                            a["hq"], a["hkv"], a["sq"], a["dq"], a["dkv"], a["scale"])


def fwd_exact(lib, **kw):
    a = dict(stream=None, q=Q, k=K, v=V, o=O, cu=CU, batch=4, hq=16, hkv=16, sq=1, dq=128, dkv=128,
             scale=0.088)
    a.update(kw)
    return lib.fmha_decode_fwd_exact(a["stream"], a["q"], a["k"], a["v"], a["o"], a["cu"], a["batch"],
                                     a["hq"], a["hkv"], a["sq"], a["dq"], a["dkv"], a["scale"])


def uni(lib, fast=False, **kw):
    a = dict(stream=None, q=Q, k=K, v=V, o=O, s=16, batch=4, hq=16, hkv=16, sq=1, dq=128, dkv=128,
             scale=0.088)
    a.update(kw)
    f = lib.fmha_decode_fwd_uniform_fast if fast else lib.fmha_decode_fwd_uniform
    return f(a["stream"], a["q"], a["k"], a["v"], a["o"], a["s"], a["batch"], a["hq"], a["hkv"], a["sq"], a["dq"],
             a["dkv"], a["scale"])


@pytest.mark.parametrize("kw,code,needle", [
    (dict(batch=-1), BAD, "batch"),
    (dict(hq=0), BAD, "head counts"),
    (dict(hkv=0), BAD, "head counts"),
    (dict(hq=16, hkv=5), BAD, "multiple"),
    # Any group size runs (the matrix-core kernel takes those above 8), but
    # not when a wave's K/V span reaches 2^30 bytes.
    (dict(hq=12 << 17, hkv=1 << 17), NOTSUP, "too large"),
    (dict(sq=2), BAD, "seqlen_q"),
    (dict(sq=0), BAD, "seqlen_q"),
    (dict(dq=128, dkv=256), BAD, "head_dim_q"),
    (dict(dq=96, dkv=96), BAD, "64, 128 or 256"),
    (dict(dq=512, dkv=512), BAD, "64, 128 or 256"),
    (dict(scale=float("nan")), BAD, "finite"),
    (dict(scale=float("inf")), BAD, "finite"),
    (dict(q=None), BAD, "non-null"),
    (dict(o=None), BAD, "non-null"),
    (dict(k=K + 8), BAD, "aligned"),
    (dict(o=O + 2), BAD, "aligned"),
    (dict(cu=None), BAD, "cu_seqlens_kv"),
    (dict(cu=CU + 2), BAD, "cu_seqlens_kv"),
    (dict(hq=1 << 20, hkv=1 << 20), BAD, "too large"),
])
def test_varlen_rejects(lib, kw, code, needle):
    assert fwd(lib, **kw) == code
    assert needle in lib.fmha_decode_last_error_detail().decode()
    assert fwd_fast(lib, **kw) == code
    assert needle in lib.fmha_decode_last_error_detail().decode()


@pytest.mark.parametrize("kw,code,needle", [
    (dict(s=-1), BAD, "seqlen_kv"),
    (dict(s=17), BAD, "seqlen_kv"),
    (dict(s=1000), BAD, "seqlen_kv"),
    (dict(hq=16 << 17, hkv=1 << 17), NOTSUP, "too large"),
    (dict(v=None), BAD, "non-null"),
])
def test_uniform_rejects(lib, kw, code, needle):
    for fast in (False, True):
        assert uni(lib, fast=fast, **kw) == code
        assert needle in lib.fmha_decode_last_error_detail().decode()


@pytest.mark.parametrize("hq,hkv", [(32, 2), (96, 8), (18, 1)])
def test_fp32_weights_group_sizes(lib, hq, hkv):
    """The fp32-weight entry runs the VALU kernel only: group sizes up to 8
    (3, 5, 6, 7 on the 4- and 8-head instantiations), nothing above."""
    assert fwd32(lib, hq=hq, hkv=hkv) == NOTSUP
    assert "at most 8" in lib.fmha_decode_last_error_detail().decode()


def strided(lib, **kw):
    a = dict(stream=None, q=Q, k=K, v=V, o=O, lens=CU, s=16, bs=16 * 16 * 128, rs=16 * 128, hs=128, batch=4,
             hq=16, hkv=16, sq=1, dq=128, dkv=128, scale=0.088)
    a.update(kw)
    return lib.fmha_decode_fwd_strided(a["stream"], a["q"], a["k"], a["v"], a["o"], a["lens"], a["s"], a["bs"],
                                       a["rs"], a["hs"], a["batch"], a["hq"], a["hkv"], a["sq"], a["dq"],
                                       a["dkv"], a["scale"])


def paged(lib, **kw):
    a = dict(stream=None, q=Q, k=K, v=V, o=O, bt=CU, bts=4, lens=CU + 64, ps=16, batch=4, hq=16, hkv=16, sq=1,
             dq=128, dkv=128, scale=0.088)
    a.update(kw)
    return lib.fmha_decode_fwd_paged(a["stream"], a["q"], a["k"], a["v"], a["o"], a["bt"], a["bts"], a["lens"],
                                     a["ps"], a["batch"], a["hq"], a["hkv"], a["sq"], a["dq"], a["dkv"],
                                     a["scale"])


@pytest.mark.parametrize("kw,code,needle", [
    (dict(s=-1), BAD, "seqlen_kv"),
    (dict(lens=None, s=17), BAD, "seqlen_kv"),
    (dict(bs=-8), BAD, "strides"),
    (dict(rs=12), BAD, "multiples of 8"),
    (dict(hs=4), BAD, "multiples of 8"),
    (dict(rs=1 << 26), BAD, "1 GiB"),
    (dict(lens=CU + 2), BAD, "seqlens_kv"),
    # Any group size runs; above 8 the matrix-core kernel's descriptor spans
    # the batches a wave touches (here 2 of 1 GiB each).
    (dict(hq=96, hkv=8, bs=1 << 29), NOTSUP, "exceeds 1 GiB"),
    (dict(k=None), BAD, "non-null"),
    (dict(dq=128, dkv=64), BAD, "head_dim_q"),
])
def test_strided_rejects(lib, kw, code, needle):
    assert strided(lib, **kw) == code
    assert needle in lib.fmha_decode_last_error_detail().decode()


@pytest.mark.parametrize("kw,code,needle", [
    (dict(ps=0), BAD, "page_size"),
    (dict(ps=24), BAD, "page_size"),
    (dict(ps=1 << 21), BAD, "page_size"),
    (dict(bt=None), BAD, "block_table"),
    (dict(lens=None), BAD, "seqlens_kv"),
    (dict(bt=CU + 2), BAD, "aligned"),
    (dict(bts=0), BAD, "block_table_stride"),
    (dict(sq=2), BAD, "seqlen_q"),
    (dict(v=None), BAD, "non-null"),
    # no workspace: group sizes above 8 only where every length up to 16
    # lies in a batch's first page
    (dict(hq=192, hkv=16, ps=8), NOTSUP, "within one page"),
])
def test_paged_rejects(lib, kw, code, needle):
    assert paged(lib, **kw) == code
    assert needle in lib.fmha_decode_last_error_detail().decode()


def splitkv(lib, **kw):
    a = dict(stream=None, q=Q, k=K, v=V, o=O, cu=CU, maxs=1000, batch=4, hq=16, hkv=16, sq=1, dq=128, dkv=128,
             scale=0.088, ws=P * 64, wsb=1 << 30)
    a.update(kw)
    return lib.fmha_decode_fwd_splitkv(a["stream"], a["q"], a["k"], a["v"], a["o"], a["cu"], a["maxs"], a["batch"],
                                       a["hq"], a["hkv"], a["sq"], a["dq"], a["dkv"], a["scale"], a["ws"], a["wsb"])


def test_splitkv_workspace_size(lib):
    f = lib.fmha_decode_splitkv_workspace_size
    assert f(0, 16, 16, 100, 128) == 0 and f(4, 16, 16, -1, 128) == 0 and f(4, 16, 16, 100, 96) == 0
    small, big = f(4, 16, 16, 100, 128), f(4, 16, 16, 10000, 128)
    assert 0 < small < big and small % 256 == 0 and big % 256 == 0
    # scores (4 B per row and query head) dominate a long row
    assert big >= 4 * 16 * 10000 * 4
    # G = 3 runs as 4 on padded copies of Q and O: the plan for Hkv * 4 heads
    # plus the two copies (4 * 8 * 4 * 128 * 2 bytes each)
    assert f(4, 24, 8, 100, 128) == f(4, 32, 8, 100, 128) + 2 * 4 * 8 * 4 * 128 * 2
    assert f(4, 56, 8, 100, 128) == f(4, 64, 8, 100, 128) + 2 * 4 * 8 * 8 * 128 * 2
    # G > 8 runs as ceil(G / 8) groups of 8 on Hkv * ceil(G / 8) launch KV
    # heads: G = 16 needs the plan for 16 KV heads of G = 8 and no copies,
    # G = 12 the same plan plus copies padded to 16 query heads per KV head
    assert f(4, 128, 8, 100, 128) == f(4, 128, 16, 100, 128)
    assert f(4, 96, 8, 100, 128) == f(4, 128, 16, 100, 128) + 2 * 4 * 8 * 16 * 128 * 2
    # MQA with G = 40 = 5 * 8: five launch KV heads, no copies
    assert f(2, 40, 1, 5000, 64) == f(2, 40, 5, 5000, 64)


@pytest.mark.parametrize("kw,code,needle", [
    (dict(maxs=-1), BAD, "max_seqlen_kv"),
    (dict(maxs=1 << 20), BAD, "too large"),
    (dict(ws=None), BAD, "workspace"),
    (dict(ws=P * 64 + 16), BAD, "256-byte"),
    (dict(wsb=1024), BAD, "too small"),
    (dict(cu=None), BAD, "cu_seqlens_kv"),
    # lengths beyond 16 take group sizes outside {1, 2, 4, 8} through a
    # padded query group in the workspace
    (dict(hq=24, hkv=8, wsb=1024), BAD, "padded query group"),
    (dict(hq=96, hkv=8, ws=None), BAD, "workspace"),
    (dict(sq=3), BAD, "seqlen_q"),
])
def test_splitkv_rejects(lib, kw, code, needle):
    assert splitkv(lib, **kw) == code
    assert needle in lib.fmha_decode_last_error_detail().decode()


def splitkv_strided(lib, **kw):
    a = dict(stream=None, q=Q, k=K, v=V, o=O, lens=CU, maxs=1000, bs=1000 * 16 * 128, rs=16 * 128, hs=128,
             batch=4, hq=16, hkv=16, sq=1, dq=128, dkv=128, scale=0.088, ws=P * 64, wsb=1 << 30)
    a.update(kw)
    return lib.fmha_decode_fwd_splitkv_strided(a["stream"], a["q"], a["k"], a["v"], a["o"], a["lens"], a["maxs"],
                                               a["bs"], a["rs"], a["hs"], a["batch"], a["hq"], a["hkv"], a["sq"],
                                               a["dq"], a["dkv"], a["scale"], a["ws"], a["wsb"])


def splitkv_paged(lib, **kw):
    a = dict(stream=None, q=Q, k=K, v=V, o=O, bt=CU, bts=64, lens=CU + 64, ps=16, maxs=1000, batch=4, hq=16,
             hkv=16, sq=1, dq=128, dkv=128, scale=0.088, ws=P * 64, wsb=1 << 30)
    a.update(kw)
    return lib.fmha_decode_fwd_splitkv_paged(a["stream"], a["q"], a["k"], a["v"], a["o"], a["bt"], a["bts"],
                                             a["lens"], a["ps"], a["maxs"], a["batch"], a["hq"], a["hkv"], a["sq"],
                                             a["dq"], a["dkv"], a["scale"], a["ws"], a["wsb"])


@pytest.mark.parametrize("kw,code,needle", [
    (dict(maxs=-1), BAD, "max_seqlen_kv"),
    (dict(bs=-8), BAD, "strides"),
    (dict(rs=12), BAD, "multiples of 8"),
    (dict(rs=1 << 20), BAD, "1 GiB"),
    (dict(lens=CU + 2), BAD, "seqlens_kv"),
    (dict(ws=None), BAD, "workspace"),
    (dict(wsb=1024), BAD, "too small"),
    (dict(hq=96, hkv=8, wsb=1024), BAD, "padded query group"),
    (dict(k=None), BAD, "non-null"),
    (dict(maxs=16, lens=None, rs=12), BAD, "multiples of 8"),   # <= 16 rows: fmha_decode_fwd_strided's checks
])
def test_splitkv_strided_rejects(lib, kw, code, needle):
    assert splitkv_strided(lib, **kw) == code
    assert needle in lib.fmha_decode_last_error_detail().decode()


@pytest.mark.parametrize("kw,code,needle", [
    (dict(maxs=-1), BAD, "max_seqlen_kv"),
    (dict(ps=24), BAD, "page_size"),
    (dict(bt=None), BAD, "block_table"),
    (dict(lens=None), BAD, "seqlens_kv"),
    (dict(bts=0), BAD, "block_table_stride"),
    (dict(ws=None), BAD, "workspace"),
    (dict(wsb=1024), BAD, "too small"),
    (dict(sq=2), BAD, "seqlen_q"),
    (dict(hq=48, hkv=16, wsb=1024), BAD, "padded query group"),
    (dict(hq=192, hkv=16, wsb=1024), BAD, "padded query group"),
])
def test_splitkv_paged_rejects(lib, kw, code, needle):
    assert splitkv_paged(lib, **kw) == code
    assert needle in lib.fmha_decode_last_error_detail().decode()


def test_splitkv_paged_bound_is_the_block_table_row(lib):
    """Lengths beyond block_table_stride * page_size count as invalid: a call
    with a larger max_seqlen_kv needs only the workspace of that bound (64
    entries of 16-row pages here).  The call is rejected for a workspace one
    byte short of it, before any launch."""
    need = lib.fmha_decode_splitkv_workspace_size(4, 16, 16, 64 * 16, 128)
    assert splitkv_paged(lib, maxs=1 << 18, wsb=need - 1) == BAD
    assert f"need {need})" in lib.fmha_decode_last_error_detail().decode()


@pytest.mark.parametrize("kw,code,needle", [
    (dict(batch=-1), BAD, "batch"),
    (dict(hq=96, hkv=8), NOTSUP, "at most 8"),
    (dict(sq=2), BAD, "seqlen_q"),
    (dict(dq=96, dkv=96), BAD, "64, 128 or 256"),
    (dict(scale=float("nan")), BAD, "finite"),
    (dict(v=None), BAD, "non-null"),
    (dict(q=Q + 4), BAD, "aligned"),
    (dict(cu=None), BAD, "cu_seqlens_kv"),
    (dict(cu=CU + 1), BAD, "cu_seqlens_kv"),
])
def test_fp32_weights_rejects(lib, kw, code, needle):
    assert fwd32(lib, **kw) == code
    assert needle in lib.fmha_decode_last_error_detail().decode()


@pytest.mark.parametrize("kw,code,needle", [
    (dict(batch=-1), BAD, "batch"),
    (dict(hq=96, hkv=8), NOTSUP, "at most 8 query heads per KV head"),
    (dict(hq=16, hkv=1), NOTSUP, "at most 8 query heads per KV head"),
    (dict(hq=16, hkv=5), BAD, "multiple"),
    (dict(sq=2), BAD, "seqlen_q"),
    (dict(dq=96, dkv=96), BAD, "64, 128 or 256"),
    (dict(scale=float("inf")), BAD, "finite"),
    (dict(k=None), BAD, "non-null"),
    (dict(o=O + 2), BAD, "aligned"),
    (dict(cu=None), BAD, "cu_seqlens_kv"),
    (dict(cu=CU + 2), BAD, "cu_seqlens_kv"),
])
def test_exact_rejects(lib, kw, code, needle):
    assert fwd_exact(lib, **kw) == code
    assert needle in lib.fmha_decode_last_error_detail().decode()


def test_batch_zero_is_a_noop(lib):
    # Nothing is launched and no pointer is needed for an empty batch.
    assert fwd(lib, batch=0, q=None, k=None, v=None, o=None, cu=None) == 0
    assert fwd_fast(lib, batch=0, q=None, k=None, v=None, o=None, cu=None) == 0
    assert fwd32(lib, batch=0, q=None, k=None, v=None, o=None, cu=None) == 0
    assert fwd_exact(lib, batch=0, q=None, k=None, v=None, o=None, cu=None) == 0
    assert uni(lib, batch=0, q=None, k=None, v=None, o=None) == 0
    assert uni(lib, fast=True, batch=0, q=None, k=None, v=None, o=None) == 0
    assert strided(lib, batch=0, q=None, k=None, v=None, o=None, lens=None) == 0
    assert paged(lib, batch=0, q=None, k=None, v=None, o=None, bt=None, lens=None) == 0
    assert splitkv(lib, batch=0, q=None, k=None, v=None, o=None, cu=None, ws=None) == 0
    assert splitkv_strided(lib, batch=0, q=None, k=None, v=None, o=None, lens=None, ws=None) == 0
    assert splitkv_paged(lib, batch=0, q=None, k=None, v=None, o=None, bt=None, lens=None, ws=None) == 0
    assert lib.fmha_decode_last_error_detail() == b""
    assert lib.fmha_decode_last_plan() == b""


def test_rejected_call_has_no_plan(lib):
    assert fwd(lib, sq=2) == BAD
    assert lib.fmha_decode_last_plan() == b""


def test_python_wrapper_raises(lib):
    import fmha_amd
    with pytest.raises(fmha_amd.FmhaDecodeError) as ei:
        fmha_amd.launch_fmha_decode(0, Q, K, V, O, CU, 4, 16, 16, 2, 128, 128, 0.1)
    assert ei.value.code == BAD and "seqlen_q" in ei.value.detail


@pytest.mark.parametrize("defines", [[], ["-DFMHA_DECODE_COMPAT_EXACT"]])
def test_compat_header_compiles(defines):
    """include/fmha_decode_compat.hpp (the drop-in for the reference's
    launch_fmha_mfma_4x4x4) compiles as host code against the C ABI, also
    routed to the exact entry point."""
    import subprocess
    import tempfile
    src = ('#include "fmha_decode_compat.hpp"\n'
           'void f(const bhalf_t* q, const bhalf_t* k, const bhalf_t* v, half_t* o, const int* cu) {\n'
           '  launch_fmha_mfma_4x4x4(dim3(1, 1, 10), dim3(256, 1, 1), 0, q, k, v, o, cu,\n'
           '                         10, 16, 16, 1, 128, 128, 0.0883883f);\n}\n')
    with tempfile.TemporaryDirectory() as d:
        p = os.path.join(d, "t.cpp")
        open(p, "w").write(src)
        r = subprocess.run(["/opt/rocm/bin/hipcc", "-std=c++17", "-fsyntax-only", "-x", "hip",
                            "--offload-arch=gfx950", "-I", os.path.join(ROOT, "include"), *defines, p],
                           capture_output=True, text=True)
        assert r.returncode == 0, r.stderr


def test_error_detail_is_per_thread(lib):
    """The detail text of a rejected call belongs to the calling thread: a
    thread making valid (empty) calls never sees another thread's text, and
    a rejecting thread always reads its own.  ctypes releases the GIL for
    the call, so the two threads' calls overlap."""
    import threading
    errors = []
    start = threading.Barrier(2)

    def rejecting():
        start.wait()
        for i in range(2000):
            rc = fwd(lib, sq=2 + i % 3)
            detail = lib.fmha_decode_last_error_detail().decode()
            if rc != BAD or f"seqlen_q must be 1 (got {2 + i % 3})" not in detail:
                errors.append(("rejecting", i, rc, detail))
                return

    def succeeding():
        start.wait()
        for i in range(2000):
            rc = fwd(lib, batch=0, q=None, k=None, v=None, o=None, cu=None)
            detail = lib.fmha_decode_last_error_detail()
            if rc != 0 or detail != b"":
                errors.append(("succeeding", i, rc, detail))
                return

    threads = [threading.Thread(target=rejecting), threading.Thread(target=succeeding)]
    for t in threads:
        t.start()
    for t in threads:
        t.join()
    assert not errors, errors[:3]


def test_header_is_plain_c():
    """include/fmha_decode.h is a C header: a C99 translation unit that calls
    every entry point compiles with gcc (declarations only, nothing runs)."""
    import subprocess
    import tempfile
    src = ('#include "fmha_decode.h"\n'
           'int f(void* s, const void* q, const void* k, const void* v, void* o, const int32_t* cu,\n'
           '      void* ws) {\n'
           '  int rc = fmha_decode_fwd(s, q, k, v, o, cu, 1, 16, 16, 1, 128, 128, 0.088f);\n'
           '  rc |= fmha_decode_fwd_fp32_weights(s, q, k, v, o, cu, 1, 16, 16, 1, 128, 128, 0.088f);\n'
           '  rc |= fmha_decode_fwd_fast(s, q, k, v, o, cu, 1, 16, 16, 1, 128, 128, 0.088f);\n'
           '  rc |= fmha_decode_fwd_exact(s, q, k, v, o, cu, 1, 16, 16, 1, 128, 128, 0.088f);\n'
           '  rc |= fmha_decode_fwd_uniform(s, q, k, v, o, 16, 1, 16, 16, 1, 128, 128, 0.088f);\n'
           '  rc |= fmha_decode_fwd_uniform_fast(s, q, k, v, o, 16, 1, 16, 16, 1, 128, 128, 0.088f);\n'
           '  rc |= fmha_decode_fwd_strided(s, q, k, v, o, cu, 16, 32768, 2048, 128, 1, 16, 16, 1, 128, 128,\n'
           '                                0.088f);\n'
           '  rc |= fmha_decode_fwd_paged(s, q, k, v, o, cu, 4, cu, 16, 1, 16, 16, 1, 128, 128, 0.088f);\n'
           '  size_t n = fmha_decode_splitkv_workspace_size(1, 16, 16, 100, 128);\n'
           '  rc |= fmha_decode_fwd_splitkv(s, q, k, v, o, cu, 100, 1, 16, 16, 1, 128, 128, 0.088f, ws, n);\n'
           '  rc |= fmha_decode_fwd_splitkv_strided(s, q, k, v, o, cu, 100, 204800, 2048, 128, 1, 16, 16, 1, 128,\n'
           '                                        128, 0.088f, ws, n);\n'
           '  rc |= fmha_decode_fwd_splitkv_paged(s, q, k, v, o, cu, 7, cu, 16, 100, 1, 16, 16, 1, 128, 128,\n'
           '                                      0.088f, ws, n);\n'
           '  const char* t = fmha_decode_error_string(rc);\n'
           '  const char* d = fmha_decode_last_error_detail();\n'
           '  d = fmha_decode_last_plan();\n'
           '  return rc + fmha_decode_version() + (t == d);\n}\n')
    with tempfile.TemporaryDirectory() as d:
        p = os.path.join(d, "t.c")
        open(p, "w").write(src)
        r = subprocess.run(["gcc", "-std=c99", "-Wall", "-Werror", "-fsyntax-only", "-I",
                            os.path.join(ROOT, "include"), p], capture_output=True, text=True)
        assert r.returncode == 0, r.stderr


def splitkv_noalloc(lib, **kw):
    a = dict(stream=None, q=Q, k=K, v=V, o=O, cu=CU, maxs=1000, batch=4, hq=16, hkv=16, sq=1, dq=128, dkv=128,
             scale=0.088)
    a.update(kw)
    return lib.fmha_decode_fwd_splitkv_noalloc(a["stream"], a["q"], a["k"], a["v"], a["o"], a["cu"], a["maxs"],
                                               a["batch"], a["hq"], a["hkv"], a["sq"], a["dq"], a["dkv"], a["scale"])


@pytest.mark.parametrize("kw,code,needle", [
    (dict(maxs=-1), BAD, "max_seqlen_kv"),
    (dict(cu=None), BAD, "cu_seqlens_kv"),
    (dict(dq=96, dkv=96), BAD, "head_dim"),
    (dict(sq=3), BAD, "seqlen_q"),
    (dict(q=None), BAD, "non-null"),
    # more scratch than the library's array holds: rejected before any GPU call
    (dict(batch=4096, hq=32, hkv=8, maxs=4096), BAD, "scratch"),
])
def test_splitkv_noalloc_rejects(lib, kw, code, needle):
    """The no-allocation entry point checks its arguments, and its scratch
    need against FMHA_DECODE_NOALLOC_SCRATCH_BYTES, on the host first."""
    assert splitkv_noalloc(lib, **kw) == code
    assert needle in lib.fmha_decode_last_error_detail().decode()


def test_noalloc_scratch_size_matches_header(lib):
    import re
    import fmha_amd
    text = open(os.path.join(ROOT, "include", "fmha_decode.h")).read()
    m = re.search(r"#define FMHA_DECODE_NOALLOC_SCRATCH_BYTES \(\(size_t\)(\d+) << (\d+)\)", text)
    assert m and int(m.group(1)) << int(m.group(2)) == fmha_amd.NOALLOC_SCRATCH_BYTES
    # a long-context batch of the size the array is meant for fits it
    assert lib.fmha_decode_splitkv_workspace_size(64, 32, 8, 4096, 128) <= fmha_amd.NOALLOC_SCRATCH_BYTES
