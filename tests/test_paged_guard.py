"""CPU checks of the paged-cache guards (fmha_amd/csrc/fmha_decode_paged.hpp:
paged_row_elem and its 32-bit-factor form paged_row_u32) that every paged
loader of the library forms its row addresses through.

Serving engines pad block tables with negative entries; a kernel that turned
one into an address would read far outside the cache and fault the GPU.
The header is compiled here for the host (tests/native/paged_guard_shim.cpp)
and driven with the tables a kernel can meet: for every layout of
block-table row, page size and length the kernels accept, each row a batch
has either maps to an offset inside the cache or is refused, a negative
entry is always refused, and every entry looked up lies inside the batch's
row of the table.  The GPU regression test of the kernels themselves is
tests/test_gpu_layouts.py::test_paged_negative_entries_give_nan.
"""
import ctypes
import os
import subprocess

import numpy as np
import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(os.path.dirname(HERE), "fmha_amd", "csrc")


@pytest.fixture(scope="module")
def guards(tmp_path_factory):
    out = str(tmp_path_factory.mktemp("guard") / "libpaged_guard.so")
    subprocess.run(["g++", "-O2", "-std=c++17", "-fPIC", "-shared", "-Wall", "-Werror", "-I" + CSRC, "-o", out,
                    os.path.join(HERE, "native", "paged_guard_shim.cpp")], check=True)
    lib = ctypes.CDLL(out)
    lib.guard_row_elem.restype = ctypes.c_int64
    lib.guard_row_elem.argtypes = [ctypes.c_int32, ctypes.c_uint32, ctypes.c_uint32, ctypes.c_uint64, ctypes.c_uint64]
    lib.guard_entries_used.restype = ctypes.c_int
    lib.guard_entries_used.argtypes = [ctypes.c_int, ctypes.c_uint32]
    lib.guard_row_u32.restype = ctypes.c_int64
    lib.guard_row_u32.argtypes = [ctypes.c_int32, ctypes.c_uint32, ctypes.c_uint32, ctypes.c_uint64, ctypes.c_uint64]
    return lib


def test_negative_entries_are_refused(guards):
    for entry in (-1, -2, -(2 ** 31), -12345):
        for row in (0, 1, 15, 16, 2 ** 20):
            for shift in (0, 4, 6, 20):
                assert guards.guard_row_elem(entry, row, shift, 16 * 4096, 4096) == -1


def test_unsigned_form_equals_the_signed_one(guards):
    """paged_row_u32 (the 32-bit-factor form the long-row loaders use) gives
    paged_row_elem's offset for every mapped entry and refuses every
    negative one: entries from -2^31 to 2^31-1, rows up to 2^24, page sizes
    1 to 2^20, the caches' page strides and row sizes."""
    rng = np.random.default_rng(5)
    entries = np.concatenate([[-(2 ** 31), -2, -1, 0, 1, 2 ** 31 - 1], rng.integers(-(2 ** 31), 2 ** 31, 2000)])
    for shift in (0, 1, 4, 6, 10, 20):
        for hkv, d in ((1, 64), (8, 128), (32, 256)):
            row_elems = hkv * d
            page_stride = (1 << shift) * row_elems
            for entry in entries[:: 7 if shift else 1]:
                for row in (0, 1, 15, 16, int(rng.integers(0, 2 ** 24))):
                    a = guards.guard_row_elem(int(entry), row, shift, page_stride, row_elems)
                    b = guards.guard_row_u32(int(entry), row, shift, page_stride, row_elems)
                    assert a == b, (int(entry), row, shift, a, b)


def test_entries_used_is_ceil_of_length_over_page(guards):
    for shift in range(0, 8):
        for S in range(0, 300):
            want = 0 if S == 0 else -(-S // (1 << shift))
            assert guards.guard_entries_used(S, shift) == want


@pytest.mark.parametrize("page_size", [1, 2, 4, 8, 16, 32, 64])
def test_every_address_a_batch_can_form_stays_in_the_cache(guards, page_size):
    """Random caches and tables with -1 padding and negative garbage: for
    each batch, every row below its length either maps inside the cache
    (slot and whole row included) or is refused, and a batch is refused as
    a whole exactly when one of the entries its rows use is negative --
    the rule each paged kernel applies (NaN outputs, nothing read)."""
    rng = np.random.default_rng(page_size)
    shift = page_size.bit_length() - 1
    for trial in range(200):
        hkv, d = [(1, 64), (2, 128), (8, 128), (4, 256)][trial % 4]
        row_elems = hkv * d
        page_stride = page_size * row_elems
        num_pages = int(rng.integers(1, 40))
        bt_stride = int(rng.integers(1, 8))
        cache_elems = num_pages * page_stride
        max_rows = min(16, bt_stride * page_size) if trial % 2 else bt_stride * page_size  # short / long rows
        for _ in range(8):
            table = rng.integers(0, num_pages, bt_stride).astype(np.int32)
            pad_from = int(rng.integers(0, bt_stride + 1))
            table[pad_from:] = -1                                   # serving-engine padding
            if rng.random() < 0.3:
                table[int(rng.integers(0, bt_stride))] = rng.choice([-2, -(2 ** 31), -7])
            S = int(rng.integers(0, max_rows + 1))
            used = guards.guard_entries_used(S, shift)
            assert used <= bt_stride                                # lookups stay in the row
            refused = bool((table[:used] < 0).any())
            any_refused = False
            for j in range(S):
                idx = j >> shift
                assert idx < used
                el = guards.guard_row_elem(int(table[idx]), j, shift, page_stride, row_elems)
                if el < 0:
                    any_refused = True
                    assert table[idx] < 0
                    continue
                assert 0 <= el and el + row_elems <= cache_elems, (el, cache_elems)
                assert el % row_elems == 0
            assert any_refused == refused
