"""CPU checks of the HIP sources for a device-compiler pitfall that no host
test can see.

hipcc (clang 22) compiles `__builtin_bit_cast(T, v[k])`, with v an
ext-vector such as u32x4 and k an index, as a cast of element 0.  The
kernels therefore convert a vector element to a scalar first
(`__builtin_bit_cast(float, (uint32_t)v[k])`).  This test finds every
variable declared as an ext-vector type in fmha_amd/csrc and fails on a
bit-cast whose operand indexes one of them without that conversion.
"""
import glob
import os
import re

from tests.conftest import ROOT

CSRC = os.path.join(ROOT, "fmha_amd", "csrc")
VECTOR_TYPES = ("u32x4", "VBuf")


def _vector_names(text):
    names = set()
    for t in VECTOR_TYPES:
        # declarations such as "u32x4 x[U];", "u32x4 lo, hi;", "const u32x4 (&kr)[NR]"
        for m in re.finditer(r"\b" + t + r"\b\s+([^;=){]+)", text):
            for part in m.group(1).split(","):
                n = re.match(r"\s*\(?&?\s*(\w+)", part)
                if n:
                    names.add(n.group(1))
    return names


def _bad_casts(text, names):
    bad = []
    for m in re.finditer(r"__builtin_bit_cast\(\s*\w+\s*,\s*(\w+)\s*\[", text):
        if m.group(1) in names:
            bad.append(text[m.start():m.start() + 60].split("\n")[0])
    return bad


def test_no_bit_cast_of_vector_elements():
    files = sorted(glob.glob(os.path.join(CSRC, "*.hpp")) + glob.glob(os.path.join(CSRC, "*.hip")))
    assert files
    found = {}
    for f in files:
        text = open(f).read()
        bad = _bad_casts(text, _vector_names(text))
        if bad:
            found[os.path.basename(f)] = bad
    assert not found, f"bit-cast of an ext-vector element without a scalar conversion: {found}"


def test_checker_catches_the_pitfall():
    text = "u32x4 x[8];\nfloat y = __builtin_bit_cast(float, x[u][k]);\n"
    assert _bad_casts(text, _vector_names(text))
    ok = "u32x4 x[8];\nfloat y = __builtin_bit_cast(float, (uint32_t)x[u][k]);\n"
    assert not _bad_casts(ok, _vector_names(ok))
