"""Build recipe for libfmha_decode.so (gfx950), used by __graft_entry__.build().

Compiles fmha_amd/csrc/fmha_decode_api.hip (the C ABI) and every part of
fmha_amd/csrc/fmha_decode_inst.hip (the kernel instantiations, one slice per
-DFMHA_DECODE_PART) with hipcc, in parallel, and links them into
fmha_amd/libfmha_decode.so, in tree, so the built library travels with the
source tree.  The objects go to fmha_amd/_build/.
"""
import concurrent.futures
import os
import re
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
LIB = os.path.join(HERE, "libfmha_decode.so")
CSRC = os.path.join(HERE, "csrc")
API_SOURCE = os.path.join(CSRC, "fmha_decode_api.hip")
INST_SOURCE = os.path.join(CSRC, "fmha_decode_inst.hip")
OBJ_DIR = os.path.join(HERE, "_build")

HIPCC_FLAGS = [
    "--offload-arch=gfx950",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    # Packed-FP32 VALU forms are kept out of every build.
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    # MFMA results in VGPRs rather than AGPRs: the matrix-core kernel reads
    # every result with VALU instructions, which cannot take AGPR operands
    # (saves one v_accvgpr_read per value).
    "-mllvm", "-amdgpu-mfma-vgpr-form",
]


def hipcc():
    return os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")


def inst_parts():
    """Number of FMHA_DECODE_PART slices, as fmha_decode_inst.hip states it."""
    m = re.search(r"FMHA_DECODE_PARTS (\d+)", open(INST_SOURCE).read())
    if not m:
        raise RuntimeError("FMHA_DECODE_PARTS missing from " + INST_SOURCE)
    return int(m.group(1))


def _run(cmd):
    res = subprocess.run(cmd, capture_output=True, text=True)
    # The host pass does not know the packed-fp32 feature name and says so.
    err = "\n".join(l for l in res.stderr.splitlines() if "packed-fp32-ops" not in l)
    return res.returncode, err


def build(verbose=False, jobs=None):
    """Compile and link the library; raises CalledProcessError on failure."""
    os.makedirs(OBJ_DIR, exist_ok=True)
    for name in os.listdir(OBJ_DIR):  # objects of an earlier part count
        if name.endswith(".o"):
            os.remove(os.path.join(OBJ_DIR, name))
    inc = ["-I" + os.path.join(ROOT, "include"), "-I" + CSRC]
    units = [(API_SOURCE, [], os.path.join(OBJ_DIR, "fmha_decode_api.o"))]
    units += [(INST_SOURCE, ["-DFMHA_DECODE_PART=%d" % p], os.path.join(OBJ_DIR, "fmha_decode_inst_%d.o" % p))
              for p in range(inst_parts())]
    cmds = [[hipcc()] + HIPCC_FLAGS + inc + defs + ["-c", "-o", obj, src] for src, defs, obj in units]
    if verbose:
        print(" ".join(cmds[0]), flush=True)
        print("... and %d parts of %s" % (len(units) - 1, os.path.basename(INST_SOURCE)), flush=True)
    jobs = jobs or min(16, os.cpu_count() or 1)
    with concurrent.futures.ThreadPoolExecutor(max_workers=jobs) as pool:
        results = list(pool.map(_run, cmds))
    failed = False
    for cmd, (rc, err) in zip(cmds, results):
        if rc != 0:
            failed = True
            sys.stderr.write(" ".join(cmd) + "\n" + err + "\n")
        elif err.strip() and verbose:
            sys.stderr.write(err + "\n")
    if failed:
        raise subprocess.CalledProcessError(1, "hipcc")
    link = [hipcc(), "--offload-arch=gfx950", "-shared", "-fPIC", "-Wl,--no-undefined", "-o", LIB + ".tmp"]
    link += [obj for _, _, obj in units]
    rc, err = _run(link)
    if rc != 0:
        sys.stderr.write(" ".join(link) + "\n" + err + "\n")
        raise subprocess.CalledProcessError(rc, link)
    os.replace(LIB + ".tmp", LIB)
    return LIB


if __name__ == "__main__":
    print(build(verbose=True))
