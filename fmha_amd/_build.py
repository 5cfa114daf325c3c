"""Build recipe for libfmha_decode.so (gfx950), used by __graft_entry__.build().

Compiles fmha_amd/csrc/*.hip with hipcc into fmha_amd/libfmha_decode.so, in
tree, so the built library travels with the source tree.
"""
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
LIB = os.path.join(HERE, "libfmha_decode.so")
SOURCES = [os.path.join(HERE, "csrc", "fmha_decode_api.hip")]

HIPCC_FLAGS = [
    "--offload-arch=gfx950",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-shared",
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


def build(verbose=False):
    """Compile the library; raises CalledProcessError on failure."""
    cmd = [hipcc()] + HIPCC_FLAGS + ["-I" + os.path.join(ROOT, "include"),
                                     "-I" + os.path.join(HERE, "csrc"),
                                     "-o", LIB + ".tmp"] + SOURCES
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    # The host pass does not know the packed-fp32 feature name and says so.
    err = "\n".join(l for l in res.stderr.splitlines() if "packed-fp32-ops" not in l)
    if res.returncode != 0:
        sys.stderr.write(err + "\n")
        raise subprocess.CalledProcessError(res.returncode, cmd)
    if err.strip() and verbose:
        sys.stderr.write(err + "\n")
    os.replace(LIB + ".tmp", LIB)
    return LIB


if __name__ == "__main__":
    print(build(verbose=True))
