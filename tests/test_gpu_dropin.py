"""The reference's own host program, unmodified, with its launches routed to
this library (oracle/_ref/fmha_dropin, built by oracle/Makefile from
/root/reference/fmha_host.cpp and oracle/dropin_main.cpp): the reference's
benchmark loop and its own CPU validation (fmha_host.cpp:434-445) run on this
library's kernel and must report success.  Its configs 0..3
(fmha_host.cpp:511-516: B=10 and 30720, H=16 and 32, D=128 and 256, its
Poisson(4) lengths) are MHA, where its CPU loop's indexing is valid; config 3
(B=30720, H=32, D=128) is the largest the CLI takes (fmha_host.cpp:485)."""
import os
import re
import subprocess

import pytest

from tests.conftest import ROOT

BIN = os.path.join(ROOT, "oracle", "_ref", "fmha_dropin")
REF_BIN = os.path.join(ROOT, "oracle", "_ref", "fmha_reference")

pytestmark = [pytest.mark.gpu,
              pytest.mark.skipif(not os.path.exists(BIN),
                                 reason="oracle/_ref/fmha_dropin not built (reference not mounted at build time)")]


@pytest.mark.parametrize("config", [0, 1, 2, 3])
def test_reference_host_validates_this_kernel(config):
    r = subprocess.run([BIN, str(config)], capture_output=True, text=True, timeout=240)
    out = r.stdout
    print(out[-1500:], flush=True)
    assert r.returncode == 0, r.stderr[-2000:]
    assert "Validation passed" in out, "reference validation did not pass"
    assert "Validation failed" not in out and "Error at" not in out
    ms = re.search(r"Average time:\s+([0-9.]+) ms", out)
    gbs = re.search(r"Memory bandwidth:\s+([0-9.]+) GB/s", out)
    assert ms and gbs
    print(f"reference harness, config {config}: {float(ms.group(1)) * 1e3:.1f} us/call, "
          f"{float(gbs.group(1)):.0f} GB/s", flush=True)
    if os.path.exists(REF_BIN):
        # the same harness with the reference's own kernel (fmha_mfma_4x4x4)
        rr = subprocess.run([REF_BIN, str(config)], capture_output=True, text=True, timeout=240)
        assert rr.returncode == 0, rr.stderr[-2000:]
        rms = re.search(r"Average time:\s+([0-9.]+) ms", rr.stdout)
        rgbs = re.search(r"Memory bandwidth:\s+([0-9.]+) GB/s", rr.stdout)
        print(f"reference harness with the reference kernel, config {config}: "
              f"{float(rms.group(1)) * 1e3:.1f} us/call, {float(rgbs.group(1)):.0f} GB/s "
              f"({'passed' if 'Validation passed' in rr.stdout else 'validation failed'})", flush=True)
