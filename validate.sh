#!/bin/bash
# Runs every configuration of both suites (BASELINE C1..C5 and the reference's
# own table) with full validation against the CPU oracle; exits non-zero if
# any configuration fails.  Build first: python3 -c 'import __graft_entry__ as g; g.build()'
set -u
ROOT=$(cd "$(dirname "$0")" && pwd)
# C1 moves 503 MB per call, less than twice the 256 MB MALL: time it over 4
# rotated input sets (2 GB) so that no call is served from the cache.
python3 "$ROOT/tests/fmha_host.py" 1 --suite baseline --validate full --iters 20 --rotate 4 && \
python3 "$ROOT/tests/fmha_host.py" all --suite baseline --validate full --iters 20 && \
python3 "$ROOT/tests/fmha_host.py" all --suite reference --validate full --iters 20 && \
python3 "$ROOT/tests/fmha_host.py" all --suite gqa --validate full --iters 20
