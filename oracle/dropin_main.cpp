// dropin_main.cpp -- the reference's own host program (fmha_host.cpp, not
// modified) built against this library: its launch_fmha_mfma_4x4x4 calls
// (fmha_host.cpp:367, :382, :437) resolve to include/fmha_decode_compat.hpp,
// i.e. to libfmha_decode.so, while its allocation, timing and CPU validation
// (do_validation, fmha_host.cpp:158-284) stay the reference's.
//
// TEST INFRASTRUCTURE ONLY (tests/test_gpu_dropin.py runs the binary).  It
// shows the one-include switch INTEGRATION.md describes on the reference's
// unmodified source: the reference headers are included first, under their
// own names; the library's drop-in is then included under a macro name, and
// the reference's calls are routed to it.  Built by oracle/Makefile into
// oracle/_ref/ where /root/reference is mounted; no reference text enters
// the repository.
#include "fmha_mfma_kernel.hpp"
#include "fmha_vectorized_fma_kernel.hpp"
#include "fmha_mfma_4x4x4_kernel.hpp"

#define launch_fmha_mfma_4x4x4 fmha_decode_dropin_launch
#include "fmha_decode_compat.hpp"

#include "fmha_host.cpp"
