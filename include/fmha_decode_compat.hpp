// fmha_decode_compat.hpp -- drop-in replacement for the reference's launch
// helper launch_fmha_mfma_4x4x4 (fmha_mfma_4x4x4_kernel.hpp:370-389).
//
// A host program written against the reference (its callers are
// fmha_host.cpp:367, :382 and :437) switches to this library by including
// this header instead of fmha_mfma_4x4x4_kernel.hpp and linking
// libfmha_decode.so; the call sites stay as they are.
//
// Differences a caller can observe:
//   * grid and block are accepted and ignored: the library computes its own
//     launch shape;
//   * K/V are read with the grouped-query head mapping (query head h uses KV
//     head h / (Hq/Hkv)); for Hq == Hkv this is the reference's indexing;
//   * an argument the library rejects throws std::runtime_error carrying the
//     library's message, where the reference either runs the D=256 kernel for
//     any head_dim other than 128 or fails later at the caller's next
//     HIP_CHECK (which throws std::runtime_error, fmha_host.cpp:26-35).
//
// fmha_decode_fwd computes the reference CPU loop's arithmetic step for step
// (fmha_host.cpp:179-244) for num_heads_q / num_heads_kv <= 2, so with the
// reference's head counts its own check (fmha_host.cpp:158-284) sees its
// own bits.  Compiled with FMHA_DECODE_COMPAT_EXACT defined, the launches go
// to fmha_decode_fwd_exact instead, which does so for groups of up to 8
// query heads per KV head and rejects larger ones.
#pragma once

#include <hip/hip_runtime.h>

#include <stdexcept>
#include <string>

#include "fmha_decode.h"

using bhalf_t = __bf16;    // same aliases as fmha_mfma_4x4x4_kernel.hpp:7-8
using half_t = _Float16;

inline void launch_fmha_mfma_4x4x4(dim3 /*grid*/, dim3 /*block*/, hipStream_t stream, const bhalf_t* Q,
                                   const bhalf_t* K, const bhalf_t* V, half_t* O, const int* cu_seqlens_kv,
                                   int batch, int num_heads_q, int num_heads_kv, int seqlen_q, int head_dim_q,
                                   int head_dim_kv, float softmax_scale) {
#ifdef FMHA_DECODE_COMPAT_EXACT
  const int rc = fmha_decode_fwd_exact(static_cast<void*>(stream), Q, K, V, O,
                                       reinterpret_cast<const int32_t*>(cu_seqlens_kv), batch, num_heads_q,
                                       num_heads_kv, seqlen_q, head_dim_q, head_dim_kv, softmax_scale);
  const char* entry = "fmha_decode_fwd_exact: ";
#else
  const int rc = fmha_decode_fwd(static_cast<void*>(stream), Q, K, V, O,
                                 reinterpret_cast<const int32_t*>(cu_seqlens_kv), batch, num_heads_q,
                                 num_heads_kv, seqlen_q, head_dim_q, head_dim_kv, softmax_scale);
  const char* entry = "fmha_decode_fwd: ";
#endif
  if (rc != FMHA_DECODE_SUCCESS) {
    throw std::runtime_error(std::string(entry) + fmha_decode_error_string(rc) + ": " +
                             fmha_decode_last_error_detail());
  }
}
