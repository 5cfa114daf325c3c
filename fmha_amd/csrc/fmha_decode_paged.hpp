// fmha_decode_paged.hpp -- guarded block-table lookups of the paged KV cache
// ([pages, page_size, Hkv, D]; row j of batch b is slot j % page_size of page
// block_table[b * stride + j / page_size]).
//
// Serving engines pad block tables with negative entries (-1).  A kernel that
// turns such an entry into an address reads far outside the cache, so every
// paged loader in this library forms a row's address only through
// paged_row_elem, which refuses a negative entry, or its 32-bit-factor form
// paged_row_u32, and treats a batch whose rows use one as invalid: its
// outputs are NaN, and the unmapped rows are never read.  Entries at or above the cache's page count are outside what
// the library can check (the C ABI does not carry the page count).
//
// Plain integer arithmetic, compiled for the device by the kernels and for
// the host by the CPU test of these guards (tests/test_paged_guard.py).
#pragma once

#include <stdint.h>

#if defined(__HIPCC__)
#define FMHA_DECODE_HD __host__ __device__ __forceinline__
#else
#define FMHA_DECODE_HD inline
#endif

namespace fmha_decode {

// Element offset of row `row` from the cache base (slot `row & (2^page_shift
// - 1)` of page `entry`), or -1 when the entry is negative (unmapped).
FMHA_DECODE_HD int64_t paged_row_elem(int32_t entry, uint32_t row, uint32_t page_shift, uint64_t page_stride,
                                      uint64_t row_elems) {
  if (entry < 0) return -1;
  const uint64_t slot = (uint64_t)(row & ((1u << page_shift) - 1u));
  return (int64_t)((uint64_t)entry * page_stride + slot * row_elems);
}

// paged_row_elem in unsigned 32-bit factors, for loaders that keep the
// arithmetic on scalar or 32-bit registers (the signed 64-bit form cost the
// single pass about 90 VGPRs): the page (0 for a negative entry) and slot of
// row `row`, and whether the entry is unmapped.  When it is not,
// page * page_stride + slot * row_elems is paged_row_elem's offset; when it
// is, the caller must read nothing for the row.
struct PagedRowU32 {
  uint32_t page;
  uint32_t slot;
  bool unmapped;
};

FMHA_DECODE_HD PagedRowU32 paged_row_u32(int32_t entry, uint32_t row, uint32_t page_shift) {
  PagedRowU32 p;
  p.unmapped = entry < 0;
  p.page = p.unmapped ? 0u : (uint32_t)entry;
  p.slot = row & ((1u << page_shift) - 1u);
  return p;
}

// Block-table entries rows [0, S) of a batch use: ceil(S / page_size).
FMHA_DECODE_HD int paged_entries_used(int S, uint32_t page_shift) {
  return S <= 0 ? 0 : (int)(((uint32_t)(S - 1) >> page_shift) + 1u);
}

}  // namespace fmha_decode
