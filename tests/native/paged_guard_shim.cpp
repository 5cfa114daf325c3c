// paged_guard_shim.cpp -- the paged-cache guards of fmha_decode_paged.hpp,
// the header the kernels include, compiled for the host so that
// tests/test_paged_guard.py can drive them on the CPU.  Test infrastructure
// only; the test compiles it with g++ into a temporary directory.
#include <stdint.h>

#include "fmha_decode_paged.hpp"

extern "C" {

int64_t guard_row_elem(int32_t entry, uint32_t row, uint32_t page_shift, uint64_t page_stride, uint64_t row_elems) {
  return fmha_decode::paged_row_elem(entry, row, page_shift, page_stride, row_elems);
}

int guard_entries_used(int S, uint32_t page_shift) { return fmha_decode::paged_entries_used(S, page_shift); }

// paged_row_u32's offset as the loaders form it (page * page_stride + slot *
// row_elems), or -1 for an unmapped entry.
int64_t guard_row_u32(int32_t entry, uint32_t row, uint32_t page_shift, uint64_t page_stride, uint64_t row_elems) {
  const fmha_decode::PagedRowU32 p = fmha_decode::paged_row_u32(entry, row, page_shift);
  if (p.unmapped) return -1;
  return (int64_t)((uint64_t)p.page * page_stride + (uint64_t)p.slot * row_elems);
}

}  // extern "C"
