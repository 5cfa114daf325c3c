// fmha_decode_splitkv.hpp -- decode attention for KV lengths beyond 16
// (split-KV), gfx950.
//
// Same semantics as the short-KV kernel, extended to any length S: fp32
// scores, max-subtracted softmax, weights rounded to bf16 *after*
// normalisation (as the reference's CPU loop does, fmha_host.cpp:209-226),
// fp32 P.V, one fp16 rounding.  Because the bf16 rounding needs the global
// max and sum before any weight is formed, the work runs in two to four
// launches over a caller-provided workspace:
//
//   1. scores:  one wave per (batch, block of 16 rows, KV-head group): the
//               block's Q and K rows are requested at once (as in the short
//               kernel), dot products, transposing butterfly (shared with
//               the short kernel); scaled scores t_j -> T, and per query head
//               the block's max m_b and sum l_b of exp(t_j - m_b).
//   2. stats:   rows of more than kPvStatBlocks blocks only: one workgroup
//               per (batch, query head): m = max_b m_b, L = sum_b l_b *
//               exp(m_b - m), loads batched, reduction order fixed
//               (deterministic).  Shorter rows skip it: each P.V wave
//               reduces its heads' block statistics itself (row_stats).
//   3. pv:      one wave per (batch, chunk of C rows, KV-head group), walking
//               the chunk in sub-blocks of NR rows with two register sets:
//               the next sub-block's V rows and scores are in flight while
//               the current one is processed.  The 64 lanes form
//               P_j = bf16(exp(t_j - m) / L) for the wave's heads into LDS,
//               then packed dot2 accumulation; the chunk's fp32 partial
//               output -> Opart, or fp16 O directly when every batch fits one
//               chunk.
//   4. combine: more than one chunk per row only: O = fp16(sum_c Opart),
//               chunks added in order.
//
// The combine stays a launch of its own: folding it into pass 3 (the last
// P.V wave of a row, found with an atomic counter, summing the partials)
// needs an agent-scope release fence in every P.V wave, an L2 writeback
// that measured about 350 ns of serialised L2 time per wave (B=256 S=1024
// Hq/Hkv 64/8 with 4 chunks per row: 584 against 250 µs; B=1 S=131072
// 32/8, 256 chunks: 137 against 106 µs).
//
// K and V are each read once; T adds 4 bytes per row and query head (written
// by 1, read by 3), the block statistics 8 bytes per 16 rows and query head,
// Opart 4*D bytes per chunk and query head.
#pragma once

#include <type_traits>

#include "fmha_decode_kernel.hpp"

namespace fmha_decode {

// How a batch's length is found (SplitArgs::len_mode).
constexpr int kLenCu = 0;       // cu[b + 1] - cu[b] (packed layout)
constexpr int kLenArray = 1;    // cu[b] holds the length itself
constexpr int kLenUniform = 2;  // every batch has max_rows rows

struct SplitArgs {
  const uint16_t* q;      // [batch, Hq, D] bf16
  const uint16_t* k;      // bf16 K rows in the launch's layout (LongRows)
  const uint16_t* v;
  uint16_t* o;            // [batch, Hq, D] fp16
  const int32_t* cu;      // packed: [batch+1] row offsets; else [batch] lengths (or null, uniform)
  float* t;               // [batch, nblk, Hq, 16] scaled scores
  float* m;               // [batch, Hq, nblk] block max
  float* l;               // [batch, Hq, nblk] block sum of exp(t - m_b)
  float* ml;              // [batch, Hq, 2] global max, global sum
  float* opart;           // [batch, Hq, nchunks, D] partial outputs
  int32_t num_heads_q;
  int32_t num_heads_kv;
  int32_t units_per_batch;  // KV-head groups per batch: ceil(Hkv / HPW)
  int32_t nblk;           // 16-row blocks per batch row: ceil(max_rows / 16)
  int32_t nchunks;        // P.V chunks per batch row: ceil(max_rows / chunk_rows)
  int32_t chunk_rows;     // C, a multiple of 16
  int32_t max_rows;       // lengths above this are invalid (NaN output)
  int32_t batch;
  float scale;
  int32_t len_mode;       // kLenCu, kLenArray or kLenUniform
  // kLayoutStrided: element strides of K/V; kLayoutPaged: page stride in
  // batch_stride, row (slot) stride in row_stride, block table and
  // log2(page_size).
  int64_t batch_stride;
  int32_t row_stride;
  int32_t head_stride;
  const int32_t* block_table;
  int32_t bt_stride;
  int32_t page_shift;
  // log2 of the sub-units per wave (scores, P.V): with fewer KV heads than a
  // wave holds, its lane groups take 2^sub_shift blocks (scores) or chunks
  // (P.V) of the same heads instead of idling (packed and strided layouts).
  int32_t sub_shift;
  // Launch KV heads per KV head in memory (>= 1): a query group larger than
  // the kernels' G runs as kv_groups groups of G on one launch, launch head
  // hk reading memory head hk / kv_groups of num_heads_kv / kv_groups.
  int32_t kv_groups;
  // 1: the statistics pass ran and ml holds each head's global max and sum;
  // 0: every P.V wave reduces its heads' block statistics (m, l) itself.
  int32_t stat_pass;
};

// KV heads of the cache in memory, and the one launch head hk reads.
__host__ __device__ __forceinline__ int kv_heads_mem(const SplitArgs& a) { return a.num_heads_kv / a.kv_groups; }
__device__ __forceinline__ int kv_head_mem(const SplitArgs& a, int hk) {
  return a.kv_groups == 1 ? hk : hk / a.kv_groups;
}

// Lane groups of a wave under SplitArgs::sub_shift: group hkl (of HPW)
// serves KV head hg * (HPW >> sub_shift) + hkl % (HPW >> sub_shift) for
// sub-unit hkl / (HPW >> sub_shift).
template <int HPW>
struct SubUnits {
  int shift;  // log2(heads per sub-unit)
  __device__ __forceinline__ explicit SubUnits(int sub_shift) : shift(ilog2(HPW) - sub_shift) {}
  __device__ __forceinline__ int heads() const { return 1 << shift; }
  __device__ __forceinline__ int unit(int hkl) const { return hkl >> shift; }
  __device__ __forceinline__ int head(uint32_t hg, int hkl) const { return (int)(hg << shift) + (hkl & (heads() - 1)); }
};

// Length of batch b (may be out of [0, max_rows]: the kernels check).
__device__ __forceinline__ int split_len(const SplitArgs& a, uint64_t b) {
  if (a.len_mode == kLenCu) return a.cu[b + 1] - a.cu[b];
  if (a.len_mode == kLenArray) return a.cu[b];
  return a.max_rows;
}
template <int LAYOUT>
__device__ __forceinline__ int split_len_l(const SplitArgs& a, uint64_t b) {
  if constexpr (LAYOUT == kLayoutPacked) return a.cu[b + 1] - a.cu[b];
  return split_len(a, b);
}

constexpr int kSplitBlockRows = kMaxSeq;  // rows per scores wave

__device__ __forceinline__ u32x4 buffer_load16_nt(__amdgpu_buffer_rsrc_t r, uint32_t voffset) {
  return buffer_load16<kPolicyStream>(r, voffset);
}

__device__ __forceinline__ float buffer_load_f32(__amdgpu_buffer_rsrc_t r, uint32_t voffset) {
  return __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(r, (int)voffset, 0, kPolicyDefault));
}


// A pointer the whole wave holds, moved to scalar registers: a buffer
// descriptor built from a value the compiler keeps in vector registers
// becomes a loop over the lanes.
__device__ __forceinline__ const uint16_t* uniform_ptr(const uint16_t* p) {
  const uint64_t v = reinterpret_cast<uint64_t>(p);
  const uint32_t lo = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)v);
  const uint32_t hi = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)(v >> 32));
  return reinterpret_cast<const uint16_t*>(((uint64_t)hi << 32) | lo);
}

// One wave's view of the K (or V) rows [lo, hi) of batch b, in one of the
// layouts of the short kernel:
//   kLayoutPacked:  rows cu[b] + j of [rows, Hkv, D];
//   kLayoutStrided: element b*batch_stride + j*row_stride + h*head_stride + d;
//   kLayoutPaged, kLayoutPagedBlock: slot j % page_size of page
//                   block_table[b][j / page_size] in a [pages, page_size,
//                   Hkv, D] cache.
// load<NR>(out, rel0) fetches rows lo + rel0 .. lo + rel0 + NR - 1 (rel0 a
// multiple of NR, lo a multiple of 16, NR <= 16): 16 bytes per lane, this
// lane's head and dims; rows at or past hi read 0 without memory access, so
// padding, neighbouring batches and unused pages are never read.
template <int D, int LAYOUT>
struct LongRows {
  static constexpr bool PAGED = LAYOUT == kLayoutPaged || LAYOUT == kLayoutPagedBlock;
  __amdgpu_buffer_rsrc_t rsrc;  // packed, strided: rows [lo, hi)
  const uint16_t* base;         // paged: the cache
  const int32_t* pages;         // paged: this batch's block-table row
  uint32_t row_bytes;           // bytes between consecutive rows (slots)
  uint32_t lane_off;            // this lane's head and dims within a row
  int lane_rows;                // rows from lo to this lane's first row (packed, strided)
  int lane_n;                   // rows from lo at which this lane's rows end (packed, strided)
  uint32_t page_shift;
  uint64_t page_stride;         // elements
  int lo, n;                    // first row, rows in range
  // Paged layouts: set once a load has met an unmapped page (a negative
  // block-table entry) among the rows in range; those rows read 0, and the
  // caller makes the batch's outputs NaN (it is invalid).  Wave-uniform: a
  // flag instead of NaN rows keeps the loads free of per-element selects
  // (which took the single pass from 206-221 to 376-382 VGPRs).
  int bad = 0;
  __device__ __forceinline__ bool any_bad() const { return bad != 0; }

  // lane_rows_: this lane's rows start that many rows after lo, and end at
  // lane_end (relative to lo, at most hi - lo): lane groups serving
  // different blocks or chunks.  Both 0 / hi - lo for the paged layouts.
  __device__ __forceinline__ void init(const SplitArgs& a, const uint16_t* t, uint32_t b, int64_t row_base, int lo_,
                                       int hi, int hk, bool head_ok, int r, int lane_rows_ = 0,
                                       int lane_end = 1 << 30) {
    lo = lo_;
    n = hi > lo_ ? hi - lo_ : 0;
    lane_rows = lane_rows_;
    lane_n = lane_end < n ? lane_end : n;
    const int hkv = kv_heads_mem(a);
    const int hm = kv_head_mem(a, hk);
    if constexpr (LAYOUT == kLayoutPacked) {
      row_bytes = (uint32_t)hkv * D * 2u;
      lane_off = head_ok ? (uint32_t)(hm * D + r * 8) * 2u : kLaneOutOfRange;
      rsrc = make_rsrc(t + ((uint64_t)row_base + lo) * hkv * D, (uint32_t)n * row_bytes);
    } else if constexpr (LAYOUT == kLayoutStrided) {
      row_bytes = (uint32_t)a.row_stride * 2u;
      lane_off = head_ok ? (uint32_t)(hm * a.head_stride + r * 8) * 2u : kLaneOutOfRange;
      const uint32_t span = n == 0 ? 0u
                                   : ((uint32_t)(n - 1) * (uint32_t)a.row_stride +
                                      (uint32_t)(hkv - 1) * (uint32_t)a.head_stride + D) * 2u;
      rsrc = make_rsrc(t + (uint64_t)b * (uint64_t)a.batch_stride + (uint64_t)lo * (uint64_t)a.row_stride, span);
    } else {
      row_bytes = (uint32_t)hkv * D * 2u;
      lane_off = head_ok ? (uint32_t)(hm * D + r * 8) * 2u : kLaneOutOfRange;
      base = t;
      pages = a.block_table + (uint64_t)b * (uint64_t)a.bt_stride;
      page_shift = (uint32_t)a.page_shift;
      page_stride = (uint64_t)a.batch_stride;
    }
  }

  // The rows of batches b0 .. b0+nb-1 through one descriptor (packed and
  // strided; lane groups serving different batches): this lane's batch b
  // has S rows (0: nothing is read).  Packed: rows relative to batch b0's
  // first, rel_rows the lane's offset (checked by the caller: rel_rows + S
  // rows stay below 2^30 bytes), the range ending at the last row any lane
  // reads; strided: the nb batches' span with max_rows rows each (checked on
  // the host).  load() then works as for init with lo = 0.
  __device__ __forceinline__ void init_multi(const SplitArgs& a, const uint16_t* t, uint32_t b0, uint32_t nb,
                                             uint32_t b, int S, int rel_rows, int hk, bool head_ok, int r) {
    static_assert(LAYOUT == kLayoutPacked || LAYOUT == kLayoutStrided, "one descriptor per wave");
    lo = 0;
    const int hkv = kv_heads_mem(a);
    const int hm = kv_head_mem(a, hk);
    if constexpr (LAYOUT == kLayoutPacked) {
      row_bytes = (uint32_t)hkv * D * 2u;
      lane_off = head_ok ? (uint32_t)(hm * D + r * 8) * 2u : kLaneOutOfRange;
      lane_rows = rel_rows;
      lane_n = rel_rows + S;
      int m = lane_n;
#pragma unroll
      for (int k = 1; k < kWaveSize; k <<= 1) m = max(m, __shfl_xor(m, k, kWaveSize));
      n = __builtin_amdgcn_readfirstlane(m);
      rsrc = make_rsrc(t + (uint64_t)a.cu[b0] * hkv * D, (uint32_t)n * row_bytes);
    } else {
      row_bytes = (uint32_t)a.row_stride * 2u;
      lane_off = head_ok ? (uint32_t)(hm * a.head_stride + r * 8) * 2u + (b - b0) * (uint32_t)a.batch_stride * 2u
                         : kLaneOutOfRange;
      lane_rows = 0;
      lane_n = S;
      n = a.max_rows;
      const uint32_t span = ((nb - 1) * (uint32_t)a.batch_stride + (uint32_t)(a.max_rows - 1) * (uint32_t)a.row_stride +
                             (uint32_t)(hkv - 1) * (uint32_t)a.head_stride + D) * 2u;
      rsrc = make_rsrc(t + (uint64_t)b0 * (uint64_t)a.batch_stride, span);
    }
  }

  // Descriptor of `rows` rows from row `row` on, inside one page.  A row past
  // the end looks up the entry of a row the wave's range has and gets an
  // empty range.  An unmapped page (a negative block-table entry) gets an
  // empty range too, nothing is read, and `bad` is set when rows > 0.
  __device__ __forceinline__ __amdgpu_buffer_rsrc_t page_rsrc(int row, int rows) {
    const int32_t entry = load_uniform_i32(pages, (uint32_t)row >> page_shift);
    // The scalar unit's form of the guard (a negative entry as page 0 with
    // an empty range).
    const PagedRowU32 pr = paged_row_u32(entry, (uint32_t)row, page_shift);
    bad |= __builtin_amdgcn_readfirstlane(rows > 0 && pr.unmapped ? 1 : 0);
    const uint32_t range = (uint32_t)__builtin_amdgcn_readfirstlane(pr.unmapped ? 0 : rows * (int)row_bytes);
    return make_rsrc(uniform_ptr(base + (uint64_t)pr.page * page_stride + (uint64_t)pr.slot * (row_bytes >> 1)),
                     range);
  }

  template <int NR>
  __device__ __forceinline__ void load(u32x4 (&out)[NR], int rel0) {
    static_assert(NR <= 16, "a sub-block fits a 16-row page");
    if constexpr (LAYOUT == kLayoutPacked || LAYOUT == kLayoutStrided) {
      // Rows past this lane's end are moved out of range (a strided range
      // can also cover other heads' padding rows).  Offsets from one
      // per-lane base plus a wave-uniform step: a per-row multiply of a
      // per-lane row kept 16-32 offsets live (several batches per wave,
      // G = 4: 256 VGPRs and 19 AGPRs against 215; the VALU P.V pass at
      // G = 1: 257 against 169).
      const int rowb = rel0 + lane_rows;
      const uint32_t off0 = lane_off + (uint32_t)rowb * row_bytes;
      const int lim = lane_n - rowb;
#pragma unroll
      for (int j = 0; j < NR; ++j)
        out[j] = buffer_load16_nt(rsrc, j < lim ? off0 + (uint32_t)j * row_bytes : kRowOutOfRange);
    } else if constexpr (LAYOUT == kLayoutPagedBlock) {
      const int valid = n - rel0 < 0 ? 0 : (n - rel0 > NR ? NR : n - rel0);
      const __amdgpu_buffer_rsrc_t pr = page_rsrc(lo + (valid > 0 ? rel0 : 0), valid);
#pragma unroll
      for (int j = 0; j < NR; ++j) out[j] = buffer_load16_nt(pr, lane_off + (uint32_t)j * row_bytes);
    } else {
#pragma unroll
      for (int j = 0; j < NR; ++j) {
        const bool ok = rel0 + j < n;
        out[j] = buffer_load16_nt(page_rsrc(lo + (ok ? rel0 + j : 0), ok ? 1 : 0), lane_off);
      }
    }
  }
};

// The rows [lo, hi) of one (batch, KV head) of a paged cache ([pages,
// page_size, Hkv, D], row j in slot j % page_size of page block_table[b][j /
// page_size]) for waves whose lane groups read different rows: the same
// init / load interface as LongRows, with per-lane addresses.  Each lane
// looks up the pages of its own rows (BLOCK, page_size >= 16: one lookup per
// 16-row block, which lies in one page).  The loads carry no branch (a
// branch in a pipelined loop makes the compiler wait for every request at
// its head): a row at or past the lane's end, or in an unmapped page (a
// negative block-table entry), reads 16 bytes of Q's first row instead --
// memory that always exists -- and is replaced by 0; an unmapped page also
// sets the lane's `bad`, and the caller makes the batch's outputs NaN (an
// invalid batch; a flag rather than NaN rows keeps the loads to one select
// per element: NaN rows took the VALU P.V pass from 245 to 352 VGPRs).
// Block-table lookups stay inside the batch's row (entry 0 for rows past
// the end), and no address is formed from a negative entry.
template <int D, bool BLOCK>
struct PagedLaneRows {
  const uint16_t* base;   // the cache at this lane's head and dims
  const uint16_t* safe;   // 16 readable bytes (Q's first row, this lane's dims)
  const int32_t* pages;   // this batch's block-table row
  uint32_t page_shift;
  uint64_t page_stride;   // elements per page
  uint64_t row_elems;     // elements per slot (Hkv * D)
  int lo, lane_rows, lane_n;
  int bad = 0;  // per lane: a load met an unmapped page among this lane's rows
  // Some lane of the wave met one (the wave's lane groups serve one batch in
  // the split passes).
  __device__ __forceinline__ bool any_bad() const { return __builtin_amdgcn_ballot_w64(bad != 0) != 0; }

  __device__ __forceinline__ void init(const SplitArgs& a, const uint16_t* t, uint32_t b, int64_t, int lo_, int hi,
                                       int hk, bool head_ok, int r, int lane_rows_ = 0, int lane_end = 1 << 30) {
    const int n = hi > lo_ ? hi - lo_ : 0;
    lo = lo_;
    lane_rows = lane_rows_;
    lane_n = head_ok ? (lane_end < n ? lane_end : n) : 0;
    base = t + (uint64_t)kv_head_mem(a, hk) * D + r * 8;
    safe = a.q + r * 8;
    pages = a.block_table + (uint64_t)b * (uint64_t)a.bt_stride;
    page_shift = (uint32_t)a.page_shift;
    page_stride = (uint64_t)a.batch_stride;
    row_elems = (uint64_t)kv_heads_mem(a) * D;
  }

  // Rows lo + rel0 + lane_rows + j, j < NR (lo and lane_rows multiples of
  // 16, rel0 a multiple of NR <= 16: with BLOCK the NR rows lie in one
  // 16-row block, hence in one page).  entries() requests their block-table
  // entries (one per row, or one with BLOCK) and load_entries() the rows
  // through them, so that a caller can request the entries a step ahead:
  // the entries and rows are vector loads, which complete in order, so
  // requesting both in one step makes every step wait a table round trip
  // after the previous rows.
  template <int NR>
  static constexpr int kEntries = BLOCK ? 1 : NR;

  template <int NR>
  __device__ __forceinline__ void entries(int32_t (&e)[kEntries<NR>], int rel0) const {
    const int row0 = rel0 + lane_rows;
    if constexpr (BLOCK) {
      const uint32_t abs0 = (uint32_t)(lo + row0);
      e[0] = pages[row0 < lane_n ? abs0 >> page_shift : 0u];
    } else {
#pragma unroll
      for (int j = 0; j < NR; ++j) {
        const uint32_t abs = (uint32_t)(lo + row0 + j);
        e[j] = pages[row0 + j < lane_n ? abs >> page_shift : 0u];
      }
    }
  }

  template <int NR>
  __device__ __forceinline__ void load_entries(u32x4 (&out)[NR], int rel0, const int32_t (&e)[kEntries<NR>]) {
    const int row0 = rel0 + lane_rows;
    u32x4 v[NR];
    bool unmapped[NR];
    // The guard in unsigned factors (paged_row_u32: a negative entry as
    // page 0, never read): the signed 64-bit form cost registers.
    if constexpr (BLOCK) {
      const bool any = row0 < lane_n;
      const PagedRowU32 pr = paged_row_u32(e[0], (uint32_t)(lo + row0), page_shift);
      const uint64_t el = (uint64_t)pr.page * page_stride + (uint64_t)pr.slot * row_elems;
#pragma unroll
      for (int j = 0; j < NR; ++j) {
        const bool ok = !pr.unmapped && row0 + j < lane_n;
        v[j] = __builtin_nontemporal_load(
            reinterpret_cast<const u32x4*>(ok ? base + el + (uint64_t)j * row_elems : safe));
        unmapped[j] = any && pr.unmapped;
      }
    } else {
#pragma unroll
      for (int j = 0; j < NR; ++j) {
        const bool ok = row0 + j < lane_n;
        const PagedRowU32 pr = paged_row_u32(e[j], (uint32_t)(lo + row0 + j), page_shift);
        const uint64_t el = (uint64_t)pr.page * page_stride + (uint64_t)pr.slot * row_elems;
        v[j] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(ok && !pr.unmapped ? base + el : safe));
        unmapped[j] = ok && pr.unmapped;
      }
    }
#pragma unroll
    for (int j = 0; j < NR; ++j) {
      const bool ok = row0 + j < lane_n && !unmapped[j];
      bad |= unmapped[j] ? 1 : 0;
#pragma unroll
      for (int k = 0; k < 4; ++k) out[j][k] = ok ? (uint32_t)v[j][k] : 0u;
    }
  }

  template <int NR>
  __device__ __forceinline__ void load(u32x4 (&out)[NR], int rel0) {
    int32_t e[kEntries<NR>];
    entries<NR>(e, rel0);
    load_entries<NR>(out, rel0, e);
  }
};

// The row loader of the split-KV passes for a layout.
template <int D, int LAYOUT>
using SplitRows = typename std::conditional<LAYOUT == kLayoutPagedLanes || LAYOUT == kLayoutPagedBlockLanes,
                                            PagedLaneRows<D, LAYOUT == kLayoutPagedBlockLanes>,
                                            LongRows<D, LAYOUT>>::type;

// First packed row of batch b (0 for the other layouts, which address rows
// per batch).
template <int LAYOUT>
__device__ __forceinline__ int64_t split_row_base(const SplitArgs& a, uint64_t b) {
  if constexpr (LAYOUT == kLayoutPacked) return a.cu[b];
  return 0;
}

// ---------------------------------------------------------------------------
// 1. scores
// ---------------------------------------------------------------------------
// Scores of 16-row block blk of batch b live at
// T[((b * nblk + blk) * Hq + query head) * 16 + row % 16]: each wave writes
// one contiguous span (its heads' 16 rows), whole cache lines.
__device__ __forceinline__ uint64_t t_block_base(const SplitArgs& a, uint64_t b, int blk) {
  return ((b * (uint64_t)a.nblk + (uint64_t)blk) * (uint64_t)a.num_heads_q) * kSplitBlockRows;
}

// One 16-row block per lane group, all of its K rows requested at once: a
// wave serves 2^sub_shift consecutive blocks (SubUnits).  The G query heads
// of a KV head are scored GH at a time against the same K registers (GH = 4
// bounds the partial sums a lane holds to 64).
template <int D, int G, int LAYOUT = kLayoutPacked>
__global__ __launch_bounds__(kBlockThreads) void splitkv_scores_kernel(SplitArgs a) {
  constexpr int LPH = D / 8;
  constexpr int HPW = kWaveSize / LPH;
  constexpr int NS = ilog2(LPH);
  constexpr int NR = kSplitBlockRows;
  constexpr int GH = G > 4 ? 4 : G;
  constexpr int V = GH * NR;
  constexpr int L = NS < ilog2(V) ? NS : ilog2(V);
  constexpr int W = (V >> NS) > 1 ? (V >> NS) : 1;
  constexpr int GS = W < NR ? W : NR;
  constexpr int C = ilog2(NR / GS);
  const int lane = threadIdx.x & (kWaveSize - 1);
  // Wave order (batch, block group, head group): consecutive waves read
  // neighbouring heads of the same rows.
  const SubUnits<HPW> su(a.sub_shift);
  const uint32_t id = blockIdx.x;
  const uint32_t upb = (uint32_t)a.units_per_batch;
  const uint32_t nwb = ((uint32_t)a.nblk + (1u << a.sub_shift) - 1) >> a.sub_shift;
  const uint32_t per_b = nwb * upb;
  const uint32_t b = id / per_b;
  if (b >= (uint32_t)a.batch) return;
  const uint32_t rem = id - b * per_b;
  const uint32_t wb = rem / upb;
  const uint32_t hg = rem - wb * upb;
  const int S = split_len_l<LAYOUT>(a, b);
  const int j0 = (int)(wb << a.sub_shift) * NR;  // the wave's first row
  if (S < 0 || S > a.max_rows || j0 >= S) return;
  const int hkl = lane / LPH;
  const int p = su.unit(hkl);           // this lane group's block of the wave
  const int hk = su.head(hg, hkl);
  const bool head_ok = hk < a.num_heads_kv;
  const int r = lane % LPH;
  const int hq = a.num_heads_q;
  const int blk = (int)(wb << a.sub_shift) + p;
  const int jb = j0 + p * NR;           // first row of this lane group's block
  const bool block_ok = jb < S;         // else past the row (and maybe past nblk): no writes
  const __amdgpu_buffer_rsrc_t q_rsrc = make_rsrc(a.q + (uint64_t)b * hq * D, (uint32_t)hq * D * 2);
  // Rows [0, S) of the batch: rows past S read 0 without access.
  SplitRows<D, LAYOUT> kv;
  kv.init(a, a.k, b, split_row_base<LAYOUT>(a, b), 0, S, hk, head_ok, r, p * NR);
  const uint32_t q_off = head_ok ? (uint32_t)(hk * G * D + r * 8) * 2u : kLaneOutOfRange;

  u32x4 qv[G];
#pragma unroll
  for (int g = 0; g < G; ++g) qv[g] = buffer_load16<kPolicyDefault>(q_rsrc, q_off + g * D * 2);
  u32x4 ks[NR];
  kv.template load<NR>(ks, j0);
  __builtin_amdgcn_sched_barrier(0);
  const bool kv_bad = kv.any_bad();

  // After the butterfly, lane r holds scores [blkl*W, blkl*W + W) of the
  // GH*NR (query head, row) pairs; lanes equal in r >> (NS - L) hold copies.
  const int blkl = r >> (NS - L);
  const bool writer = head_ok && block_ok && (r & ((1 << (NS - L)) - 1)) == 0;
  {
    // The wave's blocks' scores [Hq][16] each, written non-temporally (read
    // once, by the P.V pass): 4-6% faster on long-context shapes than
    // default-policy stores.  The range ends at the batch's last block.
    const int wblk = (int)(wb << a.sub_shift);
    const int nwblk = a.nblk - wblk < (1 << a.sub_shift) ? a.nblk - wblk : (1 << a.sub_shift);
    const __amdgpu_buffer_rsrc_t t_rsrc =
        make_rsrc(a.t + t_block_base(a, b, wblk), (uint32_t)nwblk * (uint32_t)hq * NR * 4u);
    const uint32_t t_lane = head_ok ? ((uint32_t)p * hq + (uint32_t)hk * G) * NR * 4u : kLaneOutOfRange;
#pragma unroll
    for (int g0 = 0; g0 < G; g0 += GH) {
      u32x4 qh[GH];
#pragma unroll
      for (int g = 0; g < GH; ++g) qh[g] = qv[g0 + g];
      float x[V];
      partial_scores<GH, NR>(qh, ks, x);
      TransposeReduce<LPH, V, 0>::run(x, lane);
#pragma unroll
      for (int h = 0; h < W / GS; ++h) {
        float t[GS];
        float bm = -__builtin_inff();
        const int vi0 = blkl * W + h * GS;
        const int g = g0 + vi0 / NR;
        const int jr0 = vi0 % NR;
#pragma unroll
        for (int w = 0; w < GS; ++w) {
          t[w] = x[h * GS + w] * a.scale;
          bm = jb + jr0 + w < S ? fmaxf(bm, t[w]) : bm;
        }
        // Scores of rows past S (their K rows read as 0) land in the
        // block's padding, which nothing reads as a weight.
        if (writer) {
          const uint32_t off = t_lane + (uint32_t)(g * NR + jr0) * 4u;
          if constexpr (GS % 4 == 0) {
#pragma unroll
            for (int w = 0; w < GS; w += 4) {
              const u32x4 v4 = {__builtin_bit_cast(uint32_t, t[w]), __builtin_bit_cast(uint32_t, t[w + 1]),
                                __builtin_bit_cast(uint32_t, t[w + 2]), __builtin_bit_cast(uint32_t, t[w + 3])};
              __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4_gcc, v4), t_rsrc, (int)(off + w * 4),
                                                     0, kPolicyStreamStore);
            }
          } else {
#pragma unroll
            for (int w = 0; w < GS; ++w)
              __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, t[w]), t_rsrc, (int)(off + w * 4), 0,
                                                    kPolicyStreamStore);
          }
        }
        // Every block has a valid row, so the group's max is finite for
        // finite scores.
        bm = GroupReduce<LPH, L - C, L, true>::run(bm);
        float bs = 0.0f;
#pragma unroll
        for (int w = 0; w < GS; ++w) bs += jb + jr0 + w < S ? expf(t[w] - bm) : 0.0f;
        bs = GroupReduce<LPH, L - C, L, false>::run(bs);
        if (writer && (blkl & ((1 << C) - 1)) == 0) {
          const uint64_t idx = ((uint64_t)b * hq + (uint64_t)hk * G + g) * a.nblk + blk;
          a.m[idx] = bm;
          // An unmapped page among the block's rows: a NaN sum makes every
          // weight of the batch's heads, hence its outputs, NaN.
          a.l[idx] = kv_bad ? __builtin_nanf("") : bs;
        }
      }
    }
  }
}

// Sum / max over the 64 lanes of a wave (every lane gets the result).
__device__ __forceinline__ float wave_max(float x) {
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) x = fmaxf(x, __shfl_xor(x, m, kWaveSize));
  return x;
}
__device__ __forceinline__ float wave_sum(float x) {
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) x += __shfl_xor(x, m, kWaveSize);
  return x;
}

// Max or sum over a workgroup of THREADS threads, in a fixed order (wave
// trees, then waves in index order); every thread gets the result.
template <int THREADS, bool IS_MAX>
__device__ __forceinline__ float block_reduce(float x, float* red) {
  x = IS_MAX ? wave_max(x) : wave_sum(x);
  if constexpr (THREADS == kWaveSize) {
    return x;
  } else {
    constexpr int NW = THREADS / kWaveSize;
    if ((threadIdx.x & (kWaveSize - 1)) == 0) red[threadIdx.x / kWaveSize] = x;
    __syncthreads();
    float y = red[0];
#pragma unroll
    for (int w = 1; w < NW; ++w) y = IS_MAX ? fmaxf(y, red[w]) : y + red[w];
    __syncthreads();  // red is reused by the next call
    return y;
  }
}

// ---------------------------------------------------------------------------
// 2. stats (rows of more than kPvStatBlocks blocks): per (batch, query
// head), the global max and sum of exponentials over the row's 16-row
// blocks.
// ---------------------------------------------------------------------------
// Rows of at most 16 blocks: one lane per head, all loads in flight.
#ifdef FMHA_DECODE_SHARED_KERNELS  // one translation unit emits it (not a template)
__global__ __launch_bounds__(256) void splitkv_stats_lane_kernel(SplitArgs a) {
  constexpr int NB = 16;
  const uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;  // b * Hq + h
  if (i >= (uint64_t)a.batch * a.num_heads_q) return;
  const uint64_t b = i / (uint64_t)a.num_heads_q;
  const int S = split_len(a, b);
  if (S <= 0 || S > a.max_rows) return;
  const int n = (S + kSplitBlockRows - 1) / kSplitBlockRows;
  const float* m = a.m + i * a.nblk;
  const float* l = a.l + i * a.nblk;
  float xm[NB], xl[NB];
#pragma unroll
  for (int c = 0; c < NB; ++c) {
    xm[c] = c < n ? m[c] : -__builtin_inff();
    xl[c] = c < n ? l[c] : 0.0f;
  }
  float gm = xm[0];
#pragma unroll
  for (int c = 1; c < NB; ++c) gm = fmaxf(gm, xm[c]);
  float gl = 0.0f;
#pragma unroll
  for (int c = 0; c < NB; ++c) gl += c < n ? xl[c] * expf(xm[c] - gm) : 0.0f;
  a.ml[2 * i] = gm;
  a.ml[2 * i + 1] = gl;
}
#endif  // FMHA_DECODE_SHARED_KERNELS

// Longer rows: one THREADS-thread group per head, U loads in flight per
// thread, reduction order fixed.
template <int THREADS>
__global__ __launch_bounds__(THREADS) void splitkv_stats_kernel(SplitArgs a) {
  constexpr int U = 8;
  __shared__ float red[THREADS / kWaveSize];
  const uint64_t i = blockIdx.x;  // b * Hq + h
  const int t = threadIdx.x;
  const uint64_t b = i / (uint64_t)a.num_heads_q;
  const int S = split_len(a, b);
  if (S <= 0 || S > a.max_rows) return;  // the same for every thread of the group
  const int n = (S + kSplitBlockRows - 1) / kSplitBlockRows;
  const float* m = a.m + i * a.nblk;
  const float* l = a.l + i * a.nblk;
  float vm = -__builtin_inff();
  for (int c0 = t; c0 < n; c0 += THREADS * U) {
    float xm[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int c = c0 + u * THREADS;
      xm[u] = c < n ? m[c] : -__builtin_inff();
    }
#pragma unroll
    for (int u = 0; u < U; ++u) vm = fmaxf(vm, xm[u]);
  }
  const float gm = block_reduce<THREADS, true>(vm, red);
  float vs = 0.0f;
  for (int c0 = t; c0 < n; c0 += THREADS * U) {
    float xm[U], xl[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int c = c0 + u * THREADS;
      xm[u] = c < n ? m[c] : 0.0f;
      xl[u] = c < n ? l[c] : 0.0f;
    }
#pragma unroll
    for (int u = 0; u < U; ++u) vs += c0 + u * THREADS < n ? xl[u] * expf(xm[u] - gm) : 0.0f;
  }
  const float gl = block_reduce<THREADS, false>(vs, red);
  if (t == 0) {
    a.ml[2 * i] = gm;
    a.ml[2 * i + 1] = gl;
  }
}

// The global max and sum of exp(t - max) of NS query heads (hqi[i]; ok[i]
// false: none, 0 and 1 returned) of a row of S rows, for the P.V passes:
// a.ml when the statistics pass ran, else the scores pass's block
// statistics reduced here.  The NL lanes whose lane index differs only in the bits of
// STRIDE * (NL - 1) share each head; lane k of them (k = (lane / STRIDE) %
// NL) takes blocks k, k + NL, ... (the max, then the sum of l * exp(m -
// max)), U of them in flight per head, then butterflies over the NL lanes in
// a fixed order.
template <int NL, int STRIDE, int NS>
__device__ __forceinline__ void row_stats(const SplitArgs& a, const uint64_t (&hqi)[NS], const bool (&ok)[NS], int S,
                                          int lane, float (&gm)[NS], float (&gl)[NS]) {
  if (a.stat_pass) {
#pragma unroll
    for (int i = 0; i < NS; ++i) {
      gm[i] = ok[i] ? a.ml[2 * hqi[i]] : 0.0f;
      gl[i] = ok[i] ? a.ml[2 * hqi[i] + 1] : 1.0f;
    }
    return;
  }
  constexpr int U = 4;
  const int k = (lane / STRIDE) % NL;
  const int n = (S + kSplitBlockRows - 1) / kSplitBlockRows;
  float mx[NS];
#pragma unroll
  for (int i = 0; i < NS; ++i) mx[i] = -__builtin_inff();
  for (int s0 = k; s0 < n; s0 += NL * U) {
    float x[NS][U];
#pragma unroll
    for (int i = 0; i < NS; ++i)
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int s = s0 + u * NL;
        x[i][u] = ok[i] && s < n ? a.m[hqi[i] * a.nblk + s] : -__builtin_inff();
      }
#pragma unroll
    for (int i = 0; i < NS; ++i)
#pragma unroll
      for (int u = 0; u < U; ++u) mx[i] = fmaxf(mx[i], x[i][u]);
  }
#pragma unroll
  for (int i = 0; i < NS; ++i)
#pragma unroll
    for (int d = STRIDE; d < STRIDE * NL; d <<= 1) mx[i] = fmaxf(mx[i], __shfl_xor(mx[i], d, kWaveSize));
  float sm[NS];
#pragma unroll
  for (int i = 0; i < NS; ++i) sm[i] = 0.0f;
  for (int s0 = k; s0 < n; s0 += NL * U) {
    float x[NS][U], y[NS][U];
#pragma unroll
    for (int i = 0; i < NS; ++i)
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int s = s0 + u * NL;
        const bool in = ok[i] && s < n;
        x[i][u] = in ? a.m[hqi[i] * a.nblk + s] : 0.0f;
        y[i][u] = in ? a.l[hqi[i] * a.nblk + s] : 0.0f;
      }
#pragma unroll
    for (int i = 0; i < NS; ++i)
#pragma unroll
      for (int u = 0; u < U; ++u) sm[i] += ok[i] && s0 + u * NL < n ? y[i][u] * expf(x[i][u] - mx[i]) : 0.0f;
  }
#pragma unroll
  for (int i = 0; i < NS; ++i) {
#pragma unroll
    for (int d = STRIDE; d < STRIDE * NL; d <<= 1) sm[i] += __shfl_xor(sm[i], d, kWaveSize);
    gm[i] = ok[i] ? mx[i] : 0.0f;
    gl[i] = ok[i] ? sm[i] : 1.0f;
  }
}

// ---------------------------------------------------------------------------
// 3. P.V per chunk.  DIRECT: every batch fits one chunk, so the wave writes
// fp16 O itself (and the zero / NaN rows of empty or invalid batches).
// ---------------------------------------------------------------------------
template <int D, int G, int NR>
struct PvSlots {
  static constexpr int LPH = D / 8;
  static constexpr int HPW = kWaveSize / LPH;
  static constexpr int SLOTS = HPW * G * NR;  // weights per sub-block
  static constexpr int PER_LANE = (SLOTS + kWaveSize - 1) / kWaveSize;
};

// One sub-block: weights -> LDS -> row pairs -> accumulate.  Slot
// f = lane + 64*i is (KV head f / (G*NR), query g = (f / NR) % G, row f % NR)
// of the wave's heads; valid[i] marks slots inside the chunk.
template <int D, int G, int NR>
__device__ __forceinline__ void pv_sub_block(const u32x4 (&vr)[NR], const float (&tv)[PvSlots<D, G, NR>::PER_LANE],
                                             const float (&gm)[PvSlots<D, G, NR>::PER_LANE],
                                             const float (&gsum)[PvSlots<D, G, NR>::PER_LANE],
                                             const int (&rows_left)[PvSlots<D, G, NR>::PER_LANE],
                                             bool (&slot_ok)[PvSlots<D, G, NR>::PER_LANE], uint16_t* lds_p, int hkl,
                                             int lane, float (&acc)[G][8]) {
  using P = PvSlots<D, G, NR>;
  constexpr int VP = G * kMaxSeq;
#pragma unroll
  for (int i = 0; i < P::PER_LANE; ++i) {
    const int f = lane + kWaveSize * i;
    const int jf = f % NR;
    const bool valid = slot_ok[i] && jf < rows_left[i];
    const float p = valid ? expf(tv[i] - gm[i]) / gsum[i] : 0.0f;
    if (f < P::SLOTS)
      lds_p[(f / (G * NR)) * VP + ((f / NR) % G) * kMaxSeq + jf] = __builtin_bit_cast(uint16_t, (__bf16)p);
  }
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  const uint32_t* pairs = reinterpret_cast<const uint32_t*>(lds_p + hkl * VP);
  uint32_t pp[G][(NR + 1) / 2];
#pragma unroll
  for (int g = 0; g < G; ++g)
#pragma unroll
    for (int jp = 0; jp < NR / 2; ++jp) pp[g][jp] = pairs[g * (kMaxSeq / 2) + jp];
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  accumulate_pv<G, NR>(vr, pp, acc);
}

template <int D, int G, int NR, bool DIRECT, int LAYOUT = kLayoutPacked>
__global__ __launch_bounds__(kBlockThreads) void splitkv_pv_kernel(SplitArgs a) {
  using P = PvSlots<D, G, NR>;
  constexpr int LPH = P::LPH;
  constexpr int HPW = P::HPW;
  constexpr int PL = P::PER_LANE;
  constexpr int VP = G * kMaxSeq;
  static_assert(NR % 2 == 0 && NR <= kMaxSeq, "sub-block rows");
  __shared__ __attribute__((aligned(16))) uint16_t lds_p[HPW * VP];
  const int lane = threadIdx.x & (kWaveSize - 1);
  // A wave serves 2^sub_shift consecutive chunks (one per lane group,
  // SubUnits); DIRECT launches have one chunk per batch and sub_shift = 0.
  const SubUnits<HPW> su(a.sub_shift);
  const uint32_t id = blockIdx.x;
  const uint32_t upb = (uint32_t)a.units_per_batch;
  const uint32_t nwc = ((uint32_t)a.nchunks + (1u << a.sub_shift) - 1) >> a.sub_shift;
  const uint32_t per_b = nwc * upb;
  const uint32_t b = id / per_b;
  if (b >= (uint32_t)a.batch) return;
  const uint32_t rem = id - b * per_b;
  const uint32_t wc = rem / upb;
  const uint32_t hg = rem - wc * upb;
  const int S = split_len_l<LAYOUT>(a, b);
  const bool bad = S < 0 || S > a.max_rows;
  const int roww = (int)(wc << a.sub_shift) * a.chunk_rows;  // the wave's first row
  const int hkl = lane / LPH;
  const int p = su.unit(hkl);
  const uint32_t c = (wc << a.sub_shift) + (uint32_t)p;     // this lane group's chunk
  const int row0 = (int)c * a.chunk_rows;
  const int hk = su.head(hg, hkl);
  const bool head_ok = hk < a.num_heads_kv;
  const int r = lane % LPH;
  const int hq = a.num_heads_q;
  if (bad || roww >= S) {
    // Only chunk 0 of a DIRECT launch owns the output of an empty or invalid
    // batch; the combine kernel covers them otherwise.
    if constexpr (DIRECT) {
      if (c != 0) return;
      const u32x4 fill = bad ? u32x4{0x7e007e00u, 0x7e007e00u, 0x7e007e00u, 0x7e007e00u} : u32x4{0u, 0u, 0u, 0u};
      const __amdgpu_buffer_rsrc_t o_rsrc = make_rsrc(a.o + (uint64_t)b * hq * D, (uint32_t)hq * D * 2);
      const uint32_t o_off = head_ok ? (uint32_t)(hk * G * D + r * 8) * 2u : kLaneOutOfRange;
#pragma unroll
      for (int g = 0; g < G; ++g) buffer_store16(o_rsrc, o_off + g * D * 2, fill);
    }
    return;
  }
  // Rows of this lane group's chunk (<= 0: a chunk past the row's end).
  const int rows = min(S - row0, a.chunk_rows);
  const int rows_w = min(S - roww, a.chunk_rows);  // the wave's first chunk: the most rows
  // Each lane group reads its own chunk's rows only: sub-blocks past its
  // end read 0 without access.
  SplitRows<D, LAYOUT> vrows;
  const int rowe = S - roww < (a.chunk_rows << a.sub_shift) ? S : roww + (a.chunk_rows << a.sub_shift);
  vrows.init(a, a.v, b, split_row_base<LAYOUT>(a, b), roww, rowe, hk, head_ok, r, row0 - roww,
             row0 - roww + (rows > 0 ? rows : 0));
  // This batch's scores, [nblk, Hq, 16].
  const __amdgpu_buffer_rsrc_t t_rsrc =
      make_rsrc(a.t + t_block_base(a, b, 0), (uint32_t)a.nblk * (uint32_t)hq * kSplitBlockRows * 4u);

  // Weight slot f = lane + 64*i is (wave lane group f / (G*NR), query g =
  // (f / NR) % G, row f % NR); the lane group gives its head and chunk.
  float gm[PL], gsum[PL];
  uint32_t t_off[PL];
  bool slot_ok[PL];
  int slot_rows[PL];
  uint64_t hqi[PL];
#pragma unroll
  for (int i = 0; i < PL; ++i) {
    const int f = lane + kWaveSize * i;
    const int hklf = f / (G * NR);
    const int hkf = su.head(hg, hklf);
    const int gf = (f / NR) % G;
    const int jf = f % NR;
    const int row0f = (int)((wc << a.sub_shift) + (uint32_t)su.unit(hklf)) * a.chunk_rows;
    slot_rows[i] = min(S - row0f, a.chunk_rows);
    slot_ok[i] = f < P::SLOTS && hkf < a.num_heads_kv && slot_rows[i] > 0;
    hqi[i] = (uint64_t)b * hq + hkf * G + gf;
    t_off[i] = slot_ok[i] ? (uint32_t)((row0f / kSplitBlockRows) * hq * kSplitBlockRows +
                                       (hkf * G + gf) * kSplitBlockRows + jf) * 4u
                          : kLaneOutOfRange;
  }
  // The NR lanes of a slot's (head, query) share its statistics.
  row_stats<NR, 1, PL>(a, hqi, slot_ok, S, lane, gm, gsum);

  float acc[G][8];
#pragma unroll
  for (int g = 0; g < G; ++g)
#pragma unroll
    for (int d = 0; d < 8; ++d) acc[g][d] = 0.0f;

  // Two register sets: sub-block s+1 is requested before s is processed.
  // Requests past a chunk's last row return 0 without memory access (V)
  // or read scores of other rows (or nothing, past the batch's blocks) that
  // the row check masks (T).  The wave runs as many sub-blocks as its first
  // chunk has.
  const int nsub = (rows_w + NR - 1) / NR;
  u32x4 va[NR], vb[NR];
  float ta[PL], tb[PL];
  // Per-lane page lookups on pages under 16 rows (an entry per row): each
  // sub-block's block-table entries are requested a step ahead of its rows
  // (PF).  16-row pages look up one entry per sub-block and keep the
  // registers (two more would cost the 16-row P.V its second wave per SIMD).
  constexpr bool PF = LAYOUT == kLayoutPagedLanes;
  constexpr int NE = PF ? NR : 1;
  int32_t ea[NE], eb[NE];
  auto load = [&](u32x4 (&vr)[NR], float (&tv)[PL], int s, const int32_t (&e)[NE]) {
    if constexpr (PF)
      vrows.template load_entries<NR>(vr, s * NR, e);
    else
      vrows.template load<NR>(vr, s * NR);
    // Sub-blocks never straddle a 16-row block (chunks start on multiples of 16).
    const uint32_t sub = (uint32_t)(((s * NR) / kSplitBlockRows) * hq * kSplitBlockRows +
                                    (s * NR) % kSplitBlockRows) * 4u;
#pragma unroll
    for (int i = 0; i < PL; ++i) tv[i] = buffer_load_f32(t_rsrc, t_off[i] + sub);
  };
  auto entries = [&](int32_t (&e)[NE], int s) {
    if constexpr (PF) vrows.template entries<NR>(e, s * NR);
  };
  auto left = [&](int (&rl)[PL], int s) {
#pragma unroll
    for (int i = 0; i < PL; ++i) rl[i] = slot_rows[i] - s * NR;
  };
  entries(ea, 0);
  load(va, ta, 0, ea);
  entries(eb, 1);
  for (int s = 0; s < nsub; s += 2) {
    int rl[PL];
    load(vb, tb, s + 1, eb);
    entries(ea, s + 2);
    left(rl, s);
    pv_sub_block<D, G, NR>(va, ta, gm, gsum, rl, slot_ok, lds_p, hkl, lane, acc);
    load(va, ta, s + 2, ea);
    entries(eb, s + 3);
    left(rl, s + 1);
    if (s + 1 < nsub) pv_sub_block<D, G, NR>(vb, tb, gm, gsum, rl, slot_ok, lds_p, hkl, lane, acc);
  }

  if constexpr (DIRECT) {
    const __amdgpu_buffer_rsrc_t o_rsrc = make_rsrc(a.o + (uint64_t)b * hq * D, (uint32_t)hq * D * 2);
    const uint32_t o_off = head_ok ? (uint32_t)(hk * G * D + r * 8) * 2u : kLaneOutOfRange;
#pragma unroll
    for (int g = 0; g < G; ++g) buffer_store16(o_rsrc, o_off + g * D * 2, pack_f16x8(acc[g]));
  } else {
    // Partial outputs [Hq][nchunks][D] of this batch, read by the combine
    // pass right after: default-policy stores keep them in the caches
    // (non-temporal ones measured 4-9% slower overall).
    const uint32_t part_bytes = (uint32_t)a.nchunks * D * 4u;
    const __amdgpu_buffer_rsrc_t p_rsrc =
        make_rsrc(a.opart + (uint64_t)b * hq * a.nchunks * D, (uint32_t)hq * part_bytes);
    // A lane group whose chunk starts past the row's end writes nothing.
    const uint32_t p_off = head_ok && rows > 0 ? (uint32_t)hk * G * part_bytes + (c * D + r * 8) * 4u : kLaneOutOfRange;
#pragma unroll
    for (int g = 0; g < G; ++g) {
      u32x4 lo, hi;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        lo[i] = __builtin_bit_cast(uint32_t, acc[g][i]);
        hi[i] = __builtin_bit_cast(uint32_t, acc[g][4 + i]);
      }
      __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4_gcc, lo), p_rsrc, (int)(p_off + g * part_bytes),
                                             0, kPolicyDefault);
      __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4_gcc, hi), p_rsrc,
                                             (int)(p_off + g * part_bytes + 16), 0, kPolicyDefault);
    }
  }
}

// ---------------------------------------------------------------------------
// 4. combine: O = fp16(sum over the batch's chunks of Opart), chunk order.
// ---------------------------------------------------------------------------
__device__ __forceinline__ void add8(float (&acc)[8], const u32x4& lo, const u32x4& hi) {
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    acc[k] += __builtin_bit_cast(float, (uint32_t)lo[k]);
    acc[4 + k] += __builtin_bit_cast(float, (uint32_t)hi[k]);
  }
}

// Few chunks: one lane per (batch, query head, 8 dims), U chunks in flight.
template <int D>
__global__ __launch_bounds__(256) void splitkv_combine_kernel(SplitArgs a) {
  constexpr int U = 4;
  const uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const uint64_t per_head = D / 8;
  if (i >= (uint64_t)a.batch * a.num_heads_q * per_head) return;
  const uint64_t head = i / per_head;  // b * Hq + h
  const int d0 = (int)(i - head * per_head) * 8;
  const uint64_t b = head / (uint64_t)a.num_heads_q;
  const int S = split_len(a, b);
  float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
  u32x4 out;
  if (S < 0 || S > a.max_rows) {
    out = u32x4{0x7e007e00u, 0x7e007e00u, 0x7e007e00u, 0x7e007e00u};
  } else {
    const int n = (S + a.chunk_rows - 1) / a.chunk_rows;
    const float* src = a.opart + head * a.nchunks * D + d0;
    for (int c0 = 0; c0 < n; c0 += U) {
      u32x4 lo[U], hi[U];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int c = c0 + u < n ? c0 + u : c0;
        lo[u] = *reinterpret_cast<const u32x4*>(src + (uint64_t)c * D);
        hi[u] = *reinterpret_cast<const u32x4*>(src + (uint64_t)c * D + 4);
      }
#pragma unroll
      for (int u = 0; u < U; ++u)
        if (c0 + u < n) add8(acc, lo[u], hi[u]);
    }
    out = pack_f16x8(acc);
  }
  *reinterpret_cast<u32x4*>(a.o + head * D + d0) = out;
}

// Many chunks: one THREADS-thread block per (batch, query head, slice of
// 32 dims), so that a head's partials are read by D/32 CUs and every chunk's
// slice is one 128-byte line.  Thread t sums dims [4*(t % 8), +4) of the
// slice over chunks c = t / 8 + k * CG (U = 8 chunks in flight); then the CG
// partial sums of each dim are added in order through LDS.
template <int D, int THREADS>
__global__ __launch_bounds__(THREADS) void splitkv_combine_block_kernel(SplitArgs a) {
  constexpr int SLICE = 32;
  constexpr int NSL = D / SLICE;
  constexpr int LPS = SLICE / 4;  // lanes per slice
  constexpr int CG = THREADS / LPS;
  constexpr int U = 8;
  __shared__ float part[CG][SLICE];
  const uint64_t head = blockIdx.x / NSL;  // b * Hq + h
  const int d0 = (int)(blockIdx.x - head * NSL) * SLICE;
  const int t = threadIdx.x;
  const int dl = t % LPS;
  const int cg = t / LPS;
  const uint64_t b = head / (uint64_t)a.num_heads_q;
  const int S = split_len(a, b);
  const bool bad = S < 0 || S > a.max_rows;
  const int n = bad ? 0 : (S + a.chunk_rows - 1) / a.chunk_rows;
  float acc[4] = {0, 0, 0, 0};
  const float* src = a.opart + head * a.nchunks * D + d0 + dl * 4;
  for (int c0 = cg; c0 < n; c0 += CG * U) {
    u32x4 x[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int c = c0 + u * CG < n ? c0 + u * CG : c0;
      x[u] = *reinterpret_cast<const u32x4*>(src + (uint64_t)c * D);
    }
#pragma unroll
    for (int u = 0; u < U; ++u)
      if (c0 + u * CG < n)
#pragma unroll
        for (int k = 0; k < 4; ++k) acc[k] += __builtin_bit_cast(float, (uint32_t)x[u][k]);
  }
#pragma unroll
  for (int k = 0; k < 4; ++k) part[cg][dl * 4 + k] = acc[k];
  __syncthreads();
  if (t >= SLICE / 8) return;
  // Threads 0..3 each finish 8 dims of the slice: sum over the chunk groups
  // in order, then one 16-byte fp16 store.
  float o[8] = {0, 0, 0, 0, 0, 0, 0, 0};
  for (int g = 0; g < CG; ++g)
#pragma unroll
    for (int k = 0; k < 8; ++k) o[k] += part[g][t * 8 + k];
  const u32x4 out = bad ? u32x4{0x7e007e00u, 0x7e007e00u, 0x7e007e00u, 0x7e007e00u} : pack_f16x8(o);
  *reinterpret_cast<u32x4*>(a.o + head * D + d0 + t * 8) = out;
}

}  // namespace fmha_decode
