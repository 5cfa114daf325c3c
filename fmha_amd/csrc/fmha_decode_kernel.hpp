// fmha_decode_kernel.hpp -- gfx950 decode-attention kernel (seqlen_q = 1,
// KV length 0..16 per sequence, bf16 Q/K/V, fp32 accumulation, fp16 output).
//
// Semantics restated from the reference CPU loop (fmha_host.cpp:169-245) and
// the wired-in kernel (fmha_mfma_4x4x4_kernel.hpp:243-268, :326-334): fp32 dot
// products, scale, max-subtracted softmax with a sum>0 guard, softmax weights
// rounded to bf16 before P.V, fp32 accumulation, one RNE rounding to fp16.
// Query head h reads KV head h / G with G = Hq / Hkv.
//
// Work decomposition (one wavefront = one independent unit, no block barrier):
//   * a KV head is served by LPH = D/8 consecutive lanes; lane r of the group
//     owns dims [8r, 8r+8): one 16-byte bf16x8 chunk per KV row;
//   * a wave serves HPW = 64/LPH consecutive KV heads of one batch and all G
//     query heads of each, so every K/V byte is read from HBM exactly once;
//   * each lane issues all of its Q, K and V loads (G + 2*SMAX b128 buffer
//     loads, K/V with the streaming hint) before any arithmetic, so a wave
//     keeps 2*SMAX KiB of K/V in flight; the host caps the waves per CU (by
//     reserving LDS) so that a CU holds about 80 KiB of requests, the level
//     at which MI355X streams fastest;
//   * K/V rows are fetched through a buffer resource whose num_records ends at
//     this batch's last row: rows j >= S_b (padding up to the power-of-two
//     bucket SMAX) and lanes of absent heads read 0 without touching memory.
//
// QK^T: v_dot2_f32_bf16 on the packed pairs (4 per row), then a transposing
// butterfly across the LPH lanes of the head: at each step a lane keeps one
// half of its partial sums and swaps the other half with its partner, so the
// G*SMAX scores of the head end up fully reduced and spread over the lanes
// (15 exchanges for 16 scores instead of 64 for independent butterflies).
// Softmax runs on that distribution; the bf16 weights go through 128 bytes of
// LDS per head so every lane of the head sees all of them; P.V packs row pairs
// with v_perm_b32 and accumulates with v_dot2_f32_bf16.  With fp32 weights
// (PF32, the semantics of the reference's fmha_vectorized_fma) they take 64
// bytes of LDS per query head and P.V is one fused multiply-add per element
// and row, rows in order.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "fmha_decode_paged.hpp"

namespace fmha_decode {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
// Type produced/consumed by the raw-buffer b128 builtins.
typedef uint32_t u32x4_gcc __attribute__((vector_size(16)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));

constexpr int kWaveSize = 64;
// One wave per workgroup: waves are independent, and single-wave groups let
// the dispatcher place work at wave granularity.
constexpr int kWavesPerBlock = 1;
constexpr int kBlockThreads = kWaveSize * kWavesPerBlock;
constexpr int kMaxSeq = 16;
// Buffer descriptor word 3 for gfx9-family raw buffers (32-bit data format,
// no swizzle, no index stride).
constexpr int kBufferWord3 = 0x00020000;
// Byte offsets beyond every num_records this kernel builds (all < 2^30):
// loads there return 0 and stores are dropped, with no memory access.  A lane
// of an absent head adds kLaneOutOfRange, a row past the batch's length adds
// kRowOutOfRange; the sum of both still fits 32 bits.
constexpr uint32_t kLaneOutOfRange = 0x40000000u;
constexpr uint32_t kRowOutOfRange = 0x80000000u;
// Two bf16 quiet NaNs: what the paged loaders put in place of a row whose
// page is unmapped, so that the batch's outputs turn NaN.
constexpr uint32_t kNaNBf16x2 = 0x7fc07fc0u;

// Where a batch's K/V rows live.
//   kLayoutPacked:  rows [cu[b], cu[b+1]) of a [rows, Hkv, D] tensor, or
//                   rows [b*S, b*S+S) with uniform lengths (lens == null);
//   kLayoutStrided: element (b, j, h, d) at b*batch_stride + j*row_stride +
//                   h*head_stride + d (BSHD, BHSD, padded caches), lengths
//                   from lens[b] or uniform;
//   kLayoutPaged:   a [pages, page_size, Hkv, D] cache (page_size a power of
//                   two); row j of batch b is slot j % page_size of page
//                   block_table[b*bt_stride + j / page_size]; lengths from
//                   lens[b].  seqlen_uniform holds log2(page_size) and
//                   batch_stride the page stride.
constexpr int kLayoutPacked = 0;
constexpr int kLayoutStrided = 1;
constexpr int kLayoutPaged = 2;
// Pages of at least 16 rows, for the long-row kernels: a sub-block of up to
// 16 rows (aligned to its size) lies in one page, so it needs one block-table
// lookup and one descriptor.  kLayoutPaged then means pages of 1-8 rows (one
// lookup per row).  The host picks between the two, so that no pipelined loop
// carries a branch (the compiler would wait for every request at its head).
constexpr int kLayoutPagedBlock = 3;
// The same two paged layouts read through per-lane addresses
// (PagedLaneRows; in the matrix-core short kernel, a 64-bit address per
// lane), so that the lane groups of a wave can read rows of different pages:
// sub-units (SplitArgs::sub_shift) with fewer KV heads than a wave holds.
constexpr int kLayoutPagedLanes = 4;
constexpr int kLayoutPagedBlockLanes = 5;

constexpr bool is_paged_layout(int layout) { return layout >= kLayoutPaged && layout <= kLayoutPagedBlockLanes; }

struct DecodeArgs {
  const uint16_t* q;        // [batch, Hq, D] bf16 bits
  const uint16_t* k;        // bf16 bits, layout above
  const uint16_t* v;        // bf16 bits, same layout and strides as k
  uint16_t* o;              // [batch, Hq, D] fp16 bits
  const int32_t* lens;      // packed: cu offsets [batch+1]; strided/paged: lengths [batch]; or null
  const int32_t* block_table;  // paged only
  int64_t batch_stride;     // elements (strided); page stride (paged)
  int32_t row_stride;       // elements between rows
  int32_t head_stride;      // elements between KV heads
  int32_t bt_stride;        // paged: block_table entries per batch
  int32_t max_rows;         // largest valid length (16, or page_size when smaller)
  int32_t seqlen_uniform;   // rows per batch when lens == null; paged: log2(page_size)
  int32_t num_heads_q;
  int32_t num_heads_kv;
  int32_t units_per_batch;  // waves per batch: ceil(Hkv / HPW)
  uint32_t total_units;     // batch * units_per_batch
  float scale;
  // fmha_decode_multi_kernel only: log2 of the batches per wave and of
  // num_heads_kv (a power of two below the heads a wave holds).
  int32_t sub_shift;
  int32_t hkv_shift;
  // Query heads per KV head, num_heads_q / num_heads_kv.  The kernels are
  // instantiated for G = 1, 2, 4, 8; a call with 3 runs the G = 4 kernel and
  // 5-7 the G = 8 one, the query heads at or past `group` of each KV head
  // loading and storing nothing (out-of-range offsets).
  int32_t group;
  // Packed layout with cu offsets and paged layout, else null: a word of
  // host-visible memory where the call's first wave leaves 16 x the mean
  // length (packed: 16 * (cu[batch] - cu[0]) / batch; paged: of the first
  // 4096 lengths at most), for the host to size the next call's wave cap
  // (the host cannot read the lengths of this one).
  int32_t* rows_feedback;
};

// The first wave of a packed cu_seqlens call reports 16 x its mean length to
// the host (DecodeArgs::rows_feedback): one lane, one vector store.
__device__ __forceinline__ void report_mean_rows(const DecodeArgs& a, uint32_t unit, uint32_t batch, int lane) {
  if (a.rows_feedback != nullptr && unit == 0 && lane == 0 && batch > 0) {
    const int64_t rows = (int64_t)a.lens[batch] - (int64_t)a.lens[0];
    const int64_t mean16 = rows * 16 / (int64_t)batch;
    *a.rows_feedback = (int32_t)(mean16 < 0 ? 0 : (mean16 > 0x7fffffff ? 0x7fffffff : mean16));
  }
}

// The first wave of a paged call reports 16 x the mean of the first (at
// most 4096) lengths of lens, each clamped to [0, max_rows], to the host: a
// sample, 64 loads per lane at most, a butterfly sum, one vector store.
// Every lane of the wave calls it (unit is the wave's).
__device__ __forceinline__ void report_mean_rows_sample(const DecodeArgs& a, uint32_t unit, uint32_t batch,
                                                        int lane) {
  if (a.rows_feedback == nullptr || unit != 0 || batch == 0) return;
  const int n = batch < 4096u ? (int)batch : 4096;
  int sum = 0;
#pragma unroll 16
  for (int i = lane; i < n; i += kWaveSize) {
    const int len = a.lens[i];
    sum += len < 0 ? 0 : (len > a.max_rows ? a.max_rows : len);
  }
#pragma unroll
  for (int m = 1; m < kWaveSize; m <<= 1) sum += __shfl_xor(sum, m, kWaveSize);
  if (lane == 0) *a.rows_feedback = (int32_t)((int64_t)sum * 16 / n);
}

// Byte offset of query head g of the lane's KV head from qo_off (the head's
// first query row), out of range for padding heads g >= group.  G = 1 and 2
// kernels are never padded.
template <int G>
__device__ __forceinline__ uint32_t group_row_off(uint32_t qo_off, int g, int group, int D) {
  if constexpr (G >= 4) return g < group ? qo_off + (uint32_t)(g * D * 2) : kLaneOutOfRange;
  return qo_off + (uint32_t)(g * D * 2);
}

// One batch's K/V as the kernel reads it: byte strides relative to k/v, the
// descriptor range, the length.
struct KVSpan {
  const uint16_t* k;
  const uint16_t* v;
  uint32_t records;
  uint32_t row_bytes;
  uint32_t head_bytes;
  int S;
  // kLayoutPaged: this batch's block-table row, log2(page_size), page stride
  // in elements, bytes of one row (all heads).
  const int32_t* pages;
  uint32_t page_shift;
  uint64_t page_stride;
  uint32_t row_extent;
  // kLayoutPaged: pages[0], requested together with the length (every
  // block-table row has an entry 0), so that a batch in one page waits for
  // one round trip of scalar loads, not two.
  int32_t entry0;
};

__device__ __forceinline__ constexpr int ilog2(int x) { return x <= 1 ? 0 : 1 + ilog2(x >> 1); }

__device__ __forceinline__ bf16x2 as_bf16x2(uint32_t x) { return __builtin_bit_cast(bf16x2, x); }

// A value every lane reads at the same index, from memory no kernel writes
// while this one runs (the block table): read through the constant address
// space, it becomes a scalar load that the compiler issues ahead and batches,
// where a plain load of it is a vector load whose full wait also waits for
// every K/V request issued before it.
__device__ __forceinline__ int32_t load_uniform_i32(const int32_t* p, uint64_t idx) {
  typedef const __attribute__((address_space(4))) int32_t constant_i32;
  return ((constant_i32*)p)[idx];
}

// True when rows [0, S) of a batch (S <= 16) use a negative block-table
// entry: such a batch is invalid (NaN outputs, no row read).  entry0 is
// pages[0].
__device__ __forceinline__ bool paged_rows_unmapped(const int32_t* pages, int32_t entry0, int S,
                                                    uint32_t page_shift) {
  const int n = paged_entries_used(S, page_shift);
  int32_t sign = n > 0 ? entry0 : 0;
#pragma unroll
  for (int i = 1; i < kMaxSeq; ++i) sign |= i < n ? load_uniform_i32(pages, (uint32_t)i) : 0;
  return sign < 0;
}

__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, uint32_t num_bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)num_bytes, kBufferWord3);
}

// Cache-policy operand of the buffer instructions (gfx950: bit 0 sc0, bit 1
// nt, bit 4 sc1).
//   * K and V are read exactly once: non-temporal (streaming) loads, +12% on
//     MI355X over default-policy loads.  Adding sc0 or sc1 to them changes
//     nothing measurable.
//   * O is written exactly once: stored non-temporally at device scope
//     (nt | sc1), written through the XCD's L2 without being kept there.
//     Interleaved A/B on MI355X, µs per call, device scope alone vs nt|sc1:
//     B=30720 S=16 D=128 with Hq=Hkv=32: 1270 vs 1214; Hq=32 Hkv=16: 706
//     vs 640; Hq=64 Hkv=16: 812 vs 775; S=5 D=256 Hq=Hkv=16: 452 vs 416;
//     Hq=Hkv=32 D=256: 2508 vs 2469; Hq=Hkv=16 D=128 with four input sets
//     in rotation: 647 vs 628.  Device scope alone wins (by 1.5-3%) only
//     where all of O (126 MB) fits in the 256 MB MALL and the next call
//     rewrites the same buffer: the MALL then absorbs the rewrite.  The
//     data is visible to later kernels either way.
//   * Q keeps the default policy (a non-temporal Q load measured 4% slower).
constexpr int kPolicyDefault = 0;
constexpr int kPolicyStream = 2;
constexpr int kPolicyStreamStore = 2 | 16;

template <int POLICY>
__device__ __forceinline__ u32x4 buffer_load16(__amdgpu_buffer_rsrc_t r, uint32_t voffset) {
  u32x4_gcc x = __builtin_amdgcn_raw_buffer_load_b128(r, (int)voffset, 0, POLICY);
  return __builtin_bit_cast(u32x4, x);
}

__device__ __forceinline__ void buffer_store16(__amdgpu_buffer_rsrc_t r, uint32_t voffset, u32x4 x) {
  __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4_gcc, x), r, (int)voffset, 0, kPolicyStreamStore);
}

// ---------------------------------------------------------------------------
// Lane exchanges inside the group of LPH lanes that serves one KV head.
//
// The butterfly uses partner masks, in order, from {16, 8, 7, 2, 1} (the last
// log2(LPH) of them).  Mask m pairs lane i with lane i ^ m; its split bit is
// the top bit of m.  Every mask is zero on the split bits of earlier steps, so
// partners always hold the same subset of partial sums, and the masks are
// linearly independent, so the exchanges cover all LPH lanes.
//   16: lane i^16 (crosses the two 16-lane rows of a 32-lane group)
//    8: DPP row_ror:8        (i ^ 8 inside a 16-lane row)
//    7: DPP row_half_mirror  (i ^ 7 inside an 8-lane half row)
//    2: DPP quad_perm[2,3,0,1]
//    1: DPP quad_perm[1,0,3,2]
// ---------------------------------------------------------------------------
template <int LPH>
__device__ __forceinline__ constexpr int step_mask(int s) {
  constexpr int kMasks[5] = {16, 8, 7, 2, 1};
  return kMasks[5 - ilog2(LPH) + s];
}

template <int MASK>
__device__ __forceinline__ float lane_xchg(float x) {
  const int xi = __builtin_bit_cast(int, x);
  int y;
  if constexpr (MASK == 16) {
    y = __shfl_xor(xi, 16, kWaveSize);
  } else if constexpr (MASK == 8) {
    y = __builtin_amdgcn_mov_dpp(xi, 0x128, 0xf, 0xf, false);
  } else if constexpr (MASK == 7) {
    y = __builtin_amdgcn_mov_dpp(xi, 0x141, 0xf, 0xf, false);
  } else if constexpr (MASK == 2) {
    y = __builtin_amdgcn_mov_dpp(xi, 0x4e, 0xf, 0xf, false);
  } else {
    static_assert(MASK == 1, "unsupported lane mask");
    y = __builtin_amdgcn_mov_dpp(xi, 0xb1, 0xf, 0xf, false);
  }
  return __builtin_bit_cast(float, y);
}

template <int MASK>
__device__ __forceinline__ constexpr int split_bit() { return ilog2(MASK); }

// One butterfly step over N live partial sums: lanes whose split bit is 0
// keep x[0, N/2), the others keep x[N/2, N); both halves end compacted into
// x[0, N/2).  With N == 1 the step is a plain all-reduce of x[0].
template <int MASK, int N>
__device__ __forceinline__ void butterfly_step(float* x, int lane) {
  if constexpr (N == 1) {
    x[0] += lane_xchg<MASK>(x[0]);
  } else {
    const bool upper = (lane >> split_bit<MASK>()) & 1;
#pragma unroll
    for (int i = 0; i < N / 2; ++i) {
      const float a = x[i];
      const float b = x[i + N / 2];
      const float keep = upper ? b : a;
      const float send = upper ? a : b;
      x[i] = keep + lane_xchg<MASK>(send);
    }
  }
}

template <int LPH, int V, int S>
struct TransposeReduce {
  static __device__ __forceinline__ void run(float* x, int lane) {
    if constexpr (S < ilog2(LPH)) {
      constexpr int live = (V >> S) > 1 ? (V >> S) : 1;
      butterfly_step<step_mask<LPH>(S), live>(x, lane);
      TransposeReduce<LPH, V, S + 1>::run(x, lane);
    }
  }
};

// All-reduce (max or sum) over the lanes that differ only in the split bits
// of butterfly steps [FIRST, LAST).
template <int LPH, int FIRST, int LAST, bool IS_MAX>
struct GroupReduce {
  static __device__ __forceinline__ float run(float x) {
    if constexpr (FIRST < LAST) {
      const float y = lane_xchg<step_mask<LPH>(FIRST)>(x);
      x = IS_MAX ? fmaxf(x, y) : x + y;
      return GroupReduce<LPH, FIRST + 1, LAST, IS_MAX>::run(x);
    } else {
      return x;
    }
  }
};

// Partial dot products of this lane's 8 dims: x[g*NR + j] = q_g . k_j.
// Query heads at or past `active` (padding of a group size the kernel is
// not instantiated for; a wave-uniform value) get 0 without arithmetic.
template <int G, int NR>
__device__ __forceinline__ void partial_scores(const u32x4 (&qv)[G], const u32x4 (&kr)[NR], float* x,
                                               int active = G) {
#pragma unroll
  for (int g = 0; g < G; ++g) {
    if (g >= active) {
#pragma unroll
      for (int j = 0; j < NR; ++j) x[g * NR + j] = 0.0f;
      continue;
    }
#pragma unroll
    for (int j = 0; j < NR; ++j) {
      float acc = 0.0f;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const uint32_t qw = qv[g][i];
        const uint32_t kw = kr[j][i];
        acc = __builtin_amdgcn_fdot2_f32_bf16(as_bf16x2(qw), as_bf16x2(kw), acc, false);
      }
      x[g * NR + j] = acc;
    }
  }
}

// acc[g][d] += sum_j P_g,j * V_j[d] over NR rows, rows taken in pairs:
// pp[g][jp] holds the bf16 weights of rows 2jp (low half) and 2jp+1.
// Query heads at or past `active` (wave-uniform) are skipped.
template <int G, int NR>
__device__ __forceinline__ void accumulate_pv(const u32x4 (&vr)[NR], const uint32_t (&pp)[G][(NR + 1) / 2],
                                              float (&acc)[G][8], int active = G) {
  constexpr int NP = (NR + 1) / 2;
#pragma unroll
  for (int jp = 0; jp < NP; ++jp) {
    uint32_t lo[4], hi[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint32_t v0 = vr[2 * jp][i];
      const uint32_t v1 = (2 * jp + 1 < NR) ? (uint32_t)vr[(2 * jp + 1 < NR) ? 2 * jp + 1 : 0][i] : 0u;
      lo[i] = __builtin_amdgcn_perm(v1, v0, 0x05040100u);  // (V_j[2i],   V_j+1[2i])
      hi[i] = __builtin_amdgcn_perm(v1, v0, 0x07060302u);  // (V_j[2i+1], V_j+1[2i+1])
    }
#pragma unroll
    for (int g = 0; g < G; ++g) {
      if (g >= active) continue;
      const bf16x2 pw = as_bf16x2(pp[g][jp]);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        acc[g][2 * i] = __builtin_amdgcn_fdot2_f32_bf16(as_bf16x2(lo[i]), pw, acc[g][2 * i], false);
        acc[g][2 * i + 1] = __builtin_amdgcn_fdot2_f32_bf16(as_bf16x2(hi[i]), pw, acc[g][2 * i + 1], false);
      }
    }
  }
}

// Eight fp32 values -> eight fp16 (round to nearest even), packed.
__device__ __forceinline__ u32x4 pack_f16x8(const float (&a)[8]) {
  u32x4 out;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const uint32_t h0 = __builtin_bit_cast(uint16_t, (_Float16)a[2 * i]);
    const uint32_t h1 = __builtin_bit_cast(uint16_t, (_Float16)a[2 * i + 1]);
    out[i] = h0 | (h1 << 16);
  }
  return out;
}

// ---------------------------------------------------------------------------
// Scores and masked softmax of GH query heads (g0 .. g0+GH-1 of the wave's
// KV heads) against SMAX loaded K rows, the weights written to LDS slot
// [hkl][g*16 + j] of lds_p (bf16, or fp32 with PF32; VP slots per KV head).
// Each score is the tree sum of its lanes' partial dot products over the
// butterfly masks, whatever GH is; only the lanes that hold it afterwards,
// and so the order of the softmax sums, depend on GH.
// ---------------------------------------------------------------------------
template <int D, int GH, int SMAX, bool PF32, int VP>
__device__ __forceinline__ void score_softmax(const u32x4 (&qv)[GH], const u32x4 (&kr)[SMAX], int S, float scale,
                                              int lane, uint16_t* lds_p, int g0, int active) {
  constexpr int LPH = D / 8;                 // lanes per KV head
  constexpr int NS = ilog2(LPH);             // butterfly steps
  constexpr int V = GH * SMAX;               // scores per KV head
  constexpr int L = NS < ilog2(V) ? NS : ilog2(V);  // splitting steps
  constexpr int W = (V >> NS) > 1 ? (V >> NS) : 1;  // scores per lane after the butterfly
  constexpr int GS = W < SMAX ? W : SMAX;    // scores of one query head inside a lane
  constexpr int C = ilog2(SMAX / GS);        // steps spanning one query head's lanes
  const int r = lane % LPH;
  const int hkl = lane / LPH;

  // ---- partial scores over this lane's 8 dims ----
  float x[V];
  partial_scores<GH, SMAX>(qv, kr, x, active);

  // ---- reduce over the head's lanes; lane keeps scores [blk*W, blk*W + W) ----
  TransposeReduce<LPH, V, 0>::run(x, lane);
  const int blk = r >> (NS - L);

  // ---- masked softmax (per query head) ----
  float p[W];
#pragma unroll
  for (int h0 = 0; h0 < W; h0 += GS) {
    float t[GS];
    float m = -__builtin_inff();
#pragma unroll
    for (int w = 0; w < GS; ++w) {
      const int j = (W >= SMAX) ? w : ((blk & ((1 << C) - 1)) * W + w);
      const bool ok = j < S;
      t[w] = x[h0 + w] * scale;
      m = ok ? fmaxf(m, t[w]) : m;
    }
    m = GroupReduce<LPH, L - C, L, true>::run(m);
    float sum = 0.0f;
#pragma unroll
    for (int w = 0; w < GS; ++w) {
      const int j = (W >= SMAX) ? w : ((blk & ((1 << C) - 1)) * W + w);
      const bool ok = j < S;
      t[w] = ok ? expf(t[w] - m) : 0.0f;
      sum += t[w];
    }
    sum = GroupReduce<LPH, L - C, L, false>::run(sum);
#pragma unroll
    for (int w = 0; w < GS; ++w) p[h0 + w] = (sum > 0.0f) ? (t[w] / sum) : 0.0f;
  }

  if constexpr (!PF32) {
    // ---- bf16 weights -> LDS slot [hkl][g*16 + j] ----
    uint16_t* lds_head = lds_p + hkl * VP;
#pragma unroll
    for (int w = 0; w < W; ++w) {
      const int vi = blk * W + w;
      lds_head[(g0 + vi / SMAX) * kMaxSeq + vi % SMAX] = __builtin_bit_cast(uint16_t, (__bf16)p[w]);
    }
  } else {
    // ---- fp32 weights -> LDS slot [hkl][g*16 + j] (4 bytes each) ----
    float* lds_head = reinterpret_cast<float*>(lds_p) + hkl * VP;
#pragma unroll
    for (int w = 0; w < W; ++w) {
      const int vi = blk * W + w;
      lds_head[(g0 + vi / SMAX) * kMaxSeq + vi % SMAX] = p[w];
    }
  }
}

// ---------------------------------------------------------------------------
// Scores, masked softmax and P.V of one wave whose Q, K and V registers are
// loaded (rows >= S read as 0): S valid rows (per lane group when the
// groups serve different batches), weights through LDS slot
// [hkl][g*16 + j] of lds_p, fp32 result per query head in acc.  Query heads
// at or past `active` (the padding of a group size without its own
// instantiation; wave-uniform) are neither scored nor accumulated where the
// heads are scored in several passes; a kernel that scores them in one
// pass computes the padding heads too (their Q reads as 0, their O is
// dropped), which measured faster than testing for them inside the
// unrolled loops.
// ---------------------------------------------------------------------------
template <int D, int G, int SMAX, bool PF32, bool VARLEN>
__device__ __forceinline__ void decode_core(const u32x4 (&qv)[G], const u32x4 (&kr)[SMAX], const u32x4 (&vr)[SMAX],
                                            int S, float scale, int lane, uint16_t* lds_p, float (&acc)[G][8],
                                            int active_heads = G) {
  constexpr int LPH = D / 8;                 // lanes per KV head
  constexpr int VP = G * kMaxSeq;            // LDS slots per KV head
  // Query heads per score pass: 2 for G = 8 at D <= 128, which keeps 2/G of
  // the partial scores live at once (G = 8 with 16 rows: 32 instead of 128
  // registers, 200 VGPRs in all instead of 256) (µs, B=30720 Hkv=16 D=128,
  // 1 / 2 / 4 / 8 heads per pass: G=5 S=16 1155/831/860/857, G=7 S=16
  // 1299/932/927/919; Hq=40 Hkv=8 with Poisson(4) lengths 224/218/226/254;
  // one head per pass leaves too little independent work to hide the
  // exchanges' latency), and for G = 4 in the kernels that pick a bucket per
  // wave (Hq=64 Hkv=16 Poisson(4): 317 against 327 µs); all G otherwise
  // (G = 4, uniform lengths, µs with two / one heads per pass at each one's
  // best wave cap: G=3 S=4 284/262, S=8 441/418, G=4 S=16 795/782).
  constexpr int GH = D != 256 && (G == 8 || (G == 4 && VARLEN)) ? 2 : G;
  const int active = GH < G ? active_heads : G;
  const int hkl = lane / LPH;

#pragma unroll
  for (int g0 = 0; g0 < G; g0 += GH) {
    if (g0 >= active) break;
    u32x4 qs[GH];
#pragma unroll
    for (int i = 0; i < GH; ++i) qs[i] = qv[g0 + i];
    score_softmax<D, GH, SMAX, PF32, VP>(qs, kr, S, scale, lane, lds_p, g0, active - g0);
  }

#pragma unroll
  for (int g = 0; g < G; ++g)
#pragma unroll
    for (int d = 0; d < 8; ++d) acc[g][d] = 0.0f;

  if constexpr (!PF32) {
    uint16_t* lds_head = lds_p + hkl * VP;
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");

    // ---- P.V over row pairs ----
    constexpr int NP = (SMAX + 1) / 2;
    const uint32_t* lds_pairs = reinterpret_cast<const uint32_t*>(lds_head);
    uint32_t pp[G][NP];
#pragma unroll
    for (int g = 0; g < G; ++g) {
#pragma unroll
      for (int jp = 0; jp < NP; ++jp) {
        uint32_t w2 = lds_pairs[g * (kMaxSeq / 2) + jp];
        if constexpr (SMAX == 1) w2 &= 0xffffu;  // slot 1 is not part of this bucket
        pp[g][jp] = w2;
      }
    }
    accumulate_pv<G, SMAX>(vr, pp, acc, active);
  } else {
    const float* lds_head = reinterpret_cast<const float*>(lds_p) + hkl * VP;
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    // ---- P.V row by row in row order, one fused multiply-add per element ----
#pragma unroll
    for (int g = 0; g < G; ++g) {
      if (g >= active) continue;
#pragma unroll
      for (int j = 0; j < SMAX; ++j) {
        const float w = lds_head[g * kMaxSeq + j];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const uint32_t x = vr[j][i];
          acc[g][2 * i] = __builtin_fmaf(w, __builtin_bit_cast(float, x << 16), acc[g][2 * i]);
          acc[g][2 * i + 1] = __builtin_fmaf(w, __builtin_bit_cast(float, x & 0xffff0000u), acc[g][2 * i + 1]);
        }
      }
    }
  }

}

// ---------------------------------------------------------------------------
// The reference CPU loop's arithmetic, step for step (fmha_host.cpp:179-244):
// every score a float32 sum over dims 0, 1, ..., D-1 in order, each product
// exact (bf16 x bf16) and each addition rounded; scale; max; exponentials
// rounded once from a double evaluation; their sum in row order; IEEE
// division; the weight rounded to bf16; O a float32 sum over rows in order,
// each product exact, then rounded to fp16.  The outputs are the loop's bits
// wherever its expf returns the nearest float.
//
// A bf16 x bf16 product is exact in float32, so fma(x, y, acc) is the loop's
// acc + x * y with its one rounding.  (v_dot2_f32_bf16 with a zero partner
// is not: it differed from the loop on a few outputs per million at logit
// spreads of 2-4.)
//
// Data movement.  A score is a chain of D dependent additions, so the wave's
// G * SMAX scores per KV head are spread over the lanes as register blocks:
// a lane accumulates GB query heads x JB rows of one head (GB * JB = the
// wave's scores / 64 when there are more than 64), each chain in dim order,
// so every K value it reads and widens serves GB chains and every Q value
// JB.  The operands reach the lanes through LDS as loaded (bf16), or
// widened to float32 by all lanes while they are staged when a wave has at
// most 16 scores (then most lanes have no chain, and the chains do no
// widening; with more scores float32 staging measured slower, its LDS
// traffic doubled: 697 against 617 us at B=30720 H=16 S=16 D=128), NSTAGE
// stages of D / NSTAGE dims each, which keeps the staging small enough for
// the waves per CU the stream needs:
//   * K: lane r of a head owns 16-byte chunk r of each row as loaded, so for
//     the staging its register slot j is loaded with row
//     NSTAGE * (j / NSTAGE) + (j + r / CH) % NSTAGE, chunk
//     CH * (j % NSTAGE) + r % CH (CH = chunks per stage): slot j belongs to
//     stage j % NSTAGE in every lane, every lane writes SMAX / NSTAGE rows in
//     each stage, and the slots of a stage are dead once it is written;
//   * Q: lane r writes its chunk of each query head in stage r / CH;
//   * LDS rows are padded by 16 bytes and heads by the closed form below, so
//     the block reads of each 16-lane group fall in distinct bank groups.
// Softmax: SMAX consecutive lanes per (head, query head) take the max by a
// lane exchange and the sum of exponentials as a sequential read of SMAX
// values from LDS.  P.V: one fma per output element and row, rows in order.
// ---------------------------------------------------------------------------

template <int D, int G, int SMAX, int NSTAGE>
struct ExactLayout {
  static constexpr int LPH = D / 8;
  static constexpr int HPW = kWaveSize / LPH;
  static constexpr int CH = LPH / NSTAGE;       // 16-byte bf16 chunks per row and stage
  static constexpr int N = HPW * G * SMAX;      // scores of the wave
  // At most a quarter wave of scores: the operands are staged widened to
  // float32 (WIDE), by every lane, so that the few lanes with a chain do no
  // widening in it; else as loaded (bf16), widened in the chains.  (Half a
  // wave, widened, measured no faster and took 202 VGPRs against 151 at
  // D = 256 with 16 rows.)
  static constexpr bool WIDE = N <= kWaveSize / 4;
  static constexpr int RB = CH * (WIDE ? 32 : 16) + 16;  // LDS bytes per staged row (K row or query)
  static constexpr int BL = N > kWaveSize ? N / kWaveSize : 1;  // scores per lane
  static constexpr int gb_for() {
    int gb = 1;
    while (gb * 2 <= G && gb * 2 * gb * 2 <= BL) gb *= 2;
    return BL / gb > SMAX ? BL / SMAX : gb;
  }
  static constexpr int GB = gb_for();           // query heads per block
  static constexpr int JB = BL / GB;            // rows per block
  static constexpr int GBN = G / GB;            // blocks across the query heads
  static constexpr int JBN = SMAX / JB;         // blocks across the rows
  static constexpr int NB = N / BL;             // blocks (<= 64, one per lane)
  // Head stride of the K rows in 16-byte units = JBN mod 16: the JBN rows of
  // consecutive heads that one 16-lane read touches start in distinct bank
  // groups (the row stride, RB / 16 units, is odd).
  static constexpr int KH = SMAX * RB + 16 * ((JBN - SMAX * (RB / 16) % 16 + 16) % 16);
  static constexpr int QH = G * RB;
  static constexpr int K_BYTES = HPW * KH;
  static constexpr int Q_BYTES = HPW * QH;
  static constexpr int E_BYTES = N * 4;
  static constexpr int BYTES = K_BYTES + Q_BYTES + E_BYTES;
  static_assert(LPH % NSTAGE == 0 && (SMAX % NSTAGE == 0 || SMAX == 1) && CH % 2 == 0,
                "stages must split the chunks and rows, an even number of chunks each");
  static_assert(GB * JB == BL && G % GB == 0 && SMAX % JB == 0 && NB <= kWaveSize, "score blocks");
};

// Staging budget per wave: the fewest stages (1, 2 or 4; at most the
// bucket's rows, an even number of chunks each) whose LDS stays within it.
// 12 KiB for one or two query heads per KV head, which leaves room for the
// 12-16 waves per CU that short and varying rows want (B=30720 with the
// reference's Poisson lengths: 198 / 194 us at 12 / 16 waves against 232 at
// 8), 24 KiB for wider groups, whose caps are 4-6 waves.
template <int D, int G, int SMAX>
__device__ __forceinline__ constexpr int exact_stages() {
  constexpr int budget = G <= 2 ? 12 * 1024 : 24 * 1024;
  constexpr int lph = D / 8;
  if constexpr (SMAX <= 1) {
    return 1;
  } else if constexpr (ExactLayout<D, G, SMAX, 1>::BYTES <= budget) {
    return 1;
  } else if constexpr (SMAX < 4 || lph < 8 || ExactLayout<D, G, SMAX, 2>::BYTES <= budget) {
    return 2;
  } else {
    return 4;
  }
}

// K register slot j of lane r (r < D/8): the row it is loaded with, and the
// 16-byte chunk of that row, for NSTAGE stages.  With one stage these are j
// and r, the plain load.
template <int D, int NSTAGE>
__device__ __forceinline__ int exact_k_row(int r, int j) {
  constexpr int CH = D / 8 / NSTAGE;
  return NSTAGE * (j / NSTAGE) + (j % NSTAGE + r / CH) % NSTAGE;
}

template <int D, int NSTAGE>
__device__ __forceinline__ int exact_k_chunk(int r, int j) {
  constexpr int CH = D / 8 / NSTAGE;
  return CH * (j % NSTAGE) + r % CH;
}

// One loaded 16-byte chunk (8 bf16) into the staging: as it is, or widened
// to 8 float32 (WIDE).
template <bool WIDE>
__device__ __forceinline__ void stage_chunk(unsigned char* dst, const u32x4 x) {
  if constexpr (WIDE) {
    *reinterpret_cast<u32x4*>(dst) = u32x4{x[0] << 16, x[0] & 0xffff0000u, x[1] << 16, x[1] & 0xffff0000u};
    *reinterpret_cast<u32x4*>(dst + 16) = u32x4{x[2] << 16, x[2] & 0xffff0000u, x[3] << 16, x[3] & 0xffff0000u};
  } else {
    *reinterpret_cast<u32x4*>(dst) = x;
  }
}

// The 8 dims of staged chunk c of a row as float32.
template <bool WIDE>
__device__ __forceinline__ void staged_dims(const unsigned char* row, int c, float (&f)[8]) {
  if constexpr (WIDE) {
    const float4 a = *reinterpret_cast<const float4*>(row + c * 32);
    const float4 b = *reinterpret_cast<const float4*>(row + c * 32 + 16);
    f[0] = a.x; f[1] = a.y; f[2] = a.z; f[3] = a.w;
    f[4] = b.x; f[5] = b.y; f[6] = b.z; f[7] = b.w;
  } else {
    const u32x4 x = *reinterpret_cast<const u32x4*>(row + c * 16);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const uint32_t w = x[e];
      f[2 * e] = __builtin_bit_cast(float, w << 16);
      f[2 * e + 1] = __builtin_bit_cast(float, w & 0xffff0000u);
    }
  }
}

// lds: LDS of the weights (VP bf16 slots per KV head, as decode_core), then
// ExactLayout::BYTES of staging.  kr: slot j as exact_k_row/exact_k_chunk
// say.  GROUP_S: the lane groups serve different batches, so a score lane
// takes the length of the head it scores from that head's lanes.
template <int D, int G, int SMAX, int NSTAGE, bool GROUP_S>
__device__ __forceinline__ void decode_core_exact(const u32x4 (&qv)[G], const u32x4 (&kr)[SMAX],
                                                  const u32x4 (&vr)[SMAX], int S, float scale, int lane,
                                                  uint16_t* lds_p, float (&acc)[G][8]) {
  // Every multiply and add below rounds on its own, as in the loop restated
  // (the compiler would otherwise fuse t = s * scale into t - max).
#pragma clang fp contract(off)
  using L = ExactLayout<D, G, SMAX, NSTAGE>;
  constexpr int LPH = L::LPH;
  constexpr int CH = L::CH;
  constexpr int RB = L::RB;
  constexpr int VP = G * kMaxSeq;
  constexpr int N = L::N;
  constexpr int NSLOT = (N + kWaveSize - 1) / kWaveSize;
  // Softmax slots unrolled when a lane has at most two of them; rolled
  // above, which keeps one score's registers live instead of NSLOT's.
  constexpr int SLOT_UNROLL = NSLOT <= 2 ? NSLOT : 1;
  constexpr int CH_UNROLL = CH < 4 ? CH : 4;
  constexpr int RS = ilog2(SMAX);               // row steps of the max exchange
  unsigned char* ks = reinterpret_cast<unsigned char*>(lds_p + L::HPW * VP);
  unsigned char* qz = ks + L::K_BYTES;
  float* es = reinterpret_cast<float*>(qz + L::Q_BYTES);
  const int r = lane % LPH;
  const int hkl = lane / LPH;
  const int u = r / CH;                         // the stage of this lane's own chunk

  // ---- this lane's block: head bh, query heads bg + i GBN, rows bj + t JBN ----
  const int bj = lane % L::JBN;
  const int bg = (lane / L::JBN) % L::GBN;
  const int bh = lane / (L::JBN * L::GBN);
  const bool has_block = lane < L::NB;
  float sacc[L::GB][L::JB];
#pragma unroll
  for (int i = 0; i < L::GB; ++i)
#pragma unroll
    for (int t = 0; t < L::JB; ++t) sacc[i][t] = 0.0f;

#pragma unroll
  for (int st = 0; st < NSTAGE; ++st) {
    if (st > 0) {  // every lane is done reading the previous stage
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    }
    // ---- stage st: K slots st, st + NSTAGE, ... and this lane's Q chunks ----
    // ---- (when they belong here), widened to float32                     ----
    constexpr int CB = L::WIDE ? 32 : 16;       // staged bytes per chunk
#pragma unroll
    for (int j = st; j < SMAX; j += NSTAGE)
      stage_chunk<L::WIDE>(ks + hkl * L::KH + exact_k_row<D, NSTAGE>(r, j) * RB + (r % CH) * CB, kr[j]);
    if (u == st) {
#pragma unroll
      for (int g = 0; g < G; ++g) stage_chunk<L::WIDE>(qz + hkl * L::QH + g * RB + (r % CH) * CB, qv[g]);
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    // ---- this stage's dims of the lane's block, in dim order ----
    if (has_block) {
      const unsigned char* kb = ks + bh * L::KH + bj * RB;
      const unsigned char* qb = qz + bh * L::QH + bg * RB;
      // (unrolled by at most 4: unrolled in full, the compiler hoists every
      // read of the loop and spills at D = 256)
#pragma unroll CH_UNROLL
      for (int c = 0; c < CH; ++c) {
        // 8 dims of the block's query heads and rows, widened once each
        float qf[L::GB][8], kf[L::JB][8];
#pragma unroll
        for (int i = 0; i < L::GB; ++i) staged_dims<L::WIDE>(qb + i * L::GBN * RB, c, qf[i]);
#pragma unroll
        for (int t = 0; t < L::JB; ++t) staged_dims<L::WIDE>(kb + t * L::JBN * RB, c, kf[t]);
#pragma unroll
        for (int i = 0; i < L::GB; ++i)
#pragma unroll
          for (int t = 0; t < L::JB; ++t) {
            float a = sacc[i][t];
#pragma unroll
            for (int e = 0; e < 8; ++e) a = __builtin_fmaf(qf[i][e], kf[t][e], a);
            sacc[i][t] = a;
          }
      }
    }
  }
  // ---- the scores, [head][query head][row] ----
  if (has_block) {
#pragma unroll
    for (int i = 0; i < L::GB; ++i)
#pragma unroll
      for (int t = 0; t < L::JB; ++t) es[(bh * G + bg + i * L::GBN) * SMAX + bj + t * L::JBN] = sacc[i][t];
  }
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");

  // ---- softmax: score sigma = lane + 64 sl; max over the pair's SMAX ----
  // ---- lanes (every lane takes part in the exchange), the exponential ----
  // ---- back into es[sigma]                                           ----
#pragma unroll SLOT_UNROLL
  for (int sl = 0; sl < NSLOT; ++sl) {
    const int sigma = lane + kWaveSize * sl;
    const bool in = sigma < N;
    const int c = sigma / SMAX;
    const int h = in ? c / G : 0;
    const int Sh = GROUP_S ? __shfl(S, h * LPH, kWaveSize) : S;
    const bool valid = in && sigma % SMAX < Sh;
    const float t = (in ? es[sigma] : 0.0f) * scale;
    float m = valid ? t : -__builtin_inff();
    m = GroupReduce<SMAX, 0, RS, true>::run(m);
    const float e = valid ? (float)exp((double)(t - m)) : 0.0f;
    if (in) es[sigma] = e;
  }
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  // ---- the sum in row order, the quotient, the bf16 weight ----
  // (an invalid row's exponential is +0: with at least one valid row the
  // sum is >= 1 and its weight +0; with none the sum is 0 and so is every
  // weight)
#pragma unroll SLOT_UNROLL
  for (int sl = 0; sl < NSLOT; ++sl) {
    const int sigma = lane + kWaveSize * sl;
    if (sigma < N) {
      const int c = sigma / SMAX;
      const float* row = es + c * SMAX;
      float sum = 0.0f;
#pragma unroll
      for (int jj = 0; jj < SMAX; ++jj) sum += row[jj];
      const float e = row[sigma % SMAX];
      const float p = sum > 0.0f ? e / sum : 0.0f;
      lds_p[(c / G) * VP + (c % G) * kMaxSeq + sigma % SMAX] = __builtin_bit_cast(uint16_t, (__bf16)p);
    }
  }
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");

  // ---- P.V: rows in order, one exact product per element and row ----
  // (rows at or past S have weight 0 and V 0: adding +0 changes nothing)
  const uint16_t* wrow = lds_p + hkl * VP;
#pragma unroll
  for (int g = 0; g < G; ++g) {
#pragma unroll
    for (int d = 0; d < 8; ++d) acc[g][d] = 0.0f;
    uint32_t w2[(SMAX + 1) / 2];
#pragma unroll
    for (int jp = 0; jp < (SMAX + 1) / 2; ++jp) w2[jp] = reinterpret_cast<const uint32_t*>(wrow + g * kMaxSeq)[jp];
#pragma unroll
    for (int j = 0; j < SMAX; ++j) {
      const float wf = __builtin_bit_cast(float, j % 2 == 0 ? w2[j / 2] << 16 : w2[j / 2] & 0xffff0000u);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const uint32_t vp = vr[j][i];
        acc[g][2 * i] = __builtin_fmaf(wf, __builtin_bit_cast(float, vp << 16), acc[g][2 * i]);
        acc[g][2 * i + 1] = __builtin_fmaf(wf, __builtin_bit_cast(float, vp & 0xffff0000u), acc[g][2 * i + 1]);
      }
    }
    // The sums leave as float32 values: without this the compiler fuses the
    // last multiply-add with the caller's fp16 conversion (v_fma_mix), one
    // rounding where the loop restated has two.
#pragma unroll
    for (int d = 0; d < 8; ++d) asm volatile("" : "+v"(acc[g][d]));
  }
}

// Whether a bucket takes the exact path: kernels instantiated for it (bf16
// weights, any of the VALU kernel's group sizes) and more than one row (one
// row has weight 1 and output fp16(V) on either path).
template <int G, int SMAX, bool PF32, bool EXACT>
__device__ __forceinline__ constexpr bool exact_taken() {
  static_assert(!EXACT || !PF32, "the exact path rounds the weights to bf16");
  return EXACT && SMAX > 1;
}

// LDS bytes past the weights that the exact path of buckets 2 .. SMAX_TOP
// stages through (0 when no bucket takes it).
template <int D, int G, int SMAX_TOP, bool PF32, bool VARLEN, bool EXACT>
__device__ __forceinline__ constexpr int exact_extra_bytes() {
  if constexpr (!exact_taken<G, SMAX_TOP, PF32, EXACT>()) {
    return 0;
  } else {
    int m = ExactLayout<D, G, SMAX_TOP, exact_stages<D, G, SMAX_TOP>()>::BYTES;
    if constexpr (VARLEN && SMAX_TOP > 2) {
      const int n = exact_extra_bytes<D, G, SMAX_TOP / 2, PF32, VARLEN, EXACT>();
      m = n > m ? n : m;
    }
    return m;
  }
}

// The row K slot j of lane r is loaded with (j itself outside the exact path).
template <int D, int G, int SMAX, bool PF32, bool EXACT>
__device__ __forceinline__ int exact_k_row_of(int r, int j) {
  if constexpr (exact_taken<G, SMAX, PF32, EXACT>()) return exact_k_row<D, exact_stages<D, G, SMAX>()>(r, j);
  return j;
}

// Byte offset of the K chunk slot j of lane r loads, relative to chunk r.
template <int D, int G, int SMAX, bool PF32, bool EXACT>
__device__ __forceinline__ uint32_t exact_k_delta(int r, int j) {
  if constexpr (exact_taken<G, SMAX, PF32, EXACT>())
    return (uint32_t)((exact_k_chunk<D, exact_stages<D, G, SMAX>()>(r, j) - r) * 16);
  return 0u;
}

// decode_core, or the exact core for the buckets that take it.
template <int D, int G, int SMAX, bool PF32, bool GROUP_S, bool VARLEN, bool EXACT>
__device__ __forceinline__ void decode_core_any(const u32x4 (&qv)[G], const u32x4 (&kr)[SMAX],
                                                const u32x4 (&vr)[SMAX], int S, float scale, int lane,
                                                uint16_t* lds_p, float (&acc)[G][8], int active) {
  if constexpr (exact_taken<G, SMAX, PF32, EXACT>()) {
    decode_core_exact<D, G, SMAX, exact_stages<D, G, SMAX>(), GROUP_S>(qv, kr, vr, S, scale, lane, lds_p, acc);
  } else {
    decode_core<D, G, SMAX, PF32, VARLEN>(qv, kr, vr, S, scale, lane, lds_p, acc, active);
  }
}

// ---------------------------------------------------------------------------
// One wave, one (batch, group of HPW KV heads), KV bucket SMAX >= S.
// ---------------------------------------------------------------------------
template <int D, int G, int SMAX, int LAYOUT, bool PF32, bool VARLEN, bool EXACT>
__device__ __forceinline__ void decode_unit(const DecodeArgs& a, uint32_t b, const KVSpan& kv, int hk,
                                            bool head_ok, int lane, uint16_t* lds_p) {
  constexpr int LPH = D / 8;  // lanes per KV head
  const int r = lane % LPH;
  const int hq_count = a.num_heads_q;

  const int S = kv.S;
  // ---- buffer resources and per-lane byte offsets ----
  const uint32_t q_bytes = (uint32_t)hq_count * D * 2;
  const __amdgpu_buffer_rsrc_t q_rsrc = make_rsrc(a.q + (uint64_t)b * hq_count * D, q_bytes);
  const __amdgpu_buffer_rsrc_t o_rsrc = make_rsrc(a.o + (uint64_t)b * hq_count * D, q_bytes);
  const __amdgpu_buffer_rsrc_t k_rsrc = make_rsrc(kv.k, kv.records);
  const __amdgpu_buffer_rsrc_t v_rsrc = make_rsrc(kv.v, kv.records);

  const uint32_t kv_off = head_ok ? (uint32_t)hk * kv.head_bytes + (uint32_t)r * 16u : kLaneOutOfRange;
  const int grp = G >= 4 ? a.group : G;
  const uint32_t qo_off = head_ok ? (uint32_t)(hk * grp * D + r * 8) * 2u : kLaneOutOfRange;
  // Row j's byte offset.  Packed rows past S already fall outside the
  // descriptor's range; a strided batch's range can include padding rows of
  // other heads, so there rows at or past S are moved out of range.
  uint32_t row_off[SMAX];
  row_off[0] = 0;
#pragma unroll
  for (int j = 1; j < SMAX; ++j) row_off[j] = row_off[j - 1] + kv.row_bytes;
  if constexpr (LAYOUT == kLayoutStrided) {
#pragma unroll
    for (int j = 0; j < SMAX; ++j) row_off[j] = j < S ? row_off[j] : kRowOutOfRange;
  }

  // ---- issue every load of this unit ----
  u32x4 qv[G];
#pragma unroll
  for (int g = 0; g < G; ++g) qv[g] = buffer_load16<kPolicyDefault>(q_rsrc, group_row_off<G>(qo_off, g, grp, D));
  u32x4 kr[SMAX];
  u32x4 vr[SMAX];
  if constexpr (LAYOUT != kLayoutPaged) {
#pragma unroll
    for (int j = 0; j < SMAX; ++j) {
      // The exact path loads K slot j with another row and chunk (the same
      // row and chunk r elsewhere).
      const int jr = exact_k_row_of<D, G, SMAX, PF32, EXACT>(r, j);
      const uint32_t roff = jr == j ? row_off[j]
                            : (LAYOUT == kLayoutStrided && jr >= S) ? kRowOutOfRange
                                                                    : (uint32_t)jr * kv.row_bytes;
      kr[j] = buffer_load16<kPolicyStream>(
          k_rsrc, kv_off + roff + (head_ok ? exact_k_delta<D, G, SMAX, PF32, EXACT>(r, j) : 0u));
    }
#pragma unroll
    for (int j = 0; j < SMAX; ++j) vr[j] = buffer_load16<kPolicyStream>(v_rsrc, kv_off + row_off[j]);
  } else if (kv.page_shift >= 4) {
    static_assert(!exact_taken<G, SMAX, PF32, EXACT>(), "the exact path reads the packed and strided layouts");
    // Pages of 16 rows or more: rows [0, S) (S <= 16) are slots 0..S-1 of
    // the batch's first page, one after another, so one entry and one
    // descriptor per batch cover them (empty for an unmapped entry or S =
    // 0; rows past S fall outside it and read 0 without access).
    const int32_t entry = S > 0 ? kv.entry0 : -1;
    const int64_t el = paged_row_elem(entry, 0u, kv.page_shift, kv.page_stride, kv.row_bytes >> 1);
    const uint64_t base = el < 0 ? 0u : (uint64_t)el;
    const uint32_t rec = el < 0 || S <= 0 ? 0u : (uint32_t)(S - 1) * kv.row_bytes + kv.row_extent;
    const __amdgpu_buffer_rsrc_t kp = make_rsrc(kv.k + base, rec);
    const __amdgpu_buffer_rsrc_t vp = make_rsrc(kv.v + base, rec);
#pragma unroll
    for (int j = 0; j < SMAX; ++j) kr[j] = buffer_load16<kPolicyStream>(kp, kv_off + row_off[j]);
#pragma unroll
    for (int j = 0; j < SMAX; ++j) vr[j] = buffer_load16<kPolicyStream>(vp, kv_off + row_off[j]);
  } else {
    // Row j sits in page pages[j >> page_shift] at slot j & (page_size-1):
    // one descriptor per row, spanning that row's heads, empty past S and
    // for an unmapped (negative) entry; rows past S read no entry.  The
    // caller has already turned a batch with an unmapped row into NaN, so
    // the empty range for one is a second guard.
    uint64_t row_elem[SMAX];
    uint32_t row_rec[SMAX];
#pragma unroll
    for (int j = 0; j < SMAX; ++j) {
      const int32_t entry = j < S ? load_uniform_i32(kv.pages, (uint32_t)j >> kv.page_shift) : -1;
      const int64_t el = paged_row_elem(entry, (uint32_t)j, kv.page_shift, kv.page_stride, kv.row_bytes >> 1);
      row_elem[j] = el < 0 ? 0u : (uint64_t)el;
      row_rec[j] = el < 0 ? 0u : kv.row_extent;
    }
    static_assert(!exact_taken<G, SMAX, PF32, EXACT>(), "the exact path reads the packed and strided layouts");
#pragma unroll
    for (int j = 0; j < SMAX; ++j)
      kr[j] = buffer_load16<kPolicyStream>(make_rsrc(kv.k + row_elem[j], row_rec[j]), kv_off);
#pragma unroll
    for (int j = 0; j < SMAX; ++j)
      vr[j] = buffer_load16<kPolicyStream>(make_rsrc(kv.v + row_elem[j], row_rec[j]), kv_off);
  }
  // Keep the scheduler from sinking loads into the arithmetic below: all
  // 1 + 2*SMAX requests of the unit are in flight before the first wait.
  __builtin_amdgcn_sched_barrier(0);

  float acc[G][8];
  decode_core_any<D, G, SMAX, PF32, false, VARLEN, EXACT>(qv, kr, vr, S, a.scale, lane, lds_p, acc, grp);

  // ---- fp16 (RNE) output, 16 bytes per lane per query head ----
#pragma unroll
  for (int g = 0; g < G; ++g) buffer_store16(o_rsrc, group_row_off<G>(qo_off, g, grp, D), pack_f16x8(acc[g]));
}

// Batches whose length is outside [0, max_rows] get NaN outputs so that a
// broken length table is visible in the result.
template <int D, int G>
__device__ __forceinline__ void decode_bad_length(const DecodeArgs& a, uint32_t b, int hk, bool head_ok, int lane) {
  constexpr int LPH = D / 8;
  const int r = lane % LPH;
  const uint32_t q_bytes = (uint32_t)a.num_heads_q * D * 2;
  const __amdgpu_buffer_rsrc_t o_rsrc = make_rsrc(a.o + (uint64_t)b * a.num_heads_q * D, q_bytes);
  const int grp = G >= 4 ? a.group : G;
  const uint32_t qo_off = head_ok ? (uint32_t)(hk * grp * D + r * 8) * 2u : kLaneOutOfRange;
  const u32x4 nan4 = {0x7e007e00u, 0x7e007e00u, 0x7e007e00u, 0x7e007e00u};
#pragma unroll
  for (int g = 0; g < G; ++g) buffer_store16(o_rsrc, group_row_off<G>(qo_off, g, grp, D), nan4);
}

// This batch's K/V span for the layout.  Returns false when the batch's
// length is outside [0, max_rows] (the caller then writes NaN).
template <int D, int LAYOUT, bool UNIFORM>
__device__ __forceinline__ bool batch_span(const DecodeArgs& a, uint32_t b, KVSpan& kv) {
  int S;
  uint64_t elem0;
  if constexpr (LAYOUT == kLayoutPacked) {
    int64_t row0;
    if constexpr (UNIFORM) {
      S = a.seqlen_uniform;
      row0 = (int64_t)b * S;
    } else {
      row0 = a.lens[b];
      S = a.lens[b + 1] - (int)row0;
    }
    elem0 = (uint64_t)row0 * (uint64_t)a.row_stride;
  } else if constexpr (LAYOUT == kLayoutStrided) {
    S = UNIFORM ? a.seqlen_uniform : a.lens[b];
    elem0 = (uint64_t)b * (uint64_t)a.batch_stride;
  } else {
    kv.pages = a.block_table + (uint64_t)b * a.bt_stride;
    kv.entry0 = load_uniform_i32(kv.pages, 0);
    S = a.lens[b];
    elem0 = 0;
    kv.page_shift = (uint32_t)a.seqlen_uniform;  // log2(page_size) for this layout
    kv.page_stride = (uint64_t)a.batch_stride;
    kv.row_extent = ((uint32_t)(a.num_heads_kv - 1) * (uint32_t)a.head_stride + D) * 2u;
  }
  if (S < 0 || S > a.max_rows) return false;
  kv.k = a.k + elem0;
  kv.v = a.v + elem0;
  kv.S = S;
  kv.row_bytes = (uint32_t)a.row_stride * 2u;
  kv.head_bytes = (uint32_t)a.head_stride * 2u;
  // Range of the descriptor: up to the last valid row's last head.
  if constexpr (LAYOUT == kLayoutStrided) {
    kv.records = S == 0 ? 0u
                        : ((uint32_t)(S - 1) * (uint32_t)a.row_stride +
                           (uint32_t)(a.num_heads_kv - 1) * (uint32_t)a.head_stride + D) * 2u;
  } else {
    kv.records = (uint32_t)S * kv.row_bytes;  // rows are [Hkv, D] and contiguous
  }
  return true;
}

// SB = 1, 2, 4, 8, 16: every batch has exactly seqlen_uniform <= SB rows.
// SB = 0: lengths come from a.lens and each wave picks the smallest bucket
// that holds its batch.
// PF32: softmax weights kept in fp32 and P.V as one fused multiply-add per
// row in row order (the semantics of the reference's fmha_vectorized_fma,
// fmha_vectorized_fma_kernel.hpp:243-296); otherwise weights rounded to bf16
// (the reference CPU loop and fmha_mfma_4x4x4).
template <int D, int G, int LAYOUT, int SB, bool PF32 = false, bool EXACT = false>
__global__ __launch_bounds__(kBlockThreads) void fmha_decode_fwd_kernel(DecodeArgs a) {
  constexpr int LPH = D / 8;
  constexpr int HPW = kWaveSize / LPH;
  constexpr int VP = G * kMaxSeq;
  constexpr int WB = PF32 ? 2 : 1;  // 16-bit LDS words per weight
  constexpr int XW = exact_extra_bytes<D, G, SB == 0 ? kMaxSeq : SB, PF32, SB == 0, EXACT>() / 2;  // exact staging
  __shared__ __attribute__((aligned(16))) uint16_t lds_p[kWavesPerBlock * (HPW * VP * WB + XW)];

  const int lane = threadIdx.x & (kWaveSize - 1);
  const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWaveSize);
  const uint32_t unit = blockIdx.x * kWavesPerBlock + wave;
  if (unit >= a.total_units) return;
  const uint32_t upb = (uint32_t)a.units_per_batch;
  const uint32_t b = unit / upb;
  const uint32_t hg = unit - b * upb;
  const int hk = (int)hg * HPW + lane / LPH;
  const bool head_ok = hk < a.num_heads_kv;
  uint16_t* lds_wave = lds_p + wave * (HPW * VP * WB + XW);

  if constexpr (SB == 0 && LAYOUT == kLayoutPacked) report_mean_rows(a, unit, a.total_units / upb, lane);
  if constexpr (LAYOUT == kLayoutPaged) report_mean_rows_sample(a, unit, a.total_units / upb, lane);
  KVSpan kv;
  const bool length_ok = batch_span<D, LAYOUT, SB != 0>(a, b, kv);
  // A uniform length was validated on the host; only table lengths can be
  // bad, and on a paged cache a negative block-table entry for a row the
  // batch has.
  bool valid = length_ok;
  if constexpr (LAYOUT == kLayoutPaged)
    valid = valid && !paged_rows_unmapped(kv.pages, kv.entry0, kv.S, kv.page_shift);
  if (SB == 0 && !valid) {
    decode_bad_length<D, G>(a, b, hk, head_ok, lane);
    return;
  }
  if constexpr (SB != 0) {
    decode_unit<D, G, SB, LAYOUT, PF32, false, EXACT>(a, b, kv, hk, head_ok, lane, lds_wave);
  } else {
    const int S = kv.S;
    if (S <= 1) {
      decode_unit<D, G, 1, LAYOUT, PF32, true, EXACT>(a, b, kv, hk, head_ok, lane, lds_wave);
    } else if (S <= 2) {
      decode_unit<D, G, 2, LAYOUT, PF32, true, EXACT>(a, b, kv, hk, head_ok, lane, lds_wave);
    } else if (S <= 4) {
      decode_unit<D, G, 4, LAYOUT, PF32, true, EXACT>(a, b, kv, hk, head_ok, lane, lds_wave);
    } else if (S <= 8) {
      decode_unit<D, G, 8, LAYOUT, PF32, true, EXACT>(a, b, kv, hk, head_ok, lane, lds_wave);
    } else {
      decode_unit<D, G, 16, LAYOUT, PF32, true, EXACT>(a, b, kv, hk, head_ok, lane, lds_wave);
    }
  }
}

// ---------------------------------------------------------------------------
// Batches with fewer KV heads than a wave holds (Hkv < HPW = 64 / (D/8),
// HPW a multiple of Hkv: MQA, or GQA after tensor-parallel sharding).  One
// (batch, head group) per wave would leave 1 - Hkv/HPW of the lanes idle;
// here the HPW lane groups serve R = HPW / Hkv consecutive batches, all Hkv
// heads of each (lane group hkl: batch b0 + hkl / Hkv, head hkl % Hkv).
// Packed and strided layouts: one descriptor spans the R batches' rows, each
// lane group offsets its own batch's rows and ends them at its own length.
// The KV bucket is the longest of the R lengths; arithmetic, numerics and
// the NaN of an invalid length are those of fmha_decode_fwd_kernel.
// ---------------------------------------------------------------------------

// One wave of R batches, bucket SMAX.  kbase/vbase: the wave's first batch;
// records: the descriptor range over the R batches; lane_rows: byte offset
// of this lane group's batch from kbase; S: its length (0 when invalid).
template <int D, int G, int SMAX, bool PF32, bool EXACT>
__device__ __forceinline__ void decode_multi_unit(const DecodeArgs& a, uint32_t b0, uint32_t nb, const uint16_t* kbase,
                                                  const uint16_t* vbase, uint32_t records, uint32_t lane_rows, int S,
                                                  bool bad, bool lane_ok, int sub, int hk, int lane,
                                                  uint16_t* lds_p) {
  constexpr int LPH = D / 8;
  const int r = lane % LPH;
  const int hq = a.num_heads_q;
  const uint32_t q_bytes = nb * (uint32_t)hq * D * 2u;
  const __amdgpu_buffer_rsrc_t q_rsrc = make_rsrc(a.q + (uint64_t)b0 * hq * D, q_bytes);
  const __amdgpu_buffer_rsrc_t o_rsrc = make_rsrc(a.o + (uint64_t)b0 * hq * D, q_bytes);
  const __amdgpu_buffer_rsrc_t k_rsrc = make_rsrc(kbase, records);
  const __amdgpu_buffer_rsrc_t v_rsrc = make_rsrc(vbase, records);
  const uint32_t row_bytes = (uint32_t)a.row_stride * 2u;
  const int grp = G >= 4 ? a.group : G;
  const uint32_t qo_off =
      lane_ok ? (uint32_t)sub * (uint32_t)hq * D * 2u + (uint32_t)(hk * grp * D + r * 8) * 2u : kLaneOutOfRange;
  const uint32_t kv_off =
      lane_ok ? lane_rows + (uint32_t)hk * (uint32_t)a.head_stride * 2u + (uint32_t)r * 16u : kLaneOutOfRange;
  // Rows at or past this lane group's own length are moved out of range.
  uint32_t row_off[SMAX];
#pragma unroll
  for (int j = 0; j < SMAX; ++j) row_off[j] = j < S ? (uint32_t)j * row_bytes : kRowOutOfRange;

  u32x4 qv[G];
#pragma unroll
  for (int g = 0; g < G; ++g) qv[g] = buffer_load16<kPolicyDefault>(q_rsrc, group_row_off<G>(qo_off, g, grp, D));
  u32x4 kr[SMAX];
  u32x4 vr[SMAX];
#pragma unroll
  for (int j = 0; j < SMAX; ++j) {
    // The exact path loads K slot j with another row and chunk.
    const int jr = exact_k_row_of<D, G, SMAX, PF32, EXACT>(r, j);
    const uint32_t roff = jr == j ? row_off[j] : (jr < S ? (uint32_t)jr * row_bytes : kRowOutOfRange);
    kr[j] = buffer_load16<kPolicyStream>(
        k_rsrc, kv_off + roff + (lane_ok ? exact_k_delta<D, G, SMAX, PF32, EXACT>(r, j) : 0u));
  }
#pragma unroll
  for (int j = 0; j < SMAX; ++j) vr[j] = buffer_load16<kPolicyStream>(v_rsrc, kv_off + row_off[j]);
  __builtin_amdgcn_sched_barrier(0);

  float acc[G][8];
  decode_core_any<D, G, SMAX, PF32, true, true, EXACT>(qv, kr, vr, S, a.scale, lane, lds_p, acc, grp);
  const u32x4 nan4 = {0x7e007e00u, 0x7e007e00u, 0x7e007e00u, 0x7e007e00u};
#pragma unroll
  for (int g = 0; g < G; ++g)
    buffer_store16(o_rsrc, group_row_off<G>(qo_off, g, grp, D), bad ? nan4 : pack_f16x8(acc[g]));
}

// The same for a paged cache (lengths in a.lens, log2(page_size) in
// a.seqlen_uniform, page stride in a.batch_stride): the lane groups' batches
// have their own pages, so every lane loads through its own 64-bit
// addresses, with no branch.  A lane group whose rows use a negative
// block-table entry has an invalid batch (NaN outputs) and reads nothing.
// A row with nothing to read (past the lane group's length, or a lane group
// with no valid row) reads row 0 of the first lane group whose batch has
// one (head 0) and is replaced by 0; the block-table entry looked up for
// such a row is entry 0 of its batch, so no lookup leaves the batch's table
// row, and no address is formed from an entry that was not checked.  A wave
// with no valid row reads nothing.
template <int D, int G, int SMAX, bool PF32>
__device__ __forceinline__ void decode_multi_unit_paged(const DecodeArgs& a, uint32_t b0, uint32_t nb, uint32_t b,
                                                        int S, bool bad, bool lane_ok, int sub, int hk, int lane,
                                                        uint16_t* lds_p) {
  constexpr int LPH = D / 8;
  const int r = lane % LPH;
  const int hq = a.num_heads_q;
  const uint32_t q_bytes = nb * (uint32_t)hq * D * 2u;
  const __amdgpu_buffer_rsrc_t q_rsrc = make_rsrc(a.q + (uint64_t)b0 * hq * D, q_bytes);
  const __amdgpu_buffer_rsrc_t o_rsrc = make_rsrc(a.o + (uint64_t)b0 * hq * D, q_bytes);
  const int grp = G >= 4 ? a.group : G;
  const uint32_t qo_off =
      lane_ok ? (uint32_t)sub * (uint32_t)hq * D * 2u + (uint32_t)(hk * grp * D + r * 8) * 2u : kLaneOutOfRange;

  u32x4 qv[G];
#pragma unroll
  for (int g = 0; g < G; ++g) qv[g] = buffer_load16<kPolicyDefault>(q_rsrc, group_row_off<G>(qo_off, g, grp, D));
  u32x4 kr[SMAX];
  u32x4 vr[SMAX];
  const int32_t* pages = a.block_table + (uint64_t)b * (uint64_t)a.bt_stride;
  const uint32_t shift = (uint32_t)a.seqlen_uniform;
  // This lane group's block-table entries (entry 0 for rows it does not
  // have); a negative one for a row it has makes its batch invalid.
  const bool live = lane_ok && !bad && S > 0;
  int32_t entry[SMAX];
  int32_t sign = 0;
#pragma unroll
  for (int j = 0; j < SMAX; ++j) {
    const bool ok = live && j < S;
    entry[j] = pages[ok ? (uint32_t)j >> shift : 0u];
    sign |= ok ? entry[j] : 0;
  }
  const bool unmapped = live && sign < 0;
  bad = bad || unmapped;
  const bool has = live && !unmapped;
  const uint64_t with_rows = __builtin_amdgcn_ballot_w64(has);
  if (with_rows == 0) {
#pragma unroll
    for (int j = 0; j < SMAX; ++j) kr[j] = vr[j] = u32x4{0u, 0u, 0u, 0u};
  } else {
    const uint64_t page_stride = (uint64_t)a.batch_stride;
    const uint64_t row_elems = (uint64_t)a.row_stride;
    const uint64_t lane_elem = (uint64_t)hk * (uint64_t)a.head_stride + (uint64_t)r * 8u;
    // Row 0 of the first lane group with a row (its entries all checked),
    // head 0, this lane's dims.
    const int src = (int)__builtin_ctzll(with_rows);
    const int64_t own0 = has ? paged_row_elem(entry[0], 0u, shift, page_stride, row_elems) : 0;
    const uint32_t lo0 = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(uint64_t)own0, src);
    const uint32_t hi0 = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)((uint64_t)own0 >> 32), src);
    const uint64_t safe = (((uint64_t)hi0 << 32) | lo0) + (uint64_t)r * 8u;
    uint64_t off[SMAX];
#pragma unroll
    for (int j = 0; j < SMAX; ++j) {
      const int64_t el = has && j < S ? paged_row_elem(entry[j], (uint32_t)j, shift, page_stride, row_elems) : -1;
      off[j] = el >= 0 ? (uint64_t)el + lane_elem : safe;
    }
#pragma unroll
    for (int j = 0; j < SMAX; ++j) kr[j] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(a.k + off[j]));
#pragma unroll
    for (int j = 0; j < SMAX; ++j) vr[j] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(a.v + off[j]));
#pragma unroll
    for (int j = 0; j < SMAX; ++j) {
      const bool ok = has && j < S;
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        kr[j][k] = ok ? (uint32_t)kr[j][k] : 0u;
        vr[j][k] = ok ? (uint32_t)vr[j][k] : 0u;
      }
    }
  }
  __builtin_amdgcn_sched_barrier(0);

  float acc[G][8];
  decode_core_any<D, G, SMAX, PF32, true, true, false>(qv, kr, vr, S, a.scale, lane, lds_p, acc, grp);
  const u32x4 nan4 = {0x7e007e00u, 0x7e007e00u, 0x7e007e00u, 0x7e007e00u};
#pragma unroll
  for (int g = 0; g < G; ++g)
    buffer_store16(o_rsrc, group_row_off<G>(qo_off, g, grp, D), bad ? nan4 : pack_f16x8(acc[g]));
}

// a.units_per_batch holds the batch count here, a.total_units the waves
// (ceil(batch / R)); lengths from a.lens (packed: offsets, strided and
// paged: lengths) or a.seqlen_uniform when a.lens is null (not paged).
template <int D, int G, int LAYOUT, bool PF32 = false, bool EXACT = false>
__global__ __launch_bounds__(kBlockThreads) void fmha_decode_multi_kernel(DecodeArgs a) {
  static_assert(!EXACT || LAYOUT != kLayoutPaged, "the exact path reads the packed and strided layouts");
  constexpr int LPH = D / 8;
  constexpr int HPW = kWaveSize / LPH;
  constexpr int VP = G * kMaxSeq;
  constexpr int WB = PF32 ? 2 : 1;
  constexpr int XW = exact_extra_bytes<D, G, kMaxSeq, PF32, true, EXACT>() / 2;  // exact staging
  __shared__ __attribute__((aligned(16))) uint16_t lds_p[kWavesPerBlock * (HPW * VP * WB + XW)];
  const int lane = threadIdx.x & (kWaveSize - 1);
  const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWaveSize);
  const uint32_t unit = blockIdx.x * kWavesPerBlock + wave;
  if (unit >= a.total_units) return;
  const uint32_t batch = (uint32_t)a.units_per_batch;
  if constexpr (LAYOUT == kLayoutPacked) {
    if (a.lens) report_mean_rows(a, unit, batch, lane);
  } else if constexpr (LAYOUT == kLayoutPaged) {
    report_mean_rows_sample(a, unit, batch, lane);
  }
  const uint32_t b0 = unit << a.sub_shift;
  const uint32_t nb = batch - b0 < (1u << a.sub_shift) ? batch - b0 : (1u << a.sub_shift);
  const int hkl = lane / LPH;
  const int sub = hkl >> a.hkv_shift;
  const int hk = hkl & ((1 << a.hkv_shift) - 1);
  const bool lane_ok = (uint32_t)sub < nb;
  const uint32_t b = b0 + (lane_ok ? (uint32_t)sub : 0u);
  const uint32_t row_bytes = (uint32_t)a.row_stride * 2u;
  int S;
  const uint16_t* kbase = a.k;
  const uint16_t* vbase = a.v;
  uint32_t records = 0, lane_rows = 0;
  if constexpr (LAYOUT == kLayoutPaged) {
    S = a.lens[b];
  } else if constexpr (LAYOUT == kLayoutPacked) {
    int32_t c0, ce, cb, cb1;
    if (a.lens) {
      c0 = a.lens[b0];
      ce = a.lens[b0 + nb];
      cb = a.lens[b];
      cb1 = a.lens[b + 1];
    } else {
      c0 = (int32_t)b0 * a.seqlen_uniform;
      ce = (int32_t)(b0 + nb) * a.seqlen_uniform;
      cb = (int32_t)b * a.seqlen_uniform;
      cb1 = cb + a.seqlen_uniform;
    }
    (void)ce;
    S = cb1 - cb;
    kbase = a.k + (int64_t)c0 * a.row_stride;
    vbase = a.v + (int64_t)c0 * a.row_stride;
    // This lane group's rows relative to the wave's first batch.  A batch
    // that a broken table (a huge invalid length earlier in the wave) puts
    // beyond the descriptor's reach counts as invalid too.
    const int64_t rel = (int64_t)cb - c0;
    if (rel < 0 || rel > (int64_t)((1u << 30) / row_bytes) - kMaxSeq) S = -1;
    lane_rows = (uint32_t)(rel < 0 ? 0 : rel) * row_bytes;
  } else {
    S = a.lens ? a.lens[b] : a.seqlen_uniform;
    kbase = a.k + (uint64_t)b0 * (uint64_t)a.batch_stride;
    vbase = a.v + (uint64_t)b0 * (uint64_t)a.batch_stride;
    const int rows = a.max_rows > 0 ? a.max_rows : 1;
    records = ((uint32_t)(nb - 1) * (uint32_t)a.batch_stride + (uint32_t)(rows - 1) * (uint32_t)a.row_stride +
               (uint32_t)((1 << a.hkv_shift) - 1) * (uint32_t)a.head_stride + D) * 2u;
    lane_rows = (uint32_t)sub * (uint32_t)a.batch_stride * 2u;
  }
  const bool bad = lane_ok && (S < 0 || S > a.max_rows);
  if (bad || !lane_ok) {
    // Nothing to read: every row out of range (offsets below 2^31 + 2^30).
    S = 0;
    lane_rows = 0;
  }
  // The longest length of the wave picks the bucket (a uniform value); the
  // packed descriptor ends at the last row a valid lane group reads.
  int smax = S;
  uint32_t end = LAYOUT == kLayoutPacked ? lane_rows + (uint32_t)S * row_bytes : 0u;
#pragma unroll
  for (int m = 1; m < kWaveSize; m <<= 1) {
    smax = max(smax, __shfl_xor(smax, m, kWaveSize));
    if constexpr (LAYOUT == kLayoutPacked) end = max(end, (uint32_t)__shfl_xor((int)end, m, kWaveSize));
  }
  smax = __builtin_amdgcn_readfirstlane(smax);
  if constexpr (LAYOUT == kLayoutPacked) records = (uint32_t)__builtin_amdgcn_readfirstlane((int)end);
  uint16_t* lds_wave = lds_p + wave * (HPW * VP * WB + XW);
#define FMHA_DECODE_MULTI(SM)                                                                                      \
  if constexpr (LAYOUT == kLayoutPaged)                                                                              \
    decode_multi_unit_paged<D, G, SM, PF32>(a, b0, nb, b, S, bad, lane_ok, sub, hk, lane, lds_wave);                \
  else                                                                                                               \
    decode_multi_unit<D, G, SM, PF32, EXACT>(a, b0, nb, kbase, vbase, records, lane_rows, S, bad, lane_ok, sub, hk, \
                                             lane, lds_wave)
  if (smax <= 1)
    FMHA_DECODE_MULTI(1);
  else if (smax <= 2)
    FMHA_DECODE_MULTI(2);
  else if (smax <= 4)
    FMHA_DECODE_MULTI(4);
  else if (smax <= 8)
    FMHA_DECODE_MULTI(8);
  else
    FMHA_DECODE_MULTI(16);
#undef FMHA_DECODE_MULTI
}

}  // namespace fmha_decode
