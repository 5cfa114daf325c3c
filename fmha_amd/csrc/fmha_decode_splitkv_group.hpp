// fmha_decode_splitkv_group.hpp -- the split-KV scores and P.V passes on the
// matrix cores, for query groups larger than 8 (lengths beyond 16 rows).
//
// The VALU passes (fmha_decode_splitkv.hpp) spend per lane about G * D / 8
// multiply-adds per row on Q.K^T and as many on P.V, so their time grows
// with G: the host runs a group above 8 on them as ceil(G / 8) launch KV
// heads of 8 query heads (SplitArgs::kv_groups), which reads K and V once
// but still doubles the arithmetic per doubling of G.  Here both products
// are MFMAs over 16-column tiles of query heads, as in fmha_decode_group.hpp,
// and one wave serves one KV head with all of its query heads:
//
//   * Scores: a wave takes HPW = 64 / (D/8) consecutive 16-row blocks of
//     one (batch, KV head), one block per lane group, loads their K rows as
//     the VALU pass does (LongRows, rows past the length read as 0) and
//     stages them in LDS; per 16-column tile of query heads (B operand read
//     straight from Q in the MFMA's layout) and block, S^T = K_blk . Q^T is
//     D/32 v_mfma_f32_16x16x32_bf16.  The scaled scores, the block max and
//     the block sum of exp(t - max) go to the same workspace arrays as the
//     VALU pass's, so the stats and combine kernels are shared.
//   * P.V: a wave takes one (batch, KV head, chunk) and up to TW tiles of
//     query heads; its lane groups load successive 16-row sub-blocks of the
//     chunk (HPW per round), V is transposed into LDS with v_perm as in the
//     short kernel, and per tile and sub-block the bf16 weights
//     bf16(exp(t - max) / sum) -- the row's global max and sum -- are the A
//     operand of D/16 v_mfma_f32_16x16x16_bf16 accumulating O[tile, D] over
//     the chunk's rows.  One chunk per row: fp16 O directly; otherwise fp32
//     partial outputs for the combine pass.
//
// Same numerics as the VALU passes (fp32 scores, scale, block and global
// softmax statistics, weights rounded to bf16 after normalisation, fp32
// accumulation, chunk partials summed in chunk order, one RNE rounding to
// fp16); only the order of the fp32 sums inside a product differs.  Packed
// and strided layouts read rows through LongRows' one descriptor per wave;
// on paged layouts the lane groups of a wave read rows of different pages,
// which one page's descriptor cannot cover, so PagedLaneRows gives every
// lane its own 64-bit addresses instead.  The query heads of a KV head may
// be padded (Q and O copies with a multiple of 8 heads): the kernels take
// G = num_heads_q / num_heads_kv as given.
//
// The file ends with two single passes on the same products (one launch,
// nothing through the workspace) for query groups of at most 16 with
// enough (batch, KV head) units: onepass_mfma_kernel, one workgroup per
// unit keeping the row's scores in LDS, and onepass_mfma_reg_kernel, each
// wave of the workgroup keeping its rows' scores in the registers the
// scores MFMA leaves them in.
#pragma once

#include "fmha_decode_group.hpp"
#include "fmha_decode_splitkv.hpp"

namespace fmha_decode {

// Wave barrier between LDS writes and reads of one wave.
__device__ __forceinline__ void wave_lds_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// The row loader of the matrix-core split passes for a layout: per-lane
// addresses on every paged layout.
template <int D, int LAYOUT>
using GroupRows = typename std::conditional<
    is_paged_layout(LAYOUT), PagedLaneRows<D, LAYOUT == kLayoutPagedBlock || LAYOUT == kLayoutPagedBlockLanes>,
    LongRows<D, LAYOUT>>::type;

// Grid: batch * ceil(nblk / HPW) * Hkv one-wave workgroups, workgroup
// (b * nwb + wb) * Hkv + hk serving blocks [wb * HPW, wb * HPW + HPW) of KV
// head hk of batch b (consecutive waves: neighbouring heads of the same
// rows).
template <int D, int LAYOUT>
__global__ __launch_bounds__(kBlockThreads) void splitkv_scores_group_kernel(SplitArgs a) {
  using Sh = GroupShape<D>;
  constexpr int LPH = Sh::LPH;
  constexpr int HPW = Sh::HPW;
  constexpr int NR = kSplitBlockRows;
  __shared__ __attribute__((aligned(16))) char k_lds[NR * Sh::KS];
  const int lane = threadIdx.x & (kWaveSize - 1);
  const uint32_t hkv = (uint32_t)a.num_heads_kv;
  const uint32_t nwb = ((uint32_t)a.nblk + HPW - 1) / HPW;
  const uint32_t id = blockIdx.x;
  const uint32_t hk = id % hkv;
  const uint32_t rest = id / hkv;
  const uint32_t wb = rest % nwb;
  const uint32_t b = rest / nwb;
  if (b >= (uint32_t)a.batch) return;
  const int S = split_len_l<LAYOUT>(a, b);
  const int j0 = (int)wb * HPW * NR;  // the wave's first row
  if (S < 0 || S > a.max_rows || j0 >= S) return;
  const int s = lane / LPH;  // this lane group's block of the wave
  const int r = lane % LPH;
  const int q = lane >> 4;   // MFMA lane group
  const int n = lane & 15;   // MFMA row / column
  const int hq = a.num_heads_q;
  const int G = hq / (int)hkv;
  const int tiles = (G + 15) / 16;

  // K rows of the wave's blocks (lane group s: rows j0 + 16 s + j).
  GroupRows<D, LAYOUT> kv;
  kv.init(a, a.k, b, split_row_base<LAYOUT>(a, b), 0, S, (int)hk, true, r, s * NR);
  u32x4 kr[NR];
  kv.template load<NR>(kr, j0);
  const bool kv_bad = kv.any_bad();
  // This KV head's query rows: tile t's B operands (lane (q, n): query
  // column 16 t + n, 16-byte chunks 4 cc + q), requested one tile ahead.
  const __amdgpu_buffer_rsrc_t q_rsrc =
      make_rsrc(a.q + ((uint64_t)b * hq + (uint64_t)hk * G) * D, (uint32_t)G * D * 2u);
  auto load_q = [&](bf16x8_v (&dst)[Sh::QLD], int tile) {
    const int g = tile * 16 + n;
#pragma unroll
    for (int cc = 0; cc < Sh::QLD; ++cc)
      dst[cc] = __builtin_bit_cast(
          bf16x8_v, buffer_load16<kPolicyDefault>(q_rsrc, g < G && tile < tiles
                                                              ? (uint32_t)(g * D + (4 * cc + q) * 8) * 2u
                                                              : kLaneOutOfRange));
  };
  bf16x8_v qn[Sh::QLD];
  load_q(qn, 0);
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int j = 0; j < NR; ++j) *reinterpret_cast<u32x4*>(k_lds + j * Sh::KS + s * D * 2 + r * 16) = kr[j];
  wave_lds_sync();

  // The scores of the wave's blocks.
  const int blk0 = (int)wb * HPW;
  const int nb = a.nblk - blk0 < HPW ? a.nblk - blk0 : HPW;
  const __amdgpu_buffer_rsrc_t t_rsrc =
      make_rsrc(a.t + t_block_base(a, b, blk0), (uint32_t)nb * (uint32_t)hq * NR * 4u);
  for (int tile = 0; tile < tiles; ++tile) {
    const int g = tile * 16 + n;  // this lane's query column
    const bool gok = g < G;
    bf16x8_v qb[Sh::QLD];
#pragma unroll
    for (int cc = 0; cc < Sh::QLD; ++cc) qb[cc] = qn[cc];
    if (tile + 1 < tiles) load_q(qn, tile + 1);
#pragma unroll
    for (int p = 0; p < HPW; ++p) {
      const int jb = j0 + p * NR;  // first row of block p
      if (jb >= S) break;
      f32x4_v c4 = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
      for (int cc = 0; cc < Sh::QLD; ++cc) {
        const bf16x8_v ka = *reinterpret_cast<const bf16x8_v*>(k_lds + n * Sh::KS + p * D * 2 + (4 * cc + q) * 16);
        c4 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ka, qb[cc], c4, 0, 0, 0);
      }
      // Rows 4q..4q+3 of block p for query column g; the block's max and
      // sum of exponentials over its valid rows (row jb is valid, so the
      // max is finite for finite scores).
      float x[4];
      float m = -__builtin_inff();
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        x[e] = c4[e] * a.scale;
        m = jb + 4 * q + e < S ? fmaxf(m, x[e]) : m;
      }
      m = column_reduce<true>(m);
      float sum = 0.0f;
#pragma unroll
      for (int e = 0; e < 4; ++e) sum += jb + 4 * q + e < S ? expf(x[e] - m) : 0.0f;
      sum = column_reduce<false>(sum);
      // Scores of rows past S (their K rows read as 0) land in the block's
      // padding, which nothing reads as a weight.
      if (gok) {
        const u32x4 v4 = {__builtin_bit_cast(uint32_t, x[0]), __builtin_bit_cast(uint32_t, x[1]),
                          __builtin_bit_cast(uint32_t, x[2]), __builtin_bit_cast(uint32_t, x[3])};
        __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4_gcc, v4), t_rsrc,
                                               (int)((((uint32_t)p * hq + hk * G + g) * NR + 4 * q) * 4u), 0,
                                               kPolicyStreamStore);
        if (q == 0) {
          const uint64_t idx = ((uint64_t)b * hq + (uint64_t)hk * G + g) * a.nblk + blk0 + p;
          a.m[idx] = m;
          // An unmapped page among the wave's rows: a NaN sum makes the
          // batch's weights, hence its outputs, NaN.
          a.l[idx] = kv_bad ? __builtin_nanf("") : sum;
        }
      }
    }
  }
}

// fp16 output of DPC dims per query row (8, 16 or 32 bytes) at byte offset off.
template <int DPC>
__device__ __forceinline__ void store_f16_run(__amdgpu_buffer_rsrc_t o_rsrc, uint32_t off, const float* v) {
#pragma unroll
  for (int h8 = 0; h8 < (DPC + 7) / 8; ++h8) {
    constexpr int W = DPC < 8 ? DPC : 8;
    float vals[8];
#pragma unroll
    for (int k8 = 0; k8 < 8; ++k8) vals[k8] = k8 < W ? v[h8 * 8 + (k8 < W ? k8 : 0)] : 0.0f;
    const u32x4 pk = pack_f16x8(vals);
    if constexpr (W == 8) {
      buffer_store16(o_rsrc, off + h8 * 16, pk);
    } else {
      __builtin_amdgcn_raw_buffer_store_b64(u32x2{pk[0], pk[1]}, o_rsrc, (int)off, 0, kPolicyStreamStore);
    }
  }
}

// fp16 output of P.V column n's DPC dims of one query row (dims out_dim(n,
// 0..DPC-1)) whose first element is at byte offset row_off: one contiguous
// run over the row's 16 lanes per store instruction.
template <int DPC>
__device__ __forceinline__ void store_f16_cols(__amdgpu_buffer_rsrc_t o_rsrc, uint32_t row_off, int n,
                                               const float* v) {
  if constexpr (DPC <= 8) {
    store_f16_run<DPC>(o_rsrc, row_off + (uint32_t)out_dim<DPC>(n, 0) * 2u, v);
  } else {
#pragma unroll
    for (int h8 = 0; h8 < DPC / 8; ++h8)
      store_f16_run<8>(o_rsrc, row_off + (uint32_t)out_dim<DPC>(n, 8 * h8) * 2u, v + 8 * h8);
  }
}

// Grid: units = batch * nchunks * Hkv (unit (b * nchunks + c) * Hkv + hk),
// each in TC = ceil(tiles / TW) tile chunks; ceil(units / 8) * 8 * TC
// one-wave workgroups, workgroup w serving unit ((w / 8) / TC) * 8 + w % 8
// and tile chunk (w / 8) % TC, so that the tile chunks of one unit run on
// one XCD (dispatch is round-robin over the 8 XCDs) and re-read its V from
// that XCD's L2.  DIRECT: one chunk per row (nchunks == 1), O written here.
template <int D, int TW, bool DIRECT, int LAYOUT>
__global__ __launch_bounds__(kBlockThreads) void splitkv_pv_group_kernel(SplitArgs a) {
  using Sh = GroupShape<D>;
  constexpr int LPH = Sh::LPH;
  constexpr int HPW = Sh::HPW;
  constexpr int NR = kSplitBlockRows;
  constexpr int DPC = Sh::DPC;
  __shared__ __attribute__((aligned(16))) char v_lds[HPW * Sh::VSTREAM];
  const int lane = threadIdx.x & (kWaveSize - 1);
  const uint32_t hkv = (uint32_t)a.num_heads_kv;
  const int hq = a.num_heads_q;
  const int G = hq / (int)hkv;
  const int tiles = (G + 15) / 16;
  const uint32_t tc_count = (uint32_t)((tiles + TW - 1) / TW);
  const uint32_t w = blockIdx.x;
  const uint32_t rest = w >> 3;
  const uint32_t unit = (rest / tc_count) * 8u + (w & 7u);
  const int tile0 = (int)(rest % tc_count) * TW;
  const uint32_t nchunks = (uint32_t)a.nchunks;
  if (unit >= (uint32_t)a.batch * nchunks * hkv) return;
  const uint32_t hk = unit % hkv;
  const uint32_t c = (unit / hkv) % nchunks;
  const uint32_t b = unit / hkv / nchunks;
  const int ntl = tiles - tile0 < TW ? tiles - tile0 : TW;  // > 0
  const int S = split_len_l<LAYOUT>(a, b);
  const bool bad = S < 0 || S > a.max_rows;
  const int row0 = (int)c * a.chunk_rows;
  const int q = lane >> 4;
  const int n = lane & 15;
  const __amdgpu_buffer_rsrc_t o_rsrc =
      make_rsrc(a.o + ((uint64_t)b * hq + (uint64_t)hk * G) * D, (uint32_t)G * D * 2u);
  if (bad || row0 >= S) {
    // Only a DIRECT launch (one chunk) owns the output of an empty or
    // invalid row; the combine kernel covers them otherwise.
    if constexpr (DIRECT) {
      const u32x4 fill = bad ? u32x4{0x7e007e00u, 0x7e007e00u, 0x7e007e00u, 0x7e007e00u} : u32x4{0u, 0u, 0u, 0u};
      for (int k = lane; k < ntl * 16 * (D / 8); k += kWaveSize) {
        const int g = tile0 * 16 + k / (D / 8);
        if (g < G) buffer_store16(o_rsrc, (uint32_t)(g * D + (k % (D / 8)) * 8) * 2u, fill);
      }
    }
    return;
  }
  const int s = lane / LPH;  // lane group: sub-block s of each round
  const int r = lane % LPH;
  const int rows = S - row0 < a.chunk_rows ? S - row0 : a.chunk_rows;  // > 0
  const int rounds = (rows + HPW * NR - 1) / (HPW * NR);
  // Lane group s reads rows row0 + 16 (HPW k + s) + j in round k.
  GroupRows<D, LAYOUT> vrows;
  vrows.init(a, a.v, b, split_row_base<LAYOUT>(a, b), row0, row0 + rows, (int)hk, true, r, s * NR, rows);
  const __amdgpu_buffer_rsrc_t t_rsrc =
      make_rsrc(a.t + t_block_base(a, b, 0), (uint32_t)a.nblk * (uint32_t)hq * NR * 4u);
  // The row's global max and sum for this lane's query column of each tile
  // (the four lanes q = 0..3 of a column share it).
  float gm[TW], gl[TW];
  uint64_t hqi[TW];
  bool hok[TW];
#pragma unroll
  for (int i = 0; i < TW; ++i) {
    const int g = (tile0 + i) * 16 + n;
    hok[i] = i < ntl && g < G;
    hqi[i] = (uint64_t)b * hq + (uint64_t)hk * G + (hok[i] ? g : 0);
  }
  row_stats<4, 16, TW>(a, hqi, hok, S, lane, gm, gl);
  f32x4_v acc[TW][DPC];
#pragma unroll
  for (int i = 0; i < TW; ++i)
#pragma unroll
    for (int dt = 0; dt < DPC; ++dt) acc[i][dt] = f32x4_v{0.0f, 0.0f, 0.0f, 0.0f};

  u32x4 vr[NR];
  vrows.template load<NR>(vr, 0);
  for (int k = 0; k < rounds; ++k) {
    // The round's scores (lane (q, n): rows 4q..4q+3 of sub-block p, query
    // column 16 (tile0 + i) + n), requested before the V transpose so that
    // their latency overlaps it.  Sub-blocks past the chunk's rows read
    // nothing (their weights are 0 by the row check).
    u32x4 t4[HPW][TW];
#pragma unroll
    for (int p = 0; p < HPW; ++p) {
      const int jr = (k * HPW + p) * NR;
      const int blk = (row0 + jr) / NR;
#pragma unroll
      for (int i = 0; i < TW; ++i) {
        const int g = (tile0 + i) * 16 + n;
        t4[p][i] = buffer_load16<kPolicyDefault>(
            t_rsrc, jr < rows && i < ntl && g < G ? (((uint32_t)blk * hq + hk * G + g) * NR + 4 * q) * 4u
                                                  : kLaneOutOfRange);
      }
    }
    // V^T of the round's sub-blocks: sub-block s at s * VSTREAM, 8-dim block
    // r at r * VB, dim e at e * 32 bytes, 16 rows of bf16.
    wave_lds_sync();  // the previous round's reads of v_lds are done
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int e = 0; e < 8; ++e) {
#pragma unroll
      for (int half = 0; half < 2; ++half) {
        u32x4 wv;
#pragma unroll
        for (int pp = 0; pp < 4; ++pp) {
          const int j = 8 * half + 2 * pp;
          wv[pp] = __builtin_amdgcn_perm((uint32_t)vr[j + 1][e / 2], (uint32_t)vr[j][e / 2],
                                         (e & 1) ? kPermHi : kPermLo);
        }
        *reinterpret_cast<u32x4*>(v_lds + s * Sh::VSTREAM + r * Sh::VB + e * (NR * 2) + half * 16) = wv;
      }
    }
    wave_lds_sync();
    // The next round's rows are in flight during this round's products.
    if (k + 1 < rounds) vrows.template load<NR>(vr, (k + 1) * HPW * NR);
#pragma unroll
    for (int p = 0; p < HPW; ++p) {
      const int jr = (k * HPW + p) * NR;  // sub-block's first row, relative to row0
      if (jr >= rows) break;
      const char* vs = v_lds + p * Sh::VSTREAM;
      bf16x4_v vb[DPC];
#pragma unroll
      for (int dt = 0; dt < DPC; ++dt) {
        const int dim = out_dim<DPC>(n, dt);
        vb[dt] = *reinterpret_cast<const bf16x4_v*>(vs + (dim / 8) * Sh::VB + (dim % 8) * (NR * 2) + q * 8);
      }
#pragma unroll
      for (int i = 0; i < TW; ++i) {
        if (i >= ntl) break;
        const int g = (tile0 + i) * 16 + n;
        bf16x4_v pa;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const bool valid = g < G && jr + 4 * q + e < rows;
          const float pw = valid ? expf(__builtin_bit_cast(float, (uint32_t)t4[p][i][e]) - gm[i]) / gl[i] : 0.0f;
          pa[e] = (__bf16)pw;
        }
#pragma unroll
        for (int dt = 0; dt < DPC; ++dt)
          acc[i][dt] = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(pa, vb[dt], acc[i][dt], 0, 0, 0);
      }
    }
  }

  // Lane (q, n) holds query rows 4q..4q+3 of each tile, dims out_dim(n, 0..DPC-1).
#pragma unroll
  for (int i = 0; i < TW; ++i) {
    if (i >= ntl) break;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int g = (tile0 + i) * 16 + 4 * q + e;
      float v[DPC];
#pragma unroll
      for (int dt = 0; dt < DPC; ++dt) v[dt] = acc[i][dt][e];
      if constexpr (DIRECT) {
        store_f16_cols<DPC>(o_rsrc, g < G ? (uint32_t)(g * D) * 2u : kLaneOutOfRange, n, v);
      } else {
        // Partial outputs [Hq][nchunks][D] of this batch (default policy:
        // the combine pass reads them right after).
        const uint32_t part_bytes = nchunks * D * 4u;
        const __amdgpu_buffer_rsrc_t p_rsrc =
            make_rsrc(a.opart + ((uint64_t)b * hq + (uint64_t)hk * G) * nchunks * D, (uint32_t)G * part_bytes);
        const uint32_t off = g < G ? (uint32_t)g * part_bytes + (uint32_t)(c * D) * 4u : kLaneOutOfRange;
#pragma unroll
        for (int h4 = 0; h4 < DPC / 4; ++h4) {
          const u32x4 x4 = {__builtin_bit_cast(uint32_t, v[4 * h4]), __builtin_bit_cast(uint32_t, v[4 * h4 + 1]),
                            __builtin_bit_cast(uint32_t, v[4 * h4 + 2]), __builtin_bit_cast(uint32_t, v[4 * h4 + 3])};
          __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4_gcc, x4), p_rsrc,
                                                 (int)(off + (uint32_t)out_dim<DPC>(n, 4 * h4) * 4u), 0,
                                                 kPolicyDefault);
        }
      }
    }
  }
}


// ---------------------------------------------------------------------------
// Single pass on the matrix cores: one (batch, KV head) per workgroup of NW
// waves, all of its query heads in one 16-column tile (G <= 16), K and V
// read once and nothing else in memory.
// ---------------------------------------------------------------------------
// Rows a wave takes (a multiple of the HPW 16-row blocks one round stages),
// for a row bound of nblk 16-row blocks split over NW waves.
template <int D>
constexpr int onepass_mfma_wave_rows(int nblk, int nw) {
  constexpr int RR = GroupShape<D>::HPW * kSplitBlockRows;
  return ((nblk * kSplitBlockRows + nw * RR - 1) / (nw * RR)) * RR;
}
// LDS bytes of one workgroup: the row's fp32 scores ([G][rows + 4], the
// stride off the bank period), the waves' (max, sum) per query column, and
// per wave the K rows / V transpose staging of the matrix-core passes.
template <int D>
constexpr size_t onepass_mfma_lds_bytes(int g, int nblk, int nw) {
  return (size_t)g * (nw * onepass_mfma_wave_rows<D>(nblk, nw) + 4) * 4 + (size_t)nw * 16 * 2 * 4 +
         (size_t)nw * GroupShape<D>::KV_LDS;
}

// Wave w scores rows [w R, w R + R) of the row (R = onepass_mfma_wave_rows)
// a round of HPW 16-row blocks at a time, as the split scores pass does (K
// rows staged in LDS, S^T = K_blk . Q^T on v_mfma_f32_16x16x32_bf16), into
// the workgroup's LDS, keeping per query column a running max and sum of
// exponentials; the next round's K rows are in flight during a round's
// products.  The waves exchange their (max, sum) per column and combine
// them in wave order; each wave then walks V over its rows as the split
// P.V pass does (V^T staged in LDS with v_perm, bf16(exp(t - max) / sum)
// weights as the A operand of v_mfma_f32_16x16x16_bf16), and waves 1..NW-1
// hand their sums to wave 0 through their own staging, which adds them in
// wave order and writes fp16 O.  Packed and strided layouts.
template <int D, int NW, int LAYOUT>
__global__ __launch_bounds__(kBlockThreads * NW) void onepass_mfma_kernel(SplitArgs a) {
  static_assert(LAYOUT == kLayoutPacked || LAYOUT == kLayoutStrided || LAYOUT == kLayoutPagedBlock,
                "packed, strided or pages of at least 16 rows");
  // Paged caches: every lane addresses its own rows (GroupRows), a row in
  // an unmapped page (a negative entry) is read as Q's first row and sets
  // the lane's flag; the (batch, KV head)'s outputs are then NaN.
  constexpr bool PAGED = is_paged_layout(LAYOUT);
  using Sh = GroupShape<D>;
  constexpr int LPH = Sh::LPH;
  constexpr int HPW = Sh::HPW;
  constexpr int NR = kSplitBlockRows;
  constexpr int DPC = Sh::DPC;
  constexpr int RR = HPW * NR;  // rows per round
  extern __shared__ __attribute__((aligned(16))) char onepass_mfma_lds[];
  const int lane = threadIdx.x & (kWaveSize - 1);
  const int wv = __builtin_amdgcn_readfirstlane((int)(threadIdx.x / kWaveSize));
  const uint32_t hkv = (uint32_t)a.num_heads_kv;
  const uint32_t b = blockIdx.x / hkv;
  const uint32_t hk = blockIdx.x - b * hkv;
  if (b >= (uint32_t)a.batch) return;
  const int hq = a.num_heads_q;
  const int G = hq / (int)hkv;  // <= 16
  const int S = split_len_l<LAYOUT>(a, b);
  const int q = lane >> 4;   // MFMA lane group
  const int n = lane & 15;   // MFMA row / column: this lane's query column
  const int s = lane / LPH;  // load lane group: block s of each round
  const int r = lane % LPH;
  const bool gok = n < G;
  const __amdgpu_buffer_rsrc_t o_rsrc =
      make_rsrc(a.o + ((uint64_t)b * hq + (uint64_t)hk * G) * D, (uint32_t)G * D * 2u);
  if (S <= 0 || S > a.max_rows) {
    // Empty rows give 0 (the reference loop's result), invalid ones NaN.
    if (wv != 0) return;
    const u32x4 fill = S == 0 ? u32x4{0u, 0u, 0u, 0u} : u32x4{0x7e007e00u, 0x7e007e00u, 0x7e007e00u, 0x7e007e00u};
    for (int k = lane; k < G * (D / 8); k += kWaveSize)
      buffer_store16(o_rsrc, (uint32_t)((k / (D / 8)) * D + (k % (D / 8)) * 8) * 2u, fill);
    return;
  }
  const int wrows = onepass_mfma_wave_rows<D>(a.nblk, NW);
  const int sps = NW * wrows + 4;  // floats per query column
  float* sc = reinterpret_cast<float*>(onepass_mfma_lds);
  float* pst = sc + (size_t)G * sps;  // [NW][16][2]
  char* stage = reinterpret_cast<char*>(pst + NW * 16 * 2) + (size_t)wv * Sh::KV_LDS;
  const int lo = wv * wrows;  // this wave's first row
  const int span = S - lo < 0 ? 0 : (S - lo < wrows ? S - lo : wrows);
  const int rounds = (span + RR - 1) / RR;

  // ---- K: scores of rows [lo, lo + span) -> sc, running (max, sum) ----
  GroupRows<D, LAYOUT> kv;
  kv.init(a, a.k, b, split_row_base<LAYOUT>(a, b), 0, S, (int)hk, true, r, s * NR);
  const __amdgpu_buffer_rsrc_t q_rsrc =
      make_rsrc(a.q + ((uint64_t)b * hq + (uint64_t)hk * G) * D, (uint32_t)G * D * 2u);
  bf16x8_v qb[Sh::QLD];
#pragma unroll
  for (int cc = 0; cc < Sh::QLD; ++cc)
    qb[cc] = __builtin_bit_cast(
        bf16x8_v, buffer_load16<kPolicyDefault>(q_rsrc, gok ? (uint32_t)(n * D + (4 * cc + q) * 8) * 2u : kLaneOutOfRange));
  u32x4 kr[NR];
  kv.template load<NR>(kr, lo);
  float rm = -__builtin_inff(), rl = 0.0f;  // this lane's rows of column n
  for (int k = 0; k < rounds; ++k) {
    const int j0 = lo + k * RR;
    wave_lds_sync();  // the previous round's reads of the staging are done
#pragma unroll
    for (int j = 0; j < NR; ++j) *reinterpret_cast<u32x4*>(stage + j * Sh::KS + s * D * 2 + r * 16) = kr[j];
    wave_lds_sync();
    __builtin_amdgcn_sched_barrier(0);
    // The next round's rows are in flight during this round's products
    // (past the wave's rows: rows read 0 without access, or another wave's
    // rows, never used).
    if (k + 1 < rounds) kv.template load<NR>(kr, j0 + RR);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int p = 0; p < HPW; ++p) {
      const int jb = j0 + p * NR;
      if (jb >= lo + span) break;
      f32x4_v c4 = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
      for (int cc = 0; cc < Sh::QLD; ++cc) {
        const bf16x8_v ka = *reinterpret_cast<const bf16x8_v*>(stage + n * Sh::KS + p * D * 2 + (4 * cc + q) * 16);
        c4 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ka, qb[cc], c4, 0, 0, 0);
      }
      float x[4];
      float bm = -__builtin_inff();
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        x[e] = c4[e] * a.scale;
        bm = jb + 4 * q + e < S ? fmaxf(bm, x[e]) : bm;
      }
      if (gok)
        *reinterpret_cast<float4*>(sc + (size_t)n * sps + jb + 4 * q) = float4{x[0], x[1], x[2], x[3]};
      const float mn = fmaxf(rm, bm);
      float bs = 0.0f;
#pragma unroll
      for (int e = 0; e < 4; ++e) bs += jb + 4 * q + e < S ? expf(x[e] - mn) : 0.0f;
      rl = rl * (rm == mn ? 1.0f : expf(rm - mn)) + bs;
      rm = mn;
    }
  }
  // The wave's (max, sum) per column: over its four lane groups, then
  // through LDS over the waves, in wave order.
  {
    const float cm = column_reduce<true>(rm);
    const float cl = column_reduce<false>(rl * (rm == cm ? 1.0f : expf(rm - cm)));
    if (q == 0) {
      pst[(wv * 16 + n) * 2] = cm;
      pst[(wv * 16 + n) * 2 + 1] = cl;
    }
  }
  // V rows of the wave's first round, in flight across the exchange.
  GroupRows<D, LAYOUT> vrows;
  vrows.init(a, a.v, b, split_row_base<LAYOUT>(a, b), 0, S, (int)hk, true, r, s * NR);
  u32x4 vr[NR];
  vrows.template load<NR>(vr, lo);
  // Paged: K met an unmapped page among the rows of some wave (V reads the
  // same rows through the same table).
  int poisoned = 0;
  if constexpr (PAGED)
    poisoned = __syncthreads_or(kv.bad != 0);
  else
    __syncthreads();
  float gm = -__builtin_inff();
#pragma unroll
  for (int w = 0; w < NW; ++w) gm = fmaxf(gm, pst[(w * 16 + n) * 2]);
  float gl = 0.0f;
#pragma unroll
  for (int w = 0; w < NW; ++w) {
    const float m = pst[(w * 16 + n) * 2];
    gl += m == -__builtin_inff() ? 0.0f : pst[(w * 16 + n) * 2 + 1] * (m == gm ? 1.0f : expf(m - gm));
  }

  // ---- V: rows [lo, lo + span), weights from sc ----
  f32x4_v acc[DPC];
#pragma unroll
  for (int dt = 0; dt < DPC; ++dt) acc[dt] = f32x4_v{0.0f, 0.0f, 0.0f, 0.0f};
  for (int k = 0; k < rounds; ++k) {
    const int j0 = lo + k * RR;
    wave_lds_sync();  // the previous round's reads of the staging are done
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int e = 0; e < 8; ++e) {
#pragma unroll
      for (int half = 0; half < 2; ++half) {
        u32x4 wv4;
#pragma unroll
        for (int pp = 0; pp < 4; ++pp) {
          const int j = 8 * half + 2 * pp;
          wv4[pp] = __builtin_amdgcn_perm((uint32_t)vr[j + 1][e / 2], (uint32_t)vr[j][e / 2],
                                          (e & 1) ? kPermHi : kPermLo);
        }
        *reinterpret_cast<u32x4*>(stage + s * Sh::VSTREAM + r * Sh::VB + e * (NR * 2) + half * 16) = wv4;
      }
    }
    wave_lds_sync();
    if (k + 1 < rounds) vrows.template load<NR>(vr, j0 + RR);
#pragma unroll
    for (int p = 0; p < HPW; ++p) {
      const int jb = j0 + p * NR;
      if (jb >= lo + span) break;
      const char* vs = stage + p * Sh::VSTREAM;
      bf16x4_v vb[DPC];
#pragma unroll
      for (int dt = 0; dt < DPC; ++dt) {
        const int dim = out_dim<DPC>(n, dt);
        vb[dt] = *reinterpret_cast<const bf16x4_v*>(vs + (dim / 8) * Sh::VB + (dim % 8) * (NR * 2) + q * 8);
      }
      const float4 t4 = gok ? *reinterpret_cast<const float4*>(sc + (size_t)n * sps + jb + 4 * q)
                            : float4{0.0f, 0.0f, 0.0f, 0.0f};
      const float tt[4] = {t4.x, t4.y, t4.z, t4.w};
      bf16x4_v pa;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const bool valid = gok && jb + 4 * q + e < S;
        pa[e] = (__bf16)(valid ? expf(tt[e] - gm) / gl : 0.0f);
      }
#pragma unroll
      for (int dt = 0; dt < DPC; ++dt)
        acc[dt] = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(pa, vb[dt], acc[dt], 0, 0, 0);
    }
  }

  // ---- waves 1..NW-1 -> wave 0 (each through its own staging) ----
  if constexpr (NW > 1) {
    wave_lds_sync();
    if (wv > 0) {
#pragma unroll
      for (int dt = 0; dt < DPC; ++dt)
        *reinterpret_cast<f32x4_v*>(stage + ((size_t)dt * kWaveSize + lane) * 16) = acc[dt];
    }
    __syncthreads();
    if (wv > 0) return;
    for (int w = 1; w < NW; ++w) {
      const char* ws = reinterpret_cast<char*>(pst + NW * 16 * 2) + (size_t)w * Sh::KV_LDS;
#pragma unroll
      for (int dt = 0; dt < DPC; ++dt) {
        const f32x4_v x = *reinterpret_cast<const f32x4_v*>(ws + ((size_t)dt * kWaveSize + lane) * 16);
#pragma unroll
        for (int e = 0; e < 4; ++e) acc[dt][e] += x[e];
      }
    }
  }
  // Lane (q, n) holds query rows 4q..4q+3, dims out_dim(n, 0..DPC-1).
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const int g = 4 * q + e;
    float v[DPC];
#pragma unroll
    for (int dt = 0; dt < DPC; ++dt) v[dt] = poisoned ? __builtin_nanf("") : acc[dt][e];
    store_f16_cols<DPC>(o_rsrc, g < G ? (uint32_t)(g * D) * 2u : kLaneOutOfRange, n, v);
  }
}


// ---------------------------------------------------------------------------
// Single pass on the matrix cores, the row's scores in registers.
// ---------------------------------------------------------------------------
// The v_mfma_f32_16x16x32_bf16 scores of a 16-row tile leave lane (q, n)
// (q = lane / 16, n = lane % 16) holding rows 4q..4q+3 of query column n:
// exactly its A operand of v_mfma_f32_16x16x16_bf16 in the P.V product
// (query row n, reduction index 4q + e).  So a wave that keeps its tiles'
// scores in registers needs no LDS for them, and more waves fit a CU than
// with the row's scores in LDS.  Wave w of a workgroup of NW takes rows
// [w R, w R + R), R = 16 TPW, of one (batch, KV head):
//   * K a round of HPW tiles at a time, whole rows per lane group (16 bytes
//     a lane) into a 16-row staging in LDS, read back in the A operand's
//     layout (row n, 16-byte chunks 4c + q; Q's B operand takes the same
//     chunks), the next round's rows in flight during a round's products
//     (loading the A layout straight from memory, 64 bytes of 16 rows per
//     instruction, measured 5-15% slower);
//   * its (max, sum of exp(t - max)) per query column over its rows, those
//     of the workgroup's waves exchanged through LDS and combined in wave
//     order;
//   * V rows 4q..4q+3 of each tile at dims [n D/16, n D/16 + D/16) straight
//     from memory (each load a whole row across the 16 lanes of a lane
//     group), PF tiles in flight, transposed in registers with v_perm into
//     the B operand; weights bf16(exp(t - max) / sum) with the row's global
//     max and sum;
//   * waves 1..NW-1 hand their fp32 sums to wave 0 through LDS (the K
//     staging's space), which adds them in wave order and writes fp16 O.
// Rows past the wave's range are never read (out-of-range offsets read 0).
// The tile loops are unrolled over TPW with no branch inside: the scores'
// registers need static indices, and a branch per tile made the compiler
// wait for every load in flight at each tile.  Packed and strided layouts,
// and paged ones: pages of at least 16 rows (kLayoutPagedBlock), where a
// tile lies in one page, K through per-lane page addresses (PagedLaneRows),
// V through a descriptor per tile from the tile's block-table entry, which
// each wave requests for all its tiles at the start; smaller pages
// (kLayoutPaged), every row through its own entry and a per-lane address,
// the entries requested ahead of their rows.  A negative entry among a
// (batch, KV head)'s rows makes its outputs NaN, its rows never read.
template <int D, int TPW>
constexpr int onepass_reg_pf() {
  return D == 256 || TPW >= 32 ? 2 : 4;  // V tiles in flight per wave
}
// Tiles per K staging round: a wave's lane groups (HPW) at D >= 128; at
// D = 64 with up to 16 tiles per wave (three or more waves per SIMD by
// registers), and on pages under 16 rows, half of them, two lane groups
// loading 8 rows each of one tile, which halves the staging (more waves
// per CU).
constexpr int onepass_reg_round_tiles(int d, int tpw, int layout) {
  return d == 64 && (tpw <= 16 || layout == kLayoutPaged) ? kWaveSize / (d / 8) / 2 : kWaveSize / (d / 8);
}
// LDS bytes per staged row: the round's tiles' D dims, plus padding.
constexpr int onepass_reg_stage_row(int d, int tpw, int layout) {
  return onepass_reg_round_tiles(d, tpw, layout) * d * 2 + 16;
}
// LDS of a workgroup of nw waves: the (max, sum) exchange, then each wave's
// K staging (16 rows of a round's tiles), whose space the fp32 sums of
// waves 1..nw-1 reuse once every wave is past the exchange.
template <int D>
constexpr size_t onepass_reg_stage_offset(int nw) {
  return (size_t)nw * 16 * 2 * 4;
}
template <int D>
constexpr size_t onepass_reg_lds_bytes(int nw, int tpw, int layout) {
  const size_t stage = (size_t)nw * onepass_reg_stage_row(D, tpw, layout) * kSplitBlockRows;
  const size_t red = (size_t)(nw - 1) * (D / 16) * kWaveSize * 16;
  return onepass_reg_stage_offset<D>(nw) + (stage > red ? stage : red);
}

template <int D, int TPW, int NWMAX, int LAYOUT>
__global__ __launch_bounds__(kBlockThreads * NWMAX) void onepass_mfma_reg_kernel(SplitArgs a) {
  static_assert(LAYOUT == kLayoutPacked || LAYOUT == kLayoutStrided || LAYOUT == kLayoutPagedBlock ||
                    LAYOUT == kLayoutPaged,
                "packed, strided or paged");
  constexpr bool PAGED = LAYOUT == kLayoutPagedBlock;  // pages of at least 16 rows
  constexpr bool PAGED_ROWS = LAYOUT == kLayoutPaged;  // pages under 16 rows
  constexpr int QLD = D / 32;  // 16-byte K chunks per lane per tile
  constexpr int DPC = D / 16;  // output dims per lane (one P.V MFMA each)
  constexpr int VW = DPC / 2;  // dwords of a lane's V run per row
  constexpr int PF = onepass_reg_pf<D, TPW>();
  constexpr int NR = kSplitBlockRows;
  constexpr int R = TPW * NR;
  using Sh = GroupShape<D>;
  constexpr int LPH = Sh::LPH;
  constexpr int HPW = Sh::HPW;
  constexpr int RT = onepass_reg_round_tiles(D, TPW, LAYOUT);  // tiles per staging round
  constexpr int KR = NR * RT / HPW;                            // rows a lane group loads per round
  constexpr int KSR = onepass_reg_stage_row(D, TPW, LAYOUT);   // staging bytes per row
  static_assert(TPW % RT == 0, "whole rounds");
  extern __shared__ __attribute__((aligned(16))) char onepass_reg_lds[];
  const int lane = threadIdx.x & (kWaveSize - 1);
  const int nw = (int)(blockDim.x / kWaveSize);
  const int wv = __builtin_amdgcn_readfirstlane((int)(threadIdx.x / kWaveSize));
  const uint32_t hkv = (uint32_t)a.num_heads_kv;
  const uint32_t b = blockIdx.x / hkv;
  const uint32_t hk = blockIdx.x - b * hkv;
  if (b >= (uint32_t)a.batch) return;
  const int hq = a.num_heads_q;
  const int G = hq / (int)hkv;  // <= 16
  const int S = split_len_l<LAYOUT>(a, b);
  const int q = lane >> 4;
  const int n = lane & 15;
  const bool gok = n < G;
  const __amdgpu_buffer_rsrc_t o_rsrc =
      make_rsrc(a.o + ((uint64_t)b * hq + (uint64_t)hk * G) * D, (uint32_t)G * D * 2u);
  if (S <= 0 || S > a.max_rows) {
    // Empty rows give 0 (the reference loop's result), invalid ones NaN.
    if (wv != 0) return;
    const u32x4 fill = S == 0 ? u32x4{0u, 0u, 0u, 0u} : u32x4{0x7e007e00u, 0x7e007e00u, 0x7e007e00u, 0x7e007e00u};
    for (int k = lane; k < G * (D / 8); k += kWaveSize)
      buffer_store16(o_rsrc, (uint32_t)((k / (D / 8)) * D + (k % (D / 8)) * 8) * 2u, fill);
    return;
  }
  const int lo = wv * R;
  const int span = S - lo < 0 ? 0 : (S - lo < R ? S - lo : R);
  const int nt = (span + NR - 1) / NR;
  // Pages of at least 16 rows: a tile lies in one page.  Lane t < nt holds
  // the block-table entry of the wave's tile t (entry 0, which a batch with
  // rows always has, elsewhere), requested here, long before V needs it; K
  // and V share the table, so a negative entry among them makes the
  // (batch, KV head) invalid: its outputs are NaN and the unmapped rows are
  // never read.
  int32_t tile_entry = 0;
  int unmapped = 0;
  if constexpr (PAGED) {
    const int32_t* pages = a.block_table + (uint64_t)b * (uint64_t)a.bt_stride;
    const bool has = lane < nt;
    tile_entry = pages[has ? (uint32_t)(lo + lane * NR) >> (uint32_t)a.page_shift : 0u];
    unmapped = __builtin_amdgcn_ballot_w64(has && tile_entry < 0) != 0 ? 1 : 0;
  }

  // ---- K: scores of the wave's tiles, kept in x ----
  // A round of RT tiles: lane group s loads KR rows of tile s % RT (16
  // bytes per lane, chunk r; the whole tile with RT = HPW, its rows 8 (s /
  // RT) on with RT = HPW / 2), stores them to the wave's staging, and the
  // MFMA A operands (row n, chunks 4c + q) are read back from there; the
  // next round's rows are in flight during a round's products.  Tiles past
  // the wave's rows read 0 (without memory access; on pages under 16 rows
  // from Q's first row) and are masked; the loops carry no branch, one
  // branch skips them for a wave without rows.
  const __amdgpu_buffer_rsrc_t q_rsrc =
      make_rsrc(a.q + ((uint64_t)b * hq + (uint64_t)hk * G) * D, (uint32_t)G * D * 2u);
  bf16x8_v qb[QLD];
#pragma unroll
  for (int c = 0; c < QLD; ++c)
    qb[c] = __builtin_bit_cast(
        bf16x8_v, buffer_load16<kPolicyDefault>(q_rsrc, gok ? (uint32_t)(n * D + (4 * c + q) * 8) * 2u : kLaneOutOfRange));
  const int s = lane / LPH;
  const int r = lane % LPH;
  const int ps = s % RT;        // this lane group's tile of a round
  const int ph = (s / RT) * KR;  // and its first row in it
  char* stage = onepass_reg_lds + onepass_reg_stage_offset<D>(nw) + (size_t)wv * KSR * NR;
  typename std::conditional<PAGED || PAGED_ROWS, PagedLaneRows<D, PAGED>, LongRows<D, LAYOUT>>::type kr;
  kr.init(a, a.k, b, split_row_base<LAYOUT>(a, b), lo, lo + span, (int)hk, true, r, ps * NR + ph);
  f32x4_v x[TPW];
  float m = -__builtin_inff();
  if (nt > 0) {
    u32x4 kb[KR];
    // Pages under 16 rows: each row's block-table entry, requested a round
    // ahead of its rows (entries and rows complete in request order, so
    // the entries of round k + 2 go out after the rows of round k + 1,
    // and waiting for them waits for nothing the round does not need).
    int32_t ek[PAGED_ROWS ? KR : 1];
    if constexpr (PAGED_ROWS) {
      kr.template entries<KR>(ek, 0);
      kr.template load_entries<KR>(kb, 0, ek);
      if (TPW / RT > 1) kr.template entries<KR>(ek, RT * NR);
    } else {
      kr.template load<KR>(kb, 0);
    }
#pragma unroll
    for (int k = 0; k < TPW / RT; ++k) {
      wave_lds_sync();  // the previous round's reads of the staging are done
#pragma unroll
      for (int j = 0; j < KR; ++j) *reinterpret_cast<u32x4*>(stage + (ph + j) * KSR + ps * D * 2 + r * 16) = kb[j];
      wave_lds_sync();
      __builtin_amdgcn_sched_barrier(0);
      if constexpr (PAGED_ROWS) {
        if (k + 1 < TPW / RT) {
          kr.template load_entries<KR>(kb, (k + 1) * RT * NR, ek);
          if (k + 2 < TPW / RT) kr.template entries<KR>(ek, (k + 2) * RT * NR);
        }
      } else if (k + 1 < TPW / RT) {
        kr.template load<KR>(kb, (k + 1) * RT * NR);
      }
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int p = 0; p < RT; ++p) {
        const int t = k * RT + p;
        f32x4_v c4 = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int c = 0; c < QLD; ++c) {
          const bf16x8_v ka = *reinterpret_cast<const bf16x8_v*>(stage + n * KSR + p * D * 2 + (4 * c + q) * 16);
          c4 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ka, qb[c], c4, 0, 0, 0);
        }
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          x[t][e] = c4[e] * a.scale;
          m = t * NR + 4 * q + e < span ? fmaxf(m, x[t][e]) : m;
        }
      }
    }
  } else {
#pragma unroll
    for (int t = 0; t < TPW; ++t) x[t] = f32x4_v{0.0f, 0.0f, 0.0f, 0.0f};
  }
  // The wave's (max, sum) per column, over its four lane groups.
  const float cm = column_reduce<true>(m);
  float l = 0.0f;
#pragma unroll
  for (int t = 0; t < TPW; ++t) {
#pragma unroll
    for (int e = 0; e < 4; ++e) l += t * NR + 4 * q + e < span ? expf(x[t][e] - cm) : 0.0f;
  }
  const float cl = column_reduce<false>(l);
  float* pst = reinterpret_cast<float*>(onepass_reg_lds);  // [nw][16][2]
  if (q == 0) {
    pst[(wv * 16 + n) * 2] = cm;
    pst[(wv * 16 + n) * 2 + 1] = cl;
  }
  // V rows of the wave's first tiles, in flight across the exchange.
  // A wave of pages under 16 rows has met an unmapped page among its rows
  // if its K loads have (V reads the same rows through the same table).
  if constexpr (PAGED_ROWS) unmapped = __builtin_amdgcn_ballot_w64(kr.bad != 0) != 0 ? 1 : 0;
  LongRows<D, PAGED || PAGED_ROWS ? kLayoutPacked : LAYOUT> vrw;
  if constexpr (!PAGED && !PAGED_ROWS) vrw.init(a, a.v, b, split_row_base<LAYOUT>(a, b), 0, S, (int)hk, true, 0);
  const uint32_t v_row_bytes = (uint32_t)kv_heads_mem(a) * D * 2u;       // paged: bytes per slot
  const uint32_t v_head_off = (uint32_t)kv_head_mem(a, (int)hk) * D * 2u;  // paged: this KV head in a slot
  uint32_t vr[PF][4][VW];
  // Pages under 16 rows: the entries of this lane's four rows of a tile,
  // requested PF tiles ahead of the tile's rows (after the rows of the tile
  // PF steps earlier, so waiting for them waits only for rows already due).
  int32_t ev[PAGED_ROWS ? PF : 1][4];
  const int32_t* v_pages = a.block_table + (uint64_t)b * (uint64_t)a.bt_stride;
  auto v_entries = [&](int p, int t) {
    if constexpr (PAGED_ROWS) {
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int row = t * NR + 4 * q + e;
        ev[p][e] = v_pages[row < span ? (uint32_t)(lo + row) >> (uint32_t)a.page_shift : 0u];
      }
    }
  };
  auto v_load = [&](int p, int t) {
    if constexpr (PAGED_ROWS) {
      // Per-lane addresses; a row past the wave's rows or in an unmapped
      // page reads Q's first row (memory that exists) and becomes 0.
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int row = t * NR + 4 * q + e;
        const PagedRowU32 pr = paged_row_u32(ev[p][e], (uint32_t)(lo + row), (uint32_t)a.page_shift);
        const bool ok = row < span && !pr.unmapped;
        const uint16_t* src = ok ? a.v + (uint64_t)pr.page * (uint64_t)a.batch_stride +
                                       (uint64_t)pr.slot * (v_row_bytes >> 1) + (v_head_off >> 1) + n * DPC
                                 : a.q;
        if constexpr (VW == 2) {
          const u32x2 w2 = __builtin_nontemporal_load(reinterpret_cast<const u32x2*>(src));
          vr[p][e][0] = ok ? w2[0] : 0u;
          vr[p][e][1] = ok ? w2[1] : 0u;
        } else {
#pragma unroll
          for (int h = 0; h < VW / 4; ++h) {
            const u32x4 w4 = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(src) + h);
#pragma unroll
            for (int i = 0; i < 4; ++i) vr[p][e][4 * h + i] = ok ? w4[i] : 0u;
          }
        }
      }
      return;
    }
    // Paged: the tile's page through its entry (readlane: no table round
    // trip here), a descriptor over the tile's rows in it (none when the
    // entry is unmapped: nothing is read).
    __amdgpu_buffer_rsrc_t v_rsrc;
    if constexpr (PAGED) {
      const int32_t e = __builtin_amdgcn_readlane(tile_entry, t);
      const PagedRowU32 pr = paged_row_u32(e, (uint32_t)(lo + t * NR), (uint32_t)a.page_shift);
      const int rows = pr.unmapped ? 0 : (span - t * NR < 0 ? 0 : (span - t * NR < NR ? span - t * NR : NR));
      v_rsrc = make_rsrc(uniform_ptr(a.v + (uint64_t)pr.page * (uint64_t)a.batch_stride +
                                     (uint64_t)pr.slot * (v_row_bytes >> 1)),
                         (uint32_t)rows * v_row_bytes);
    } else {
      v_rsrc = vrw.rsrc;
    }
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int row = t * NR + 4 * q + e;
      uint32_t off;
      if constexpr (PAGED)  // from the tile's first row
        off = row < span ? v_head_off + (uint32_t)(4 * q + e) * v_row_bytes + (uint32_t)(n * DPC * 2) : kRowOutOfRange;
      else
        off = row < span ? vrw.lane_off + (uint32_t)(lo + row) * vrw.row_bytes + (uint32_t)(n * DPC * 2)
                         : kRowOutOfRange;
      if constexpr (VW == 2) {
        const u32x2 w2 = __builtin_bit_cast(
            u32x2, __builtin_amdgcn_raw_buffer_load_b64(v_rsrc, (int)off, 0, kPolicyStream));
        vr[p][e][0] = w2[0];
        vr[p][e][1] = w2[1];
      } else {
#pragma unroll
        for (int h = 0; h < VW / 4; ++h) {
          const u32x4 w4 = buffer_load16_nt(v_rsrc, off + (uint32_t)h * 16u);
#pragma unroll
          for (int i = 0; i < 4; ++i) vr[p][e][4 * h + i] = w4[i];
        }
      }
    }
  };
  if constexpr (PAGED_ROWS) {
#pragma unroll
    for (int p = 0; p < PF; ++p) v_entries(p, p);
  }
#pragma unroll
  for (int p = 0; p < PF; ++p) v_load(p, p);
  if constexpr (PAGED_ROWS) {
#pragma unroll
    for (int p = 0; p < PF; ++p) v_entries(p, p + PF);
  }
  const int poisoned = PAGED || PAGED_ROWS ? __syncthreads_or(unmapped) : (__syncthreads(), 0);
  float gm = -__builtin_inff();
  for (int w = 0; w < nw; ++w) gm = fmaxf(gm, pst[(w * 16 + n) * 2]);
  float gl = 0.0f;
  for (int w = 0; w < nw; ++w) {
    const float mw = pst[(w * 16 + n) * 2];
    gl += mw == -__builtin_inff() ? 0.0f : pst[(w * 16 + n) * 2 + 1] * (mw == gm ? 1.0f : expf(mw - gm));
  }

  // ---- V: weights from x ----
  f32x4_v acc[DPC];
#pragma unroll
  for (int dt = 0; dt < DPC; ++dt) acc[dt] = f32x4_v{0.0f, 0.0f, 0.0f, 0.0f};
  if (nt > 0) {
#pragma unroll
    for (int t = 0; t < TPW; ++t) {
      bf16x4_v pa;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const bool valid = gok && t * NR + 4 * q + e < span;
        pa[e] = (__bf16)(valid ? expf(x[t][e] - gm) / gl : 0.0f);
      }
      const int p = t % PF;
#pragma unroll
      for (int dt = 0; dt < DPC; ++dt) {
        const uint32_t sel = (dt & 1) ? kPermHi : kPermLo;
        const u32x2 w2 = {__builtin_amdgcn_perm(vr[p][1][dt / 2], vr[p][0][dt / 2], sel),
                          __builtin_amdgcn_perm(vr[p][3][dt / 2], vr[p][2][dt / 2], sel)};
        acc[dt] = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(pa, __builtin_bit_cast(bf16x4_v, w2), acc[dt], 0, 0, 0);
      }
      if (t + PF < TPW) {
        v_load(p, t + PF);
        if (t + 2 * PF < TPW) v_entries(p, t + 2 * PF);
      }
      __builtin_amdgcn_sched_barrier(0);
    }
  }

  // ---- waves 1..nw-1 -> wave 0 ----
  if (nw > 1) {
    f32x4_v* red = reinterpret_cast<f32x4_v*>(onepass_reg_lds + onepass_reg_stage_offset<D>(nw));
    if (wv > 0) {
#pragma unroll
      for (int dt = 0; dt < DPC; ++dt) red[((size_t)(wv - 1) * DPC + dt) * kWaveSize + lane] = acc[dt];
    }
    __syncthreads();
    if (wv > 0) return;
    for (int w = 1; w < nw; ++w) {
#pragma unroll
      for (int dt = 0; dt < DPC; ++dt) {
        const f32x4_v y = red[((size_t)(w - 1) * DPC + dt) * kWaveSize + lane];
#pragma unroll
        for (int e = 0; e < 4; ++e) acc[dt][e] += y[e];
      }
    }
  }
  // Lane (q, n) holds query rows 4q..4q+3, dims [n DPC, n DPC + DPC);
  // NaN for a (batch, KV head) that met an unmapped page.
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const int g = 4 * q + e;
    float v[DPC];
#pragma unroll
    for (int dt = 0; dt < DPC; ++dt) v[dt] = poisoned ? __builtin_nanf("") : acc[dt][e];
    store_f16_run<DPC>(o_rsrc, g < G ? (uint32_t)(g * D + n * DPC) * 2u : kLaneOutOfRange, v);
  }
}

}  // namespace fmha_decode
