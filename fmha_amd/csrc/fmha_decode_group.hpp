// fmha_decode_group.hpp -- gfx950 decode attention on the matrix cores for
// any number of query heads per KV head (G = Hq / Hkv >= 1), KV length 0..16
// per sequence, bf16 Q/K/V, fp32 accumulation, fp16 output.
//
// Same semantics as fmha_decode_fwd_kernel (the reference CPU loop,
// fmha_host.cpp:169-245, with KV head h / G): fp32 scores, scale, masked
// max-subtracted softmax with a sum > 0 guard, weights rounded to bf16 after
// normalisation, fp32 P.V, one RNE rounding to fp16.  Only the order of the
// fp32 sums differs (matrix-core accumulation).
//
// Why a second kernel: the VALU kernel spends about 4*G*S v_dot2 per lane on
// Q.K^T plus a butterfly over G*S partial scores, so from G = 4 its waves
// compute for about as long as their loads take, and it holds G query
// vectors in registers (G <= 8).  Here the two products are MFMAs:
//
//   * A "stream" is one (batch, KV head); stream sigma = b * Hkv + h owns
//     query rows [sigma*G, sigma*G + G) of Q and O, so the query rows of
//     consecutive streams are contiguous whatever Hkv is.  A wave takes HPW =
//     64 / (D/8) consecutive streams (several batches when Hkv < HPW) and
//     loads K and V exactly like the VALU kernel: D/8 lanes per stream, one
//     16-byte chunk of one row per lane and instruction, all rows issued at
//     once, rows past a stream's length out of range.
//   * Query columns are taken in tiles of 16 (an MFMA's N): NS = 4 streams
//     of 4 columns for G <= 4, NS = 2 of 8 for G <= 8, one stream per tile
//     above (query heads [16c, 16c + 16) of tile c); columns at or past G
//     are padding that is never stored.  A wave handles HPW / NS tiles;
//     larger groups take ceil(G / 16) waves per stream group, each loading
//     the K/V of only the streams its tiles use (a stream whose tiles two
//     waves share is read by both, on one XCD, so that the second read hits
//     its L2).  The query rows of a wave's
//     tiles are one contiguous range of Q; each lane loads its column's query
//     words straight into the B operand (8 dims per MFMA step), so Q takes
//     no LDS.
//   * K goes to LDS as rows; per tile and stream S^T = K_p . Q^T is D/32
//     v_mfma_f32_16x16x32_bf16 (A = 16 K rows of stream p, B = the tile's 16
//     query columns), each column keeping its own stream's pass.  No product
//     ever mixes two streams' data, so a non-finite value in one stream
//     cannot reach another.
//   * The 16x16 accumulator holds, per lane, rows 4q..4q+3 of one query
//     column: the softmax reduces over those 4 values and across the 4 lane
//     groups (v_permlane16/32_swap), and the bf16 weights it leaves are
//     already the A operand of a v_mfma_f32_16x16x16_bf16 (rows 4q..4q+3 of
//     query i in lane (q, i)).
//   * V is transposed into LDS with v_perm from the coalesced registers
//     ([stream][8-dim block][dim][16 rows], 16 bytes of padding per block),
//     over the K rows, which are dead by then; per tile and stream P.V is
//     D/16 MFMAs, each output row keeping its own stream's; column n covers
//     dims [n*D/16, (n+1)*D/16) (D <= 128; at D = 256 two runs of 8,
//     out_dim) so each lane stores whole 8/16-byte runs.
//   * 48 MFMAs per wave for G <= 16 at every D.
#pragma once

#include "fmha_decode_kernel.hpp"

namespace fmha_decode {

typedef __bf16 bf16x8_v __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4_v __attribute__((ext_vector_type(4)));
typedef float f32x4_v __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

struct GroupArgs {
  const uint16_t* q;       // [streams * G, D] bf16 bits (= [batch, Hq, D])
  const uint16_t* k;       // bf16 bits, packed, strided or paged (LAYOUT)
  const uint16_t* v;
  uint16_t* o;             // [batch, Hq, D] fp16 bits
  const int32_t* lens;     // packed: [batch + 1] row offsets; strided: [batch] lengths; or null
  int32_t seqlen_uniform;  // rows per batch when lens is null
  int32_t max_rows;        // longest valid length (16; strided: the rows each batch has, capped at 16)
  int64_t batch_stride;    // strided: elements between batches; paged: between pages
  int32_t row_stride;      // elements between rows (packed: Hkv * D)
  int32_t head_stride;     // elements between KV heads (packed: D)
  int32_t num_heads_kv;
  int32_t group;           // G = Hq / Hkv
  uint32_t streams;        // batch * Hkv
  uint32_t stream_groups;  // ceil(streams / HPW)
  int32_t tiles_per_stream;  // ceil(G / 16): 16-row query tiles per stream
  int32_t chunks;          // waves per stream group: ceil(HPW * tiles_per_stream / HPW) = tiles_per_stream
  uint32_t waves;          // grid size (>= stream_groups * chunks)
  float scale;
  const int32_t* block_table;  // paged: [batch, bt_stride] page indices
  int32_t bt_stride;
};

template <int D>
struct GroupShape {
  static constexpr int LPH = D / 8;               // lanes per stream (one 16-byte chunk each)
  static constexpr int HPW = kWaveSize / LPH;     // streams per wave
  static constexpr int KS = HPW * D * 2 + 16;     // LDS bytes per K row (all streams) + padding
  static constexpr int VB = 8 * kMaxSeq * 2 + 16; // LDS bytes per 8-dim block of V^T + padding
  static constexpr int VSTREAM = (D / 8) * VB;    // LDS bytes of one stream's V^T
  static constexpr int DPC = D / 16;              // output dims per P.V column
  static constexpr int QLD = D / 32;              // 16-byte Q loads per lane per tile
  // K rows are dead once every tile's scores are formed, so V^T reuses them.
  static constexpr int KV_LDS = (kMaxSeq * KS > HPW * VSTREAM) ? kMaxSeq * KS : HPW * VSTREAM;
  static constexpr int lds_bytes() { return KV_LDS; }
};

__device__ __forceinline__ int shfl_i(int x, int src) { return __shfl(x, src, kWaveSize); }

// Max or sum over lanes l, l^16, l^32, l^48 (one column of a 16x16 MFMA
// tile).  v_permlane16_swap / v_permlane32_swap with both operands x return
// x of this lane and of its partner (l^16, l^32), in some order: combining
// the two halves needs no lane select and gives every lane the same bits.
template <bool IS_MAX>
__device__ __forceinline__ float column_reduce(float x) {
  const auto a = __builtin_amdgcn_permlane16_swap(__builtin_bit_cast(uint32_t, x), __builtin_bit_cast(uint32_t, x),
                                                  false, false);
  const float a0 = __builtin_bit_cast(float, (uint32_t)a[0]);
  const float a1 = __builtin_bit_cast(float, (uint32_t)a[1]);
  x = IS_MAX ? fmaxf(a0, a1) : a0 + a1;
  const auto b = __builtin_amdgcn_permlane32_swap(__builtin_bit_cast(uint32_t, x), __builtin_bit_cast(uint32_t, x),
                                                  false, false);
  const float b0 = __builtin_bit_cast(float, (uint32_t)b[0]);
  const float b1 = __builtin_bit_cast(float, (uint32_t)b[1]);
  return IS_MAX ? fmaxf(b0, b1) : b0 + b1;
}

// v_perm selector: low halves / high halves of two dwords (lo, hi) -> one dword.
constexpr uint32_t kPermLo = 0x05040100u;
constexpr uint32_t kPermHi = 0x07060302u;

// Output dim of P.V column n's dt-th value (dt < DPC = D / 16): n * DPC +
// dt up to 8 dims per column; above (D = 256), column n takes dims [128h +
// 8n, 128h + 8n + 8) for h = dt / 8, so each store instruction of a row
// (one per h) covers 256 contiguous bytes over the row's 16 lanes rather
// than every other 16 bytes of 512 (half-written lines doubled the HBM
// write bytes), and the V^T reads land on distinct banks.
template <int DPC>
__device__ __forceinline__ int out_dim(int n, int dt) {
  return DPC <= 8 ? n * DPC + dt : (dt / 8) * 128 + n * 8 + dt % 8;
}

// One wave: HPW consecutive streams of stream group sg (wave-local stream
// p = 0..HPW-1), KV bucket SMAX, query tiles [chunk*TW, chunk*TW + TW) of the
// group's tile list (TW = HPW / NS tiles per wave).  A tile's 16 columns hold
// NS streams of CPS = 16 / NS query columns each: with NS > 1 (G <= CPS)
// tile tau holds streams [tau*NS, tau*NS + NS) and column n query head n %
// CPS of stream tau*NS + n / CPS; with NS = 1 tile tau holds query heads
// [16c, 16c + 16) of stream tau / TPS, c = tau % TPS (TPS = ceil(G / 16)).
// Columns whose query head is at or past G are padding, never stored.  The
// rows of a wave's tiles are one contiguous range [R0, R0 + nrows) of Q.
// LANES: kbase and vbase are this lane's own addresses (its stream's row 0
// plus its 16-byte chunk) and load_rows its rows to read (0 for a lane that
// reads nothing); kv_off and records are then unused.
template <int D, int SMAX, int NS, bool LANES>
__device__ __forceinline__ void group_unit(const GroupArgs& a, uint32_t sg, int chunk, int lane, int S,
                                           uint32_t kv_off, const uint16_t* kbase, const uint16_t* vbase,
                                           uint32_t row_bytes, uint32_t records, uint64_t bad_mask, char* lds,
                                           int load_rows) {
  using Sh = GroupShape<D>;
  constexpr int LPH = Sh::LPH;
  constexpr int HPW = Sh::HPW;
  constexpr int TW = HPW / NS;   // tiles per wave
  constexpr int CPS = 16 / NS;   // query columns per stream in a tile
  const int s = lane / LPH;
  const int r = lane % LPH;
  const int q = lane >> 4;   // MFMA lane group
  const int n = lane & 15;   // MFMA row / column inside the 16x16 tile
  const int G = a.group;
  const int TPS = a.tiles_per_stream;  // 1 when NS > 1

  char* k_lds = lds;
  char* v_lds = lds;  // written after the last read of k_lds

  // ---- this wave's tiles and query rows ----
  const uint32_t sigma0 = sg * HPW;
  const int nstreams = (int)min(a.streams - sigma0, (uint32_t)HPW);  // valid streams of the group
  const int ntiles_group = ((nstreams + NS - 1) / NS) * TPS;
  const int tau0 = chunk * TW;
  const int ntiles = min(ntiles_group - tau0, TW);                    // > 0
  const int tau1 = tau0 + ntiles - 1;
  const int R0 = (tau0 / TPS) * NS * G + (tau0 % TPS) * 16;
  const int p1 = min((tau1 / TPS) * NS + NS, nstreams) - 1;
  const int nrows = p1 * G + min(16 * (tau1 % TPS) + 16, G) - R0;     // <= 16 * TW
  const uint64_t qrow0 = (uint64_t)sigma0 * G + R0;
  const __amdgpu_buffer_rsrc_t q_rsrc = make_rsrc(a.q + qrow0 * D, (uint32_t)nrows * D * 2u);
  const __amdgpu_buffer_rsrc_t o_rsrc = make_rsrc(a.o + qrow0 * D, (uint32_t)nrows * D * 2u);

  // ---- issue every load: the query words straight into the B operand of
  //      the score MFMA (lane (q, n): 8 dims of column n's query row per
  //      step), K rows, V rows ----
  const int slot_col = n / CPS;  // stream slot of this lane's column
  bf16x8_v qb[TW][Sh::QLD];
#pragma unroll
  for (int i = 0; i < TW; ++i) {
    const int tau = tau0 + i;
    const int p_col = (tau / TPS) * NS + slot_col;
    const int g_col = (tau % TPS) * 16 + n % CPS;
    // Padding columns (and tiles past the wave's) read nothing: zero scores, never used.
    const bool col_ok = i < ntiles && g_col < G && p_col < nstreams;
    const uint32_t qoff = col_ok ? (uint32_t)((p_col * G + g_col - R0) * D + 8 * q) * 2u : kLaneOutOfRange;
#pragma unroll
    for (int cc = 0; cc < Sh::QLD; ++cc)
      qb[i][cc] = __builtin_bit_cast(bf16x8_v, buffer_load16<kPolicyDefault>(q_rsrc, qoff + (uint32_t)cc * 64u));
  }
  u32x4 kr[SMAX];
  u32x4 vr[SMAX];
  if constexpr (LANES) {
    // Rows j < load_rows, row_stride elements apart; zeros beyond, as the
    // descriptor form's out-of-range rows.
    const uint32_t row_elems = (uint32_t)a.row_stride;
#pragma unroll
    for (int j = 0; j < SMAX; ++j) {
      kr[j] = u32x4{0u, 0u, 0u, 0u};
      if (j < load_rows) kr[j] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(kbase + j * row_elems));
    }
#pragma unroll
    for (int j = 0; j < SMAX; ++j) {
      vr[j] = u32x4{0u, 0u, 0u, 0u};
      if (j < load_rows) vr[j] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(vbase + j * row_elems));
    }
  } else {
    const __amdgpu_buffer_rsrc_t k_rsrc = make_rsrc(kbase, records);
    const __amdgpu_buffer_rsrc_t v_rsrc = make_rsrc(vbase, records);
#pragma unroll
    for (int j = 0; j < SMAX; ++j)
      kr[j] = buffer_load16<kPolicyStream>(k_rsrc, kv_off + (j < S ? (uint32_t)j * row_bytes : kRowOutOfRange));
#pragma unroll
    for (int j = 0; j < SMAX; ++j)
      vr[j] = buffer_load16<kPolicyStream>(v_rsrc, kv_off + (j < S ? (uint32_t)j * row_bytes : kRowOutOfRange));
  }
  __builtin_amdgcn_sched_barrier(0);

  // ---- K rows to LDS ----
#pragma unroll
  for (int j = 0; j < SMAX; ++j) *reinterpret_cast<u32x4*>(k_lds + j * Sh::KS + s * D * 2 + r * 16) = kr[j];
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");

  // ---- per tile: one S^T = K_p . Q^T pass per stream, each column keeping
  //      its own stream's; masked softmax; bf16 weights stay in registers ----
  bf16x4_v pa[TW];
  const int krow = n < SMAX ? n : 0;  // K rows past the bucket are never valid: any finite row will do
#pragma unroll
  for (int i = 0; i < TW; ++i) {
    pa[i] = bf16x4_v{0, 0, 0, 0};
    if (i >= ntiles) continue;
    const int tau = tau0 + i;
    const int pt = (tau / TPS) * NS;    // the tile's first stream
    const int p_col = pt + slot_col;
    f32x4_v st;
#pragma unroll
    for (int k = 0; k < NS; ++k) {
      const int p = min(pt + k, HPW - 1);
      f32x4_v c4 = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
      for (int cc = 0; cc < Sh::QLD; ++cc) {
        const bf16x8_v ka = *reinterpret_cast<const bf16x8_v*>(k_lds + krow * Sh::KS + p * D * 2 + (4 * cc + q) * 16);
        c4 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ka, qb[i][cc], c4, 0, 0, 0);
      }
      if (k == 0) {
        st = c4;
      } else {
#pragma unroll
        for (int e = 0; e < 4; ++e) st[e] = slot_col == k ? c4[e] : st[e];
      }
    }
    // Masked softmax over the 16 rows of this lane's query column: rows
    // 4q..4q+3 here, the rest in lanes n + 16, n + 32, n + 48.
    int S_col = __builtin_amdgcn_readlane(S, min(pt, HPW - 1) * LPH);
#pragma unroll
    for (int k = 1; k < NS; ++k) {
      const int S_k = __builtin_amdgcn_readlane(S, min(pt + k, HPW - 1) * LPH);
      S_col = slot_col == k ? S_k : S_col;
    }
    float x[4];
    float m = -__builtin_inff();
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      x[e] = st[e] * a.scale;
      m = (4 * q + e < S_col) ? fmaxf(m, x[e]) : m;
    }
    m = column_reduce<true>(m);
    float sum = 0.0f;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      x[e] = (4 * q + e < S_col) ? expf(x[e] - m) : 0.0f;
      sum += x[e];
    }
    sum = column_reduce<false>(sum);
#pragma unroll
    for (int e = 0; e < 4; ++e) pa[i][e] = (__bf16)((sum > 0.0f) ? (x[e] / sum) : 0.0f);
    // A stream with an invalid length gets NaN weights, so every output of
    // its columns is NaN (NaN times any V value, zero included).
    if ((bad_mask >> (uint32_t)(min(p_col, HPW - 1) * LPH)) & 1u)
      pa[i] = bf16x4_v{__builtin_nanf(""), __builtin_nanf(""), __builtin_nanf(""), __builtin_nanf("")};
  }

  // ---- V^T to LDS (over the K rows, whose last read is above): block r of
  //      stream s, [dim e][16 rows], from the row registers ----
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll
  for (int e = 0; e < 8; ++e) {
#pragma unroll
    for (int half = 0; half < 2; ++half) {
      u32x4 w;
#pragma unroll
      for (int pp = 0; pp < 4; ++pp) {
        const int j0 = 8 * half + 2 * pp;
        const uint32_t v0 = j0 < SMAX ? (uint32_t)vr[j0 < SMAX ? j0 : 0][e / 2] : 0u;
        const uint32_t v1 = j0 + 1 < SMAX ? (uint32_t)vr[j0 + 1 < SMAX ? j0 + 1 : 0][e / 2] : 0u;
        w[pp] = __builtin_amdgcn_perm(v1, v0, (e & 1) ? kPermHi : kPermLo);
      }
      *reinterpret_cast<u32x4*>(v_lds + s * Sh::VSTREAM + r * Sh::VB + e * (kMaxSeq * 2) + half * 16) = w;
    }
  }
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");

  // ---- per tile: one P.V pass per stream, each row keeping its own
  //      stream's; lane (q, n) ends with rows 4q..4q+3 of the tile, dims
  //      [n*DPC, n*DPC + DPC) ----
  constexpr int DPC = Sh::DPC;
#pragma unroll
  for (int i = 0; i < TW; ++i) {
    if (i >= ntiles) continue;
    const int tau = tau0 + i;
    const int pt = (tau / TPS) * NS;
    const int c16 = (tau % TPS) * 16;
    f32x4_v acc[DPC];
#pragma unroll
    for (int k = 0; k < NS; ++k) {
      const char* vs = v_lds + min(pt + k, HPW - 1) * Sh::VSTREAM;
#pragma unroll
      for (int dt = 0; dt < DPC; ++dt) {
        const int dim = out_dim<DPC>(n, dt);
        const bf16x4_v vb =
            *reinterpret_cast<const bf16x4_v*>(vs + (dim / 8) * Sh::VB + (dim % 8) * (kMaxSeq * 2) + q * 8);
        const f32x4_v c4 =
            __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(pa[i], vb, f32x4_v{0.0f, 0.0f, 0.0f, 0.0f}, 0, 0, 0);
        if (k == 0) {
          acc[dt] = c4;
        } else {
#pragma unroll
          for (int e = 0; e < 4; ++e) acc[dt][e] = (4 * q + e) / CPS == k ? c4[e] : acc[dt][e];
        }
      }
    }
    // ---- fp16 (RNE) output: row 4q + e is query head c16 + (4q+e) % CPS of
    //      stream pt + (4q+e) / CPS ----
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int p = pt + (4 * q + e) / CPS;
      const int g = c16 + (4 * q + e) % CPS;
      const uint32_t off =
          (g < G && p < nstreams) ? (uint32_t)((p * G + g - R0) * D + out_dim<DPC>(n, 0)) * 2u : kLaneOutOfRange;
#pragma unroll
      for (int h8 = 0; h8 < (DPC + 7) / 8; ++h8) {
        constexpr int W = DPC < 8 ? DPC : 8;  // dims per store
        float vals[8];
#pragma unroll
        for (int k8 = 0; k8 < 8; ++k8) vals[k8] = k8 < W ? acc[h8 * 8 + (k8 < W ? k8 : 0)][e] : 0.0f;
        const u32x4 pk = pack_f16x8(vals);
        if constexpr (W == 8) {
          buffer_store16(o_rsrc, off + h8 * 256, pk);  // out_dim(n, 8 * h8) = out_dim(n, 0) + 128 * h8
        } else {
          __builtin_amdgcn_raw_buffer_store_b64(u32x2{pk[0], pk[1]}, o_rsrc, (int)off, 0, kPolicyStreamStore);
        }
      }
    }
  }
}

// Grid: a.waves one-wave workgroups.  Workgroup w serves stream group
// ((w / 8) / chunks) * 8 + w % 8 and tile chunk (w / 8) % chunks, so the
// chunks of one stream group (G > 16) run on one XCD (dispatch is
// round-robin over the 8 XCDs) at nearly the same time and their K/V re-reads
// hit its L2; with chunks == 1 it is stream group w.
// SB = 1, 2, 4, 8, 16: uniform lengths (lens == null, seqlen_uniform <= SB);
// SB = 0: lengths from lens (or uniform), the bucket chosen per wave.
// LAYOUT: kLayoutPacked (rows [lens[b], lens[b+1]) of [rows, Hkv, D]) or
// kLayoutStrided (element (b, j, h, d) at b*batch_stride + j*row_stride +
// h*head_stride + d, lengths lens[b]); one descriptor spans the wave's
// streams from its first batch (the host bounds that span below 1 GiB).
// kLayoutPaged: row j of batch b in slot j of page block_table[b *
// bt_stride] (pages batch_stride elements apart), lengths lens[b]; launched
// only where a wave's streams share one batch (Hkv a multiple of HPW) and
// no length the wave accepts (max_rows) reaches past that first page, so
// the descriptor is based at the page.  A negative entry, or a wave whose
// streams would span batches, makes the batch invalid (NaN output) and
// nothing of it is read.  kLayoutPagedLanes: the same rows through a 64-bit
// address per lane, for waves whose streams span batches (Hkv below HPW or
// not a multiple of it), each lane looking up its own batch's page.
template <int D, int SB, int NS, int LAYOUT>
__global__ __launch_bounds__(kBlockThreads) void fmha_decode_group_kernel(GroupArgs a) {
  static_assert(LAYOUT == kLayoutPacked || LAYOUT == kLayoutStrided || LAYOUT == kLayoutPaged ||
                    LAYOUT == kLayoutPagedLanes,
                "one descriptor per wave, or one address per lane");
  constexpr bool LANES = LAYOUT == kLayoutPagedLanes;
  using Sh = GroupShape<D>;
  constexpr int LPH = Sh::LPH;
  constexpr int HPW = Sh::HPW;
  constexpr int TW = HPW / NS;  // tiles per wave
  __shared__ __attribute__((aligned(16))) char lds[Sh::lds_bytes()];

  const int lane = threadIdx.x & (kWaveSize - 1);
  const uint32_t w = blockIdx.x;
  const uint32_t chunks = (uint32_t)a.chunks;
  const uint32_t rest = w >> 3;
  const uint32_t sg = (rest / chunks) * 8u + (w & 7u);
  const int chunk = (int)(rest % chunks);
  if (sg >= a.stream_groups) return;
  const uint32_t sigma0 = sg * HPW;
  const int nstreams = (int)min(a.streams - sigma0, (uint32_t)HPW);
  if (((nstreams + NS - 1) / NS) * a.tiles_per_stream <= chunk * TW) return;

  // ---- this lane's stream: batch, head, first element relative to the
  //      wave's base (its first batch) ----
  const int s = lane / LPH;
  const int r = lane % LPH;
  const uint32_t Hkv = (uint32_t)a.num_heads_kv;
  const uint32_t sig = sigma0 + (uint32_t)s;
  const bool sok = sig < a.streams;
  const uint32_t bq = sok ? sig / Hkv : 0u;
  const uint32_t h = sok ? sig - bq * Hkv : 0u;
  const uint32_t b_first = sigma0 / Hkv;
  const uint32_t row_bytes = (uint32_t)a.row_stride * 2u;
  int S;
  bool bad;
  uint64_t base_elem;
  int64_t lane_elem;  // row 0 of this lane's stream, relative to base_elem
  uint32_t end;       // byte just past the last row this lane reads
  if constexpr (LAYOUT == kLayoutPacked) {
    int64_t row_first, row0;
    if (a.lens) {
      row_first = a.lens[b_first];
      row0 = a.lens[bq];
      S = (int)(a.lens[bq + 1] - row0);
    } else {
      S = a.seqlen_uniform;
      row_first = (int64_t)b_first * S;
      row0 = (int64_t)bq * S;
    }
    const int64_t rel = row0 - row_first;
    // A length outside [0, max_rows] (max_rows <= 16), or a table that puts
    // this batch beyond the reach of the wave's descriptor, makes the stream
    // invalid (NaN output).
    bad = sok && (S < 0 || S > a.max_rows || rel < 0 ||
                  (rel + kMaxSeq) * (int64_t)row_bytes >= (int64_t)kLaneOutOfRange);
    base_elem = (uint64_t)row_first * a.row_stride;
    lane_elem = rel * a.row_stride + (int64_t)h * a.head_stride;
    end = (sok && !bad && S > 0) ? (uint32_t)((rel + S) * (int64_t)row_bytes) : 0u;
  } else if constexpr (LAYOUT == kLayoutPaged) {
    S = a.lens[bq];
    const int32_t entry = __builtin_amdgcn_readfirstlane(a.block_table[(int64_t)b_first * a.bt_stride]);
    bad = sok && (S < 0 || S > a.max_rows || (S > 0 && entry < 0) || bq != b_first);
    base_elem = entry < 0 ? 0u : (uint64_t)(uint32_t)entry * (uint64_t)a.batch_stride;
    lane_elem = (int64_t)h * a.head_stride;
    end = (sok && !bad && S > 0) ? (uint32_t)((lane_elem + (int64_t)(S - 1) * a.row_stride + D) * 2) : 0u;
  } else if constexpr (LANES) {
    S = sok ? a.lens[bq] : 0;
    const int32_t entry = a.block_table[(int64_t)bq * a.bt_stride];
    bad = sok && (S < 0 || S > a.max_rows || (S > 0 && entry < 0));
    base_elem = 0;
    lane_elem = (sok && !bad && S > 0) ? (int64_t)entry * a.batch_stride + (int64_t)h * a.head_stride : 0;
    end = 0u;
  } else {
    S = a.lens ? a.lens[bq] : a.seqlen_uniform;
    bad = sok && (S < 0 || S > a.max_rows);
    base_elem = (uint64_t)b_first * (uint64_t)a.batch_stride;
    lane_elem = (int64_t)(bq - b_first) * a.batch_stride + (int64_t)h * a.head_stride;
    end = (sok && !bad && S > 0) ? (uint32_t)((lane_elem + (int64_t)(S - 1) * a.row_stride + D) * 2) : 0u;
  }
  if (!sok || bad) S = 0;
  // With one stream per tile and several tiles per stream (G > 16), a
  // chunk's tiles use only some of the group's streams: the other lanes load
  // nothing (those streams' K/V belong to another chunk's tiles).
  const int tps = a.tiles_per_stream;
  const int tau0 = chunk * TW;
  const int tau1 = min(tau0 + TW, ((nstreams + NS - 1) / NS) * tps) - 1;
  const bool used = s >= (tau0 / tps) * NS && s < (tau1 / tps) * NS + NS;
  const uint32_t kv_off =
      (sok && !bad && used && !LANES) ? (uint32_t)(lane_elem * 2) + (uint32_t)r * 16u : kLaneOutOfRange;
  const int load_rows = (sok && !bad && used) ? S : 0;
  // Descriptor range: the end of the last row any lane reads; bucket: the
  // longest length of the wave; invalid streams as a bit per stream.
  int smax = S;
#pragma unroll
  for (int m = 1; m < kWaveSize; m <<= 1) {
    smax = max(smax, __shfl_xor(smax, m, kWaveSize));
    end = max(end, (uint32_t)__shfl_xor((int)end, m, kWaveSize));
  }
  const uint32_t records = (uint32_t)__builtin_amdgcn_readfirstlane((int)end);
  smax = __builtin_amdgcn_readfirstlane(smax);
  const uint64_t bad_mask = __ballot(bad && r == 0);
  const uint16_t* kbase = LANES ? a.k + lane_elem + r * 8 : a.k + base_elem;
  const uint16_t* vbase = LANES ? a.v + lane_elem + r * 8 : a.v + base_elem;

#define FMHA_GROUP_UNIT(SM) \
  group_unit<D, SM, NS, LANES>(a, sg, chunk, lane, S, kv_off, kbase, vbase, row_bytes, records, bad_mask, lds, load_rows)
  if constexpr (SB != 0) {
    FMHA_GROUP_UNIT(SB);
  } else {
    if (smax <= 1)
      FMHA_GROUP_UNIT(1);
    else if (smax <= 2)
      FMHA_GROUP_UNIT(2);
    else if (smax <= 4)
      FMHA_GROUP_UNIT(4);
    else if (smax <= 8)
      FMHA_GROUP_UNIT(8);
    else
      FMHA_GROUP_UNIT(16);
  }
#undef FMHA_GROUP_UNIT
}

// ---------------------------------------------------------------------------
// Query-group padding for the long-row paths (split-KV, single pass, paged
// short kernel), whose kernels exist for G in {1, 2, 4, 8}: another G runs
// on copies of Q and O with GP (4 or 8) rows per stream.  The copy for query
// heads [g0, g0 + gn) of every stream (gn <= GP; G > 8 takes several such
// slices in turn) holds Q row sigma*G + g0 + g at row sigma*GP + g for g < gn
// and zero rows above; the O rows go back the same way.  One thread per
// 16-byte chunk; every index is checked against the element counts.
// ---------------------------------------------------------------------------
constexpr int kPadThreads = 256;

// Defined in one translation unit only (FMHA_DECODE_SHARED_KERNELS): they
// are not templates, so every other one must not emit them again.
#ifdef FMHA_DECODE_SHARED_KERNELS
__global__ __launch_bounds__(kPadThreads) void pad_query_group_kernel(const uint16_t* q, uint16_t* qp,
                                                                       uint64_t streams, int G, int g0, int gn,
                                                                       int GP, int D) {
  const uint64_t cpr = (uint64_t)(D / 8);  // 16-byte chunks per row
  const uint64_t i = (uint64_t)blockIdx.x * kPadThreads + threadIdx.x;
  if (i >= streams * (uint64_t)GP * cpr) return;
  const uint64_t row = i / cpr;
  const uint64_t c = i - row * cpr;
  const uint64_t sigma = row / (uint64_t)GP;
  const int g = (int)(row - sigma * (uint64_t)GP);
  u32x4 x = {0u, 0u, 0u, 0u};
  if (g < gn) x = *reinterpret_cast<const u32x4*>(q + ((sigma * (uint64_t)G + g0 + g) * D + c * 8));
  *reinterpret_cast<u32x4*>(qp + (row * D + c * 8)) = x;
}

__global__ __launch_bounds__(kPadThreads) void unpad_output_group_kernel(const uint16_t* op, uint16_t* o,
                                                                          uint64_t streams, int G, int g0, int gn,
                                                                          int GP, int D) {
  const uint64_t cpr = (uint64_t)(D / 8);
  const uint64_t i = (uint64_t)blockIdx.x * kPadThreads + threadIdx.x;
  if (i >= streams * (uint64_t)gn * cpr) return;
  const uint64_t row = i / cpr;  // row of the slice: stream sigma, head g
  const uint64_t c = i - row * cpr;
  const uint64_t sigma = row / (uint64_t)gn;
  const uint64_t g = row - sigma * (uint64_t)gn;
  *reinterpret_cast<u32x4*>(o + ((sigma * (uint64_t)G + g0 + g) * D + c * 8)) =
      *reinterpret_cast<const u32x4*>(op + ((sigma * (uint64_t)GP + g) * D + c * 8));
}
#endif  // FMHA_DECODE_SHARED_KERNELS

}  // namespace fmha_decode
