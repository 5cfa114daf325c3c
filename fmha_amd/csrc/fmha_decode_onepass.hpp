// fmha_decode_onepass.hpp -- single-pass decode attention for KV lengths
// beyond 16 when there are enough (batch, KV-head group) units to fill the
// GPU without splitting rows, gfx950.
//
// Same semantics as the split-KV path: fp32 scores, global max and sum,
// weights rounded to bf16 after normalisation (fmha_host.cpp:209-226), fp32
// P.V, one fp16 rounding.  One wave per (batch, group of HPW KV heads), as in
// the short kernel, in three phases:
//
//   1. K: 16-row sub-blocks with two register sets (two sub-blocks in flight,
//      a set refilled as soon as it is scored; 8-row ones, with their
//      block-table entries requested two sub-blocks ahead, when every lane
//      looks up its own rows' pages); dot products and the
//      transposing butterfly of the short kernel; scaled scores -> LDS.  The
//      first two V sub-blocks are requested at the end of this phase.
//   2. softmax in the wave: per (KV head, query head) the max and the sum of
//      exponentials over the row, read back from LDS by the head's lanes;
//      bf16 weights -> LDS.
//   3. V: sub-blocks of NRV rows with two register sets, refilled as they
//      are consumed; packed bf16 weight pairs from LDS, dot2 accumulation;
//      fp16 O.
//
// K and V are each read once and nothing else touches memory (no workspace),
// in one launch.  LDS per wave: HPW * G * (6 SP + 8) bytes (fp32 scores and
// bf16 weights for SP = the row bound rounded up to 32, each (KV head, query
// head) row padded by one dword, so that the softmax lanes, one row each,
// and the P.V lane groups fall in different banks).  Both loops run an even
// number of sub-blocks with no branch inside, so every wait is a fixed count:
// an odd row's last sub-block pairs with one past its end, whose requests
// read 0 without memory access, whose scores land in LDS padding the softmax
// never reads and whose weights are 0.
#pragma once

#include "fmha_decode_splitkv.hpp"

namespace fmha_decode {

template <int D, int G>
struct OnepassShape {
  static constexpr int LPH = D / 8;
  static constexpr int HPW = kWaveSize / LPH;
  static constexpr int NRV = G >= 8 ? 8 : 16;  // V rows per sub-block (register budget)
};

// 16-row blocks each of NW waves sharing a row takes (an even number, so
// the loops' paired sub-blocks always have room), for a row bound of nblk.
constexpr int onepass_wave_blocks(int nblk, int nw) { return ((nblk + nw - 1) / nw + 1) / 2 * 2; }

// LDS row stride for a row bound of nblk 16-row blocks split over NW waves.
constexpr int onepass_lds_rows(int nblk, int nw = 1) { return nw * onepass_wave_blocks(nblk, nw) * kSplitBlockRows; }

// LDS strides for sp rows: fp32 scores (floats) and bf16 weights (halves),
// both an odd number of dwords.
constexpr int onepass_score_stride(int sp) { return sp + 1; }
constexpr int onepass_weight_stride(int sp) { return sp + 2; }

// LDS bytes of one unit with sp rows: the scores and weights of the row,
// and with NW > 1 waves the P.V partial sums of waves 1..NW-1 (16-byte
// aligned after the weights).
template <int D, int G>
constexpr size_t onepass_lds_bytes(int sp, int nw = 1) {
  const size_t rows = (size_t)OnepassShape<D, G>::HPW * G * (onepass_score_stride(sp) * 4 + onepass_weight_stride(sp) * 2);
  return nw == 1 ? rows : (rows + 15) / 16 * 16 + (size_t)(nw - 1) * kWaveSize * G * 8 * 4;
}

// MULTI: several batches per wave (fewer KV heads than a wave holds,
// SplitArgs::sub_shift > 0; packed and strided layouts through one
// descriptor over the batches, paged caches through per-lane page lookups,
// kLayoutPagedLanes / kLayoutPagedBlockLanes); otherwise one batch per wave
// with its length read once for the whole wave.
// WPE: waves per SIMD the compiler schedules for (amdgpu_waves_per_eu; 1
// gives the same code as no hint).  2 for one batch per wave of eight query
// heads per KV head on pages of 16 rows or more with rows of up to four
// 16-row blocks, where the default schedule measured slower (same 250
// VGPRs; µs, 1 / 2: B=16384 S=24 Hq/Hkv 64/8 432 / 349, B=5461 S=24 153 /
// 127, B=2730 S=48 145 / 119; but B=1024 S=128 115 / 134).  Elsewhere 2
// measured equal (one-row pages, packed) or made the compiler spill
// (several batches per wave).
// NW: waves per unit (a workgroup of NW waves, one batch): wave w
// scores and multiplies rows [w * R, w * R + R) of the row (R =
// onepass_wave_blocks * 16), the scores of all of them shared through LDS
// for the softmax (each wave reduces the whole row, in the order one wave
// would, and forms the weights of its own rows); waves 1..NW-1 hand their
// P.V sums to wave 0 through LDS, which adds them in wave order.  For rows
// with too few (batch, KV-head group) units to fill the GPU one wave each.
// ROWS8: 8-row sub-blocks, half the registers of 16-row ones (123 against
// 208 VGPRs at G = 4 on pages under 16 rows with one batch per wave, 145
// against 242 at G = 8 packed), for more waves per CU where the LDS leaves
// room for them.
template <int D, int G, int LAYOUT = kLayoutPacked, bool MULTI = false, int WPE = 1, int NW = 1, bool ROWS8 = false>
__global__ __launch_bounds__(kBlockThreads * NW) __attribute__((amdgpu_waves_per_eu(WPE))) void onepass_decode_kernel(
    SplitArgs a) {
  static_assert(NW == 1 || !MULTI, "waves sharing a row serve one batch");
  static_assert(!ROWS8 || ((LAYOUT == kLayoutPaged || LAYOUT == kLayoutPagedBlock) && !MULTI) ||
                    LAYOUT == kLayoutPacked || LAYOUT == kLayoutStrided,
                "8-row sub-blocks: per-row pages one batch per wave, or one descriptor");
  using P = OnepassShape<D, G>;
  constexpr int LPH = P::LPH;
  constexpr int HPW = P::HPW;
  // Per-lane page lookups (several batches per wave on a paged cache).
  constexpr bool LANES = LAYOUT == kLayoutPagedLanes || LAYOUT == kLayoutPagedBlockLanes;
  // Per-lane lookups: 8-row sub-blocks for K and for V (4-row ones for V
  // with eight query heads per KV head), which leave room for two waves per
  // SIMD with a lookup and a 64-bit address per row on pages under 16 rows
  // (16-row sub-blocks took 416 registers at G = 4, 8-row V sub-blocks 300
  // at G = 8) and for three on larger pages.
  constexpr int NRV = LANES || ROWS8 ? (G >= 8 ? 4 : 8) : P::NRV;
  constexpr int NS = ilog2(LPH);
  constexpr int NR = LANES || ROWS8 ? 8 : kSplitBlockRows;
  constexpr int GH = G > 4 ? 4 : G;  // query heads scored per pass (partial sums per lane <= 64)
  constexpr int VS = GH * NR;
  constexpr int L = NS < ilog2(VS) ? NS : ilog2(VS);
  constexpr int W = (VS >> NS) > 1 ? (VS >> NS) : 1;
  constexpr int LPG = LPH / G;  // lanes per query head in the softmax phase
  static_assert(LPG >= 1, "at most LPH query heads per KV head");
  extern __shared__ __attribute__((aligned(16))) float onepass_lds[];

  const int lane = threadIdx.x & (kWaveSize - 1);
  const int wv = NW == 1 ? 0 : __builtin_amdgcn_readfirstlane((int)(threadIdx.x / kWaveSize));
  const int hkl = lane / LPH;
  const int r = lane % LPH;
  const int hq = a.num_heads_q;
  const u32x4 nan4 = {0x7e007e00u, 0x7e007e00u, 0x7e007e00u, 0x7e007e00u};
  uint32_t b0, nb, b;
  int sub, hk, S, smax, rel_rows = 0;
  bool head_ok, bad = false;
  if constexpr (!MULTI) {
    // One (batch, KV-head group) per wave; the length is the wave's.
    const uint32_t unit = blockIdx.x;
    const uint32_t upb = (uint32_t)a.units_per_batch;
    b = unit / upb;
    if (b >= (uint32_t)a.batch) return;
    const uint32_t hg = unit - b * upb;
    b0 = b;
    nb = 1;
    sub = 0;
    hk = (int)hg * HPW + hkl;
    head_ok = hk < a.num_heads_kv;
    S = split_len_l<LAYOUT>(a, b);
    smax = S;
    if (S <= 0 || S > a.max_rows) {
      // Empty rows give 0 (the reference loop's result), invalid ones NaN.
      if (wv != 0) return;
      const __amdgpu_buffer_rsrc_t o_rsrc = make_rsrc(a.o + (uint64_t)b * hq * D, (uint32_t)hq * D * 2);
      const uint32_t qo_off = head_ok ? (uint32_t)(hk * G * D + r * 8) * 2u : kLaneOutOfRange;
      const u32x4 fill = S == 0 ? u32x4{0u, 0u, 0u, 0u} : nan4;
#pragma unroll
      for (int g = 0; g < G; ++g) buffer_store16(o_rsrc, qo_off + g * D * 2, fill);
      return;
    }
  } else {
    // The lane groups serve 2^sub_shift consecutive batches (SubUnits);
    // lengths are per lane group and the loops run to the longest.
    const SubUnits<HPW> su(a.sub_shift);
    const uint32_t unit = blockIdx.x;
    const uint32_t upb = (uint32_t)a.units_per_batch;
    const uint32_t bw = unit / upb;
    b0 = bw << a.sub_shift;
    if (b0 >= (uint32_t)a.batch) return;
    const uint32_t hg = unit - bw * upb;
    nb = (uint32_t)a.batch - b0 < (1u << a.sub_shift) ? (uint32_t)a.batch - b0 : (1u << a.sub_shift);
    sub = su.unit(hkl);
    const bool lane_ok = (uint32_t)sub < nb;
    b = b0 + (lane_ok ? (uint32_t)sub : 0u);
    hk = su.head(hg, hkl);
    head_ok = lane_ok && hk < a.num_heads_kv;
    S = split_len_l<LAYOUT>(a, b);
    bad = lane_ok && (S < 0 || S > a.max_rows);
    if constexpr (LAYOUT == kLayoutPacked) {
      // This batch's rows relative to the wave's first batch; one that a
      // broken table puts beyond the descriptor's reach counts as invalid.
      const int64_t rel = (int64_t)a.cu[b] - a.cu[b0];
      if (rel < 0 || rel > (int64_t)((1u << 30) / ((uint32_t)kv_heads_mem(a) * D * 2u)) - a.max_rows) bad = lane_ok;
      else rel_rows = (int)rel;
    }
    if (bad || !lane_ok) {
      S = 0;
      rel_rows = 0;
    }
    smax = S;
#pragma unroll
    for (int k = 1; k < kWaveSize; k <<= 1) smax = max(smax, __shfl_xor(smax, k, kWaveSize));
    smax = __builtin_amdgcn_readfirstlane(smax);
    if (smax == 0) {
      // Empty rows give 0 (the reference loop's result), invalid ones NaN.
      const __amdgpu_buffer_rsrc_t o_rsrc = make_rsrc(a.o + (uint64_t)b0 * hq * D, nb * (uint32_t)hq * D * 2u);
      const uint32_t qo_off =
          head_ok ? (uint32_t)sub * (uint32_t)hq * D * 2u + (uint32_t)(hk * G * D + r * 8) * 2u : kLaneOutOfRange;
      const u32x4 fill = bad ? nan4 : u32x4{0u, 0u, 0u, 0u};
#pragma unroll
      for (int g = 0; g < G; ++g) buffer_store16(o_rsrc, qo_off + g * D * 2, fill);
      return;
    }
  }
  const uint32_t q_bytes = nb * (uint32_t)hq * D * 2u;
  const __amdgpu_buffer_rsrc_t o_rsrc = make_rsrc(a.o + (uint64_t)b0 * hq * D, q_bytes);
  const uint32_t qo_off =
      head_ok ? (uint32_t)sub * (uint32_t)hq * D * 2u + (uint32_t)(hk * G * D + r * 8) * 2u : kLaneOutOfRange;
  const int sp = onepass_lds_rows(a.nblk, NW);
  const int sps = onepass_score_stride(sp);   // floats
  const int spw = onepass_weight_stride(sp);  // halves (even: the P.V reads pairs)
  float* sc = onepass_lds + (size_t)hkl * G * sps;                                          // [G][sps] fp32
  uint16_t* pw = reinterpret_cast<uint16_t*>(onepass_lds + (size_t)HPW * G * sps) + (size_t)hkl * G * spw;  // [G][spw]

  // Rows [0, S) of each lane group's batch: later rows read 0 without access.
  static_assert(!LANES || MULTI, "per-lane page lookups serve several batches per wave");
  SplitRows<D, LAYOUT> krows, vrows;
  if constexpr (!MULTI || LANES) {
    // One batch per wave, or per-lane pages: each lane group addresses its
    // own batch's rows.
    const int64_t row_base = split_row_base<LAYOUT>(a, b);
    krows.init(a, a.k, b, row_base, 0, S, hk, head_ok, r);
    vrows.init(a, a.v, b, row_base, 0, S, hk, head_ok, r);
  } else {
    krows.init_multi(a, a.k, b0, nb, b, S, rel_rows, hk, head_ok, r);
    vrows.init_multi(a, a.v, b0, nb, b, S, rel_rows, hk, head_ok, r);
  }
  const __amdgpu_buffer_rsrc_t q_rsrc = make_rsrc(a.q + (uint64_t)b0 * hq * D, q_bytes);

  u32x4 qv[G];
#pragma unroll
  for (int g = 0; g < G; ++g) qv[g] = buffer_load16<kPolicyDefault>(q_rsrc, qo_off + g * D * 2);

  // ---- 1. scores of every row -> LDS ----
  const int blkl = r >> (NS - L);
  const bool writer = (r & ((1 << (NS - L)) - 1)) == 0;
  // This wave's rows [lo, lo + span): the whole row with NW = 1.
  const int wrows = onepass_wave_blocks(a.nblk, NW) * NR;
  const int lo = wv * wrows;
  const int span = NW == 1 ? smax : (smax - lo < 0 ? 0 : (smax - lo < wrows ? smax - lo : wrows));
  const int sk0 = lo / NR;                              // first sub-block
  const int nsub = ((span + NR - 1) / NR + 1) / 2 * 2;  // even
  auto load_k = [&](u32x4 (&kr)[NR], int s) { krows.template load<NR>(kr, s * NR); };
  // Per-lane lookups: each sub-block's block-table entries (one per row on
  // pages under 16 rows, else one) are requested two sub-blocks ahead,
  // between the row requests of the two register sets.  Vector loads
  // complete in order, so entries requested with their own rows would make
  // every refill wait for the rows before it (one sub-block in flight, and
  // a table round trip each).
  constexpr int NE = LANES ? PagedLaneRows<D, LAYOUT == kLayoutPagedBlockLanes>::template kEntries<NR> : 1;
  constexpr int NEV = LANES ? PagedLaneRows<D, LAYOUT == kLayoutPagedBlockLanes>::template kEntries<NRV> : 1;
  auto entries_k = [&](int32_t (&e)[NE], int s) {
    if constexpr (LANES) krows.template entries<NR>(e, s * NR);
  };
  auto fill_k = [&](u32x4 (&kr)[NR], int s, const int32_t (&e)[NE]) {
    if constexpr (LANES) krows.template load_entries<NR>(kr, s * NR, e);
  };
  auto score = [&](const u32x4 (&kr)[NR], int s) {
#pragma unroll
    for (int g0 = 0; g0 < G; g0 += GH) {
      u32x4 qh[GH];
#pragma unroll
      for (int g = 0; g < GH; ++g) qh[g] = qv[g0 + g];
      float x[VS];
      partial_scores<GH, NR>(qh, kr, x);
      TransposeReduce<LPH, VS, 0>::run(x, lane);
      if (writer) {
#pragma unroll
        for (int w = 0; w < W; ++w) {
          const int vi = blkl * W + w;
          sc[(g0 + vi / NR) * sps + s * NR + vi % NR] = x[w] * a.scale;
        }
      }
    }
  };
  const int sv0 = lo / NRV;    // this wave's first V sub-block
  int32_t eva[NEV], evb[NEV];  // per-lane lookups: the next V entries
  {
    // Two sub-blocks in flight: a register set is refilled as soon as it has
    // been scored (past the row's end the refills read 0 without access).
    // The scheduling barriers keep the compiler from interleaving a refill
    // with the scoring of the other set, which would make it wait for both.
    u32x4 ka[NR], kb[NR];
    if constexpr (LANES) {
      // In flight at the top of each pass: rows s, entries s + 2, rows s + 1
      // (the last pass refills nothing: rows past every lane's end would
      // still be read, from Q's first row).
      int32_t ea[NE], eb[NE];
      entries_k(ea, sk0);
      entries_k(eb, sk0 + 1);
      __builtin_amdgcn_sched_barrier(0);
      fill_k(ka, sk0, ea);
      __builtin_amdgcn_sched_barrier(0);
      entries_k(ea, sk0 + 2);
      __builtin_amdgcn_sched_barrier(0);
      fill_k(kb, sk0 + 1, eb);
      __builtin_amdgcn_sched_barrier(0);
      int s = sk0;
      for (; s + 2 < sk0 + nsub; s += 2) {
        score(ka, s);
        __builtin_amdgcn_sched_barrier(0);
        entries_k(eb, s + 3);
        __builtin_amdgcn_sched_barrier(0);
        fill_k(ka, s + 2, ea);
        __builtin_amdgcn_sched_barrier(0);
        score(kb, s + 1);
        __builtin_amdgcn_sched_barrier(0);
        entries_k(ea, s + 4);
        __builtin_amdgcn_sched_barrier(0);
        fill_k(kb, s + 3, eb);
        __builtin_amdgcn_sched_barrier(0);
      }
      // The first V entries, behind the last K rows.
      vrows.template entries<NRV>(eva, sv0 * NRV);
      vrows.template entries<NRV>(evb, (sv0 + 1) * NRV);
      __builtin_amdgcn_sched_barrier(0);
      score(ka, s);
      __builtin_amdgcn_sched_barrier(0);
      score(kb, s + 1);
      __builtin_amdgcn_sched_barrier(0);
    } else {
      load_k(ka, sk0);
      __builtin_amdgcn_sched_barrier(0);
      load_k(kb, sk0 + 1);
      __builtin_amdgcn_sched_barrier(0);
      for (int s = sk0; s < sk0 + nsub; s += 2) {
        score(ka, s);
        __builtin_amdgcn_sched_barrier(0);
        load_k(ka, s + 2);
        __builtin_amdgcn_sched_barrier(0);
        score(kb, s + 1);
        __builtin_amdgcn_sched_barrier(0);
        load_k(kb, s + 3);
        __builtin_amdgcn_sched_barrier(0);
      }
    }
  }
  // The first two V sub-blocks are requested before the softmax, which they
  // do not depend on, so they arrive while it runs.
  using VBuf = u32x4[NRV];
  VBuf va, vb;
  auto load_v = [&](u32x4 (&vr)[NRV], int s) { vrows.template load<NRV>(vr, s * NRV); };
  if constexpr (LANES) {
    vrows.template load_entries<NRV>(va, sv0 * NRV, eva);
    __builtin_amdgcn_sched_barrier(0);
    vrows.template entries<NRV>(eva, (sv0 + 2) * NRV);
    __builtin_amdgcn_sched_barrier(0);
    vrows.template load_entries<NRV>(vb, (sv0 + 1) * NRV, evb);
    __builtin_amdgcn_sched_barrier(0);
  } else {
    load_v(va, sv0);
    __builtin_amdgcn_sched_barrier(0);
    load_v(vb, sv0 + 1);
    __builtin_amdgcn_sched_barrier(0);
  }
  // An unmapped page among rows [0, S) (seen by the K phase, which reads
  // them all): the batch is invalid (per lane group with MULTI, whose lane
  // groups serve different batches).
  bool poisoned;
  if constexpr (NW == 1) {
    poisoned = krows.bad != 0;
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  } else {
    // Every wave's scores are in LDS; any wave's unmapped page poisons the row.
    poisoned = __syncthreads_or(krows.bad != 0) != 0;
  }

  // ---- 2. softmax per (KV head, query head): lane r takes query head
  // r % G and rows r / G, r / G + LPG, ... ----
  {
    const int g = r % G;
    const int j0 = r / G;
    float* t = sc + g * sps;
    float m = -__builtin_inff();
    for (int j = j0; j < S; j += LPG) m = fmaxf(m, t[j]);
#pragma unroll
    for (int msk = G; msk < LPH; msk <<= 1) m = fmaxf(m, __shfl_xor(m, msk, kWaveSize));
    float l = 0.0f;
    uint16_t* p = pw + g * spw;
    if constexpr (NW == 1) {
      for (int j = j0; j < S; j += LPG) {
        const float e = expf(t[j] - m);
        t[j] = e;
        l += e;
      }
#pragma unroll
      for (int msk = G; msk < LPH; msk <<= 1) l += __shfl_xor(l, msk, kWaveSize);
      const int pad = (smax + 2 * NRV - 1) / (2 * NRV) * (2 * NRV);  // rows the V phase reads weights for
      for (int j = j0; j < pad; j += LPG)
        p[j] = j < S ? __builtin_bit_cast(uint16_t, (__bf16)(l > 0.0f ? t[j] / l : 0.0f)) : (uint16_t)0;
    } else {
      // The scores are shared: the exponentials are formed again for this
      // wave's own rows rather than stored (the same values, the same sum).
      for (int j = j0; j < S; j += LPG) l += expf(t[j] - m);
#pragma unroll
      for (int msk = G; msk < LPH; msk <<= 1) l += __shfl_xor(l, msk, kWaveSize);
      const int pad = lo + (span + 2 * NRV - 1) / (2 * NRV) * (2 * NRV);  // rows this wave's V phase reads
      for (int j = lo + j0; j < pad; j += LPG)
        p[j] = j < S ? __builtin_bit_cast(uint16_t, (__bf16)(l > 0.0f ? expf(t[j] - m) / l : 0.0f)) : (uint16_t)0;
    }
  }
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");

  // ---- 3. P.V ----
  float acc[G][8];
#pragma unroll
  for (int g = 0; g < G; ++g)
#pragma unroll
    for (int d = 0; d < 8; ++d) acc[g][d] = 0.0f;
  const int nsv = ((span + NRV - 1) / NRV + 1) / 2 * 2;  // even
  auto pv = [&](const u32x4 (&vr)[NRV], int s) {
    uint32_t pp[G][NRV / 2];
#pragma unroll
    for (int g = 0; g < G; ++g) {
      const uint32_t* pairs = reinterpret_cast<const uint32_t*>(pw + g * spw + s * NRV);
#pragma unroll
      for (int jp = 0; jp < NRV / 2; ++jp) pp[g][jp] = pairs[jp];
    }
    accumulate_pv<G, NRV>(vr, pp, acc);
  };
  if constexpr (LANES) {
    // As the K phase: rows s, entries s + 2, rows s + 1 in flight.
    int s = sv0;
    for (; s + 2 < sv0 + nsv; s += 2) {
      pv(va, s);
      __builtin_amdgcn_sched_barrier(0);
      vrows.template entries<NRV>(evb, (s + 3) * NRV);
      __builtin_amdgcn_sched_barrier(0);
      vrows.template load_entries<NRV>(va, (s + 2) * NRV, eva);
      __builtin_amdgcn_sched_barrier(0);
      pv(vb, s + 1);
      __builtin_amdgcn_sched_barrier(0);
      vrows.template entries<NRV>(eva, (s + 4) * NRV);
      __builtin_amdgcn_sched_barrier(0);
      vrows.template load_entries<NRV>(vb, (s + 3) * NRV, evb);
      __builtin_amdgcn_sched_barrier(0);
    }
    pv(va, s);
    __builtin_amdgcn_sched_barrier(0);
    pv(vb, s + 1);
  } else {
    for (int s = sv0; s < sv0 + nsv; s += 2) {
      pv(va, s);
      __builtin_amdgcn_sched_barrier(0);
      load_v(va, s + 2);
      __builtin_amdgcn_sched_barrier(0);
      pv(vb, s + 1);
      __builtin_amdgcn_sched_barrier(0);
      load_v(vb, s + 3);
      __builtin_amdgcn_sched_barrier(0);
    }
  }
  if constexpr (NW > 1) {
    // Waves 1..NW-1 hand their sums to wave 0 (LDS after the weights),
    // which adds them in wave order.
    float* red = reinterpret_cast<float*>(
        reinterpret_cast<char*>(onepass_lds) +
        ((size_t)HPW * G * (sps * 4 + spw * 2) + 15) / 16 * 16);
    if (wv > 0) {
#pragma unroll
      for (int g = 0; g < G; ++g)
#pragma unroll
        for (int d = 0; d < 8; d += 4)
          *reinterpret_cast<float4*>(red + (((size_t)(wv - 1) * G + g) * kWaveSize + lane) * 8 + d) =
              float4{acc[g][d], acc[g][d + 1], acc[g][d + 2], acc[g][d + 3]};
    }
    __syncthreads();
    if (wv > 0) return;
    for (int w = 1; w < NW; ++w)
#pragma unroll
      for (int g = 0; g < G; ++g)
#pragma unroll
        for (int d = 0; d < 8; d += 4) {
          const float4 x = *reinterpret_cast<const float4*>(red + (((size_t)(w - 1) * G + g) * kWaveSize + lane) * 8 + d);
          acc[g][d] += x.x;
          acc[g][d + 1] += x.y;
          acc[g][d + 2] += x.z;
          acc[g][d + 3] += x.w;
        }
  }
#pragma unroll
  for (int g = 0; g < G; ++g) {
    if constexpr (MULTI)
      buffer_store16(o_rsrc, qo_off + g * D * 2, bad || poisoned ? nan4 : pack_f16x8(acc[g]));
    else
      buffer_store16(o_rsrc, qo_off + g * D * 2, poisoned ? nan4 : pack_f16x8(acc[g]));
  }
}

}  // namespace fmha_decode
