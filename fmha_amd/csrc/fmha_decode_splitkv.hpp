// fmha_decode_splitkv.hpp -- decode attention for KV lengths beyond 16
// (split-KV), gfx950.
//
// Same semantics as the short-KV kernel, extended to any length S: fp32
// scores, max-subtracted softmax, weights rounded to bf16 *after*
// normalisation (as the reference's CPU loop does, fmha_host.cpp:209-226),
// fp32 P.V, one fp16 rounding.  Because the bf16 rounding needs the global
// max and sum before any weight is formed, the work runs in four launches
// over a caller-provided workspace:
//
//   1. scores:  wave = (batch, KV-head group, chunk of C rows).  16-row
//               sub-blocks: K loads, dot products, transposing butterfly
//               (shared with the short kernel), scaled scores t_j -> T, and
//               the chunk's running (max m_c, sum l_c of exp(t - m_c)).
//   2. stats:   lane = (batch, query head): m = max_c m_c,
//               L = sum_c l_c * exp(m_c - m).
//   3. pv:      wave = (batch, KV-head group, chunk): per sub-block the 64
//               lanes form P_j = bf16(exp(t_j - m) / L) for the wave's heads
//               into LDS, then V loads and packed dot2 accumulation; the
//               chunk's fp32 partial output -> Opart (or fp16 O directly when
//               every batch fits one chunk).
//   4. combine: lane = (batch, query head, 8 dims): O = fp16(sum_c Opart).
//
// K and V are each read once; T, the stats and Opart add 4 bytes per row per
// query head and 4*D bytes per chunk per query head.
#pragma once

#include "fmha_decode_kernel.hpp"

namespace fmha_decode {

struct SplitArgs {
  const uint16_t* q;      // [batch, Hq, D] bf16
  const uint16_t* k;      // [rows, Hkv, D] bf16, packed by cu
  const uint16_t* v;
  uint16_t* o;            // [batch, Hq, D] fp16
  const int32_t* cu;      // [batch+1]
  float* t;               // [batch, Hq, t_stride] scaled scores
  float* m;               // [batch, Hq, nchunks] chunk max
  float* l;               // [batch, Hq, nchunks] chunk sum of exp(t - m_c)
  float* ml;              // [batch, Hq, 2] global max, global sum
  float* opart;           // [batch, Hq, nchunks, D] partial outputs
  int32_t num_heads_q;
  int32_t num_heads_kv;
  int32_t units_per_batch;
  int32_t nchunks;        // chunks per batch row (max_rows / chunk_rows, rounded up)
  int32_t chunk_rows;     // C, a multiple of 16
  int32_t max_rows;       // lengths above this are invalid (NaN output)
  int32_t t_stride;       // nchunks * chunk_rows
  int32_t batch;
  uint32_t total_units;   // batch * units_per_batch
  float scale;
};

// Decodes a split wave id into (batch, head group, chunk) and the batch's
// K/V range.  Returns false for an empty chunk or an invalid length.
template <int D>
__device__ __forceinline__ bool split_wave(const SplitArgs& a, uint32_t& b, int& hk, bool& head_ok, int& row0,
                                           int& S, int64_t& base, int lane) {
  constexpr int LPH = D / 8;
  constexpr int HPW = kWaveSize / LPH;
  const uint32_t id = blockIdx.x * kWavesPerBlock + __builtin_amdgcn_readfirstlane(threadIdx.x / kWaveSize);
  const uint32_t nch = (uint32_t)a.nchunks;
  const uint32_t unit = id / nch;
  const uint32_t c = id - unit * nch;
  if (unit >= a.total_units) return false;
  const uint32_t upb = (uint32_t)a.units_per_batch;
  b = unit / upb;
  const uint32_t hg = unit - b * upb;
  hk = (int)hg * HPW + lane / LPH;
  head_ok = hk < a.num_heads_kv;
  base = a.cu[b];
  S = a.cu[b + 1] - (int)base;
  row0 = (int)c * a.chunk_rows;
  return S >= 0 && S <= a.max_rows && row0 < S;
}

// ---------------------------------------------------------------------------
// 1. scores
// ---------------------------------------------------------------------------
template <int D, int G>
__global__ __launch_bounds__(kBlockThreads) void splitkv_scores_kernel(SplitArgs a) {
  constexpr int LPH = D / 8;
  constexpr int NS = ilog2(LPH);
  constexpr int NR = 16;
  constexpr int V = G * NR;
  constexpr int L = NS < ilog2(V) ? NS : ilog2(V);
  constexpr int W = (V >> NS) > 1 ? (V >> NS) : 1;
  constexpr int GS = W < NR ? W : NR;
  constexpr int C = ilog2(NR / GS);
  const int lane = threadIdx.x & (kWaveSize - 1);
  uint32_t b;
  int hk, row0, S;
  bool head_ok;
  int64_t base;
  if (!split_wave<D>(a, b, hk, head_ok, row0, S, base, lane)) return;
  const int r = lane % LPH;
  const int hq = a.num_heads_q;
  const uint32_t row_bytes = (uint32_t)a.num_heads_kv * D * 2;
  const __amdgpu_buffer_rsrc_t q_rsrc = make_rsrc(a.q + (uint64_t)b * hq * D, (uint32_t)hq * D * 2);
  const __amdgpu_buffer_rsrc_t k_rsrc = make_rsrc(a.k + (uint64_t)base * a.num_heads_kv * D, (uint32_t)S * row_bytes);
  const uint32_t kv_off = head_ok ? (uint32_t)(hk * D + r * 8) * 2u : kLaneOutOfRange;
  const uint32_t q_off = head_ok ? (uint32_t)(hk * G * D + r * 8) * 2u : kLaneOutOfRange;

  u32x4 qv[G];
#pragma unroll
  for (int g = 0; g < G; ++g) qv[g] = buffer_load16<kPolicyDefault>(q_rsrc, q_off + g * D * 2);

  const int blk = r >> (NS - L);
  // Heads whose scores this lane holds after the butterfly: W/GS groups.
  float run_m[W / GS];
  float run_l[W / GS];
#pragma unroll
  for (int h = 0; h < W / GS; ++h) {
    run_m[h] = -__builtin_inff();
    run_l[h] = 0.0f;
  }
  const int row_end = min(S, row0 + a.chunk_rows);
  for (int j0 = row0; j0 < row_end; j0 += NR) {
    u32x4 kr[NR];
#pragma unroll
    for (int j = 0; j < NR; ++j)
      kr[j] = buffer_load16<kPolicyStream>(k_rsrc, kv_off + (uint32_t)(j0 + j) * row_bytes);
    float x[V];
    partial_scores<G, NR>(qv, kr, x);
    TransposeReduce<LPH, V, 0>::run(x, lane);
#pragma unroll
    for (int h = 0; h < W / GS; ++h) {
      float t[GS];
      float bm = -__builtin_inff();
#pragma unroll
      for (int w = 0; w < GS; ++w) {
        const int vi = blk * W + h * GS + w;
        const int row = j0 + vi % NR;
        t[w] = x[h * GS + w] * a.scale;
        bm = row < S ? fmaxf(bm, t[w]) : bm;
        if (head_ok && row < S) a.t[((uint64_t)b * hq + hk * G + vi / NR) * a.t_stride + row] = t[w];
      }
      bm = GroupReduce<LPH, L - C, L, true>::run(bm);
      const float nm = fmaxf(run_m[h], bm);  // finite: every sub-block has a valid row
      float bs = 0.0f;
#pragma unroll
      for (int w = 0; w < GS; ++w) {
        const int row = j0 + (blk * W + h * GS + w) % NR;
        bs += row < S ? expf(t[w] - nm) : 0.0f;
      }
      bs = GroupReduce<LPH, L - C, L, false>::run(bs);
      run_l[h] = run_l[h] * expf(run_m[h] - nm) + bs;
      run_m[h] = nm;
    }
  }
  if (!head_ok) return;
  const int c = row0 / a.chunk_rows;
#pragma unroll
  for (int h = 0; h < W / GS; ++h) {
    const int g = (blk * W + h * GS) / NR;
    const uint64_t idx = ((uint64_t)b * hq + hk * G + g) * a.nchunks + c;
    a.m[idx] = run_m[h];
    a.l[idx] = run_l[h];
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

// ---------------------------------------------------------------------------
// 2. stats: per (batch, query head), the global max and sum of exponentials.
// Few chunks: one lane per head.  Many chunks: one wave per head, lanes
// striding the chunks (lane order is fixed, so results are deterministic).
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(64) void splitkv_stats_wave_kernel(SplitArgs a) {
  const uint64_t i = blockIdx.x;  // b * Hq + h
  const int lane = threadIdx.x;
  const uint64_t b = i / (uint64_t)a.num_heads_q;
  const int S = a.cu[b + 1] - a.cu[b];
  if (S <= 0 || S > a.max_rows) return;
  const int n = (S + a.chunk_rows - 1) / a.chunk_rows;
  const float* m = a.m + i * a.nchunks;
  const float* l = a.l + i * a.nchunks;
  float gm = -__builtin_inff();
  for (int c = lane; c < n; c += kWaveSize) gm = fmaxf(gm, m[c]);
  gm = wave_max(gm);
  float gl = 0.0f;
  for (int c = lane; c < n; c += kWaveSize) gl += l[c] * expf(m[c] - gm);
  gl = wave_sum(gl);
  if (lane == 0) {
    a.ml[2 * i] = gm;
    a.ml[2 * i + 1] = gl;
  }
}

__global__ __launch_bounds__(256) void splitkv_stats_kernel(SplitArgs a) {
  const uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= (uint64_t)a.batch * a.num_heads_q) return;
  const uint64_t b = i / (uint64_t)a.num_heads_q;
  const int S = a.cu[b + 1] - a.cu[b];
  if (S <= 0 || S > a.max_rows) return;
  const int n = (S + a.chunk_rows - 1) / a.chunk_rows;
  const float* m = a.m + i * a.nchunks;
  const float* l = a.l + i * a.nchunks;
  float gm = -__builtin_inff();
  for (int c = 0; c < n; ++c) gm = fmaxf(gm, m[c]);
  float gl = 0.0f;
  for (int c = 0; c < n; ++c) gl += l[c] * expf(m[c] - gm);
  a.ml[2 * i] = gm;
  a.ml[2 * i + 1] = gl;
}

// ---------------------------------------------------------------------------
// 3. P.V per chunk.  DIRECT: every batch fits one chunk, so the wave writes
// fp16 O itself (and the zero / NaN rows of empty or invalid batches).
// ---------------------------------------------------------------------------
template <int D, int G, bool DIRECT>
__global__ __launch_bounds__(kBlockThreads) void splitkv_pv_kernel(SplitArgs a) {
  constexpr int LPH = D / 8;
  constexpr int HPW = kWaveSize / LPH;
  constexpr int NR = 16;
  constexpr int VP = G * kMaxSeq;
  constexpr int SLOTS = HPW * G * NR;                        // weights per sub-block
  constexpr int PER_LANE = (SLOTS + kWaveSize - 1) / kWaveSize;
  __shared__ __attribute__((aligned(16))) uint16_t lds_p[HPW * VP];
  const int lane = threadIdx.x & (kWaveSize - 1);
  uint32_t b = 0;
  int hk = 0, row0 = -1, S = 0;
  bool head_ok = false;
  int64_t base = 0;
  const bool live = split_wave<D>(a, b, hk, head_ok, row0, S, base, lane);
  const int r = lane % LPH;
  const int hkl = lane / LPH;
  const int hq = a.num_heads_q;
  if (!live) {
    // Only chunk 0 of a DIRECT launch owns the output of an empty or invalid
    // batch; everything else has nothing to do.
    if constexpr (DIRECT) {
      const uint32_t id = blockIdx.x * kWavesPerBlock + __builtin_amdgcn_readfirstlane(threadIdx.x / kWaveSize);
      if (id >= a.total_units * (uint32_t)a.nchunks || row0 != 0) return;
      const bool bad = S < 0 || S > a.max_rows;
      const u32x4 fill = bad ? u32x4{0x7e007e00u, 0x7e007e00u, 0x7e007e00u, 0x7e007e00u} : u32x4{0u, 0u, 0u, 0u};
      const __amdgpu_buffer_rsrc_t o_rsrc = make_rsrc(a.o + (uint64_t)b * hq * D, (uint32_t)hq * D * 2);
      const uint32_t o_off = head_ok ? (uint32_t)(hk * G * D + r * 8) * 2u : kLaneOutOfRange;
#pragma unroll
      for (int g = 0; g < G; ++g) buffer_store16(o_rsrc, o_off + g * D * 2, fill);
    }
    return;
  }
  const uint32_t row_bytes = (uint32_t)a.num_heads_kv * D * 2;
  const __amdgpu_buffer_rsrc_t v_rsrc = make_rsrc(a.v + (uint64_t)base * a.num_heads_kv * D, (uint32_t)S * row_bytes);
  const uint32_t kv_off = head_ok ? (uint32_t)(hk * D + r * 8) * 2u : kLaneOutOfRange;
  const int hk0 = hk - hkl;  // first KV head of this wave

  // The weight slots this lane forms: slot f = lane + 64*i covers
  // (head hkl_f, query g_f, row j_f) of the wave's heads.
  float gm[PER_LANE], gsum[PER_LANE];
#pragma unroll
  for (int i = 0; i < PER_LANE; ++i) {
    const int f = lane + kWaveSize * i;
    const int hkf = hk0 + f / (G * NR);
    const int gf = (f / NR) % G;
    const bool ok = f < SLOTS && hkf < a.num_heads_kv;
    const uint64_t hqi = (uint64_t)b * hq + hkf * G + gf;
    gm[i] = ok ? a.ml[2 * hqi] : 0.0f;
    gsum[i] = ok ? a.ml[2 * hqi + 1] : 1.0f;
  }

  float acc[G][8];
#pragma unroll
  for (int g = 0; g < G; ++g)
#pragma unroll
    for (int d = 0; d < 8; ++d) acc[g][d] = 0.0f;

  const int row_end = min(S, row0 + a.chunk_rows);
  for (int j0 = row0; j0 < row_end; j0 += NR) {
    u32x4 vr[NR];
#pragma unroll
    for (int j = 0; j < NR; ++j)
      vr[j] = buffer_load16<kPolicyStream>(v_rsrc, kv_off + (uint32_t)(j0 + j) * row_bytes);
    // Weights of this sub-block: exp(t - m) / L rounded to bf16, 0 past S.
#pragma unroll
    for (int i = 0; i < PER_LANE; ++i) {
      const int f = lane + kWaveSize * i;
      const int hlf = f / (G * NR);
      const int gf = (f / NR) % G;
      const int jf = f % NR;
      const int hkf = hk0 + hlf;
      const int row = j0 + jf;
      float p = 0.0f;
      if (f < SLOTS && hkf < a.num_heads_kv && row < S) {
        const float t = a.t[((uint64_t)b * hq + hkf * G + gf) * a.t_stride + row];
        p = expf(t - gm[i]) / gsum[i];
      }
      if (f < SLOTS) lds_p[hlf * VP + gf * kMaxSeq + jf] = __builtin_bit_cast(uint16_t, (__bf16)p);
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    const uint32_t* pairs = reinterpret_cast<const uint32_t*>(lds_p + hkl * VP);
    uint32_t pp[G][NR / 2];
#pragma unroll
    for (int g = 0; g < G; ++g)
#pragma unroll
      for (int jp = 0; jp < NR / 2; ++jp) pp[g][jp] = pairs[g * (kMaxSeq / 2) + jp];
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    accumulate_pv<G, NR>(vr, pp, acc);
  }

  if constexpr (DIRECT) {
    const __amdgpu_buffer_rsrc_t o_rsrc = make_rsrc(a.o + (uint64_t)b * hq * D, (uint32_t)hq * D * 2);
    const uint32_t o_off = head_ok ? (uint32_t)(hk * G * D + r * 8) * 2u : kLaneOutOfRange;
#pragma unroll
    for (int g = 0; g < G; ++g) buffer_store16(o_rsrc, o_off + g * D * 2, pack_f16x8(acc[g]));
  } else {
    if (!head_ok) return;
    const int c = row0 / a.chunk_rows;
#pragma unroll
    for (int g = 0; g < G; ++g) {
      float* dst = a.opart + (((uint64_t)b * hq + hk * G + g) * a.nchunks + c) * D + r * 8;
      u32x4 lo, hi;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        lo[i] = __builtin_bit_cast(uint32_t, acc[g][i]);
        hi[i] = __builtin_bit_cast(uint32_t, acc[g][4 + i]);
      }
      *reinterpret_cast<u32x4*>(dst) = lo;
      *reinterpret_cast<u32x4*>(dst + 4) = hi;
    }
  }
}

// ---------------------------------------------------------------------------
// 4. combine: O = fp16(sum over the batch's chunks of Opart), chunk order.
// ---------------------------------------------------------------------------
template <int D>
__global__ __launch_bounds__(256) void splitkv_combine_kernel(SplitArgs a) {
  const uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const uint64_t per_head = D / 8;
  if (i >= (uint64_t)a.batch * a.num_heads_q * per_head) return;
  const uint64_t head = i / per_head;  // b * Hq + h
  const int d0 = (int)(i - head * per_head) * 8;
  const uint64_t b = head / (uint64_t)a.num_heads_q;
  const int S = a.cu[b + 1] - a.cu[b];
  float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
  u32x4 out;
  if (S < 0 || S > a.max_rows) {
    out = u32x4{0x7e007e00u, 0x7e007e00u, 0x7e007e00u, 0x7e007e00u};
  } else {
    const int n = (S + a.chunk_rows - 1) / a.chunk_rows;
    const float* src = a.opart + head * a.nchunks * D + d0;
    for (int c = 0; c < n; ++c) {
      const u32x4 lo = *reinterpret_cast<const u32x4*>(src + (uint64_t)c * D);
      const u32x4 hi = *reinterpret_cast<const u32x4*>(src + (uint64_t)c * D + 4);
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        acc[k] += __builtin_bit_cast(float, (uint32_t)lo[k]);
        acc[4 + k] += __builtin_bit_cast(float, (uint32_t)hi[k]);
      }
    }
    out = pack_f16x8(acc);
  }
  *reinterpret_cast<u32x4*>(a.o + head * D + d0) = out;
}

// Many chunks: one 256-thread block per (batch, query head); thread t sums
// dims [8*(t % (D/8)), +8) over chunks c = t / (D/8) + k * CG, then the CG
// partial sums of each dim group are added in order through LDS.
template <int D>
__global__ __launch_bounds__(256) void splitkv_combine_block_kernel(SplitArgs a) {
  constexpr int DG = D / 8;
  constexpr int CG = 256 / DG;
  __shared__ float part[CG][D];
  const uint64_t head = blockIdx.x;  // b * Hq + h
  const int t = threadIdx.x;
  const int dg = t % DG;
  const int cg = t / DG;
  const uint64_t b = head / (uint64_t)a.num_heads_q;
  const int S = a.cu[b + 1] - a.cu[b];
  const bool bad = S < 0 || S > a.max_rows;
  const int n = bad ? 0 : (S + a.chunk_rows - 1) / a.chunk_rows;
  float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
  const float* src = a.opart + head * a.nchunks * D + dg * 8;
  for (int c = cg; c < n; c += CG) {
    const u32x4 lo = *reinterpret_cast<const u32x4*>(src + (uint64_t)c * D);
    const u32x4 hi = *reinterpret_cast<const u32x4*>(src + (uint64_t)c * D + 4);
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      acc[k] += __builtin_bit_cast(float, (uint32_t)lo[k]);
      acc[4 + k] += __builtin_bit_cast(float, (uint32_t)hi[k]);
    }
  }
#pragma unroll
  for (int k = 0; k < 8; ++k) part[cg][dg * 8 + k] = acc[k];
  __syncthreads();
  if (cg != 0) return;
#pragma unroll
  for (int k = 0; k < 8; ++k) acc[k] = 0.0f;
  for (int g = 0; g < CG; ++g)
#pragma unroll
    for (int k = 0; k < 8; ++k) acc[k] += part[g][dg * 8 + k];
  const u32x4 out = bad ? u32x4{0x7e007e00u, 0x7e007e00u, 0x7e007e00u, 0x7e007e00u} : pack_f16x8(acc);
  *reinterpret_cast<u32x4*>(a.o + head * D + dg * 8) = out;
}

}  // namespace fmha_decode
