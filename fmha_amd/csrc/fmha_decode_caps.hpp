// fmha_decode_caps.hpp -- the in-flight budget model that sizes the short
// kernels' waves per CU (the host reserves unused LDS per workgroup so that
// only that many waves fit on a CU).  Host code only: shared by the library
// (fmha_decode_api.hip) and the measurement aid that replays a kernel's
// traffic with the same caps (tests/profiling/stream_ceiling.hip).
#pragma once

#include <cstdint>

namespace fmha_decode {
namespace host {

// Each wave issues all of its loads at once, and MI355X streams fastest with
// a bounded amount of them in flight per CU: 80 KiB for the one- and
// two-head kernels with known lengths (3 waves of the S=16, D=128 unit: 7.13
// TB/s, against 6.63 TB/s uncapped; 6 waves of the S=5, D=256 unit); tiny
// units (S=1) want every wave the registers allow (kMaxWavesPerCU: no cap).
constexpr int kInflightBytesPerCU = 80 * 1024;
constexpr int kMaxWavesPerCU = 32;

// The in-flight budget model behind every short-kernel launch's waves per
// CU.  A wave of the g-head kernel serving `rows` K/V rows (a mean) and G
// query heads per KV head moves a unit of 2 rows + c G KiB (each row 1 KiB of
// K and 1 KiB of V per wave at any head dim, each query head 1 KiB of Q in
// and 1 KiB of O out, which c weighs: 2 counts them in full, 1 at half,
// their loads being few and their stores leaving nothing to wait for);
// MI355X streams fastest with a bounded amount in flight per CU, A + B rows
// KiB, larger for longer rows, whose waves compute longer between requests.
// The cap is floor((A + B rows) / (2 rows + c G)) waves, at least `floor`,
// none from 16 on (every wave the registers allow).
struct WaveBudget {
  int a_kib;   // A
  int b2_kib;  // 2 B (KiB per row, in halves)
  int c;       // KiB per query head
  int floor;
};

inline int budget_waves(const WaveBudget& m, int rows16, int g_real) {
  // Numerator and denominator in 1/32 KiB: rows16 = 16 rows.
  const int64_t num = 32LL * m.a_kib + (int64_t)m.b2_kib * rows16;
  const int64_t den = 4LL * rows16 + 32LL * m.c * g_real;
  const int64_t w = num / den;
  if (w >= 16) return kMaxWavesPerCU;
  return w < m.floor ? m.floor : (int)w;
}

// Budgets of the tree-order kernels, by kernel (g query heads, head dim dq)
// and how the wave learns its lengths: known on the host with one batch per
// wave, or bucket_per_wave (lengths on the device, or several batches per
// wave).  The fitted ones come from tests/profiling/cap_sweep.py at B=30720
// (15360 at D = 256), Hkv = 16 at D = 128 and 8 otherwise, S = 1-16, G =
// 3-8 (102 shapes, two sweeps averaged): the lowest mean time over the
// swept shapes that keeps the cap of every benchmark configuration, mean
// and worst time over the best cap 1.003 and 1.023 to 1.015 and 1.091 per
// kernel, against 1.003-1.027 and 1.016-1.196 for the per-shape rules they
// replace (profiles/fmha_decode_wave_caps.md).
//   * 1 or 2 query heads, lengths known: 80 KiB flat (3 waves of the 34 KiB
//     S=16 D=128 unit, 7.13 TB/s against 6.63 uncapped; 6 of the 12 KiB S=5
//     D=256 unit, 6.60 against 6.05).
//   * 1 or 2 with lengths on the device: 144 KiB flat (their waves first
//     wait for the length, so they carry requests for a shorter part of
//     their life; B=30720 S=5 D=256 µs for 4/6/8/10/12/16 waves
//     643/504/446/433/423/427, Poisson(4) lengths H=16 D=128
//     291/233/206/198/191/191).
//   * 4-head kernel, lengths known: one pass over all four query heads, its
//     best cap falling with the rows faster than a flat budget does: (40 +
//     6 rows, c = 1) at D = 128, (90 + rows / 2, c = 1, at least 4 waves) at
//     D = 64, (78 + 2 rows, c = 1, at least 4) at D = 256.
//   * 8-head kernel, lengths known: 200 KiB flat at D = 128 (two query heads
//     per pass), (212 + rows / 2, c = 1) at D = 64, (54 + 8 rows, c = 1) at
//     D = 256.
//   * 8-head kernel at D = 128 with lengths on the device: (120 + 7.5 rows)
//     (B=30720, µs against 200 KiB flat: Hq/Hkv 32/4 S=16 212.3 / 252.2,
//     128/16 S=16 922.4 / 1006.0, 64/8 S=16 475.3 / 510.9).
//   * the 4- and 8-head kernels otherwise (a bucket per wave, scoring two
//     query heads per pass at D <= 128): 200 KiB flat (G=4 S=16 Poisson µs
//     for 4/5/6/7/8 waves 429/374/341/323/316; G=8 S=8 670/615/631/655/662).
inline WaveBudget tree_order_budget(int g, int dq, bool device_lengths, bool bucket_per_wave) {
  if (!bucket_per_wave && g == 4)
    return dq == 64 ? WaveBudget{90, 1, 1, 4} : dq == 128 ? WaveBudget{40, 12, 1, 3} : WaveBudget{78, 4, 1, 4};
  if (!bucket_per_wave && g == 8 && dq != 128)
    return dq == 64 ? WaveBudget{212, 1, 1, 3} : WaveBudget{54, 16, 1, 3};
  if (device_lengths && g == 8 && dq == 128) return WaveBudget{120, 15, 2, 4};
  if (g >= 4) return WaveBudget{200, 0, 2, g >= 8 ? 4 : 3};
  if (device_lengths) return WaveBudget{144, 0, 2, 3};
  return WaveBudget{kInflightBytesPerCU / 1024, 0, 2, 3};
}

}  // namespace host
}  // namespace fmha_decode
