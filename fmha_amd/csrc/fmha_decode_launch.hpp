// fmha_decode_launch.hpp -- host-side launchers of the decode kernels.
//
// Shared by fmha_decode_api.hip (argument checks, plans and kernel choice
// behind the C ABI) and fmha_decode_inst.hip, which is compiled once per
// part (FMHA_DECODE_PART): each part explicitly instantiates one slice of
// the launchers below, and with them their kernels, so that the library's
// few hundred kernel instantiations compile in parallel.  The extern
// template declarations at the end keep every other translation unit from
// instantiating them again.
#pragma once

#include <hip/hip_runtime.h>

#include <atomic>
#include <cstdint>
#include <cstdlib>

#include "fmha_decode_caps.hpp"
#include "fmha_decode_group.hpp"
#include "fmha_decode_kernel.hpp"
#include "fmha_decode_onepass.hpp"
#include "fmha_decode_splitkv.hpp"
#include "fmha_decode_splitkv_group.hpp"

namespace fmha_decode {
namespace host {

using fmha_decode::DecodeArgs;
using fmha_decode::SplitArgs;
using fmha_decode::kBlockThreads;
using fmha_decode::kWaveSize;
using fmha_decode::kWavesPerBlock;

// Appends one launch of the current entry-point call to the calling
// thread's plan text (fmha_decode_last_plan): printf-style, launches
// separated by "; ".  Defined in fmha_decode_api.hip.
void plan_note(const char* fmt, ...) __attribute__((format(printf, 1, 2)));

// Names of the K/V layouts in plan text.
inline const char* layout_name(int layout) {
  switch (layout) {
    case fmha_decode::kLayoutPacked: return "packed";
    case fmha_decode::kLayoutStrided: return "strided";
    case fmha_decode::kLayoutPaged: return "paged";
    case fmha_decode::kLayoutPagedLanes: return "paged_lanes";
    case fmha_decode::kLayoutPagedBlock: return "paged16";
    default: return "paged16_lanes";
  }
}


// Dynamic LDS bytes that leave room for exactly `waves` one-wave workgroups
// on a CU with `lds_per_cu` bytes (0 when no cap is needed).
inline size_t lds_reserve_for(int waves, int lds_per_cu, size_t static_lds) {
  if (waves >= kMaxWavesPerCU || lds_per_cu <= 0) return 0;
  // Midway between the per-group share that fits `waves` groups and the one
  // that would fit `waves + 1`, so allocation granularity cannot tip it.
  const size_t hi = (size_t)lds_per_cu / waves;
  const size_t lo = (size_t)lds_per_cu / (waves + 1);
  const size_t per_group = (hi + lo) / 2;
  return per_group > static_lds ? per_group - static_lds : 0;
}

// LDS bytes per CU of the current device, queried once per device.
inline int lds_per_cu() {
  constexpr int kMaxDevices = 64;
  static std::atomic<int> cache[kMaxDevices];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return 0;
  const bool cacheable = dev >= 0 && dev < kMaxDevices;
  if (cacheable) {
    const int v = cache[dev].load(std::memory_order_relaxed);
    if (v > 0) return v;
  }
  int bytes = 0;
  if (hipDeviceGetAttribute(&bytes, hipDeviceAttributeMaxSharedMemoryPerMultiprocessor, dev) != hipSuccess) return 0;
  if (cacheable) cache[dev].store(bytes, std::memory_order_relaxed);
  return bytes;
}

// Compute units of the current device, queried once per device.
inline int device_cus() {
  constexpr int kMaxDevices = 64;
  static std::atomic<int> cache[kMaxDevices];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return 0;
  const bool cacheable = dev >= 0 && dev < kMaxDevices;
  if (cacheable) {
    const int v = cache[dev].load(std::memory_order_relaxed);
    if (v > 0) return v;
  }
  int n = 0;
  if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) return 0;
  if (cacheable) cache[dev].store(n, std::memory_order_relaxed);
  return n;
}

// Static LDS of a kernel, queried once (a property of the code object).
template <auto KERNEL>
size_t static_lds() {
  static const size_t bytes = [] {
    hipFuncAttributes attr;
    return hipFuncGetAttributes(&attr, reinterpret_cast<const void*>(KERNEL)) == hipSuccess ? attr.sharedSizeBytes
                                                                                           : size_t(0);
  }();
  return bytes;
}

// Dynamic LDS that caps KERNEL at `waves` one-wave workgroups per CU.
template <auto KERNEL>
size_t lds_reserve_kernel(int waves) {
  return lds_reserve_for(waves, lds_per_cu(), static_lds<KERNEL>());
}

template <int D, int G, int LAYOUT, int SB, bool PF32, bool EXACT = false>
hipError_t launch_one(const DecodeArgs& a, int waves_per_cu, hipStream_t stream) {
  constexpr auto kernel = fmha_decode::fmha_decode_fwd_kernel<D, G, LAYOUT, SB, PF32, EXACT>;
  plan_note("short(numerics=%s D=%d G=%d layout=%s bucket=%s%d waves_per_cu=%d)",
            EXACT ? "exact" : PF32 ? "fp32_weights" : "fast", D, G, layout_name(LAYOUT), SB == 0 ? "per_wave<=" : "",
            SB == 0 ? 16 : SB, waves_per_cu);
  const uint32_t blocks = (a.total_units + kWavesPerBlock - 1) / kWavesPerBlock;
  hipLaunchKernelGGL(kernel, dim3(blocks), dim3(kBlockThreads), lds_reserve_kernel<kernel>(waves_per_cu), stream, a);
  return hipGetLastError();
}

// sb: 0 = lengths from a.lens (bucket picked per wave), else the uniform
// length's power-of-two bucket.  The paged layout always reads lengths.
// PF32: fp32 softmax weights (instantiated for the packed layout only).
// EXACT: the exact-arithmetic kernels (packed layout, G = 1).
template <int D, int G, int LAYOUT, bool PF32, bool EXACT = false>
hipError_t launch_bucket(const DecodeArgs& a, int sb, int w, hipStream_t stream) {
  if constexpr (LAYOUT == fmha_decode::kLayoutPaged) {
    return launch_one<D, G, LAYOUT, 0, PF32, EXACT>(a, w, stream);
  } else {
    switch (sb) {
      case 0: return launch_one<D, G, LAYOUT, 0, PF32, EXACT>(a, w, stream);
      case 1: return launch_one<D, G, LAYOUT, 1, PF32, EXACT>(a, w, stream);
      case 2: return launch_one<D, G, LAYOUT, 2, PF32, EXACT>(a, w, stream);
      case 4: return launch_one<D, G, LAYOUT, 4, PF32, EXACT>(a, w, stream);
      case 8: return launch_one<D, G, LAYOUT, 8, PF32, EXACT>(a, w, stream);
      default: return launch_one<D, G, LAYOUT, 16, PF32, EXACT>(a, w, stream);
    }
  }
}

template <int D, int LAYOUT, bool PF32>
hipError_t launch_group(const DecodeArgs& a, int g, int sb, int w, hipStream_t stream) {
  switch (g) {
    case 1: return launch_bucket<D, 1, LAYOUT, PF32>(a, sb, w, stream);
    case 2: return launch_bucket<D, 2, LAYOUT, PF32>(a, sb, w, stream);
    case 4: return launch_bucket<D, 4, LAYOUT, PF32>(a, sb, w, stream);
    default: return launch_bucket<D, 8, LAYOUT, PF32>(a, sb, w, stream);
  }
}

template <int LAYOUT, bool PF32 = false>
hipError_t launch_dim(const DecodeArgs& a, int d, int g, int sb, int w, hipStream_t stream) {
  switch (d) {
    case 64: return launch_group<64, LAYOUT, PF32>(a, g, sb, w, stream);
    case 128: return launch_group<128, LAYOUT, PF32>(a, g, sb, w, stream);
    default: return launch_group<256, LAYOUT, PF32>(a, g, sb, w, stream);
  }
}

template <int D, int G, int LAYOUT, bool PF32, bool EXACT = false>
hipError_t launch_multi_one(const DecodeArgs& a, int waves_per_cu, hipStream_t stream) {
  constexpr auto kernel = fmha_decode::fmha_decode_multi_kernel<D, G, LAYOUT, PF32, EXACT>;
  plan_note("short_multi(numerics=%s D=%d G=%d layout=%s batches_per_wave=%d waves_per_cu=%d)",
            EXACT ? "exact" : PF32 ? "fp32_weights" : "fast", D, G, layout_name(LAYOUT), 1 << a.sub_shift,
            waves_per_cu);
  const uint32_t blocks = (a.total_units + kWavesPerBlock - 1) / kWavesPerBlock;
  hipLaunchKernelGGL(kernel, dim3(blocks), dim3(kBlockThreads), lds_reserve_kernel<kernel>(waves_per_cu), stream, a);
  return hipGetLastError();
}

template <int LAYOUT, bool PF32>
hipError_t launch_multi(const DecodeArgs& a, int d, int g, int w, hipStream_t stream) {
#define FMHA_DECODE_MULTI_G(DD)                                                  \
  switch (g) {                                                                   \
    case 1: return launch_multi_one<DD, 1, LAYOUT, PF32>(a, w, stream);          \
    case 2: return launch_multi_one<DD, 2, LAYOUT, PF32>(a, w, stream);          \
    case 4: return launch_multi_one<DD, 4, LAYOUT, PF32>(a, w, stream);          \
    default: return launch_multi_one<DD, 8, LAYOUT, PF32>(a, w, stream);         \
  }
  switch (d) {
    case 64: FMHA_DECODE_MULTI_G(64)
    case 128: FMHA_DECODE_MULTI_G(128)
    default: FMHA_DECODE_MULTI_G(256)
  }
#undef FMHA_DECODE_MULTI_G
}

// The exact-arithmetic kernels: packed layout, G query heads per KV head
// (1, 2, 4, 8; 3 and 5-7 run on the 4- and 8-head kernels as padded
// groups); multi: R batches per wave (fewer KV heads than a wave holds).
// Known lengths (sb > 0, the uniform entry point) take them for G <= 2
// only, the groups whose default numerics they are; above, only
// fmha_decode_fwd_exact reaches them, with lengths on the device.
template <int D, int G>
hipError_t launch_exact(const DecodeArgs& a, bool multi, int sb, int w, hipStream_t stream) {
  if (multi) return launch_multi_one<D, G, kLayoutPacked, false, true>(a, w, stream);
  if constexpr (G <= 2) {
    return launch_bucket<D, G, kLayoutPacked, false, true>(a, sb, w, stream);
  } else {
    (void)sb;
    return launch_one<D, G, kLayoutPacked, 0, false, true>(a, w, stream);
  }
}

template <int D, int NS, int LAYOUT>
hipError_t launch_mfma_one(const fmha_decode::GroupArgs& g, int waves_per_cu, hipStream_t stream) {
  constexpr auto kernel = fmha_decode::fmha_decode_group_kernel<D, 0, NS, LAYOUT>;
  plan_note("short_matrix_core(D=%d G=%d layout=%s streams_per_tile=%d waves_per_cu=%d)", D, (int)g.group,
            layout_name(LAYOUT), NS, waves_per_cu);
  hipLaunchKernelGGL(kernel, dim3(g.waves), dim3(kBlockThreads), lds_reserve_kernel<kernel>(waves_per_cu), stream, g);
  return hipGetLastError();
}

template <int D, int LAYOUT>
hipError_t launch_mfma_d(const fmha_decode::GroupArgs& g, int ns, int w, hipStream_t stream) {
  switch (ns) {
    case 1: return launch_mfma_one<D, 1, LAYOUT>(g, w, stream);
    case 2: return launch_mfma_one<D, 2, LAYOUT>(g, w, stream);
    default:
      if constexpr (fmha_decode::GroupShape<D>::HPW >= 4) return launch_mfma_one<D, 4, LAYOUT>(g, w, stream);
      else return launch_mfma_one<D, 2, LAYOUT>(g, w, stream);
  }
}

template <int LAYOUT>
hipError_t launch_mfma_layout(const fmha_decode::GroupArgs& g, int dq, int ns, int w, hipStream_t stream) {
  if constexpr (LAYOUT == fmha_decode::kLayoutPaged || LAYOUT == fmha_decode::kLayoutPagedLanes) {
    // Paged caches reach the matrix-core kernel for groups above 8 only:
    // one stream per 16-column tile.
    if (ns != 1) return hipErrorInvalidValue;
    switch (dq) {
      case 64: return launch_mfma_one<64, 1, LAYOUT>(g, w, stream);
      case 128: return launch_mfma_one<128, 1, LAYOUT>(g, w, stream);
      default: return launch_mfma_one<256, 1, LAYOUT>(g, w, stream);
    }
  } else {
    switch (dq) {
      case 64: return launch_mfma_d<64, LAYOUT>(g, ns, w, stream);
      case 128: return launch_mfma_d<128, LAYOUT>(g, ns, w, stream);
      default: return launch_mfma_d<256, LAYOUT>(g, ns, w, stream);
    }
  }
}

// Per-CU wave caps of the two streaming passes (dynamic LDS reservation).
// Scores waves request 16 KiB of K plus G KiB of Q at once; P.V waves keep
// two 16-row (8-row for G = 8) sub-blocks of V in flight.  Swept apart
// (µs at scores caps 4 / 6 / 8 / 12 / 16, P.V at 8; Hq/Hkv 32/8 D=128):
// B=64 S=4096 210.8/192.7/190.9/188.7/187.9, B=8 S=32768
// 213.9/194.0/191.7/189.9/190.3, B=1 S=131072 116.8/107.7/106.7/104.4/105.2;
// Hq=Hkv=16 B=16 S=8192 and the matrix-core passes (64/8 B=256 S=1024)
// flat from 6 up.  P.V caps of 4-12 are within 1% everywhere.
constexpr int kSplitScoresWavesPerCU = 12;
constexpr int kSplitPvWavesPerCU = 8;

// Rows longer than 16 go through one pass (onepass_decode_kernel: one wave
// per batch and head group, no workspace traffic, one launch) when there are
// at least 512 such units and the row's scores and weights fit the wave's
// LDS budget; otherwise through the four split-KV launches.  Measured
// (µs, split -> one pass, 8 waves per CU): B=2048 Hq=32 Hkv=8 S=128 201 ->
// 171; B=4096 S=64 206 -> 178; B=16384 S=24 327 -> 296; B=256 S=256 (512
// units) 69 -> 58; B=128 S=256 (256 units) 43 -> 49 and B=16 S=256 23 -> 49,
// where a wave's walk over its row outlasts split-KV's shorter waves.
constexpr int64_t kOnepassMinUnits = 512;
constexpr size_t kOnepassMaxLdsPerWave = 40 * 1024;
// Waves per CU of the single pass: 8, and 4 for one or two query heads per
// KV head with rows of at most 48 (three 16-row blocks), whose waves compute
// little per byte (µs at 4 / 8 waves, D=128 unless given: B=16384 S=24
// Hq/Hkv 16/16 497.5 / 545.9, 16/8 S=32 341.4 / 363.8, B=8192 S=48 32/16
// 503.2 / 539.2, B=4096 S=32 16/16 D=256 326.0 / 344.4; longer rows are
// flat or faster at 8, B=1024 S=128 16/16 172.8 / 163.8; G = 4 and 8 flat
// from 8 up).
constexpr int kOnepassWavesPerCU = 8;
constexpr int kOnepassWavesPerCUNarrow = 4;
// Pages under 16 rows, one or two query heads per KV head: 12 (157 VGPRs
// leave room), the per-row page lookups wanting more waves in flight (µs at
// 4 or 8 / 12: B=5461 S=24 Hq/Hkv 8/8 158 / 108, B=2730 S=48 129 / 102,
// B=16384 S=24 16/16 895 / 597, S=48 1391 / 1065; 16-row pages measured
// 2-6% slower at 12 and keep the caps above).
constexpr int kOnepassWavesPerCUPagedRows = 12;
// Waves per CU the LDS must hold for the 8-row sub-blocks of the one-batch
// paged single pass on rows of more than four blocks (launch_onepass_dg).
constexpr int kOnepassRows8MinWaves = 12;

// Waves of the single pass: ceil(batch / 2^sub_shift) batch groups times
// the KV-head groups of one.
inline int64_t onepass_waves(const SplitArgs& a) {
  return (((int64_t)a.batch + (1 << a.sub_shift) - 1) >> a.sub_shift) * a.units_per_batch;
}

template <int D, int G>
bool onepass_fits(const SplitArgs& a) {
  return onepass_waves(a) >= kOnepassMinUnits &&
         fmha_decode::onepass_lds_bytes<D, G>(fmha_decode::onepass_lds_rows(a.nblk)) <= kOnepassMaxLdsPerWave;
}

// The single pass with two waves per unit (a workgroup sharing one row)
// for rows with fewer than kOnepassMinUnits units: from 192 units with one
// or two query heads per KV head and from 384 with four (eight take the
// matrix cores), if a unit's LDS stays within kOnepassMaxLdsPerGroup.  Two
// waves against the split passes (µs, D = 128 unless given, packed): B=64
// S=256 Hq/Hkv 16/16 25.6 / 30.8, B=120 S=128 16/16 26.0 / 28.7, B=200
// S=256 8/8 38.2 / 42.7, B=100 S=512 16/16 70.4 / 76.7, B=200 S=96 32/8
// 25.6 / 31.5, D=64 B=64 S=256 32/32 28.1 / 30.9, D=256 B=60 S=160 16/8
// 17.9 / 23.0 (240 units); fewer units lose (B=128 S=256 32/8, 256 units:
// 38.9 / 37.0; B=64 S=256 32/8 36.7 / 25.1; B=32 S=1024 16/16 59.2 /
// 51.4), and four or eight waves per row measured slower than two wherever
// two applied.  Packed caches, and strided ones up to 16 blocks (BHSD:
// B=64 S=256 16/16 30.8 / 32.2, B=200 S=96 32/8 25.7 / 31.3, but B=100
// S=512 16/16 85.1 / 79.2); paged ones keep the split passes (within 1%
// either way).  FMHA_DECODE_ONEPASS_WAVES=1 turns it off (for sweeps).
constexpr size_t kOnepassMaxLdsPerGroup = 64 * 1024;
constexpr int kOnepassGroupNW = 2;

template <int D, int G, int LAYOUT>
bool onepass_group_fits(const SplitArgs& a) {
  if (const char* e = std::getenv("FMHA_DECODE_ONEPASS_WAVES"))
    if (std::atoi(e) == 1) return false;
  // One batch per unit: with fewer KV heads than a wave's lane groups the
  // rest would idle (µs, packed, D = 256, two-wave single pass / split
  // passes with the lane groups on other blocks: B=488 S=1024 4/1 152.0 /
  // 99-102, B=244 S=2048 2/1 116.3 / 96-104).
  constexpr int HPW = kWaveSize / (D / 8);
  const int64_t units = onepass_waves(a);
  return G <= 4 && a.num_heads_kv >= HPW && units < kOnepassMinUnits && units >= (G <= 2 ? 192 : 384) &&
         a.nblk >= 2 * kOnepassGroupNW &&
         (LAYOUT == fmha_decode::kLayoutPacked || a.nblk <= 16) &&
         fmha_decode::onepass_lds_bytes<D, G>(fmha_decode::onepass_lds_rows(a.nblk, kOnepassGroupNW),
                                              kOnepassGroupNW) <= kOnepassMaxLdsPerGroup;
}

template <auto KERNEL>
hipError_t launch_onepass_kernel(const SplitArgs& a, size_t need, int waves, hipStream_t stream) {
  const size_t cap = lds_reserve_kernel<KERNEL>(waves);
  hipLaunchKernelGGL(KERNEL, dim3((uint32_t)onepass_waves(a)), dim3(kBlockThreads), need > cap ? need : cap, stream,
                     a);
  return hipGetLastError();
}

template <int D, int G, int LAYOUT, bool MULTI>
hipError_t launch_onepass_dg(const SplitArgs& a, hipStream_t stream) {
  const size_t need = fmha_decode::onepass_lds_bytes<D, G>(fmha_decode::onepass_lds_rows(a.nblk));
  int waves = LAYOUT == fmha_decode::kLayoutPaged && G <= 2 ? kOnepassWavesPerCUPagedRows
              : !MULTI && G <= 2 && a.nblk <= 3     ? kOnepassWavesPerCUNarrow
                                                    : kOnepassWavesPerCU;
  if constexpr (LAYOUT == fmha_decode::kLayoutPagedBlockLanes) {
    // 16-row pages with per-lane lookups (three waves per SIMD fit): 8 or
    // 12 waves per CU, whichever leaves the last round of waves fuller --
    // each wave is one pass of about equal length, so a launch runs in
    // rounds (µs, 8 / 12 waves per CU: 4/1 D=128 S=96, 2605 waves, 113 /
    // 87; S=64, 3907 waves, 95 / 99; S=24, 10417 waves, 112 / 108; 8/1
    // D=256 S=96 150 / 107; 2/1 D=64 S=64 87 / 90).  Ties take 12.
    const int64_t w = onepass_waves(a);
    const int64_t cus = device_cus() > 0 ? device_cus() : 256;
    auto slots = [&](int64_t c) { return (w + c * cus - 1) / (c * cus) * c; };
    waves = slots(12) <= slots(8) ? 12 : 8;
  }
  // FMHA_DECODE_ONEPASS_WAVES_PER_CU=n: n waves per CU instead (sweeps).
  if (const char* e = std::getenv("FMHA_DECODE_ONEPASS_WAVES_PER_CU"))
    if (std::atoi(e) > 0) waves = std::atoi(e);
  if constexpr (LAYOUT == fmha_decode::kLayoutPaged && !MULTI) {
    // Pages under 16 rows, one batch per wave: 8-row sub-blocks and more
    // waves per CU on rows of up to four blocks, and on rows of five or six
    // where the LDS holds kOnepassRows8MinWaves waves (µs, one-row pages,
    // 16-row sub-blocks at 8 or 12 waves / 8-row ones, B sized for 512 MB
    // of K and V unless given: Hq/Hkv 32/8 D=128 S=24 130 / 105, S=96 102 /
    // 90, B=2048 S=96 145 / 140; 64/8 S=24 156 / 120, S=48 139 / 116; 8/8
    // S=24 104 / 97; D=64 32/8 S=24 131 / 107, 64/8 S=48 156 / 137; D=256
    // 64/8 S=96 118 / 98; where the LDS holds 8 waves the 16-row ones stay
    // ahead: D=64 32/8 S=96 111 / 118, D=128 64/8 S=96 124 / 136; and on
    // rows of eight blocks with more waves than one round at 8 per CU:
    // B=2048 S=128 32/8 185 / 201, B=4096 366 / 388).
    bool rows8 = a.nblk <= 4 || (a.nblk <= 6 && need * kOnepassRows8MinWaves <= (size_t)lds_per_cu());
    if (const char* e = std::getenv("FMHA_DECODE_ONEPASS_ROWS8")) rows8 = std::atoi(e) != 0;
    if (rows8) {
      if (!std::getenv("FMHA_DECODE_ONEPASS_WAVES_PER_CU")) waves = 16;
      plan_note("onepass(D=%d G=%d layout=%s batches_per_wave=1 blocks=%d waves_per_cu=%d rows=8)", D, G,
                layout_name(LAYOUT), a.nblk, waves);
      return launch_onepass_kernel<fmha_decode::onepass_decode_kernel<D, G, LAYOUT, false, 1, 1, true>>(a, need, waves,
                                                                                                      stream);
    }
  }
  if constexpr (LAYOUT == fmha_decode::kLayoutPagedBlock && !MULTI && G >= 4) {
    // Pages of 16 rows or more, one batch per wave: 8-row sub-blocks at 16
    // waves per CU for groups of 8 (rows of up to three blocks at D = 64,
    // six at D = 128, any at D = 256) and of 4 at D = 128 on rows of up to
    // three (µs, B sized for 512 MB of K and V, 16-row sub-blocks / 8-row:
    // 64/8 D=256 S=24 132.5 / 113.6, S=128 110.3 / 87.0; D=128 S=24 121.5 /
    // 113.9, S=96 126.0 / 119.5, but S=128 112.9 / 142.6; D=64 S=96 142.9 /
    // 150.7; 32/8 D=128 S=48 99.6 / 94.3).
    bool rows8 = G == 8 ? (D == 256 || a.nblk <= (D == 128 ? 6 : 3)) : D == 128 && a.nblk <= 3;
    if (const char* e = std::getenv("FMHA_DECODE_ONEPASS_ROWS8")) rows8 = std::atoi(e) != 0;
    if (rows8) {
      if (!std::getenv("FMHA_DECODE_ONEPASS_WAVES_PER_CU")) waves = 16;
      plan_note("onepass(D=%d G=%d layout=%s batches_per_wave=1 blocks=%d waves_per_cu=%d rows=8)", D, G,
                layout_name(LAYOUT), a.nblk, waves);
      return launch_onepass_kernel<fmha_decode::onepass_decode_kernel<D, G, LAYOUT, false, 1, 1, true>>(a, need, waves,
                                                                                                      stream);
    }
  }
  if constexpr ((LAYOUT == fmha_decode::kLayoutPacked || LAYOUT == fmha_decode::kLayoutStrided) && G >= 4) {
    // One descriptor per wave, groups of 8 on rows of up to four blocks
    // (any at D = 256), groups of 4 on rows of up to two: 8-row sub-blocks
    // at 16 waves per CU (µs, packed, B sized for 512 MB of K and V unless
    // given, 16-row sub-blocks at 8 waves / 8-row ones: Hq/Hkv 16/2 D=128
    // S=24 123.5 / 110.4, S=48 117.1 / 107.1; 64/8 S=24 117.4 / 112.4; 8/1
    // D=64 S=24 123.0 / 117.3; 64/8 D=256 S=48 113.7 / 104.1, S=128 94.1 /
    // 91.8, B=2048 S=128 380.2 / 371.8; 4/1 D=64 S=24 103.6 / 97.6, D=128
    // 100.3 / 97.1; but 32/8 D=64 S=48 98.8 / 100.1, S=128 114.5 / 116.8;
    // 64/8 D=128 B=4096 S=96 298.5 / 320.1).
    // FMHA_DECODE_ONEPASS_ROWS8=0 or 1 turns them off or on (sweeps).
    bool rows8 = G == 8 ? (D == 256 || a.nblk <= 4) : a.nblk <= 2;
    if (const char* e = std::getenv("FMHA_DECODE_ONEPASS_ROWS8")) rows8 = std::atoi(e) != 0;
    if (rows8) {
      if (!std::getenv("FMHA_DECODE_ONEPASS_WAVES_PER_CU")) waves = 16;
      plan_note("onepass(D=%d G=%d layout=%s batches_per_wave=%d blocks=%d waves_per_cu=%d rows=8)", D, G,
                layout_name(LAYOUT), 1 << a.sub_shift, a.nblk, waves);
      return launch_onepass_kernel<fmha_decode::onepass_decode_kernel<D, G, LAYOUT, MULTI, 1, 1, true>>(a, need, waves,
                                                                                                      stream);
    }
  }
  plan_note("onepass(D=%d G=%d layout=%s batches_per_wave=%d blocks=%d waves_per_cu=%d)", D, G, layout_name(LAYOUT),
            1 << a.sub_shift, a.nblk, waves);
  // 16-row pages, eight query heads per KV head, rows of up to four blocks
  // that keep 16-row sub-blocks (D = 64, four blocks; or the 8-row form
  // turned off): the kernel scheduled for two waves per SIMD.
  if constexpr (!MULTI && G == 8 && LAYOUT == fmha_decode::kLayoutPagedBlock)
    if (a.nblk <= 4)
      return launch_onepass_kernel<fmha_decode::onepass_decode_kernel<D, G, LAYOUT, MULTI, 2>>(a, need, waves, stream);
  return launch_onepass_kernel<fmha_decode::onepass_decode_kernel<D, G, LAYOUT, MULTI>>(a, need, waves, stream);
}

// The single pass with kOnepassGroupNW waves per unit, one batch per unit.
template <int D, int G, int LAYOUT>
hipError_t launch_onepass_group(const SplitArgs& a, hipStream_t stream) {
  constexpr int NW = kOnepassGroupNW;
  const size_t need = fmha_decode::onepass_lds_bytes<D, G>(fmha_decode::onepass_lds_rows(a.nblk, NW), NW);
  plan_note("onepass_group(D=%d G=%d layout=%s waves_per_row=%d blocks=%d)", D, G, layout_name(LAYOUT), NW, a.nblk);
  hipLaunchKernelGGL((fmha_decode::onepass_decode_kernel<D, G, LAYOUT, false, 1, NW>), dim3((uint32_t)onepass_waves(a)),
                     dim3(kBlockThreads * NW), need, stream, a);
  return hipGetLastError();
}


// Launchers of the kernels every long-row path shares, defined once in the
// part that owns them (fmha_decode_inst.hip, FMHA_DECODE_PART 0).
// The statistics pass of split-KV (rows of more than kPvStatBlocks blocks):
// the global max and sum per (batch, query head).
void launch_split_stats(const SplitArgs& a, hipStream_t stream);
// The combine pass of split-KV (more than one chunk per row): the partial
// outputs summed in chunk order.
void launch_split_combine(const SplitArgs& a, int d, hipStream_t stream);

// Rows of up to this many 16-row blocks: every split-KV P.V wave reduces its
// heads' block statistics itself (no statistics pass; µs with the pass /
// without: B=256 S=1024 Hq/Hkv 64/8 222 / 218, B=128 S=256 32/8 41 / 37).
constexpr int kPvStatBlocks = 64;

// Q rows copied to, and O rows back from, a query group padded to GP rows
// per (batch, KV head) stream (fmha_decode_group.hpp).
hipError_t launch_pad_query_group(const uint16_t* q, uint16_t* qp, uint64_t streams, int G, int GP, int D,
                                  hipStream_t stream);
hipError_t launch_unpad_output_group(const uint16_t* op, uint16_t* o, uint64_t streams, int G, int GP, int D,
                                     hipStream_t stream);

// Returned by the long-row launchers with onepass_only when the single pass
// does not apply (nothing launched).
constexpr hipError_t kOnepassNotTaken = hipErrorNotReady;

// The matrix-core single pass with the row's scores in LDS
// (onepass_mfma_kernel): NW waves per (batch, KV head), for groups of at
// most 16 query heads per KV head (after padding) on packed and strided
// caches, rows of at least 8 blocks and at least 512 units, where the
// register single pass below does not apply: D = 256 rows of up to 40
// blocks, one wave per row within 80 KiB of LDS.  At D = 128 and 64 the
// register pass measured faster wherever this one fits, and takes those
// rows.  Against the matrix-core split passes (µs, packed, B x Hq/Hkv x S;
// NW = 1 / 2 / 4 / split):
//   D = 128: 1024 x 64/8 x 160: 127.9 / 156.1 / 166.7 / 145.9; x 256:
//   199.7 / 191.6 / 205.9 / 220.4; 512 x 64/8 x 512: 200.8 / 189.3 / 258.0
//   / 220.0; 256 x 64/8 x 1024: 255.5 / 202.4 / 217.2 / 219.1; x 1536:
//   468.9 / 484.6 / 299.2 / 360.7; 128 x 64/8 x 2048: 588.9 / 320.3 / 195.8
//   / 223.1; 512 x 16/1 x 600: 52.9 / 36.9 / 43.8 / 66.1; 512 x 128/8 x 512
//   (G = 16): 250.8 / 216.6 / 259.9 / 252.2; 64 x 96/8 x 300 (G = 12): 36.7
//   / 30.4 / 38.2 / 46.9;
//   D = 256: 256 x 32/4 x 500: 85.3 / 102.5 / 104.6 / 100.6 (the register
//   single pass: 93.2 with 16 tiles per wave, 96.4 with 8);
//   D = 64: 600 x 8/1 x 1200: 145.5 / 81.3 / 81.7 / 68.4.
// At D = 256 one wave per row within 80 KiB.
// FMHA_DECODE_ONEPASS_MFMA=0 turns it off and =1, 2, 4 forces the waves
// per row wherever the LDS fits (for sweeps).
constexpr int64_t kOnepassMfmaMinUnits = 512;
constexpr int kOnepassMfmaMinBlocks = 8;

// Waves per row of the matrix-core single pass for a, or 0 where it does
// not apply.
template <int D, int LAYOUT>
int onepass_mfma_waves(const SplitArgs& a) {
  // Pages of 16 rows or more too (µs, D = 256, G = 8, the split passes /
  // this pass: B=122 S=512 64/8 111.5 / 105.0, B=977 S=512 8/1 112.4 /
  // 104.7); pages under 16 rows, a lookup per row, keep the split passes
  // (B=160 S=640 64/8 200.5 / 314.5, B=977 S=512 8/1 116.5 / 124.9).
  if constexpr (LAYOUT != fmha_decode::kLayoutPacked && LAYOUT != fmha_decode::kLayoutStrided &&
                LAYOUT != fmha_decode::kLayoutPagedBlock) {
    return 0;
  } else {
    const int g = a.num_heads_q / a.num_heads_kv;
    const int64_t units = (int64_t)a.batch * a.num_heads_kv;
    if (g > 16 || units < kOnepassMfmaMinUnits || units > INT32_MAX) return 0;
    auto lds = [&](int nw) { return fmha_decode::onepass_mfma_lds_bytes<D>(g, a.nblk, nw); };
    if (const char* e = std::getenv("FMHA_DECODE_ONEPASS_MFMA")) {
      const int v = std::atoi(e);
      if (v == 0) return 0;
      if (v == 1 || v == 2 || v == 4) return lds(v) <= 160 * 1024 ? v : 0;
    }
    if (a.nblk < kOnepassMfmaMinBlocks) return 0;
    if constexpr (D == 256) {
      return lds(1) <= 80 * 1024 ? 1 : 0;
    } else {
      return 0;  // the register single pass takes these rows
    }
  }
}

template <int D, int LAYOUT>
hipError_t launch_onepass_mfma(const SplitArgs& a, int nw, hipStream_t stream) {
  const int g = a.num_heads_q / a.num_heads_kv;
  const size_t need = fmha_decode::onepass_mfma_lds_bytes<D>(g, a.nblk, nw);
  plan_note("onepass_matrix_core(D=%d G=%d layout=%s waves_per_row=%d blocks=%d)", D, g, layout_name(LAYOUT), nw,
            a.nblk);
  const dim3 grid((uint32_t)((int64_t)a.batch * a.num_heads_kv));
  switch (nw) {
    case 1:
      hipLaunchKernelGGL((fmha_decode::onepass_mfma_kernel<D, 1, LAYOUT>), grid, dim3(kBlockThreads), need, stream, a);
      break;
    case 4:
      hipLaunchKernelGGL((fmha_decode::onepass_mfma_kernel<D, 4, LAYOUT>), grid, dim3(kBlockThreads * 4), need, stream,
                         a);
      break;
    default:
      hipLaunchKernelGGL((fmha_decode::onepass_mfma_kernel<D, 2, LAYOUT>), grid, dim3(kBlockThreads * 2), need, stream,
                         a);
      break;
  }
  return hipGetLastError();
}

// The matrix-core single pass with the row's scores in registers
// (onepass_mfma_reg_kernel): workgroups of ceil(nblk / TPW) <= 8 waves, TPW
// 16-row tiles per wave (8 up to 32 blocks, 16 up to 128, 32 beyond at D <=
// 128: rows of up to 4096 at D <= 128, 2048 at D = 256), for groups of at
// most 16 query heads per KV head (after padding), at least
// 128-256 (batch, KV head) units (kOnepassRegMinUnitsWide / Small / 256)
// and kOnepassRegMinBlocks
// blocks (at D = 256 more than kOnepassReg256LdsBlocks) on packed,
// strided and paged caches (one-row pages, µs against the split passes:
// B=256 S=1024 64/8 189.3 / 241.6, B=128 S=256 32/8 27.4 / 45.5; 16-row
// pages: B=256 S=1024 64/8
// 178.6 / 228.4, B=128 S=2048 64/8 177.9 / 232.6, B=64 S=4096 32/8 177.7 /
// 199.3, B=128 S=256 32/8 25.8 / 38.2).  Against the LDS
// single pass at its best waves per row (µs, packed, D = 128, B x Hq/Hkv x
// S): 256 x 64/8 x 1024 173.7 / 202.6, 512 x 64/8 x 512 179.2 / 189.7, 1024 x
// 64/8 x 256 188.9 / 190.7, 128 x 64/8 x 2048 174.5 / 194.7, 256 x 64/8 x
// 1536 261.9 / 297.8, 512 x 16/1 x 600 31.5 / 36.6, 512 x 128/8 x 512 188.1
// / 216.5, 64 x 96/8 x 300 26.0 / 30.4, 1024 x 64/8 x 160 123.9 / 127.7,
// 4096 x 8/1 x 256 91.1 / 99.1 (x
// 128: 97.6 / 95.4); against the split passes at D = 64: 2048 x 64/8 x 256
// 206.4 / 274.3, 1024 x 32/4 x 512 106.3 / 142.0, 4096 x 32/4 x 128 101.8 /
// 147.6, 600 x 8/1 x 1200 65.1 / 68.4.  Eight tiles per wave against 16
// (same shapes): 179.0 / 173.7, 179.2 / 183.3, 188.9 / 186.9, 34.1 / 31.5,
// 188.1 / 190.3, 26.0 / 32.4, 123.9 / 125.4.  32 tiles (256 VGPRs, 20 bytes
// of scratch per lane, V two tiles ahead) against the split passes: 64 x
// 32/8 x 4096 175.1 / 189.9, 128 x 64/8 x 4096 348.5 / 427.9, 128 x 32/8 x
// 3000 268.5 / 280.0, 256 x 16/2 x 4096 181.5 / 218.9, D=64 512 x 16/1 x
// 4000 104.3 / 174.3.  FMHA_DECODE_ONEPASS_REG=0 turns it off, =8, 16 or
// 32 forces the tiles per wave (32 at D <= 128; for sweeps).
constexpr int kOnepassRegMaxWaves = 8;
// Rows of fewer blocks keep the split passes (three blocks: µs, 8/8
// B=200 S=40, 14.1 against 13.1).
constexpr int kOnepassRegMinBlocks = 4;
// At D = 256 the LDS single pass (one wave per row) keeps rows of up to
// this many blocks and the register pass takes longer ones, 16 tiles per
// wave (µs, Hq/Hkv 32/4, LDS / register: B=256 S=500 84.9 / 93.2, B=512
// S=600 205.3 / 225.9; B=256 S=768 206.3 / 135.3, S=1024 272.1 / 176.5,
// B=512 S=900 373.3 / 323.6, 64/8 B=256 S=1536 699.7 / 524.5; against the
// matrix-core split passes B=128 S=2048 187.6 / 174.9, 64/8 B=64 S=2000
// 194.7 / 173.4, 96/8 B=128 S=1024 223.4 / 193.8; 8 tiles per wave were
// slower at every length swept).
constexpr int kOnepassReg256LdsBlocks = 40;
// Fewer (batch, KV head) units than kOnepassMfmaMinUnits still fill the
// CUs with several waves per row: at D = 128 from 128 units for groups of 5
// and more (the matrix-core split passes the alternative) and 256 below
// (the VALU ones), at D = 64 from 128, at D = 256 from 192.  µs, packed,
// register pass / split passes: D = 128 16/2 B=128 S=1024 (256 units) 29.8
// / 47.9, 64/8 B=32 S=1024 28.6 / 47.1, B=48 S=2048 79.3 / 99.7, 32/8 B=32
// S=4096 93.1 / 104.5, 16/4 B=64 S=512 16.9 / 26.7; 64/8 B=16 S=4096 (128
// units) 66.0 / 72.1, S=1024 24.7 / 33.7; fewer lose, 64/8 B=8 S=4096 (64
// units) 60.9 / 47.4, and so do groups of 4 at 128, 32/8 B=16 S=4096 66.0 /
// 61.0.  D = 64: 64/8 B=32 S=2048 31.1 / 54.6, B=16 27.4 / 35.5, 16/4 B=32
// S=2048 26.6 / 32.4.  D = 256: 64/8 B=32 S=1024 49.9 / 61.6, 32/4 B=48
// S=1536 60.5 / 69.2, but 64/8 B=16 S=2048 (128 units) 68.0 / 63.4.
constexpr int64_t kOnepassRegMinUnitsWide = 128;
constexpr int64_t kOnepassRegMinUnitsSmall = 256;
constexpr int64_t kOnepassRegMinUnits256 = 192;
// Waves of the one-wave VALU single pass below which groups of at most 4
// take the register single pass first (launch_split_dg).
constexpr int64_t kOnepassRegBeforeWaves = 1024;

// Tiles per wave of the register single pass for a, or 0 where it does not
// apply.
template <int D, int LAYOUT>
int onepass_reg_tiles(const SplitArgs& a) {
  if constexpr (LAYOUT != fmha_decode::kLayoutPacked && LAYOUT != fmha_decode::kLayoutStrided &&
                LAYOUT != fmha_decode::kLayoutPagedBlock && LAYOUT != fmha_decode::kLayoutPaged) {
    return 0;
  } else {
    const int g = a.num_heads_q / a.num_heads_kv;
    const int64_t units = (int64_t)a.batch * a.num_heads_kv;
    const int64_t min_units = D == 128  ? (g >= 5 ? kOnepassRegMinUnitsWide : kOnepassRegMinUnitsSmall)
                              : D == 64 ? kOnepassRegMinUnitsWide
                                        : kOnepassRegMinUnits256;
    if (g > 16 || units < min_units || units > INT32_MAX) return 0;
    int tpw = a.nblk <= 32 ? 8 : a.nblk <= 128 ? 16 : 32;
    // Paged caches at D = 64: 8 tiles per wave up to 64 blocks, 32 beyond
    // (16 took the per-row-page kernel to 171 VGPRs, two waves per SIMD; µs,
    // 8 / 16 / 32 tiles: one-row pages B=244 S=1024 32/8 113.3 / 131.6 /
    // 130.0, B=976 S=2048 8/1 - / 138.7 / 122.9; 16-row pages B=976 S=2048
    // 8/1 - / 114.7 / 104.7, B=128 S=2048 32/8 - / 118.8 / 109.7).
    if (D == 64 && (LAYOUT == fmha_decode::kLayoutPaged || LAYOUT == fmha_decode::kLayoutPagedBlock))
      tpw = a.nblk <= 64 ? 8 : 32;
    if (const char* e = std::getenv("FMHA_DECODE_ONEPASS_REG")) {
      tpw = std::atoi(e);
    } else if (D == 256) {
      if (a.nblk <= kOnepassReg256LdsBlocks) return 0;
      tpw = 16;
    } else if (a.nblk < (g > 8 && D <= 128 && LAYOUT != fmha_decode::kLayoutPaged ? 2 : kOnepassRegMinBlocks)) {
      // Groups above 8 (a 16-column tile full or nearly so) from two blocks,
      // against the matrix-core split passes (µs, D = 128, Hq/Hkv 128/8,
      // split / register pass: packed B=3000 S=40 150.9 / 127.2, B=2604
      // S=48 144.3 / 120.9, B=4096 S=32 172.0 / 159.6, B=5208 S=24 198.0 /
      // 196.5; 16-row pages S=40 168.3 / 151.8, S=24 242.1 / 230.8; one-row
      // pages, a lookup per row, keep the split passes: S=24 252.6 / 289.0).
      return 0;
    }
    if (tpw != 8 && tpw != 16 && !(tpw == 32 && D <= 128)) return 0;
    const int nw = (a.nblk + tpw - 1) / tpw;
    return nw <= kOnepassRegMaxWaves && fmha_decode::onepass_reg_lds_bytes<D>(nw, tpw, LAYOUT) <= 160 * 1024 ? tpw : 0;
  }
}

template <int D, int LAYOUT>
hipError_t launch_onepass_reg(const SplitArgs& a, int tpw, hipStream_t stream) {
  const int g = a.num_heads_q / a.num_heads_kv;
  const int nw = (a.nblk + tpw - 1) / tpw;
  const size_t need = fmha_decode::onepass_reg_lds_bytes<D>(nw, tpw, LAYOUT);
  plan_note("onepass_matrix_core_regs(D=%d G=%d layout=%s waves_per_row=%d tiles_per_wave=%d blocks=%d)", D, g,
            layout_name(LAYOUT), nw, tpw, a.nblk);
  const dim3 grid((uint32_t)((int64_t)a.batch * a.num_heads_kv));
  const dim3 block((uint32_t)(kBlockThreads * nw));
  if (tpw == 8) {
    hipLaunchKernelGGL((fmha_decode::onepass_mfma_reg_kernel<D, 8, kOnepassRegMaxWaves, LAYOUT>), grid, block, need,
                       stream, a);
  } else if (tpw == 16) {
    hipLaunchKernelGGL((fmha_decode::onepass_mfma_reg_kernel<D, 16, kOnepassRegMaxWaves, LAYOUT>), grid, block, need,
                       stream, a);
  } else {
    if constexpr (D <= 128)
      hipLaunchKernelGGL((fmha_decode::onepass_mfma_reg_kernel<D, 32, kOnepassRegMaxWaves, LAYOUT>), grid, block, need,
                         stream, a);
    else
      return hipErrorInvalidValue;  // onepass_reg_tiles gives 32 only at D <= 128
  }
  return hipGetLastError();
}

// Groups of at most 4 (on the VALU launcher) that the register single pass
// takes where the VALU single pass does not hold the row: every such group
// at D = 128, groups of 4 at D = 64, whose 16-column query tile then holds
// 4 heads (µs, packed, register pass / split: 32/8 B=1024 S=512 216.5 /
// 257.4, 16/4 B=256 S=1000 52.4 / 74.6); with one or two heads per tile the
// VALU passes stay ahead there (16/8 B=512 S=600 130.8 / 115.7, 32/32
// B=128 S=2048 424.7 / 341.8).
template <int D, int G>
constexpr bool kRegSmallGroups = G <= 4 && (D == 128 || (D == 64 && G == 4));

// The register single pass's layout for a VALU launcher layout: pages of
// either size whichever way the VALU passes address them.
template <int LAYOUT>
constexpr int RegLayout = LAYOUT == fmha_decode::kLayoutPagedBlockLanes ? fmha_decode::kLayoutPagedBlock
                          : LAYOUT == fmha_decode::kLayoutPagedLanes    ? fmha_decode::kLayoutPaged
                                                                        : LAYOUT;
template <int LAYOUT>
constexpr bool kPagedLayout = LAYOUT == fmha_decode::kLayoutPaged || LAYOUT == fmha_decode::kLayoutPagedLanes ||
                              LAYOUT == fmha_decode::kLayoutPagedBlock ||
                              LAYOUT == fmha_decode::kLayoutPagedBlockLanes;

// LAYOUT: how the K/V rows are addressed (fmha_decode::LongRows).
// onepass_only: launch the single pass if it applies with every lane group
// busy, on rows of at most eight 16-row blocks at D = 128 and 256 (with
// several batches per wave: two at D = 128, four at D = 64), else nothing
// (kOnepassNotTaken), for callers that run the split passes elsewhere.
template <int D, int G, int LAYOUT>
hipError_t launch_split_dg(const SplitArgs& a, hipStream_t stream, bool onepass_only = false) {
  // With fewer KV heads than a wave holds, its lane groups serve 2^shift
  // batches (single pass), blocks (scores) or chunks (P.V) instead of
  // idling: packed and strided layouts, whose descriptor spans the rows
  // (the paged ones address one page at a time).
  constexpr int HPW = kWaveSize / (D / 8);
  constexpr bool LANES = LAYOUT == fmha_decode::kLayoutPagedLanes || LAYOUT == fmha_decode::kLayoutPagedBlockLanes;
  int shift = 0;
  if (LAYOUT == fmha_decode::kLayoutPacked || LAYOUT == fmha_decode::kLayoutStrided || LANES)
    while ((a.num_heads_kv << (shift + 1)) <= HPW && HPW % (a.num_heads_kv << (shift + 1)) == 0) ++shift;
  // The single pass spans 2^shift batches with one descriptor: for the
  // strided layout only when their span stays below 1 GiB.  On paged caches
  // (LANES) its lane groups look up their own batches' pages.
  // Against the split passes, which leave most lane groups idle with one
  // or two chunks per row, that pays for rows of a few 16-row blocks (µs,
  // 16-row pages, split / single pass: B=16384 S=48 4/1 D=64 191 / 49, D=128
  // 202 / 91, 1/1 195 / 88; B=8192 S=96 4/1 D=64 145 / 56).  With the
  // lookups made two sub-blocks ahead (one per row on pages under 16 rows,
  // one per sub-block on larger ones): rows of up to eight blocks, four for
  // groups of 8 at D <= 128 (three on 16-row pages) and six for groups of 4
  // at D = 64, beyond which the register single pass is faster (µs, single
  // pass against the matrix-core passes, B sized for 512 MB of K and V;
  // one-row pages: 4/1 D=64 S=24 117 / 446, S=96 111 / 140, S=128 140 /
  // 119; D=128 S=24 110 / 237, S=128 87 / 93; D=256 S=24 110 / 160, S=128
  // 86 / 111; 8/1 D=64 S=24 136 / 453, S=64 150 / 183, S=96 201 / 141;
  // D=128 S=24 134 / 242, S=64 118 / 134, S=96 129 / 108; D=256 S=24 132 /
  // 188, S=128 107 / 119; 16-row pages: 8/1 D=128 S=48 121 / 146, S=64
  // 131 / 114; D=64 S=48 158 / 230, S=64 164 / 154; D=256 S=96 107 / 124;
  // 4/1 D=256 S=128 83 / 108, where the one-batch single pass took 91).
  // Pages under 16 rows at D >= 128 with up to 4 query heads per KV head:
  // longer rows too, ten blocks at D = 128 and any the single pass holds at
  // D = 256 (the per-lane split passes beyond it), where the other choices
  // are the register single pass and the one-batch single pass, half of
  // whose lane groups idle (µs, one-row pages, other / per-lane: D=128
  // B=8192 S=160 1/1 152 / 105, 4/1 155 / 112, but S=256 184 / 248; D=256
  // B=4096 S=384 4/1 329 / 257, 1/1 312 / 244; B=977 S=512 4/1 162 / 117
  // on the split passes).  16-row pages keep the one-batch single pass at
  // D = 256 (B=6144 S=256 4/1 266 / 330).
  // FMHA_DECODE_LANES_BLOCKS=n: n blocks instead (sweeps).
  int lanes_blocks = LAYOUT == fmha_decode::kLayoutPagedLanes
                         ? (G == 8 ? (D <= 128 ? 4 : 8) : D == 64 ? (G == 4 ? 6 : 8) : D == 128 ? 10 : 1 << 20)
                     : G == 8 && D <= 128 ? 3
                     : G == 4 && D == 64  ? 6
                                          : 8;
  if (const char* e = std::getenv("FMHA_DECODE_LANES_BLOCKS")) lanes_blocks = std::atoi(e);
  const bool lanes_onepass = LANES && a.nblk <= lanes_blocks;
  if (!LANES || (D == 256 && LAYOUT != fmha_decode::kLayoutPagedLanes) || lanes_onepass) {
    SplitArgs ao = a;
    ao.sub_shift = LANES && !lanes_onepass ? 0 : shift;
    if (LAYOUT == fmha_decode::kLayoutStrided && shift > 0) {
      const int64_t span = ((int64_t)((1 << shift) - 1) * a.batch_stride + (int64_t)(a.max_rows - 1) * a.row_stride +
                            (int64_t)(fmha_decode::kv_heads_mem(a) - 1) * a.head_stride + D) * 2;
      if (span >= (int64_t(1) << 30)) ao.sub_shift = 0;
    }
    ao.units_per_batch = (a.num_heads_kv + (HPW >> ao.sub_shift) - 1) / (HPW >> ao.sub_shift);
    // onepass_only: waves with no idle lane groups, on rows up to where the
    // single pass measured faster than the matrix-core passes: four 16-row
    // blocks at D = 64, six at D = 128 (with several batches per wave, and
    // with one on packed and strided caches, where the register single pass
    // takes longer rows) and eight otherwise (µs, single pass against the
    // matrix cores: Hq/Hkv 8/1 packed D=128 B=16384 S=64 105 / 121 split,
    // B=10922 S=96 110 / 123, B=8192 S=128 140 / 117; D=64 B=21845 S=96 150
    // / 138; BHSD D=256 B=21845 S=24 137 / 184, D=128 B=43690 S=24 142 /
    // 161, D=64 B=43690 S=48 150 / 176; 64/8 D=128 against the register
    // single pass B=4096 S=64 205 / 211, B=2730 S=96 205 / 202, B=2048 S=128
    // 221 / 199).
    constexpr bool kRegLonger = D == 128 && (LAYOUT == fmha_decode::kLayoutPacked || LAYOUT == fmha_decode::kLayoutStrided);
    const int only_nblk =
        shift > 0 ? (D == 64 ? 4 : D == 128 ? 6 : 8) : (D == 64 ? a.nblk : kRegLonger ? 6 : 8);
    // Groups of at most 4, one batch per wave, with fewer than
    // kOnepassRegBeforeWaves waves of the one-wave pass (too few to fill the
    // CUs): the register single pass below instead where it applies (µs,
    // 32/8 S=256, one-wave / register: B=256, 512 waves, 58.4 / 49.4;
    // B=512, 1024 waves, 90.5 / 93.7).
    constexpr bool kRegRows = kRegSmallGroups<D, G> && (LAYOUT == fmha_decode::kLayoutPacked ||
                                                        LAYOUT == fmha_decode::kLayoutStrided || kPagedLayout<LAYOUT>);
    bool reg_first = false;
    // Groups of 4 at D = 64 on rows of more than four blocks with several
    // batches per wave on packed and strided caches: the register pass too
    // (µs, packed, single pass / register pass: 4/1 B=15625 S=128 116.4 /
    // 87.2, B=12500 S=160 133.8 / 97.6, B=20833 S=96 101.6 / 89.7, 8/2
    // B=15625 S=128 188.1 / 175.0; BHSD 4/1 S=160 148.3 / 90.2; but 4/1
    // B=31250 S=64 92.9 / 110.9).
    constexpr bool kRegMulti64 =
        D == 64 && G == 4 && (LAYOUT == fmha_decode::kLayoutPacked || LAYOUT == fmha_decode::kLayoutStrided);
    if constexpr (kRegRows)
      reg_first = !onepass_only &&
                  ((ao.sub_shift == 0 && onepass_waves(ao) < kOnepassRegBeforeWaves) ||
                   (kRegMulti64 && ao.sub_shift > 0 && a.nblk > 4)) &&
                  onepass_reg_tiles<D, RegLayout<LAYOUT>>(a) > 0;
    if (!reg_first && onepass_fits<D, G>(ao) && (!onepass_only || (ao.sub_shift == shift && a.nblk <= only_nblk))) {
      if constexpr (LAYOUT == fmha_decode::kLayoutPacked || LAYOUT == fmha_decode::kLayoutStrided || LANES)
        if (ao.sub_shift > 0) return launch_onepass_dg<D, G, LAYOUT, true>(ao, stream);
      constexpr int OL = LAYOUT == fmha_decode::kLayoutPagedLanes        ? fmha_decode::kLayoutPaged
                         : LAYOUT == fmha_decode::kLayoutPagedBlockLanes ? fmha_decode::kLayoutPagedBlock
                                                                         : LAYOUT;
      // Pages under 16 rows with G = 8: a descriptor per row for eight
      // query heads' registers spills SGPRs into VGPR lanes, and beyond
      // six 16-row blocks (four at D = 64, eight at D = 256) the split
      // passes run those rows faster (one-row pages, Hq/Hkv 64/8, µs, single
      // pass against split: B=16384 S=24 424 / 455, B=4096 S=64 220 / 259,
      // B=2730 S=96 229 / 247, B=2048 S=128 265 / 239, B=1365 S=192 340 /
      // 243; D=64 B=12288 S=32 183 / 261, B=6144 S=64 202 / 251, B=4096
      // S=96 265 / 251; D=256 48/8 B=1024 S=128 224 / 242, B=512 S=256
      // 314 / 231).  G <= 4 keeps the single pass (32/8: 185 against 221 µs,
      // B=16384 S=24 357 / 388, 16/16 D=256 352 / 368; D=64 111 / 141).
      if (OL != fmha_decode::kLayoutPaged || G < 8 || a.nblk <= (D == 64 ? 4 : D == 128 ? 6 : 8))
        return launch_onepass_dg<D, G, OL, false>(ao, stream);
    }
  }
  if (onepass_only) return kOnepassNotTaken;
  if constexpr ((kRegSmallGroups<D, G> || G == 8) && kPagedLayout<LAYOUT>) {
    // Paged caches: the register single pass, as below for groups of at
    // most 4, and for groups of 8 on the pages under 16 rows that the
    // planner leaves to the VALU passes (half a wave of KV heads or more).
    if (const int tpw = onepass_reg_tiles<D, RegLayout<LAYOUT>>(a))
      return launch_onepass_reg<D, RegLayout<LAYOUT>>(a, tpw, stream);
  }
  if constexpr (G <= 4 && (LAYOUT == fmha_decode::kLayoutPacked || LAYOUT == fmha_decode::kLayoutStrided)) {
    // Rows the one-wave single pass does not hold, of at least 4 blocks,
    // with enough (batch, KV head) units: the matrix-core single pass, its
    // query tile mostly padding; one query head per KV head keeps the
    // two-wave single pass where that applies (µs, packed, D = 128, against
    // the split passes or the two-wave single pass: B=128 S=256 32/8 25.7 /
    // 37.1, B=256 S=512 89.2 / 99.3, B=128 S=1024 88.9 / 101.9, B=64 S=2048
    // 89.2 / 103.7, 16/4 B=128 S=256 17.0 / 25.8, B=256 S=64 12.7 / 17.1,
    // 8/2 B=512 S=128 16.5 / 25.0, 32/8 B=200 S=96 19.2 / 25.7, 32/16 B=64
    // S=256 25.0 / 28.9, B=64 S=2048 170.6 / 177.7, 16/16 B=64 S=2048 170.3
    // / 175.7; G = 1 with the two-wave pass up to 64 blocks: 8/8 B=200
    // S=256 42.3 / 37.9, 16/16 B=100 S=512 76.5 / 69.7, 8/8 B=96 S=64 12.1 /
    // 10.1 (beyond: 16/16 B=64 S=2048 170.3 / 175.7); three blocks:
    // 8/8 B=200 S=40 14.1 / 13.1 split; where the one-wave pass holds the
    // row it stays ahead: 32/8 B=512 S=256 93.7 / 90.5, 16/16 B=128 S=1024
    // 173.1 / 163.8).
    SplitArgs ag = a;
    ag.sub_shift = 0;
    const bool group_fits = onepass_group_fits<D, G, LAYOUT>(ag);
    if (G == 1 && group_fits && a.nblk <= 64) return launch_onepass_group<D, G, LAYOUT>(ag, stream);
    if constexpr (kRegSmallGroups<D, G>)
      if (const int tpw = onepass_reg_tiles<D, LAYOUT>(a)) return launch_onepass_reg<D, LAYOUT>(a, tpw, stream);
    // Too few units for one wave each: two waves per unit.
    if (group_fits) return launch_onepass_group<D, G, LAYOUT>(ag, stream);
  }
  // P.V sub-block rows (register budget: pages under 16 rows address every
  // row on its own, a descriptor or a 64-bit address per row; 16 rows there
  // leave one wave per SIMD).
  constexpr int NR = G >= 8 || LAYOUT == fmha_decode::kLayoutPaged || LAYOUT == fmha_decode::kLayoutPagedLanes ? 8 : 16;
  SplitArgs as = a;
  as.sub_shift = shift;
  as.units_per_batch = (a.num_heads_kv + (HPW >> shift) - 1) / (HPW >> shift);
  const int64_t upb = as.units_per_batch;
  as.stat_pass = a.nblk > kPvStatBlocks;
  const int64_t score_waves = (int64_t)a.batch * ((a.nblk + (1 << shift) - 1) >> shift) * upb;
  const int64_t nwc = (a.nchunks + (1 << shift) - 1) >> shift;  // P.V waves per unit
  const int64_t pv_waves = (int64_t)a.batch * nwc * upb;
  if (score_waves > INT32_MAX || pv_waves > INT32_MAX) return hipErrorInvalidValue;
  // The combine grid has one workgroup per (batch, query head, 32 dims).
  if ((uint64_t)a.batch * (uint64_t)a.num_heads_q * (D / 32) > UINT32_MAX) return hipErrorInvalidValue;
  const int passes = 2 + as.stat_pass + (a.nchunks > 1);
  plan_note("split(D=%d G=%d layout=%s sub_units=%d blocks=%d chunk_rows=%d chunks=%d passes=%d)", D, G,
            layout_name(LAYOUT), 1 << shift, a.nblk, a.chunk_rows, a.nchunks, passes);
  {
    constexpr auto kernel = fmha_decode::splitkv_scores_kernel<D, G, LAYOUT>;
    hipLaunchKernelGGL(kernel, dim3((uint32_t)score_waves), dim3(kBlockThreads),
                       lds_reserve_kernel<kernel>(kSplitScoresWavesPerCU), stream, as);
  }
  if (as.stat_pass) launch_split_stats(as, stream);
  if (a.nchunks == 1) {
    // One chunk per batch: the P.V wave writes O itself, one chunk per wave.
    constexpr auto kernel = fmha_decode::splitkv_pv_kernel<D, G, NR, true, LAYOUT>;
    SplitArgs ad = a;
    ad.stat_pass = as.stat_pass;
    const uint32_t waves = (uint32_t)a.batch * (uint32_t)a.units_per_batch;
    hipLaunchKernelGGL(kernel, dim3(waves), dim3(kBlockThreads), lds_reserve_kernel<kernel>(kSplitPvWavesPerCU),
                       stream, ad);
    return hipGetLastError();
  }
  {
    constexpr auto kernel = fmha_decode::splitkv_pv_kernel<D, G, NR, false, LAYOUT>;
    hipLaunchKernelGGL(kernel, dim3((uint32_t)pv_waves), dim3(kBlockThreads),
                       lds_reserve_kernel<kernel>(kSplitPvWavesPerCU), stream, as);
  }
  launch_split_combine(a, D, stream);
  return hipGetLastError();
}

template <int D, int LAYOUT>
hipError_t launch_split_d(const SplitArgs& a, int g, hipStream_t stream, bool onepass_only) {
  switch (g) {
    case 1: return launch_split_dg<D, 1, LAYOUT>(a, stream, onepass_only);
    case 2: return launch_split_dg<D, 2, LAYOUT>(a, stream, onepass_only);
    case 4: return launch_split_dg<D, 4, LAYOUT>(a, stream, onepass_only);
    default: return launch_split_dg<D, 8, LAYOUT>(a, stream, onepass_only);
  }
}

template <int LAYOUT>
hipError_t launch_split_layout(const SplitArgs& a, int d, int g, hipStream_t stream, bool onepass_only = false) {
  switch (d) {
    case 64: return launch_split_d<64, LAYOUT>(a, g, stream, onepass_only);
    case 128: return launch_split_d<128, LAYOUT>(a, g, stream, onepass_only);
    default: return launch_split_d<256, LAYOUT>(a, g, stream, onepass_only);
  }
}

// Split-KV on the matrix cores (fmha_decode_splitkv_group.hpp): a's KV heads
// are the cache's (kv_groups = 1) and G = num_heads_q / num_heads_kv any
// size.  Scores, the statistics pass for rows of more than kPvStatBlocks
// blocks, P.V (O directly with one chunk per row), combine.
// P.V waves take TW tiles of 16 query heads, their accumulators TW * D/16 *
// 4 VGPRs: 2 tiles (G <= 32 in one wave) at D = 64 and 128, one at D = 256.
template <int D, int LAYOUT>
hipError_t launch_split_group_d(const SplitArgs& a, hipStream_t stream) {
  if constexpr (LAYOUT == fmha_decode::kLayoutPacked || LAYOUT == fmha_decode::kLayoutStrided ||
                LAYOUT == fmha_decode::kLayoutPagedBlock || LAYOUT == fmha_decode::kLayoutPaged)
    if (const int tpw = onepass_reg_tiles<D, LAYOUT>(a)) return launch_onepass_reg<D, LAYOUT>(a, tpw, stream);
  if constexpr (LAYOUT == fmha_decode::kLayoutPacked || LAYOUT == fmha_decode::kLayoutStrided ||
                LAYOUT == fmha_decode::kLayoutPagedBlock)
    if (const int nw = onepass_mfma_waves<D, LAYOUT>(a)) return launch_onepass_mfma<D, LAYOUT>(a, nw, stream);
  constexpr int HPW = kWaveSize / (D / 8);
  constexpr int TW = D == 256 ? 1 : 2;
  const int64_t g = a.num_heads_q / a.num_heads_kv;
  const int64_t tiles = (g + 15) / 16;
  const int64_t tc = (tiles + TW - 1) / TW;
  const int64_t score_waves = (int64_t)a.batch * ((a.nblk + HPW - 1) / HPW) * a.num_heads_kv;
  const int64_t units = (int64_t)a.batch * a.nchunks * a.num_heads_kv;
  const int64_t pv_waves = (units + 7) / 8 * 8 * tc;
  if (score_waves > INT32_MAX || pv_waves > INT32_MAX ||
      (uint64_t)a.batch * (uint64_t)a.num_heads_q * (D / 32) > UINT32_MAX)
    return hipErrorInvalidValue;
  SplitArgs am = a;
  am.stat_pass = a.nblk > kPvStatBlocks;
  plan_note("split_matrix_core(D=%d G=%d layout=%s blocks=%d chunk_rows=%d chunks=%d passes=%d)", D, (int)g,
            layout_name(LAYOUT), a.nblk, a.chunk_rows, a.nchunks, 2 + am.stat_pass + (a.nchunks > 1));
  {
    constexpr auto kernel = fmha_decode::splitkv_scores_group_kernel<D, LAYOUT>;
    hipLaunchKernelGGL(kernel, dim3((uint32_t)score_waves), dim3(kBlockThreads),
                       lds_reserve_kernel<kernel>(kSplitScoresWavesPerCU), stream, am);
  }
  if (am.stat_pass) launch_split_stats(am, stream);
  if (a.nchunks == 1) {
    constexpr auto kernel = fmha_decode::splitkv_pv_group_kernel<D, TW, true, LAYOUT>;
    hipLaunchKernelGGL(kernel, dim3((uint32_t)pv_waves), dim3(kBlockThreads),
                       lds_reserve_kernel<kernel>(kSplitPvWavesPerCU), stream, am);
    return hipGetLastError();
  }
  {
    constexpr auto kernel = fmha_decode::splitkv_pv_group_kernel<D, TW, false, LAYOUT>;
    hipLaunchKernelGGL(kernel, dim3((uint32_t)pv_waves), dim3(kBlockThreads),
                       lds_reserve_kernel<kernel>(kSplitPvWavesPerCU), stream, am);
  }
  launch_split_combine(a, D, stream);
  return hipGetLastError();
}

template <int LAYOUT>
hipError_t launch_split_group_layout(const SplitArgs& a, int d, hipStream_t stream) {
  switch (d) {
    case 64: return launch_split_group_d<64, LAYOUT>(a, stream);
    case 128: return launch_split_group_d<128, LAYOUT>(a, stream);
    default: return launch_split_group_d<256, LAYOUT>(a, stream);
  }
}

// Explicitly instantiated in fmha_decode_inst.hip (one part each).
#ifndef FMHA_DECODE_INSTANTIATING
extern template hipError_t launch_group<64, kLayoutPacked, false>(const DecodeArgs&, int, int, int, hipStream_t);
extern template hipError_t launch_group<64, kLayoutPacked, true>(const DecodeArgs&, int, int, int, hipStream_t);
extern template hipError_t launch_group<64, kLayoutStrided, false>(const DecodeArgs&, int, int, int, hipStream_t);
extern template hipError_t launch_group<64, kLayoutPaged, false>(const DecodeArgs&, int, int, int, hipStream_t);
extern template hipError_t launch_group<128, kLayoutPacked, false>(const DecodeArgs&, int, int, int, hipStream_t);
extern template hipError_t launch_group<128, kLayoutPacked, true>(const DecodeArgs&, int, int, int, hipStream_t);
extern template hipError_t launch_group<128, kLayoutStrided, false>(const DecodeArgs&, int, int, int, hipStream_t);
extern template hipError_t launch_group<128, kLayoutPaged, false>(const DecodeArgs&, int, int, int, hipStream_t);
extern template hipError_t launch_group<256, kLayoutPacked, false>(const DecodeArgs&, int, int, int, hipStream_t);
extern template hipError_t launch_group<256, kLayoutPacked, true>(const DecodeArgs&, int, int, int, hipStream_t);
extern template hipError_t launch_group<256, kLayoutStrided, false>(const DecodeArgs&, int, int, int, hipStream_t);
extern template hipError_t launch_group<256, kLayoutPaged, false>(const DecodeArgs&, int, int, int, hipStream_t);
extern template hipError_t launch_exact<64, 1>(const DecodeArgs&, bool, int, int, hipStream_t);
extern template hipError_t launch_exact<64, 2>(const DecodeArgs&, bool, int, int, hipStream_t);
extern template hipError_t launch_exact<64, 4>(const DecodeArgs&, bool, int, int, hipStream_t);
extern template hipError_t launch_exact<64, 8>(const DecodeArgs&, bool, int, int, hipStream_t);
extern template hipError_t launch_exact<128, 1>(const DecodeArgs&, bool, int, int, hipStream_t);
extern template hipError_t launch_exact<128, 2>(const DecodeArgs&, bool, int, int, hipStream_t);
extern template hipError_t launch_exact<128, 4>(const DecodeArgs&, bool, int, int, hipStream_t);
extern template hipError_t launch_exact<128, 8>(const DecodeArgs&, bool, int, int, hipStream_t);
extern template hipError_t launch_exact<256, 1>(const DecodeArgs&, bool, int, int, hipStream_t);
extern template hipError_t launch_exact<256, 2>(const DecodeArgs&, bool, int, int, hipStream_t);
extern template hipError_t launch_exact<256, 4>(const DecodeArgs&, bool, int, int, hipStream_t);
extern template hipError_t launch_exact<256, 8>(const DecodeArgs&, bool, int, int, hipStream_t);
extern template hipError_t launch_multi<kLayoutPacked, false>(const DecodeArgs&, int, int, int, hipStream_t);
extern template hipError_t launch_multi<kLayoutPacked, true>(const DecodeArgs&, int, int, int, hipStream_t);
extern template hipError_t launch_multi<kLayoutStrided, false>(const DecodeArgs&, int, int, int, hipStream_t);
extern template hipError_t launch_multi<kLayoutPaged, false>(const DecodeArgs&, int, int, int, hipStream_t);
extern template hipError_t launch_mfma_d<64, kLayoutPacked>(const GroupArgs&, int, int, hipStream_t);
extern template hipError_t launch_mfma_d<64, kLayoutStrided>(const GroupArgs&, int, int, hipStream_t);
extern template hipError_t launch_mfma_d<128, kLayoutPacked>(const GroupArgs&, int, int, hipStream_t);
extern template hipError_t launch_mfma_d<128, kLayoutStrided>(const GroupArgs&, int, int, hipStream_t);
extern template hipError_t launch_mfma_d<256, kLayoutPacked>(const GroupArgs&, int, int, hipStream_t);
extern template hipError_t launch_mfma_d<256, kLayoutStrided>(const GroupArgs&, int, int, hipStream_t);
extern template hipError_t launch_split_d<64, kLayoutPacked>(const SplitArgs&, int, hipStream_t, bool);
extern template hipError_t launch_split_d<64, kLayoutStrided>(const SplitArgs&, int, hipStream_t, bool);
extern template hipError_t launch_split_d<64, kLayoutPaged>(const SplitArgs&, int, hipStream_t, bool);
extern template hipError_t launch_split_d<64, kLayoutPagedLanes>(const SplitArgs&, int, hipStream_t, bool);
extern template hipError_t launch_split_d<64, kLayoutPagedBlock>(const SplitArgs&, int, hipStream_t, bool);
extern template hipError_t launch_split_d<64, kLayoutPagedBlockLanes>(const SplitArgs&, int, hipStream_t, bool);
extern template hipError_t launch_split_d<128, kLayoutPacked>(const SplitArgs&, int, hipStream_t, bool);
extern template hipError_t launch_split_d<128, kLayoutStrided>(const SplitArgs&, int, hipStream_t, bool);
extern template hipError_t launch_split_d<128, kLayoutPaged>(const SplitArgs&, int, hipStream_t, bool);
extern template hipError_t launch_split_d<128, kLayoutPagedLanes>(const SplitArgs&, int, hipStream_t, bool);
extern template hipError_t launch_split_d<128, kLayoutPagedBlock>(const SplitArgs&, int, hipStream_t, bool);
extern template hipError_t launch_split_d<128, kLayoutPagedBlockLanes>(const SplitArgs&, int, hipStream_t, bool);
extern template hipError_t launch_split_d<256, kLayoutPacked>(const SplitArgs&, int, hipStream_t, bool);
extern template hipError_t launch_split_d<256, kLayoutStrided>(const SplitArgs&, int, hipStream_t, bool);
extern template hipError_t launch_split_d<256, kLayoutPaged>(const SplitArgs&, int, hipStream_t, bool);
extern template hipError_t launch_split_d<256, kLayoutPagedLanes>(const SplitArgs&, int, hipStream_t, bool);
extern template hipError_t launch_split_d<256, kLayoutPagedBlock>(const SplitArgs&, int, hipStream_t, bool);
extern template hipError_t launch_split_d<256, kLayoutPagedBlockLanes>(const SplitArgs&, int, hipStream_t, bool);
extern template hipError_t launch_split_group_d<64, kLayoutPacked>(const SplitArgs&, hipStream_t);
extern template hipError_t launch_split_group_d<64, kLayoutStrided>(const SplitArgs&, hipStream_t);
extern template hipError_t launch_split_group_d<64, kLayoutPaged>(const SplitArgs&, hipStream_t);
extern template hipError_t launch_split_group_d<64, kLayoutPagedBlock>(const SplitArgs&, hipStream_t);
extern template hipError_t launch_split_group_d<128, kLayoutPacked>(const SplitArgs&, hipStream_t);
extern template hipError_t launch_split_group_d<128, kLayoutStrided>(const SplitArgs&, hipStream_t);
extern template hipError_t launch_split_group_d<128, kLayoutPaged>(const SplitArgs&, hipStream_t);
extern template hipError_t launch_split_group_d<128, kLayoutPagedBlock>(const SplitArgs&, hipStream_t);
extern template hipError_t launch_split_group_d<256, kLayoutPacked>(const SplitArgs&, hipStream_t);
extern template hipError_t launch_split_group_d<256, kLayoutStrided>(const SplitArgs&, hipStream_t);
extern template hipError_t launch_split_group_d<256, kLayoutPaged>(const SplitArgs&, hipStream_t);
extern template hipError_t launch_split_group_d<256, kLayoutPagedBlock>(const SplitArgs&, hipStream_t);
#endif

}  // namespace host
}  // namespace fmha_decode
