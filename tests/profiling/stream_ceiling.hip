// stream_ceiling -- measurement aid: the decode kernel's memory traffic
// without its arithmetic.
//
// For a uniform-length configuration (B, Hq, Hkv, S, D) this launches the same
// grid as fmha_decode_fwd_kernel (one wave per batch and group of 64/(D/8) KV
// heads), reserves the same LDS per workgroup (the library's per-CU wave
// cap), and issues the same buffer loads (Q with the default policy, K and V
// non-temporal, rows past S out of range) and, unless --no-write, the same
// non-temporal device-scope O stores.  The stored value is the XOR of the
// loaded words, so every load is consumed.  The time it takes is the ceiling
// the memory system allows for exactly this access pattern; the decode
// kernel's time over it is the share its arithmetic and reductions cost.
//
//   stream_ceiling B Hq Hkv S D [--sets N] [--iters N] [--no-write] [--waves W]
//   (S in {1, 4, 5, 16}; D = 128 with G in {1, 2, 5, 8, 32}, or D = 256 with G = 1)
//
// Prints one JSON line: median µs per call over --iters calls (HIP events per
// call, after 5 warm-up calls), algorithmic TB/s with the same byte count as
// the decode kernel (Q + K + V + O), the waves-per-CU cap used.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <vector>

#include "fmha_decode_caps.hpp"
#include "fmha_decode_kernel.hpp"

using namespace fmha_decode;

#define CHECK(x)                                                                   \
  do {                                                                             \
    hipError_t e_ = (x);                                                           \
    if (e_ != hipSuccess) {                                                        \
      std::fprintf(stderr, "%s:%d %s\n", __FILE__, __LINE__, hipGetErrorString(e_)); \
      std::exit(1);                                                                \
    }                                                                              \
  } while (0)

template <int D, int G, int SB, bool WRITE>
__global__ __launch_bounds__(64) void stream_kernel(const uint16_t* q, const uint16_t* k, const uint16_t* v,
                                                    uint16_t* o, int hq, int hkv, int S, uint32_t units,
                                                    uint32_t upb) {
  constexpr int LPH = D / 8;
  constexpr int HPW = 64 / LPH;
  const int lane = threadIdx.x;
  const uint32_t unit = blockIdx.x;
  if (unit >= units) return;
  const uint32_t b = unit / upb;
  const uint32_t hg = unit - b * upb;
  const int hk = (int)hg * HPW + lane / LPH;
  const int r = lane % LPH;
  const bool head_ok = hk < hkv;
  const uint32_t q_bytes = (uint32_t)hq * D * 2;
  const __amdgpu_buffer_rsrc_t q_rsrc = make_rsrc(q + (uint64_t)b * hq * D, q_bytes);
  const __amdgpu_buffer_rsrc_t o_rsrc = make_rsrc(o + (uint64_t)b * hq * D, q_bytes);
  const uint32_t row_bytes = (uint32_t)hkv * D * 2;
  const uint64_t elem0 = (uint64_t)b * S * hkv * D;
  const __amdgpu_buffer_rsrc_t k_rsrc = make_rsrc(k + elem0, (uint32_t)S * row_bytes);
  const __amdgpu_buffer_rsrc_t v_rsrc = make_rsrc(v + elem0, (uint32_t)S * row_bytes);
  const uint32_t kv_off = head_ok ? (uint32_t)hk * D * 2 + (uint32_t)r * 16u : kLaneOutOfRange;
  const uint32_t qo_off = head_ok ? (uint32_t)(hk * G * D + r * 8) * 2u : kLaneOutOfRange;
  u32x4 qv[G], kr[SB], vr[SB];
#pragma unroll
  for (int g = 0; g < G; ++g) qv[g] = buffer_load16<kPolicyDefault>(q_rsrc, qo_off + g * D * 2);
#pragma unroll
  for (int j = 0; j < SB; ++j) kr[j] = buffer_load16<kPolicyStream>(k_rsrc, kv_off + j * row_bytes);
#pragma unroll
  for (int j = 0; j < SB; ++j) vr[j] = buffer_load16<kPolicyStream>(v_rsrc, kv_off + j * row_bytes);
  __builtin_amdgcn_sched_barrier(0);
  u32x4 x = kr[0] ^ vr[0];
#pragma unroll
  for (int j = 1; j < SB; ++j) x ^= kr[j] ^ vr[j];
#pragma unroll
  for (int g = 0; g < G; ++g) {
    const u32x4 y = x ^ qv[g];
    if (WRITE) {
      buffer_store16(o_rsrc, qo_off + g * D * 2, y);
    } else if (y[0] == 0x12345678u && y[1] == 0x9abcdef0u) {
      // Practically never taken; keeps the loads live without a store.
      buffer_store16(o_rsrc, qo_off + g * D * 2, y);
    }
  }
}

// The library's cap for known lengths, one batch per wave: its in-flight
// budget model (fmha_decode_caps.hpp) for the kernel of the call's group
// (1, 2, 4 for G = 3-4, 8 for G = 5-8 and the VALU replay of larger
// groups); 32: no cap.  g: the real group size.
int waves_for(int rows, int g, int d) {
  const int gk = g <= 2 ? g : (g <= 4 ? 4 : 8);
  using fmha_decode::host::budget_waves;
  using fmha_decode::host::tree_order_budget;
  return budget_waves(tree_order_budget(gk, d, false, false), 16 * rows, g);
}

size_t lds_reserve(int waves, size_t static_lds) {
  int dev = 0, lds = 0;
  CHECK(hipGetDevice(&dev));
  CHECK(hipDeviceGetAttribute(&lds, hipDeviceAttributeMaxSharedMemoryPerMultiprocessor, dev));
  if (waves >= 32 || lds <= 0) return 0;
  const size_t hi = (size_t)lds / waves, lo = (size_t)lds / (waves + 1), per = (hi + lo) / 2;
  return per > static_lds ? per - static_lds : 0;
}

template <int D, int G, int SB, bool WRITE>
void run(int B, int hq, int hkv, int S, int sets, int iters, int waves) {
  constexpr int HPW = 64 / (D / 8);
  const uint32_t upb = (uint32_t)((hkv + HPW - 1) / HPW);
  const uint32_t units = upb * (uint32_t)B;
  const size_t q_elems = (size_t)B * hq * D, kv_elems = (size_t)B * S * hkv * D;
  std::vector<uint16_t*> bufs;
  for (int s = 0; s < sets; ++s) {
    uint16_t *q, *k, *v, *o;
    CHECK(hipMalloc(&q, q_elems * 2));
    CHECK(hipMalloc(&k, kv_elems * 2 + 16));
    CHECK(hipMalloc(&v, kv_elems * 2 + 16));
    CHECK(hipMalloc(&o, q_elems * 2));
    CHECK(hipMemset(q, 0x3c, q_elems * 2));
    CHECK(hipMemset(k, 0x3c, kv_elems * 2));
    CHECK(hipMemset(v, 0x3c, kv_elems * 2));
    bufs.insert(bufs.end(), {q, k, v, o});
  }
  const int w = waves > 0 ? waves : waves_for(S, hq / hkv, D);
  const auto kern = stream_kernel<D, G, SB, WRITE>;
  const size_t dyn = lds_reserve(w, 0);
  hipEvent_t e0, e1;
  CHECK(hipEventCreate(&e0));
  CHECK(hipEventCreate(&e1));
  std::vector<float> t;
  for (int i = 0; i < iters + 5; ++i) {
    uint16_t** p = &bufs[4 * (i % sets)];
    CHECK(hipEventRecord(e0, 0));
    hipLaunchKernelGGL(kern, dim3(units), dim3(64), dyn, 0, p[0], p[1], p[2], p[3], hq, hkv, S, units, upb);
    CHECK(hipGetLastError());
    CHECK(hipEventRecord(e1, 0));
    CHECK(hipEventSynchronize(e1));
    float ms = 0;
    CHECK(hipEventElapsedTime(&ms, e0, e1));
    if (i >= 5) t.push_back(ms);
  }
  std::sort(t.begin(), t.end());
  const double med_us = t[t.size() / 2] * 1e3;
  const double bytes = 2.0 * q_elems * 2 + 2.0 * kv_elems * 2;
  std::printf(
      "{\"B\": %d, \"Hq\": %d, \"Hkv\": %d, \"S\": %d, \"D\": %d, \"writes\": %s, \"input_sets\": %d, "
      "\"waves_per_cu\": %d, \"us_per_call_median\": %.1f, \"tb_s\": %.3f}\n",
      B, hq, hkv, S, D, WRITE ? "true" : "false", sets, w, med_us, bytes / med_us / 1e6);
  std::fflush(stdout);
  for (uint16_t* p : bufs) CHECK(hipFree(p));
  CHECK(hipEventDestroy(e0));
  CHECK(hipEventDestroy(e1));
}

template <int D, int G, bool WRITE>
bool by_len(int B, int hq, int hkv, int S, int sets, int iters, int waves) {
  switch (S) {
    case 1: run<D, G, 1, WRITE>(B, hq, hkv, S, sets, iters, waves); return true;
    case 4: run<D, G, 4, WRITE>(B, hq, hkv, S, sets, iters, waves); return true;
    case 5: run<D, G, 5, WRITE>(B, hq, hkv, S, sets, iters, waves); return true;
    case 16: run<D, G, 16, WRITE>(B, hq, hkv, S, sets, iters, waves); return true;
    default: return false;
  }
}

template <bool WRITE>
bool dispatch(int B, int hq, int hkv, int S, int D, int sets, int iters, int waves) {
  const int g = hq / hkv;
  if (D == 128 && g == 1) return by_len<128, 1, WRITE>(B, hq, hkv, S, sets, iters, waves);
  if (D == 128 && g == 2) return by_len<128, 2, WRITE>(B, hq, hkv, S, sets, iters, waves);
  if (D == 128 && g == 3) return by_len<128, 3, WRITE>(B, hq, hkv, S, sets, iters, waves);
  if (D == 128 && g == 4) return by_len<128, 4, WRITE>(B, hq, hkv, S, sets, iters, waves);
  if (D == 128 && g == 5) return by_len<128, 5, WRITE>(B, hq, hkv, S, sets, iters, waves);
  if (D == 128 && g == 8) return by_len<128, 8, WRITE>(B, hq, hkv, S, sets, iters, waves);
  if (D == 128 && g == 32) return by_len<128, 32, WRITE>(B, hq, hkv, S, sets, iters, waves);
  if (D == 256 && g == 1) return by_len<256, 1, WRITE>(B, hq, hkv, S, sets, iters, waves);
  return false;
}

int main(int argc, char** argv) {
  if (argc < 6) {
    std::fprintf(stderr, "usage: %s B Hq Hkv S D [--sets N] [--iters N] [--no-write] [--waves W]\n", argv[0]);
    return 2;
  }
  const int B = std::atoi(argv[1]), hq = std::atoi(argv[2]), hkv = std::atoi(argv[3]);
  const int S = std::atoi(argv[4]), D = std::atoi(argv[5]);
  int sets = 1, iters = 50, waves = 0;
  bool write = true;
  for (int i = 6; i < argc; ++i) {
    if (!std::strcmp(argv[i], "--sets") && i + 1 < argc) sets = std::atoi(argv[++i]);
    else if (!std::strcmp(argv[i], "--iters") && i + 1 < argc) iters = std::atoi(argv[++i]);
    else if (!std::strcmp(argv[i], "--waves") && i + 1 < argc) waves = std::atoi(argv[++i]);
    else if (!std::strcmp(argv[i], "--no-write")) write = false;
    else { std::fprintf(stderr, "unknown argument %s\n", argv[i]); return 2; }
  }
  if (B <= 0 || hq <= 0 || hkv <= 0 || hq % hkv || sets < 1 || iters < 1) {
    std::fprintf(stderr, "bad sizes\n");
    return 2;
  }
  const bool ok = write ? dispatch<true>(B, hq, hkv, S, D, sets, iters, waves)
                        : dispatch<false>(B, hq, hkv, S, D, sets, iters, waves);
  if (!ok) {
    std::fprintf(stderr, "shape not built into this aid (S in {1,4,5,16}; D=128 with G in {1,2,3,4,5,8,32}, or D=256 with G=1)\n");
    return 2;
  }
  return 0;
}
