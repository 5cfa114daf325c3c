// ref_shim.cpp -- builds the reference's own source, unmodified and in place
// (/root/reference/fmha_host.cpp, which includes the reference kernel
// headers), into oracle/_ref/libfmha_ref.so and exposes a C ABI over it.
//
// TEST INFRASTRUCTURE ONLY: used by tests/ (oracle pinning, GPU comparison
// with the reference kernels) and bench.py's cpu_baseline leg.  The reference
// source never enters this repository; the recipe is oracle/Makefile and the
// build needs /root/reference, so it only happens where the reference is
// mounted.  The built library travels with the tree like any other .so.
//
// The reference's main() is renamed so the translation unit links as a
// library; nothing else in the reference text is touched.
#define main fmha_reference_main
#include "fmha_host.cpp"
#undef main
// The fourth variant, which fmha_host.cpp does not include.
#include "fmha_mfma_16x16x16_v3_kernel.hpp"

#include <cstdint>

extern "C" {

// fmha_host.cpp:58-72: FMHAConfig::generate_seqlens_kv (mt19937(42), Poisson(4)
// rejected outside [2, max_seqlen_kv]).
void ref_generate_seqlens(int batch, int max_seqlen_kv, int32_t* out) {
  FMHAConfig cfg(batch, 1, 1, 1, max_seqlen_kv, 128, 128);
  std::vector<int> s = cfg.generate_seqlens_kv();
  for (int i = 0; i < batch; i++) out[i] = s[i];
}

// fmha_host.cpp:158-284: the reference CPU loop.  Fills ref_o (fp16 bits,
// [batch, Hq, D]) and compares it with gpu_o using the reference rule;
// returns 1 if do_validation reported success.  The reference indexes K/V
// with the query head, so only Hq == Hkv is meaningful.
int ref_do_validation(int batch, int hq, int hkv, int d, const int32_t* cu, const uint16_t* q, const uint16_t* k,
                      const uint16_t* v, uint16_t* ref_o, const uint16_t* gpu_o) {
  int max_s = 0;
  std::vector<int> seqlens(batch), cus(batch + 1);
  for (int b = 0; b <= batch; b++) cus[b] = cu[b];
  for (int b = 0; b < batch; b++) {
    seqlens[b] = cu[b + 1] - cu[b];
    if (seqlens[b] > max_s) max_s = seqlens[b];
  }
  FMHAConfig cfg(batch, hq, hkv, 1, max_s, d, d);
  bool ok = do_validation(cfg, seqlens, cus, (bhalf_t*)q, (bhalf_t*)k, (bhalf_t*)v, (half_t*)ref_o,
                          (half_t*)gpu_o);
  return ok ? 1 : 0;
}

// fmha_mfma_4x4x4_kernel.hpp:370-389 with the grid and block that
// fmha_host.cpp:358-359 computes.  Valid only for Hq == Hkv, Hq % 16 == 0,
// D in {128, 256} and every length in [1, 16].
int ref_launch_mfma_4x4x4(void* stream, const void* Q, const void* K, const void* V, void* O, const int32_t* cu,
                          int batch, int hq, int hkv, int d, float scale) {
  dim3 grid(1, (hq + 15) / 16, batch);
  dim3 block(256, 1, 1);
  launch_fmha_mfma_4x4x4(grid, block, (hipStream_t)stream, (const bhalf_t*)Q, (const bhalf_t*)K, (const bhalf_t*)V,
                         (half_t*)O, cu, batch, hq, hkv, 1, d, d, scale);
  return (int)hipGetLastError();
}

// fmha_vectorized_fma (fmha_vectorized_fma_kernel.hpp:69-331) with the grid
// its header documents, (1, ceil(Hq/16), B) x 256.  Same validity limits.
int ref_launch_vectorized_fma(void* stream, const void* Q, const void* K, const void* V, void* O,
                              const int32_t* cu, int batch, int hq, int hkv, int d, float scale) {
  dim3 grid(1, (hq + 15) / 16, batch);
  dim3 block(256, 1, 1);
  hipLaunchKernelGGL(fmha_vectorized_fma, grid, block, 0, (hipStream_t)stream, (const bhalf_t*)Q,
                     (const bhalf_t*)K, (const bhalf_t*)V, (half_t*)O, cu, batch, hq, hkv, 1, d, d, scale);
  return (int)hipGetLastError();
}

// fmha_mfma (fmha_mfma_kernel.hpp:51-239): one query head per 256-thread
// workgroup, grid (1, Hq, B) as README.md:173-179 documents.  Every global
// access stays inside the batch's rows [cu[b], cu[b+1]) and the head's D
// elements: K and V rows r < seqlen_kv only (:119-122, :194-197), Q by D/8
// threads (:107-110), O dims < D (:236).  Valid for Hq == Hkv (K/V indexed with the
// query head), D in {64, 128, 256}, every length in [1, 16] (the LDS tile is
// 16 rows).
int ref_launch_mfma(void* stream, const void* Q, const void* K, const void* V, void* O, const int32_t* cu, int batch,
                    int hq, int hkv, int d, float scale) {
  dim3 grid(1, hq, batch);
  dim3 block(256, 1, 1);
  hipLaunchKernelGGL(fmha_mfma, grid, block, 0, (hipStream_t)stream, (const bhalf_t*)Q, (const bhalf_t*)K,
                     (const bhalf_t*)V, (half_t*)O, cu, batch, hq, hkv, 1, d, d, scale);
  return (int)hipGetLastError();
}

// fmha_mfma_v3 (fmha_mfma_16x16x16_v3_kernel.hpp:51-291), grid (1, Hq, B)
// from its header (:47).  K rows r < seqlen_kv (:123-126); V rows clamped to
// [0, seqlen_kv - 1] (:213-218), in range for lengths >= 1.  Same validity
// limits as fmha_mfma.
int ref_launch_mfma_v3(void* stream, const void* Q, const void* K, const void* V, void* O, const int32_t* cu,
                       int batch, int hq, int hkv, int d, float scale) {
  dim3 grid(1, hq, batch);
  dim3 block(256, 1, 1);
  hipLaunchKernelGGL(fmha_mfma_v3, grid, block, 0, (hipStream_t)stream, (const bhalf_t*)Q, (const bhalf_t*)K,
                     (const bhalf_t*)V, (half_t*)O, cu, batch, hq, hkv, 1, d, d, scale);
  return (int)hipGetLastError();
}

}  // extern "C"
