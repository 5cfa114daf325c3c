// fmha_decode_api.hip -- C ABI of libfmha_decode.so: argument checks, launch
// shape and kernel selection for the gfx950 decode-attention kernel.
//
// Replaces the reference's launch helper launch_fmha_mfma_4x4x4
// (fmha_mfma_4x4x4_kernel.hpp:370-389), which takes a caller-computed grid,
// runs the D=256 kernel for any head_dim other than 128 and reports nothing;
// here every argument is checked before the GPU is touched and the library
// computes its own grid.
#include <hip/hip_runtime.h>

#include <atomic>
#include <cmath>
#include <cstdarg>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <mutex>

#include "fmha_decode.h"
#include "fmha_decode_launch.hpp"

namespace fmha_decode {
namespace host {
namespace {
// The launches of this thread's most recent entry-point call.
thread_local char g_plan[1024] = "";
}  // namespace

void plan_note(const char* fmt, ...) {
  size_t n = std::strlen(g_plan);
  if (n > 0 && n + 2 < sizeof(g_plan)) {
    std::memcpy(g_plan + n, "; ", 3);
    n += 2;
  }
  if (n + 1 >= sizeof(g_plan)) return;
  va_list ap;
  va_start(ap, fmt);
  std::vsnprintf(g_plan + n, sizeof(g_plan) - n, fmt, ap);
  va_end(ap);
}
}  // namespace host
}  // namespace fmha_decode

namespace {

// Launchers and their instantiations: fmha_decode_launch.hpp,
// fmha_decode_inst.hip.
using namespace fmha_decode::host;

thread_local char g_detail[256] = "";

// Start of an entry-point call: no rejection detail, no launch yet.
void begin_call() {
  g_detail[0] = '\0';
  fmha_decode::host::g_plan[0] = '\0';
}

int reject(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  std::vsnprintf(g_detail, sizeof(g_detail), fmt, ap);
  va_end(ap);
  return code;
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// Batches with fewer KV heads than a wave holds: the wave serves R = HPW /
// Hkv batches (fmha_decode_multi_kernel).  Returns log2 R (0: not used).
int multi_shift(int hkv, int dq) {
  const int hpw = kWaveSize / (dq / 8);
  int shift = 0;
  while ((hkv << (shift + 1)) <= hpw && hpw % (hkv << (shift + 1)) == 0) ++shift;
  return shift;
}

// G values the VALU kernel is instantiated for.
bool valu_group(int g) { return g == 1 || g == 2 || g == 4 || g == 8; }

// The VALU instantiation a call with G query heads per KV head runs: G for
// 1, 2, 4, 8; 4 for 3 and 8 for 5-7 (the extra query heads load and store
// nothing, DecodeArgs::group); 0 above 8.
int valu_kernel_group(int g) {
  if (valu_group(g)) return g;
  if (g == 3) return 4;
  if (g >= 5 && g <= 7) return 8;
  return 0;
}

// Waves per CU of the tree-order kernels: rows16 = 16 x the K/V rows per
// batch (a mean), g_real the call's query heads per KV head on the g-head
// kernel.
int waves_per_cu_for(int rows16, int g, int g_real, int dq, bool device_lengths, bool bucket_per_wave) {
  return budget_waves(tree_order_budget(g, dq, device_lengths, bucket_per_wave), rows16, g_real);
}

// Pages under 16 rows and pages of 16 with one batch per wave, 1 or 2 query
// heads: 216 KiB flat, the page lookups coming before any K/V request
// (B=30720 D=128, µs for 4/5/6/8/12/16 waves: 16-row pages Hq/Hkv 16/16
// S=16 678/653/645/665/682/680, 32/16 S=4 335/282/250/227/224/227; one-row
// pages S=16 771/721/693/703/715/721, S=8 470/426/403/382/377/378).
constexpr WaveBudget kPagedBudget{216, 0, 2, 3};

// Waves per CU for the exact-arithmetic kernels (rows16 and g_real as for
// waves_per_cu_for).  Their waves compute longer than the tree-order ones
// (sequential score sums staged through LDS), so fewer of their waves have
// requests in flight at a time and the CU needs more of them: 144 KiB per
// CU with known lengths, 200 KiB with lengths on the device (whose waves
// also wait for the lengths first); at least 4 waves, 5 for groups of 2 (C4
// with known lengths, µs at 4 / 5 / 6 / 8 waves: 665.8 / 652.7 / 667.1 /
// 691.4) and 6 for groups of 4 or more.  Sweep at B=30720 (µs, best cap /
// this model's / the tree-order kernel): known lengths Hq/Hkv 16/16 S=16
// D=128 613.7 (4) / 613.7 (4) / 610.2, 32/16 S=16 665.0 (4) / 665.0 (4) /
// 645.6, 32/32 S=16 D=256 2466.9 (4) / 2466.9 (4) / 2481.2, 16/16 S=5
// D=256 440.0 (16) / 442.1 (12) / 416.9; device lengths 16/16 S=16 616.9
// (4) / 626.1 (6; 5 here) / 614.6, 32/16 S=16 650.7 (6) / 650.7 (6) /
// 645.7, 32/32 S=16 D=256 2504.1 (6) / 2504.1 (6) / 2505.3.
int waves_per_cu_exact(int rows16, int g, int g_real, bool device_lengths) {
  const WaveBudget m{device_lengths ? 200 : 144, 0, 2, g >= 4 ? 6 : 3 + g};
  return budget_waves(m, rows16, g_real);
}

// Smallest power-of-two bucket >= s (s in [0, 16]); 0 selects bucket 1.
int bucket_for(int s) {
  int b = 1;
  while (b < s) b <<= 1;
  return b;
}

// Checks every entry point shares.  Any group size G = Hq / Hkv passes here;
// the kernel choice rejects what a path cannot run.
int check_common(const void* Q, const void* K, const void* V, void* O, int32_t batch, int32_t hq,
                 int32_t hkv, int32_t seqlen_q, int32_t dq, int32_t dkv, float scale, bool kv_may_be_null) {
  if (batch < 0) return reject(FMHA_DECODE_ERROR_INVALID_VALUE, "batch must be >= 0 (got %d)", batch);
  if (hq <= 0 || hkv <= 0)
    return reject(FMHA_DECODE_ERROR_INVALID_VALUE, "head counts must be > 0 (num_heads_q=%d, num_heads_kv=%d)", hq,
                  hkv);
  if (hq % hkv != 0)
    return reject(FMHA_DECODE_ERROR_INVALID_VALUE, "num_heads_q (%d) must be a multiple of num_heads_kv (%d)", hq,
                  hkv);
  if (seqlen_q != 1) return reject(FMHA_DECODE_ERROR_INVALID_VALUE, "seqlen_q must be 1 (got %d)", seqlen_q);
  if (dq != dkv)
    return reject(FMHA_DECODE_ERROR_INVALID_VALUE, "head_dim_q (%d) must equal head_dim_kv (%d)", dq, dkv);
  if (dq != 64 && dq != 128 && dq != 256)
    return reject(FMHA_DECODE_ERROR_INVALID_VALUE, "head_dim must be 64, 128 or 256 (got %d)", dq);
  if (!std::isfinite(scale)) return reject(FMHA_DECODE_ERROR_INVALID_VALUE, "softmax_scale must be finite");
  // Byte sizes of one batch's Q/O rows and of one batch's K/V span must fit
  // the 31-bit buffer ranges the kernel builds.
  if ((int64_t)hq * dq * 2 >= (int64_t(1) << 31) ||
      (int64_t)hkv * dq * 2 * FMHA_DECODE_MAX_SEQLEN_KV >= (int64_t(1) << 31))
    return reject(FMHA_DECODE_ERROR_INVALID_VALUE, "head count too large (num_heads_q=%d, num_heads_kv=%d)", hq, hkv);
  if (batch == 0) return FMHA_DECODE_SUCCESS;
  if (!Q || !O) return reject(FMHA_DECODE_ERROR_INVALID_VALUE, "Q and O must be non-null");
  // K and V may be null only when no row can be read (uniform seqlen_kv == 0).
  if ((!K || !V) && !kv_may_be_null)
    return reject(FMHA_DECODE_ERROR_INVALID_VALUE, "K and V must be non-null");
  if (!aligned16(Q) || !aligned16(K) || !aligned16(V) || !aligned16(O))
    return reject(FMHA_DECODE_ERROR_INVALID_VALUE, "Q, K, V and O must be 16-byte aligned");
  return FMHA_DECODE_SUCCESS;
}

// Fills the layout-independent fields, picks the wave cap and launches.
// rows16: 16 x the KV rows per batch used to size the per-CU wave cap (the
// uniform length, or an estimate when lengths live on the device, which
// device_lengths says); numerics selects the tree-order bf16-weight kernels
// (kBf16Weights), the fp32-weight ones or the exact-arithmetic ones (packed
// layout only, G <= 8).
enum class Numerics { kBf16Weights, kFp32Weights, kExact };

int launch(void* stream, int layout, DecodeArgs a, int32_t batch, int32_t dq, int sb, int rows16,
           bool device_lengths, Numerics numerics = Numerics::kBf16Weights) {
  const bool fp32_weights = numerics == Numerics::kFp32Weights;
  const bool exact = numerics == Numerics::kExact;
  const int heads_per_wave = kWaveSize / (dq / 8);
  const int64_t upb = (a.num_heads_kv + heads_per_wave - 1) / heads_per_wave;
  const int64_t units = upb * batch;
  if (units > (int64_t)UINT32_MAX - kWavesPerBlock)
    return reject(FMHA_DECODE_ERROR_INVALID_VALUE, "batch too large (%d)", batch);
  a.units_per_batch = (int32_t)upb;
  a.total_units = (uint32_t)units;
  a.group = a.num_heads_q / a.num_heads_kv;
  const int g = valu_kernel_group(a.group);
  if (g == 0)
    return reject(FMHA_DECODE_ERROR_NOT_SUPPORTED, "num_heads_q / num_heads_kv must be at most 8 here (got %d)",
                  a.group);
  hipStream_t s = static_cast<hipStream_t>(stream);
  hipError_t err;
  if (exact && layout != fmha_decode::kLayoutPacked)
    return reject(FMHA_DECODE_ERROR_NOT_SUPPORTED, "the exact kernels read the packed layout");
  // Fewer KV heads than a wave holds: R batches per wave, every lane busy
  // (paged: per-lane page lookups and addresses).  Strided only when R
  // batches' spans fit one descriptor.
  const int shift = fp32_weights && layout != fmha_decode::kLayoutPacked ? 0 : multi_shift(a.num_heads_kv, dq);
  bool multi = shift > 0;
  if (multi && layout == fmha_decode::kLayoutStrided) {
    const int64_t rows = a.max_rows > 0 ? a.max_rows : 1;
    const int64_t span = ((int64_t)((1 << shift) - 1) * a.batch_stride + (rows - 1) * a.row_stride +
                          (int64_t)(a.num_heads_kv - 1) * a.head_stride + dq) * 2;
    multi = span < (int64_t(1) << 30);
  }
  int w = exact ? waves_per_cu_exact(rows16, g, a.group, device_lengths)
               : waves_per_cu_for(rows16, g, a.group, dq, device_lengths, device_lengths || multi || sb == 0);
  if (layout == fmha_decode::kLayoutPaged && !multi) {
    if (g <= 2) {
      w = budget_waves(kPagedBudget, rows16, a.group);
    } else {
      // Three or more query heads per KV head: the page lookups come first
      // here too, and the byte model's cap (5 at 16 rows) leaves the CU
      // short of requests: at least 8 waves for groups of 3-4 at D <= 128,
      // 6 otherwise (B=30720 D=128, µs at the model's cap / this floor:
      // one-row pages 32/8 S=16 472.9 / 402.1, S=12 385.5 / 353.8, 24/8 S=16
      // 443.6 / 395.2, 64/8 S=12 490.4 / 441.7, S=16 550.1 / 521.4; 16-row
      // pages 32/8 S=16 436.5 / 404.1, 64/8 S=12 461.8 / 420.9, S=16 499.1 /
      // 505.0; D=64 32/8 S=16 245.6 / 211.3; D=256 B=15360 32/8 S=16 407.0
      // / 399.9 at 6, 408.9 at 8); rows of a whole 16-row page keep the
      // model's cap above four query heads (64/8 S=16 499.1 at 5 / 517.7 at
      // 6).
      const bool page_rows = a.seqlen_uniform >= 4 && rows16 >= 16 * 16;  // paged: log2(page size)
      const int floor = dq <= 128 && a.group <= 4 ? 8 : page_rows ? 0 : 6;
      if (w < floor) w = floor;
    }
  }
  // Waves that serve several batches (each lane group its own length and
  // rows) want at least 8 per CU at D <= 128 (B=30720 with lengths on the
  // device, µs at the byte model's cap / 8 waves: Hq/Hkv 8/1 S=16 79.0 /
  // 65.0, 4/1 60.4 / 56.6, 2/1 51.6 / 48.4, 8/2 109.5 / 102.7, D=64 8/1
  // 49.1 / 38.6; short rows and D = 256 flat).
  if (multi && dq <= 128 && w < 8) w = 8;
  // FMHA_DECODE_WAVE_CAP=<waves per CU> overrides the cap (for sweeps).
  if (const char* e = std::getenv("FMHA_DECODE_WAVE_CAP")) {
    const int v = std::atoi(e);
    if (v > 0) w = v;
  }
  if (exact) {
    if (multi) {
      int hs = 0;
      while ((1 << hs) < a.num_heads_kv) ++hs;
      a.sub_shift = shift;
      a.hkv_shift = hs;
      a.units_per_batch = batch;
      a.total_units = (uint32_t)(((int64_t)batch + (1 << shift) - 1) >> shift);
    }
#define FMHA_DECODE_EXACT_G(DD)                                    \
  switch (g) {                                                     \
    case 1: err = launch_exact<DD, 1>(a, multi, sb, w, s); break;  \
    case 2: err = launch_exact<DD, 2>(a, multi, sb, w, s); break;  \
    case 4: err = launch_exact<DD, 4>(a, multi, sb, w, s); break;  \
    default: err = launch_exact<DD, 8>(a, multi, sb, w, s); break; \
  }
    switch (dq) {
      case 64: FMHA_DECODE_EXACT_G(64) break;
      case 128: FMHA_DECODE_EXACT_G(128) break;
      default: FMHA_DECODE_EXACT_G(256) break;
    }
#undef FMHA_DECODE_EXACT_G
    if (err != hipSuccess) return reject((int)err, "kernel launch failed: %s", hipGetErrorString(err));
    return FMHA_DECODE_SUCCESS;
  }
  if (multi) {
    int hs = 0;
    while ((1 << hs) < a.num_heads_kv) ++hs;
    a.sub_shift = shift;
    a.hkv_shift = hs;
    a.units_per_batch = batch;  // the batch count, for this kernel
    a.total_units = (uint32_t)(((int64_t)batch + (1 << shift) - 1) >> shift);
    switch (layout) {
      case fmha_decode::kLayoutPacked:
        err = fp32_weights ? launch_multi<fmha_decode::kLayoutPacked, true>(a, dq, g, w, s)
                           : launch_multi<fmha_decode::kLayoutPacked, false>(a, dq, g, w, s);
        break;
      case fmha_decode::kLayoutStrided: err = launch_multi<fmha_decode::kLayoutStrided, false>(a, dq, g, w, s); break;
      default: err = launch_multi<fmha_decode::kLayoutPaged, false>(a, dq, g, w, s); break;
    }
    if (err != hipSuccess) return reject((int)err, "kernel launch failed: %s", hipGetErrorString(err));
    return FMHA_DECODE_SUCCESS;
  }
  switch (layout) {
    case fmha_decode::kLayoutPacked:
      err = fp32_weights ? launch_dim<fmha_decode::kLayoutPacked, true>(a, dq, g, sb, w, s)
                         : launch_dim<fmha_decode::kLayoutPacked>(a, dq, g, sb, w, s);
      break;
    case fmha_decode::kLayoutStrided: err = launch_dim<fmha_decode::kLayoutStrided>(a, dq, g, sb, w, s); break;
    default: err = launch_dim<fmha_decode::kLayoutPaged>(a, dq, g, sb, w, s); break;
  }
  if (err != hipSuccess) return reject((int)err, "kernel launch failed: %s", hipGetErrorString(err));
  return FMHA_DECODE_SUCCESS;
}

// ---------------------------------------------------------------------------
// Matrix-core kernel (fmha_decode_group_kernel): packed layout, any G.
// ---------------------------------------------------------------------------

// Kernel choice for the packed and strided layouts, G query heads per KV
// head: the VALU kernel for G <= 8 (3 and 5-7 on its 4- and 8-head
// instantiations), the matrix-core kernel above.  With the VALU kernel's
// wave caps it is the faster of the two or within 2% at every G <= 8 shape
// measured (B=30720, µs VALU / MFMA: D=128 Hkv=16 G=3 S=8 418/469, S=16
// 754/763, G=5 S=16 834/889, G=7 S=8 595/634, G=8 S=16 966/1002; D=64
// Hkv=8 G=5 S=16 191/210, G=7 S=16 206/225; D=256 Hkv=8 B=15360 G=6 S=16
// 435/692).
// FMHA_DECODE_GQA_KERNEL=mfma runs the matrix-core kernel for every G, =valu
// keeps the VALU kernel wherever it exists (for comparisons).
// Long rows, by the launch's group (g_launch = launch query heads per launch
// KV head: 8 for G = 5-8 and, as kv_groups groups of 8, for every G > 8):
// the matrix-core split passes for G > 8 and for G = 5-8 on the packed,
// strided and 16-row-page layouts, and on pages under 16 rows when the
// batch has fewer KV heads than half a wave (hkv launch KV heads, head dim
// d); the VALU passes otherwise.  Against the VALU passes at G = 8 and 5-7
// (µs, each at its best chunk size; D = 128 unless given): B=8 S=32768
// Hq/Hkv 64/8 232 vs 223, B=256 S=1024 64/8 233 vs 221, B=64 S=4096 64/8
// 219 vs 218, 32/4 125 vs 123, 8/1 52 vs 46, D=64 B=32 64/8 99 vs 87,
// D=256 B=16 64/8 115 vs 108, 40/8 236 vs 227; BHSD 64/8 B=8 260 vs 211;
// 16-row pages 250 vs 233; one-row pages 64/8 B=64 273 vs 381 (the VALU
// passes' per-row descriptors against per-lane addresses), 8/1 92 vs 66.
// At G = 4 the VALU split passes stay faster (B=64 S=4096 32/8 189 vs 206);
// groups of at most 4 on rows the one-wave single pass does not hold take
// the register single pass on the matrix cores from the VALU launcher
// (launch_split_dg) where it applies.
// FMHA_DECODE_GQA_KERNEL=valu keeps every G on the VALU passes (G > 8 on
// ceil(G / 8) launch KV heads of 8 query heads), =mfma puts every G on the
// matrix cores.
bool gqa_kernel_forced(const char* kind) {
  const char* e = std::getenv("FMHA_DECODE_GQA_KERNEL");
  return e && std::strcmp(e, kind) == 0;
}

bool split_on_matrix_cores(int g_launch, int kv_groups, int layout, int hkv, int d, int max_rows) {
  if (gqa_kernel_forced("valu")) return false;
  if (gqa_kernel_forced("mfma")) return true;
  if (kv_groups > 1) return true;
  const int hpw = kWaveSize / (d / 8);
  const bool lanes = 2 * hkv <= hpw && hpw % (2 * hkv) == 0;
  if (g_launch < 8) return false;
  if (layout != fmha_decode::kLayoutPaged) return true;
  return lanes;
}

bool use_mfma_kernel(int g) {
  if (const char* e = std::getenv("FMHA_DECODE_GQA_KERNEL"))
    if (std::strcmp(e, "mfma") == 0) return true;
  return valu_kernel_group(g) == 0;
}

// Streams per 16-column query tile: 4 for G <= 4, 2 for G <= 8, else 1
// (capped at the streams a wave holds).
int mfma_streams_per_tile(int64_t g, int hpw) {
  const int ns = g <= 4 ? 4 : (g <= 8 ? 2 : 1);
  return ns < hpw ? ns : hpw;
}

// a: the fields base_args and the entry points fill (packed: lens = cu
// offsets or null with seqlen_uniform, row and head strides of [rows, Hkv,
// D]; strided: lens = lengths or null, strides, max_rows).  rows_hint as for
// launch().
int launch_mfma(void* stream, int layout, const DecodeArgs& a, int32_t batch, int32_t dq, int rows_hint) {
  const int hpw = kWaveSize / (dq / 8);
  const int64_t hkv = a.num_heads_kv;
  const int64_t g = a.num_heads_q / a.num_heads_kv;
  // One descriptor covers a wave's streams, which span at most hpw / hkv + 2
  // batches; that byte range must stay below the out-of-range offsets (2^30).
  const int64_t batches = hpw / hkv + 2;
  if (layout == fmha_decode::kLayoutPacked) {
    const int64_t row_bytes = hkv * dq * 2;
    if (row_bytes * FMHA_DECODE_MAX_SEQLEN_KV * batches >= (int64_t(1) << 30))
      return reject(FMHA_DECODE_ERROR_NOT_SUPPORTED, "num_heads_kv * head_dim too large (%lld)", (long long)(hkv * dq));
  } else if (layout == fmha_decode::kLayoutPagedLanes) {
    // 64-bit addresses per lane: no descriptor to bound.
  } else if (layout == fmha_decode::kLayoutPaged) {
    // One batch's rows within its first page (paged_mfma_layout).
    const int64_t rows = a.max_rows > 0 ? a.max_rows : 1;
    const int64_t span = ((rows - 1) * a.row_stride + (hkv - 1) * a.head_stride + dq) * 2;
    if (span >= (int64_t(1) << 30))
      return reject(FMHA_DECODE_ERROR_NOT_SUPPORTED, "num_heads_kv * head_dim too large (%lld)", (long long)(hkv * dq));
  } else {
    const int64_t rows = a.max_rows > 0 ? a.max_rows : 1;
    const int64_t span = ((batches - 1) * a.batch_stride + (rows - 1) * a.row_stride + (hkv - 1) * a.head_stride + dq) * 2;
    if (span >= (int64_t(1) << 30))
      return reject(FMHA_DECODE_ERROR_NOT_SUPPORTED,
                    "K/V span of %lld batches exceeds 1 GiB for the matrix-core kernel (group size %lld)",
                    (long long)batches, (long long)g);
  }
  const int ns = mfma_streams_per_tile(g, hpw);
  const int64_t tps = ns > 1 ? 1 : (g + 15) / 16;  // tiles per stream = waves per stream group
  const int64_t streams = (int64_t)batch * hkv;
  const int64_t groups = (streams + hpw - 1) / hpw;
  const int64_t waves = tps == 1 ? groups : 8 * tps * ((groups + 7) / 8);
  if (streams > (int64_t)UINT32_MAX || waves > (int64_t)INT32_MAX)
    return reject(FMHA_DECODE_ERROR_INVALID_VALUE, "batch too large (%d)", batch);
  fmha_decode::GroupArgs ga = {};
  ga.q = a.q;
  ga.k = a.k;
  ga.v = a.v;
  ga.o = a.o;
  ga.lens = a.lens;
  ga.seqlen_uniform = a.seqlen_uniform;
  ga.max_rows = a.max_rows;
  ga.batch_stride = a.batch_stride;
  ga.row_stride = a.row_stride;
  ga.head_stride = a.head_stride;
  ga.num_heads_kv = a.num_heads_kv;
  ga.group = (int32_t)g;
  ga.streams = (uint32_t)streams;
  ga.stream_groups = (uint32_t)groups;
  ga.tiles_per_stream = (int32_t)tps;
  ga.chunks = (int32_t)tps;
  ga.waves = (uint32_t)waves;
  ga.scale = a.scale;
  ga.block_table = a.block_table;
  ga.bt_stride = a.bt_stride;
  // Waves per CU, from sweeps (B=30720, S=16, µs for 4/5/6/8 waves; the
  // kernel's 17 KiB of LDS and 172-215 VGPRs allow 8): the best cap follows
  // the tiles a wave computes more than its bytes.  D=128: 4 (G=3
  // 773/810/813/818, G=12 1126/1167/1164/1190); 8 where a stream group's
  // query heads take more than one wave (G > 16: their K/V re-reads are L2
  // hits, so a wave brings mostly Q and O; MQA G=32 Hkv=1
  // 132/121/124/117); D=64: 6 (Hkv=8, G=5 227/194/210/207, G=12
  // 400/320/317/316 with an earlier form); D=256: 4 (G=3 557/483/484/488/490
  // for 3/4/5/6/8, G=5 603/633/637/638/632, an earlier form).  Waves of
  // under 32 KiB (short rows) run uncapped (G=5 at S=4 725/569/476/417/413
  // for 3/4/5/6/8, an earlier form).
  const int64_t qrows = g <= 16 ? hpw * g : 16 * hpw;
  const int64_t unit_bytes = 2LL * rows_hint * hpw * dq * 2 + 2LL * qrows * dq * 2;
  int w = dq == 64 ? 6 : (tps >= 2 ? 8 : 4);
  if (unit_bytes < 32 * 1024) w = kMaxWavesPerCU;
  if (const char* e = std::getenv("FMHA_DECODE_WAVE_CAP")) {  // as in launch(): for sweeps
    const int v = std::atoi(e);
    if (v > 0) w = v;
  }
  hipStream_t s = static_cast<hipStream_t>(stream);
  const hipError_t err = layout == fmha_decode::kLayoutPacked
                             ? launch_mfma_layout<fmha_decode::kLayoutPacked>(ga, dq, ns, w, s)
                         : layout == fmha_decode::kLayoutPaged
                             ? launch_mfma_layout<fmha_decode::kLayoutPaged>(ga, dq, ns, w, s)
                         : layout == fmha_decode::kLayoutPagedLanes
                             ? launch_mfma_layout<fmha_decode::kLayoutPagedLanes>(ga, dq, ns, w, s)
                             : launch_mfma_layout<fmha_decode::kLayoutStrided>(ga, dq, ns, w, s);
  if (err != hipSuccess) return reject((int)err, "kernel launch failed: %s", hipGetErrorString(err));
  return FMHA_DECODE_SUCCESS;
}

DecodeArgs base_args(const void* Q, const void* K, const void* V, void* O, int32_t hq, int32_t hkv, float scale) {
  DecodeArgs a = {};
  a.q = static_cast<const uint16_t*>(Q);
  a.k = static_cast<const uint16_t*>(K);
  a.v = static_cast<const uint16_t*>(V);
  a.o = static_cast<uint16_t*>(O);
  a.num_heads_q = hq;
  a.num_heads_kv = hkv;
  a.group = hq / hkv;
  a.scale = scale;
  a.max_rows = FMHA_DECODE_MAX_SEQLEN_KV;
  return a;
}

// Rows per batch assumed when lengths come from a device array (the host
// cannot see them): the reference's own varlen workload, Poisson(4) lengths
// in [2, 16], averages 4.3 rows, and its best cap is the 4-row one.
constexpr int kVarlenRowsHint = 4;

// Mean-length feedback for the packed cu_seqlens and the paged entry
// points.  The best
// wave cap depends on the rows per batch (4-row batches: 8 waves per CU;
// 16-row batches: 3, 7% faster than under the 4-row cap at B=30720 H=16
// D=128), which the host cannot read without a synchronisation.  So the
// first wave of each call writes 16 x its mean length, 16 * (cu[batch] -
// cu[0]) / batch, into one word of pinned host memory per device, and the
// next call on that device sizes its cap from it (the default 4-row cap
// until a call has reported).  Decoding loops call with lengths that change
// by one row per step, so the previous call's mean is a close estimate; a
// stale or foreign value changes speed, never results.  The word is
// allocated on the first call that is not being captured into a graph (a
// capture does not report), never freed, and read without a lock.  The
// paged short kernels report likewise into a second word of the same
// allocation (kPagedFeedbackWord), the mean of a sample of their lengths
// (the first 4096): with 16-row pages their best cap follows the rows as
// the packed kernels' does (B=30720 S=16 Hq/Hkv 16/16, µs at 5 waves per
// CU / the 4-row cap of 14: 644 / 684).
constexpr int kPagedFeedbackWord = 8;
constexpr int kMaxFeedbackDevices = 64;
std::atomic<int32_t*> g_feedback[kMaxFeedbackDevices];
std::atomic<bool> g_feedback_failed[kMaxFeedbackDevices];
std::mutex g_feedback_mutex;

int32_t* feedback_word(void* stream, bool may_allocate = true) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxFeedbackDevices) return nullptr;
  int32_t* word = g_feedback[dev].load(std::memory_order_acquire);
  if (word || !may_allocate || g_feedback_failed[dev].load(std::memory_order_relaxed)) return word;
  hipStreamCaptureStatus capture = hipStreamCaptureStatusNone;
  if (hipStreamIsCapturing(static_cast<hipStream_t>(stream), &capture) != hipSuccess ||
      capture != hipStreamCaptureStatusNone)
    return nullptr;
  std::lock_guard<std::mutex> lock(g_feedback_mutex);
  word = g_feedback[dev].load(std::memory_order_acquire);
  if (word) return word;
  void* host = nullptr;
  void* mapped = nullptr;
  if (hipHostMalloc(&host, 64, hipHostMallocMapped | hipHostMallocCoherent | hipHostMallocPortable) != hipSuccess ||
      hipHostGetDevicePointer(&mapped, host, 0) != hipSuccess) {
    (void)hipGetLastError();  // no feedback on this device: the default cap
    g_feedback_failed[dev].store(true, std::memory_order_relaxed);
    return nullptr;
  }
  for (int i = 0; i < 16; ++i) static_cast<volatile int32_t*>(host)[i] = 0;
  word = static_cast<int32_t*>(mapped);
  g_feedback[dev].store(word, std::memory_order_release);
  return word;
}

// 16 x the rows per batch for the wave cap of a cu_seqlens call: the mean
// the last reporting call left (within [1, max_rows] rows), or the default.
int feedback_rows16(const int32_t* word, int max_rows) {
  const int32_t mean16 = word ? __atomic_load_n(word, __ATOMIC_RELAXED) : 0;
  int rows16 = mean16 > 0 ? mean16 : 16 * kVarlenRowsHint;
  if (rows16 > 16 * max_rows) rows16 = 16 * max_rows;
  return rows16 < 16 ? 16 : rows16;
}

// ---------------------------------------------------------------------------
// Split-KV (lengths beyond 16)
// ---------------------------------------------------------------------------
constexpr size_t kWorkspaceAlign = 256;

size_t align_up(size_t x) { return (x + kWorkspaceAlign - 1) / kWorkspaceAlign * kWorkspaceAlign; }

struct SplitPlan {
  int chunk_rows = 16;
  int nchunks = 1;
  int nblk = 1;
  int64_t units = 0;
  size_t off_t = 0, off_m = 0, off_l = 0, off_ml = 0, off_opart = 0, total = 0;
};

// P.V waves the VALU split pass aims for.  A wave keeps two sub-blocks of V
// in flight: 2 * 16 rows of 1 KiB (the wave's heads' share of a row) for
// G <= 4, half that for G = 8 (8-row sub-blocks), and less again when the
// batch has fewer KV heads than a wave holds (idle lanes).  The target is
// 512 waves of the full kind, scaled up by those two factors, so that the V
// requests in flight per CU stay about the same and the pass runs in one
// round of long waves: fewer, longer chunks also mean fewer partial outputs
// to combine.  Measured against a fixed 2048 (µs): B=1 S=131072 Hq=32 Hkv=8
// D=128 118.4 -> 105.5; B=64 S=4096 200.5 -> 188.7; B=16 Hq=16 Hkv=8 S=8192
// D=256 186.7 -> 175.5; B=32 Hq=64 Hkv=8 S=8192 234.0 -> 216.5; B=4 Hq=32
// Hkv=4 S=32768 D=64 (half the lanes idle) 72.0 -> 72.1.
int64_t split_target_waves(int hq, int hkv, int d) {
  const int heads_per_wave = kWaveSize / (d / 8);
  const int g = hq / hkv;
  const int active = hkv < heads_per_wave ? hkv : heads_per_wave;
  return (int64_t)512 * (g >= 8 ? 2 : 1) * heads_per_wave / active;
}

// Scores: one wave per 16-row block.  P.V: chunks of C rows (C in
// {64, ..., 1024}, or the rows' own multiple of 16 when shorter), the
// largest that still gives the pass's target wave count where the work
// allows.  VALU passes: split_target_waves waves of HPW KV heads (1024 rows
// against 512 measured 0-3% faster where it keeps that count: B=256 S=1024
// Hq=32 Hkv=8 192.9 -> 187.9 µs).  Matrix-core passes (kv_groups launch KV
// heads per cache head): one wave per (batch, cache KV head, chunk, pair of
// 16-column tiles; one tile at D = 256), 2048 of them for groups of up to 8
// query heads and 1024 above (whose waves fill their tiles), half that at
// D = 256 (µs by C = 256 / 512 / 1024: B=8 S=32768 64/8 239/226/223, 40/8
// 244/233/227; B=64 S=4096 32/4 129/123/122, 64/4 (G = 16) 150/143/136;
// B=8 S=32768 8/1 48/55/74 (C = 128: 46); D=64 B=32 S=4096 64/8
// 90/87/91; D=256 B=16 S=4096 64/8 110/108/136; MQA B=8 S=32768 32/1
// 72/82/111).
SplitPlan plan_split(int64_t batch, int hq, int hkv, int max_rows, int d, int kv_groups, int layout) {
  SplitPlan p;
  const int heads_per_wave = kWaveSize / (d / 8);
  const int64_t upb = (hkv + heads_per_wave - 1) / heads_per_wave;
  p.units = upb * batch;
  int64_t per_chunk = p.units;  // P.V waves per chunk of every batch
  int64_t target = split_target_waves(hq, hkv, d);
  if (split_on_matrix_cores(hq / hkv, kv_groups, layout, hkv, d, max_rows)) {
    const int hkv_mem = hkv / kv_groups;
    const int g_mem = hq / hkv_mem;
    const int tw = d == 256 ? 1 : 2;
    per_chunk = batch * hkv_mem * (((g_mem + 15) / 16 + tw - 1) / tw);
    target = (g_mem <= 8 ? 2048 : 1024) / (d == 256 ? 2 : 1);
  }
  int c = 1024;
  while (c > 64 && per_chunk * ((max_rows + c - 1) / c) < target) c /= 2;
  // Pages of fewer than 16 rows put every row at its own place in memory:
  // the P.V waves, which walk their chunk a sub-block at a time, then wait
  // on scattered requests, and shorter chunks (more waves) hide that (µs by
  // C = 128 / 256 / 512 / 1024 on one-row pages, B=64 S=4096 Hq=32 Hkv=8:
  // 243/220/227/309; B=8 S=32768: 239/230/256/312; Hq=64 Hkv=8
  // 268/251/314/387; B=16 S=8192 16/16: 206/193/195/255; matrix cores,
  // B=64 S=4096 64/4: 245/219/-/274).
  if (layout == fmha_decode::kLayoutPaged && c > 256) c = 256;
  // Fewer KV heads than a wave holds, on the VALU passes: a P.V wave's
  // 2^shift lane groups take chunks of one row, so rows get at least 2^shift
  // chunks where chunks of 64 rows or more allow it: on paged caches for any
  // shift (µs, 16-row pages, chunks as before / now: B=2048 S=512 Hq/Hkv
  // 4/1 192 / 121, B=1024 S=1024 140 / 115, B=2048 S=512 8/2 254 / 216, D=64
  // 2/1 80 / 65; one-row pages B=2048 S=512 4/1 141 / 118, D=64 2/1 88 /
  // 64), on packed and strided ones from four lane groups up (packed B=2048
  // S=512 4/1 123 / 115, D=64 2/1 66 / 62; with two, 8/2, 195 / 210).
  if (!split_on_matrix_cores(hq / hkv, kv_groups, layout, hkv, d, max_rows)) {
    int shift = 0;
    while ((hkv << (shift + 1)) <= heads_per_wave && heads_per_wave % (hkv << (shift + 1)) == 0) ++shift;
    if (shift >= (fmha_decode::is_paged_layout(layout) ? 1 : 2))
      while (c > 64 && ((int64_t)c << shift) > max_rows) c /= 2;
  }
  // FMHA_DECODE_SPLIT_CHUNK=<64|...|2048> overrides C (for sweeps; the
  // workspace size follows, and a launch checks its workspace against it).
  if (const char* e = std::getenv("FMHA_DECODE_SPLIT_CHUNK")) {
    const int v = std::atoi(e);
    if (v >= 64 && v <= 2048 && (v & (v - 1)) == 0) c = v;
  }
  const int fit = max_rows <= 16 ? 16 : (max_rows + 15) / 16 * 16;  // no longer than the rows need
  if (c > fit) c = fit;
  p.chunk_rows = c;
  p.nchunks = max_rows <= 0 ? 1 : (max_rows + c - 1) / c;
  p.nblk = max_rows <= 0 ? 1 : (max_rows + fmha_decode::kSplitBlockRows - 1) / fmha_decode::kSplitBlockRows;
  const size_t heads = (size_t)batch * hq;
  size_t off = 0;
  p.off_t = off;
  off += align_up(heads * (size_t)p.nblk * fmha_decode::kSplitBlockRows * 4);
  p.off_m = off;
  off += align_up(heads * (size_t)p.nblk * 4);
  p.off_l = off;
  off += align_up(heads * (size_t)p.nblk * 4);
  p.off_ml = off;
  off += align_up(heads * 2 * 4);
  p.off_opart = off;
  if (p.nchunks > 1) off += align_up(heads * (size_t)p.nchunks * d * 4);
  p.total = off;
  return p;
}

}  // namespace

namespace {

// Numerics of the default entry points (fmha_decode_fwd, _uniform, and
// fmha_decode_fwd_splitkv up to 16 rows) for G query heads per KV head: the
// reference loop's arithmetic up to 2, the group sizes of the reference's
// own configurations and of BASELINE, where it costs at most 1% at B=30720
// but for short rows at D = 256 (S=5: 440 against 417 us; the measurements
// at waves_per_cu_exact); the tree-order kernels above, where the exact
// ones measured 2-45% slower (Hq/Hkv 64/16 S=16 +4.5% with known lengths,
// 64/16 Poisson(4) +20%, 80/16 and 128/16 S=16 +14-16%, 8/1 S=16 +16%,
// D=64 40/8 +45%).
Numerics default_numerics(int g) { return g <= 2 ? Numerics::kExact : Numerics::kBf16Weights; }

// The packed cu_seqlens entry points.  kExact: the reference loop's
// arithmetic for G <= 8; G > 8 has no exact kernel and is rejected
// (fmha_decode_fwd_exact).  kBf16Weights: the tree-order kernels, the VALU
// kernel for G <= 8 and the matrix-core kernel above (or for every G under
// FMHA_DECODE_GQA_KERNEL=mfma).
int fwd_cu(void* stream, const void* Q, const void* K, const void* V, void* O, const int32_t* cu_seqlens_kv,
           int32_t batch, int32_t num_heads_q, int32_t num_heads_kv, int32_t seqlen_q, int32_t head_dim_q,
           int32_t head_dim_kv, float softmax_scale, Numerics numerics, bool exact_only) {
  begin_call();
  int rc = check_common(Q, K, V, O, batch, num_heads_q, num_heads_kv, seqlen_q, head_dim_q, head_dim_kv,
                        softmax_scale, false);
  if (rc != FMHA_DECODE_SUCCESS || batch == 0) return rc;
  const int g = num_heads_q / num_heads_kv;
  if (exact_only && valu_kernel_group(g) == 0)
    return reject(FMHA_DECODE_ERROR_NOT_SUPPORTED,
                  "the exact path takes at most 8 query heads per KV head (got %d)", g);
  if (!cu_seqlens_kv) return reject(FMHA_DECODE_ERROR_INVALID_VALUE, "cu_seqlens_kv must be non-null");
  if ((reinterpret_cast<uintptr_t>(cu_seqlens_kv) & 3u) != 0)
    return reject(FMHA_DECODE_ERROR_INVALID_VALUE, "cu_seqlens_kv must be 4-byte aligned");
  DecodeArgs a = base_args(Q, K, V, O, num_heads_q, num_heads_kv, softmax_scale);
  a.lens = cu_seqlens_kv;
  a.row_stride = num_heads_kv * head_dim_q;
  a.head_stride = head_dim_q;
  const bool mfma = numerics == Numerics::kBf16Weights && use_mfma_kernel(g);
  if (mfma) return launch_mfma(stream, fmha_decode::kLayoutPacked, a, batch, head_dim_q, kVarlenRowsHint);
  a.rows_feedback = feedback_word(stream);
  return launch(stream, fmha_decode::kLayoutPacked, a, batch, head_dim_q, 0,
                feedback_rows16(a.rows_feedback, FMHA_DECODE_MAX_SEQLEN_KV), true, numerics);
}

// The uniform entry points, numerics as fwd_cu.
int fwd_uniform(void* stream, const void* Q, const void* K, const void* V, void* O, int32_t seqlen_kv,
                int32_t batch, int32_t num_heads_q, int32_t num_heads_kv, int32_t seqlen_q, int32_t head_dim_q,
                int32_t head_dim_kv, float softmax_scale, Numerics numerics) {
  begin_call();
  if (seqlen_kv < 0 || seqlen_kv > FMHA_DECODE_MAX_SEQLEN_KV)
    return reject(FMHA_DECODE_ERROR_INVALID_VALUE, "seqlen_kv must lie in [0, %d] (got %d)",
                  FMHA_DECODE_MAX_SEQLEN_KV, seqlen_kv);
  int rc = check_common(Q, K, V, O, batch, num_heads_q, num_heads_kv, seqlen_q, head_dim_q, head_dim_kv,
                        softmax_scale, seqlen_kv == 0);
  if (rc != FMHA_DECODE_SUCCESS || batch == 0) return rc;
  DecodeArgs a = base_args(Q, K, V, O, num_heads_q, num_heads_kv, softmax_scale);
  a.seqlen_uniform = seqlen_kv;
  a.row_stride = num_heads_kv * head_dim_q;
  a.head_stride = head_dim_q;
  const int g = num_heads_q / num_heads_kv;
  if (numerics != Numerics::kExact && use_mfma_kernel(g))
    return launch_mfma(stream, fmha_decode::kLayoutPacked, a, batch, head_dim_q, seqlen_kv);
  return launch(stream, fmha_decode::kLayoutPacked, a, batch, head_dim_q, bucket_for(seqlen_kv), 16 * seqlen_kv,
                false, numerics);
}

}  // namespace

extern "C" int fmha_decode_fwd(void* stream, const void* Q, const void* K, const void* V, void* O,
                               const int32_t* cu_seqlens_kv, int32_t batch, int32_t num_heads_q,
                               int32_t num_heads_kv, int32_t seqlen_q, int32_t head_dim_q, int32_t head_dim_kv,
                               float softmax_scale) {
  const int g = num_heads_kv > 0 ? num_heads_q / num_heads_kv : 0;
  return fwd_cu(stream, Q, K, V, O, cu_seqlens_kv, batch, num_heads_q, num_heads_kv, seqlen_q, head_dim_q,
                head_dim_kv, softmax_scale, default_numerics(g), false);
}

extern "C" int fmha_decode_fwd_fast(void* stream, const void* Q, const void* K, const void* V, void* O,
                                    const int32_t* cu_seqlens_kv, int32_t batch, int32_t num_heads_q,
                                    int32_t num_heads_kv, int32_t seqlen_q, int32_t head_dim_q, int32_t head_dim_kv,
                                    float softmax_scale) {
  return fwd_cu(stream, Q, K, V, O, cu_seqlens_kv, batch, num_heads_q, num_heads_kv, seqlen_q, head_dim_q,
                head_dim_kv, softmax_scale, Numerics::kBf16Weights, false);
}

extern "C" int fmha_decode_fwd_fp32_weights(void* stream, const void* Q, const void* K, const void* V, void* O,
                                            const int32_t* cu_seqlens_kv, int32_t batch, int32_t num_heads_q,
                                            int32_t num_heads_kv, int32_t seqlen_q, int32_t head_dim_q,
                                            int32_t head_dim_kv, float softmax_scale) {
  return fwd_cu(stream, Q, K, V, O, cu_seqlens_kv, batch, num_heads_q, num_heads_kv, seqlen_q, head_dim_q,
                head_dim_kv, softmax_scale, Numerics::kFp32Weights, false);
}

extern "C" int fmha_decode_fwd_exact(void* stream, const void* Q, const void* K, const void* V, void* O,
                                     const int32_t* cu_seqlens_kv, int32_t batch, int32_t num_heads_q,
                                     int32_t num_heads_kv, int32_t seqlen_q, int32_t head_dim_q, int32_t head_dim_kv,
                                     float softmax_scale) {
  return fwd_cu(stream, Q, K, V, O, cu_seqlens_kv, batch, num_heads_q, num_heads_kv, seqlen_q, head_dim_q,
                head_dim_kv, softmax_scale, Numerics::kExact, true);
}

extern "C" int fmha_decode_fwd_uniform(void* stream, const void* Q, const void* K, const void* V, void* O,
                                       int32_t seqlen_kv, int32_t batch, int32_t num_heads_q, int32_t num_heads_kv,
                                       int32_t seqlen_q, int32_t head_dim_q, int32_t head_dim_kv,
                                       float softmax_scale) {
  const int g = num_heads_kv > 0 ? num_heads_q / num_heads_kv : 0;
  return fwd_uniform(stream, Q, K, V, O, seqlen_kv, batch, num_heads_q, num_heads_kv, seqlen_q, head_dim_q,
                     head_dim_kv, softmax_scale, default_numerics(g));
}

extern "C" int fmha_decode_fwd_uniform_fast(void* stream, const void* Q, const void* K, const void* V, void* O,
                                            int32_t seqlen_kv, int32_t batch, int32_t num_heads_q,
                                            int32_t num_heads_kv, int32_t seqlen_q, int32_t head_dim_q,
                                            int32_t head_dim_kv, float softmax_scale) {
  return fwd_uniform(stream, Q, K, V, O, seqlen_kv, batch, num_heads_q, num_heads_kv, seqlen_q, head_dim_q,
                     head_dim_kv, softmax_scale, Numerics::kBf16Weights);
}

extern "C" int fmha_decode_fwd_strided(void* stream, const void* Q, const void* K, const void* V, void* O,
                                       const int32_t* seqlens_kv, int32_t seqlen_kv, int64_t kv_batch_stride,
                                       int64_t kv_row_stride, int64_t kv_head_stride, int32_t batch,
                                       int32_t num_heads_q, int32_t num_heads_kv, int32_t seqlen_q,
                                       int32_t head_dim_q, int32_t head_dim_kv, float softmax_scale) {
  begin_call();
  if (seqlen_kv < 0 || (!seqlens_kv && seqlen_kv > FMHA_DECODE_MAX_SEQLEN_KV))
    return reject(FMHA_DECODE_ERROR_INVALID_VALUE,
                  "seqlen_kv must be >= 0, and <= %d when seqlens_kv is null (got %d)", FMHA_DECODE_MAX_SEQLEN_KV,
                  seqlen_kv);
  const int cap = seqlen_kv < FMHA_DECODE_MAX_SEQLEN_KV ? seqlen_kv : FMHA_DECODE_MAX_SEQLEN_KV;
  int rc = check_common(Q, K, V, O, batch, num_heads_q, num_heads_kv, seqlen_q, head_dim_q, head_dim_kv,
                        softmax_scale, cap == 0);
  if (rc != FMHA_DECODE_SUCCESS || batch == 0) return rc;
  if (kv_batch_stride < 0 || kv_row_stride < 0 || kv_head_stride < 0)
    return reject(FMHA_DECODE_ERROR_INVALID_VALUE, "K/V strides must be >= 0");
  if ((kv_batch_stride | kv_row_stride | kv_head_stride) & 7)
    return reject(FMHA_DECODE_ERROR_INVALID_VALUE, "K/V strides must be multiples of 8 elements (16 bytes)");
  // Bytes one batch's descriptor may span must stay below 2^30.
  const int64_t extent = cap == 0 ? 0
                                  : (int64_t)(cap - 1) * kv_row_stride +
                                        (int64_t)(num_heads_kv - 1) * kv_head_stride + head_dim_q;
  if (extent * 2 >= (int64_t(1) << 30))
    return reject(FMHA_DECODE_ERROR_INVALID_VALUE, "one batch's K/V span exceeds 1 GiB");
  if (seqlens_kv && (reinterpret_cast<uintptr_t>(seqlens_kv) & 3u) != 0)
    return reject(FMHA_DECODE_ERROR_INVALID_VALUE, "seqlens_kv must be 4-byte aligned");
  DecodeArgs a = base_args(Q, K, V, O, num_heads_q, num_heads_kv, softmax_scale);
  a.lens = seqlens_kv;
  a.seqlen_uniform = seqlens_kv ? 0 : seqlen_kv;
  a.max_rows = cap;
  a.batch_stride = kv_batch_stride;
  a.row_stride = (int32_t)kv_row_stride;
  a.head_stride = (int32_t)kv_head_stride;
  const int sb = seqlens_kv ? 0 : bucket_for(seqlen_kv);
  const int rows_hint = seqlens_kv ? (cap < kVarlenRowsHint ? cap : kVarlenRowsHint) : seqlen_kv;
  if (use_mfma_kernel(num_heads_q / num_heads_kv))
    return launch_mfma(stream, fmha_decode::kLayoutStrided, a, batch, head_dim_q, rows_hint);
  return launch(stream, fmha_decode::kLayoutStrided, a, batch, head_dim_q, sb, 16 * rows_hint, seqlens_kv != nullptr);
}

namespace {

int log2_pow2(int x) {
  int shift = 0;
  while ((1 << shift) < x) ++shift;
  return shift;
}

int paged_checks(const void* Q, const void* K_cache, const void* V_cache, void* O, const int32_t* block_table,
                 int32_t block_table_stride, const int32_t* seqlens_kv, int32_t page_size, int32_t batch,
                 int32_t num_heads_q, int32_t num_heads_kv, int32_t seqlen_q, int32_t head_dim_q,
                 int32_t head_dim_kv, float softmax_scale) {
  int rc = check_common(Q, K_cache, V_cache, O, batch, num_heads_q, num_heads_kv, seqlen_q, head_dim_q, head_dim_kv,
                        softmax_scale, false);
  if (rc != FMHA_DECODE_SUCCESS || batch == 0) return rc;
  if (page_size < 1 || (page_size & (page_size - 1)) != 0 || page_size > (1 << 20))
    return reject(FMHA_DECODE_ERROR_INVALID_VALUE, "page_size must be a power of two in [1, 2^20] (got %d)",
                  page_size);
  if (!block_table || !seqlens_kv)
    return reject(FMHA_DECODE_ERROR_INVALID_VALUE, "block_table and seqlens_kv must be non-null");
  if (((reinterpret_cast<uintptr_t>(block_table) | reinterpret_cast<uintptr_t>(seqlens_kv)) & 3u) != 0)
    return reject(FMHA_DECODE_ERROR_INVALID_VALUE, "block_table and seqlens_kv must be 4-byte aligned");
  if (block_table_stride < 1)
    return reject(FMHA_DECODE_ERROR_INVALID_VALUE, "block_table_stride must be >= 1 (got %d)", block_table_stride);
  return FMHA_DECODE_SUCCESS;
}

// Rows a block-table row can map: lengths above this get NaN, so no batch
// reads past its own row of the table.
int32_t paged_capacity(int32_t block_table_stride, int32_t page_size, int32_t max_rows) {
  const int64_t cap = (int64_t)block_table_stride * page_size;
  return cap < max_rows ? (int32_t)cap : max_rows;
}

// Groups above 8 on a paged cache run on the matrix-core short kernel when
// every length the call accepts (cap) lies within a batch's first page: one
// descriptor per wave based at that page where the wave's streams share a
// batch (num_heads_kv a multiple of the streams a wave holds), else an
// address per lane.  The kernel's layout, or -1 when rows may span pages.
int paged_mfma_layout(int32_t page_size, int32_t cap, int32_t num_heads_kv, int32_t head_dim) {
  if (cap > page_size) return -1;
  const int hpw = kWaveSize / (head_dim / 8);
  return num_heads_kv % hpw == 0 ? fmha_decode::kLayoutPaged : fmha_decode::kLayoutPagedLanes;
}

// The short kernel over a paged cache; lengths above max_rows (<= 16) give NaN.
int paged_short(void* stream, const void* Q, const void* K_cache, const void* V_cache, void* O,
                const int32_t* block_table, int32_t block_table_stride, const int32_t* seqlens_kv, int32_t page_size,
                int32_t max_rows, int32_t batch, int32_t num_heads_q, int32_t num_heads_kv, int32_t head_dim_q,
                float softmax_scale) {
  max_rows = paged_capacity(block_table_stride, page_size, max_rows);
  DecodeArgs a = base_args(Q, K_cache, V_cache, O, num_heads_q, num_heads_kv, softmax_scale);
  if (valu_kernel_group(num_heads_q / num_heads_kv) == 0) {
    const int layout = paged_mfma_layout(page_size, max_rows, num_heads_kv, head_dim_q);
    if (layout < 0)
      return reject(FMHA_DECODE_ERROR_NOT_SUPPORTED,
                    "num_heads_q / num_heads_kv above 8 (got %d) needs lengths up to %d within one page (page_size "
                    "%d) here",
                    num_heads_q / num_heads_kv, max_rows, page_size);
    a.lens = seqlens_kv;
    a.block_table = block_table;
    a.bt_stride = block_table_stride;
    a.row_stride = num_heads_kv * head_dim_q;
    a.head_stride = head_dim_q;
    a.batch_stride = (int64_t)page_size * num_heads_kv * head_dim_q;
    a.max_rows = max_rows;
    return launch_mfma(stream, layout, a, batch, head_dim_q, max_rows < kVarlenRowsHint ? max_rows : kVarlenRowsHint);
  }
  a.lens = seqlens_kv;
  a.block_table = block_table;
  a.bt_stride = block_table_stride;
  a.seqlen_uniform = log2_pow2(page_size);
  a.row_stride = num_heads_kv * head_dim_q;
  a.head_stride = head_dim_q;
  a.batch_stride = (int64_t)page_size * num_heads_kv * head_dim_q;
  a.max_rows = max_rows;
  // The paged calls' own feedback word (32 bytes past the packed calls').
  int32_t* word = feedback_word(stream);
  a.rows_feedback = word ? word + kPagedFeedbackWord : nullptr;
  return launch(stream, fmha_decode::kLayoutPaged, a, batch, head_dim_q, 0, feedback_rows16(a.rows_feedback, max_rows),
                true);
}

}  // namespace

extern "C" int fmha_decode_fwd_paged(void* stream, const void* Q, const void* K_cache, const void* V_cache, void* O,
                                     const int32_t* block_table, int32_t block_table_stride,
                                     const int32_t* seqlens_kv, int32_t page_size, int32_t batch,
                                     int32_t num_heads_q, int32_t num_heads_kv, int32_t seqlen_q,
                                     int32_t head_dim_q, int32_t head_dim_kv, float softmax_scale) {
  begin_call();
  int rc = paged_checks(Q, K_cache, V_cache, O, block_table, block_table_stride, seqlens_kv, page_size, batch,
                        num_heads_q, num_heads_kv, seqlen_q, head_dim_q, head_dim_kv, softmax_scale);
  if (rc != FMHA_DECODE_SUCCESS || batch == 0) return rc;
  return paged_short(stream, Q, K_cache, V_cache, O, block_table, block_table_stride, seqlens_kv, page_size,
                     FMHA_DECODE_MAX_SEQLEN_KV, batch, num_heads_q, num_heads_kv, head_dim_q, softmax_scale);
}

namespace {

// Query heads per KV head the long-row kernels (instantiated for 1, 2, 4, 8)
// run a call with G of them: G itself for 1, 2, 4, 8; 4 for 3 and 8 for 5-7
// (query-group padding); above 8 the next multiple of 8, as G / 8 rounded up
// launch KV heads of 8 per KV head; 0 for G < 1.
int long_row_group(int g) { return g > 8 ? (g + 7) / 8 * 8 : valu_kernel_group(g); }

// Bytes of one query-group-padded copy of Q or O ([batch, Hkv * GP, D]),
// aligned for the workspace.
size_t group_pad_bytes(int64_t batch, int hkv, int gp, int d) {
  return align_up((size_t)batch * (size_t)hkv * (size_t)gp * (size_t)d * 2);
}

}  // namespace

extern "C" size_t fmha_decode_splitkv_workspace_size(int32_t batch, int32_t num_heads_q, int32_t num_heads_kv,
                                                     int32_t max_seqlen_kv, int32_t head_dim) {
  if (batch <= 0 || num_heads_q <= 0 || num_heads_kv <= 0 || max_seqlen_kv < 0 ||
      (head_dim != 64 && head_dim != 128 && head_dim != 256))
    return 0;
  const int g = num_heads_q % num_heads_kv == 0 ? num_heads_q / num_heads_kv : 0;
  // The plan of whichever passes the layout takes: the larger of the packed
  // layout's and the short-page layout's, which can differ.
  auto plan_total = [&](int hq, int hkv, int kvg) {
    const size_t a = plan_split(batch, hq, hkv, max_seqlen_kv, head_dim, kvg, fmha_decode::kLayoutPacked).total;
    const size_t b = plan_split(batch, hq, hkv, max_seqlen_kv, head_dim, kvg, fmha_decode::kLayoutPaged).total;
    return a > b ? a : b;
  };
  if (g == 0 || valu_group(g)) return plan_total(num_heads_q, num_heads_kv, 1);
  // G > 8: ns groups of 8 per KV head on Hkv * ns launch KV heads; Q and O
  // copies unless G is a multiple of 8.  G = 3, 5-7: the copies padded to
  // 4 or 8, and the plan for Hkv * GP heads.
  const int gp = long_row_group(g);
  const int ns = g > 8 ? gp / 8 : 1;
  const size_t pad = gp == g ? 0 : 2 * group_pad_bytes(batch, num_heads_kv, gp, head_dim);
  return pad + plan_total(num_heads_kv * gp, num_heads_kv * ns, ns);
}

namespace {

// Checks shared by the split-KV entry points, then the plan and the
// layout-independent fields of the launch.  kv_span_bytes: the largest byte
// range one wave's K/V descriptor covers in the caller's layout (must stay
// below 2^30, as must one batch's scores and partial outputs).
int split_prepare(int layout, const void* Q, const void* K, const void* V, void* O, int32_t max_seqlen_kv,
                  int32_t batch, int32_t num_heads_q, int32_t num_heads_kv, int32_t kv_groups, int32_t head_dim,
                  float softmax_scale, void* workspace, size_t workspace_bytes, int64_t kv_span_bytes, SplitArgs& a) {
  const SplitPlan plan = plan_split(batch, num_heads_q, num_heads_kv, max_seqlen_kv, head_dim, kv_groups, layout);
  const int64_t padded_rows = (int64_t)plan.nblk * fmha_decode::kSplitBlockRows;
  const int64_t part_bytes = (int64_t)num_heads_q * plan.nchunks * head_dim * 4;  // one batch's partials
  if (kv_span_bytes >= (int64_t(1) << 30) || padded_rows * num_heads_q * 4 >= (int64_t(1) << 30) ||
      part_bytes >= (int64_t(1) << 30))
    return reject(FMHA_DECODE_ERROR_INVALID_VALUE, "max_seqlen_kv too large for this head count (%d)", max_seqlen_kv);
  if (!workspace) return reject(FMHA_DECODE_ERROR_INVALID_VALUE, "workspace must be non-null");
  if ((reinterpret_cast<uintptr_t>(workspace) & (kWorkspaceAlign - 1)) != 0)
    return reject(FMHA_DECODE_ERROR_INVALID_VALUE, "workspace must be 256-byte aligned");
  if (workspace_bytes < plan.total)
    return reject(FMHA_DECODE_ERROR_INVALID_VALUE, "workspace too small (%zu bytes, need %zu)", workspace_bytes,
                  plan.total);
  if (plan.units * plan.nblk > (int64_t)INT32_MAX || (int64_t)batch * num_heads_q > (int64_t)INT32_MAX)
    return reject(FMHA_DECODE_ERROR_INVALID_VALUE, "batch * heads * blocks too large");
  char* ws = static_cast<char*>(workspace);
  a = SplitArgs{};
  a.q = static_cast<const uint16_t*>(Q);
  a.k = static_cast<const uint16_t*>(K);
  a.v = static_cast<const uint16_t*>(V);
  a.o = static_cast<uint16_t*>(O);
  a.t = reinterpret_cast<float*>(ws + plan.off_t);
  a.m = reinterpret_cast<float*>(ws + plan.off_m);
  a.l = reinterpret_cast<float*>(ws + plan.off_l);
  a.ml = reinterpret_cast<float*>(ws + plan.off_ml);
  a.opart = reinterpret_cast<float*>(ws + plan.off_opart);
  a.num_heads_q = num_heads_q;
  a.num_heads_kv = num_heads_kv;
  a.kv_groups = kv_groups;
  a.units_per_batch = (int32_t)(plan.units / batch);
  a.nblk = plan.nblk;
  a.nchunks = plan.nchunks;
  a.chunk_rows = plan.chunk_rows;
  a.max_rows = max_seqlen_kv;
  a.batch = batch;
  a.scale = softmax_scale;
  return FMHA_DECODE_SUCCESS;
}

int split_launch(void* stream, int layout, const SplitArgs& a, int32_t head_dim) {
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int g = a.num_heads_q / a.num_heads_kv;
  hipError_t err;
  // Paged caches with fewer KV heads than a wave holds read through
  // per-lane addresses, so that the idle lane groups take other blocks or
  // chunks of the same heads (sub-units, as on packed caches).
  const int hpw = kWaveSize / (head_dim / 8);
  const bool lanes = 2 * a.num_heads_kv <= hpw && hpw % (2 * a.num_heads_kv) == 0;
  // The VALU long-row kernels; onepass_only: their single pass or nothing.
  auto valu = [&](bool onepass_only) -> hipError_t {
    switch (layout) {
      case fmha_decode::kLayoutPacked:
        return launch_split_layout<fmha_decode::kLayoutPacked>(a, head_dim, g, s, onepass_only);
      case fmha_decode::kLayoutStrided:
        return launch_split_layout<fmha_decode::kLayoutStrided>(a, head_dim, g, s, onepass_only);
      case fmha_decode::kLayoutPaged:
        return lanes ? launch_split_layout<fmha_decode::kLayoutPagedLanes>(a, head_dim, g, s, onepass_only)
                     : launch_split_layout<fmha_decode::kLayoutPaged>(a, head_dim, g, s, onepass_only);
      default:
        return lanes ? launch_split_layout<fmha_decode::kLayoutPagedBlockLanes>(a, head_dim, g, s, onepass_only)
                     : launch_split_layout<fmha_decode::kLayoutPagedBlock>(a, head_dim, g, s, onepass_only);
    }
  };
  if (split_on_matrix_cores(a.num_heads_q / a.num_heads_kv, a.kv_groups, layout, a.num_heads_kv, head_dim,
                            a.max_rows)) {
    // Groups of 5-8 on rows that the VALU single pass holds (enough waves,
    // a row's scores in LDS, every lane group busy) take it on rows of at
    // most 64 at D = 128, 128 at D = 256 and any it holds at D = 64 (with
    // several batches per wave: 96 at D = 128, 64 at D = 64, 128 at D =
    // 256; launch_split_dg's onepass_only): one launch against four (µs, packed,
    // D = 128 unless given, matrix-core split vs single pass: B=16384 S=24
    // Hq/Hkv 64/8 486 vs 332, B=4096 S=64 64/8 230 vs 204, B=2048 S=128
    // 225 vs 221, D=256 B=1024 S=128 48/8 246 vs 207, D=64 B=12288 S=32
    // 343 vs 165, B=4096 S=96 216 vs 201, MQA-like 8/1 D=64 B=16384 S=64
    // 87 vs 67, D=256 B=8192 S=64 135 vs 119).  Longer rows favour the
    // split: D=128 S=160 224 vs 237, D=256 S=256 222 vs 252, 8/1 S=48 124
    // vs 148.  One-row pages with per-lane lookups: launch_split_dg's rule.
    if (g == 8 && a.kv_groups == 1 && !gqa_kernel_forced("mfma")) {
      err = valu(true);
      if (err != kOnepassNotTaken) {
        if (err != hipSuccess) return reject((int)err, "kernel launch failed: %s", hipGetErrorString(err));
        return FMHA_DECODE_SUCCESS;
      }
    }
    // The matrix cores take the cache's KV heads with all of their query
    // heads (a group above 8: ns * 8 of them, the same workspace plan).
    SplitArgs m = a;
    m.num_heads_kv = fmha_decode::kv_heads_mem(a);
    m.kv_groups = 1;
    m.sub_shift = 0;
    switch (layout) {
      case fmha_decode::kLayoutPacked:
        err = launch_split_group_layout<fmha_decode::kLayoutPacked>(m, head_dim, s);
        break;
      case fmha_decode::kLayoutStrided:
        err = launch_split_group_layout<fmha_decode::kLayoutStrided>(m, head_dim, s);
        break;
      case fmha_decode::kLayoutPaged:
        err = launch_split_group_layout<fmha_decode::kLayoutPaged>(m, head_dim, s);
        break;
      default:
        err = launch_split_group_layout<fmha_decode::kLayoutPagedBlock>(m, head_dim, s);
        break;
    }
    if (err != hipSuccess) return reject((int)err, "kernel launch failed: %s", hipGetErrorString(err));
    return FMHA_DECODE_SUCCESS;
  }
  err = valu(false);
  if (err != hipSuccess) return reject((int)err, "kernel launch failed: %s", hipGetErrorString(err));
  return FMHA_DECODE_SUCCESS;
}

int split_check_workspace_args(int32_t max_seqlen_kv) {
  if (max_seqlen_kv < 0) return reject(FMHA_DECODE_ERROR_INVALID_VALUE, "max_seqlen_kv must be >= 0");
  return FMHA_DECODE_SUCCESS;
}

// Runs body(Q, O, num_heads_q, num_heads_kv, kv_groups, workspace,
// workspace_bytes) for a long-row call, whose kernels exist for G in {1, 2,
// 4, 8}.  G = 3 and 5-7 run as 4 and 8 on copies of Q and O padded to that
// many query heads per KV head, placed at the start of the workspace (the
// rest goes to the body), made and read back around it on the same stream.
// G > 8 runs as ns = ceil(G / 8) groups of 8 on one launch: the body sees
// Hkv * ns launch KV heads, launch head h reading KV head h / ns (kv_groups
// = ns), so that K and V are read once, and Q and O padded to ns * 8 query
// heads per KV head (no copies when G is a multiple of 8).
template <class BODY>
int with_group_padding(void* stream, const void* Q, void* O, int32_t batch, int32_t hq, int32_t hkv, int32_t d,
                       void* workspace, size_t workspace_bytes, BODY body) {
  const int g = hq / hkv;
  if (valu_group(g)) return body(Q, O, hq, hkv, 1, workspace, workspace_bytes);
  const int gp = long_row_group(g);
  const int ns = g > 8 ? gp / 8 : 1;
  if (gp == g) return body(Q, O, hq, hkv * ns, ns, workspace, workspace_bytes);
  const size_t pb = group_pad_bytes(batch, hkv, gp, d);
  if (!workspace) return reject(FMHA_DECODE_ERROR_INVALID_VALUE, "workspace must be non-null");
  if ((reinterpret_cast<uintptr_t>(workspace) & (kWorkspaceAlign - 1)) != 0)
    return reject(FMHA_DECODE_ERROR_INVALID_VALUE, "workspace must be 256-byte aligned");
  if (workspace_bytes < 2 * pb)
    return reject(FMHA_DECODE_ERROR_INVALID_VALUE, "workspace too small (%zu bytes) for the padded query group",
                  workspace_bytes);
  char* ws = static_cast<char*>(workspace);
  uint16_t* qp = reinterpret_cast<uint16_t*>(ws);
  uint16_t* op = reinterpret_cast<uint16_t*>(ws + pb);
  hipStream_t st = static_cast<hipStream_t>(stream);
  const uint64_t streams = (uint64_t)batch * (uint64_t)hkv;
  const uint64_t pad_chunks = streams * (uint64_t)gp * (uint64_t)(d / 8);
  // The output copy has G <= GP rows per stream: fewer blocks than the input copy.
  if ((pad_chunks + fmha_decode::kPadThreads - 1) / fmha_decode::kPadThreads > (uint64_t)INT32_MAX)
    return reject(FMHA_DECODE_ERROR_INVALID_VALUE, "batch too large (%d)", batch);
  hipError_t err = launch_pad_query_group(static_cast<const uint16_t*>(Q), qp, streams, g, gp, d, st);
  if (err != hipSuccess) return reject((int)err, "kernel launch failed: %s", hipGetErrorString(err));
  const int rc = body(qp, op, hkv * gp, hkv * ns, ns, ws + 2 * pb, workspace_bytes - 2 * pb);
  if (rc != FMHA_DECODE_SUCCESS) return rc;
  err = launch_unpad_output_group(op, static_cast<uint16_t*>(O), streams, g, gp, d, st);
  if (err != hipSuccess) return reject((int)err, "kernel launch failed: %s", hipGetErrorString(err));
  return FMHA_DECODE_SUCCESS;
}
}  // namespace

namespace {

// fmha_decode_fwd_splitkv with the workspace given; may_allocate: whether the
// short route may allocate the mean-length feedback word.
int splitkv_packed(void* stream, const void* Q, const void* K, const void* V, void* O, const int32_t* cu_seqlens_kv,
                   int32_t max_seqlen_kv, int32_t batch, int32_t num_heads_q, int32_t num_heads_kv,
                   int32_t seqlen_q, int32_t head_dim_q, int32_t head_dim_kv, float softmax_scale, void* workspace,
                   size_t workspace_bytes, bool may_allocate) {
  int rc = check_common(Q, K, V, O, batch, num_heads_q, num_heads_kv, seqlen_q, head_dim_q, head_dim_kv,
                        softmax_scale, false);
  if (rc != FMHA_DECODE_SUCCESS || batch == 0) return rc;
  if (!cu_seqlens_kv) return reject(FMHA_DECODE_ERROR_INVALID_VALUE, "cu_seqlens_kv must be non-null");
  if ((reinterpret_cast<uintptr_t>(cu_seqlens_kv) & 3u) != 0)
    return reject(FMHA_DECODE_ERROR_INVALID_VALUE, "cu_seqlens_kv must be 4-byte aligned");
  if ((rc = split_check_workspace_args(max_seqlen_kv)) != FMHA_DECODE_SUCCESS) return rc;
  const int rows_hint = max_seqlen_kv < kVarlenRowsHint ? max_seqlen_kv : kVarlenRowsHint;
  // One batch's K/V rows (up to nblk * 16) are addressed through one range.
  const int64_t row_bytes = (int64_t)num_heads_kv * head_dim_q * 2;
  const int64_t padded_rows = ((int64_t)max_seqlen_kv + 15) / 16 * 16;
  const int64_t span = (padded_rows > 16 ? padded_rows : 16) * row_bytes;
  if (max_seqlen_kv <= FMHA_DECODE_MAX_SEQLEN_KV) {
    // Rows that fit the short kernels take them (same numerics, lengths above
    // max_seqlen_kv give NaN there too); the workspace is checked but unused.
    DecodeArgs d = base_args(Q, K, V, O, num_heads_q, num_heads_kv, softmax_scale);
    d.lens = cu_seqlens_kv;
    d.row_stride = num_heads_kv * head_dim_q;
    d.head_stride = head_dim_q;
    d.max_rows = max_seqlen_kv;
    const Numerics numerics = default_numerics(num_heads_q / num_heads_kv);
    if (numerics != Numerics::kExact && use_mfma_kernel(num_heads_q / num_heads_kv))
      return launch_mfma(stream, fmha_decode::kLayoutPacked, d, batch, head_dim_q, rows_hint);
    SplitArgs unused;
    rc = split_prepare(fmha_decode::kLayoutPacked, Q, K, V, O, max_seqlen_kv, batch, num_heads_q, num_heads_kv, 1,
                       head_dim_q, softmax_scale, workspace, workspace_bytes, span, unused);
    if (rc != FMHA_DECODE_SUCCESS) return rc;
    d.rows_feedback = feedback_word(stream, may_allocate);
    return launch(stream, fmha_decode::kLayoutPacked, d, batch, head_dim_q, 0,
                  feedback_rows16(d.rows_feedback, max_seqlen_kv), true, numerics);
  }
  return with_group_padding(
      stream, Q, O, batch, num_heads_q, num_heads_kv, head_dim_q, workspace, workspace_bytes,
      [&](const void* q, void* o, int32_t hq, int32_t hkv, int32_t kvg, void* ws, size_t ws_bytes) {
        SplitArgs a;
        int rc2 = split_prepare(fmha_decode::kLayoutPacked, q, K, V, o, max_seqlen_kv, batch, hq, hkv, kvg,
                                head_dim_q, softmax_scale, ws, ws_bytes, span, a);
        if (rc2 != FMHA_DECODE_SUCCESS) return rc2;
        a.cu = cu_seqlens_kv;
        a.len_mode = fmha_decode::kLenCu;
        return split_launch(stream, fmha_decode::kLayoutPacked, a, head_dim_q);
      });
}

// Scratch of fmha_decode_fwd_splitkv_noalloc: the split-KV workspace as a
// device array, one copy per GPU (each holds it from load until the process
// ends).  Host code never uses the array's name as an address: the device
// address comes from hipGetSymbolAddress, once per device.
constexpr size_t kNoAllocScratchBytes = (size_t)FMHA_DECODE_NOALLOC_SCRATCH_BYTES;
static __device__ __align__(256) unsigned char scratch[kNoAllocScratchBytes];
std::atomic<void*> g_scratch[kMaxFeedbackDevices];
std::mutex g_scratch_mutex;

// This device's scratch address, or null (detail set) when it cannot be had.
void* scratch_address(int* rc) {
  int dev = 0;
  hipError_t err = hipGetDevice(&dev);
  if (err != hipSuccess) {
    *rc = reject((int)err, "hipGetDevice failed: %s", hipGetErrorString(err));
    return nullptr;
  }
  if (dev < 0 || dev >= kMaxFeedbackDevices) {
    *rc = reject(FMHA_DECODE_ERROR_NOT_SUPPORTED, "device %d is beyond the %d this library serves", dev,
                 kMaxFeedbackDevices);
    return nullptr;
  }
  void* p = g_scratch[dev].load(std::memory_order_acquire);
  if (p) return p;
  std::lock_guard<std::mutex> lock(g_scratch_mutex);
  p = g_scratch[dev].load(std::memory_order_acquire);
  if (p) return p;
  err = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
  if (err != hipSuccess || p == nullptr) {
    *rc = reject(err != hipSuccess ? (int)err : FMHA_DECODE_ERROR_NOT_SUPPORTED,
                 "no device address for the scratch array: %s", hipGetErrorString(err));
    return nullptr;
  }
  g_scratch[dev].store(p, std::memory_order_release);
  return p;
}

}  // namespace

extern "C" int fmha_decode_fwd_splitkv(void* stream, const void* Q, const void* K, const void* V, void* O,
                                       const int32_t* cu_seqlens_kv, int32_t max_seqlen_kv, int32_t batch,
                                       int32_t num_heads_q, int32_t num_heads_kv, int32_t seqlen_q,
                                       int32_t head_dim_q, int32_t head_dim_kv, float softmax_scale,
                                       void* workspace, size_t workspace_bytes) {
  begin_call();
  return splitkv_packed(stream, Q, K, V, O, cu_seqlens_kv, max_seqlen_kv, batch, num_heads_q, num_heads_kv,
                        seqlen_q, head_dim_q, head_dim_kv, softmax_scale, workspace, workspace_bytes, true);
}

extern "C" int fmha_decode_fwd_splitkv_noalloc(void* stream, const void* Q, const void* K, const void* V, void* O,
                                               const int32_t* cu_seqlens_kv, int32_t max_seqlen_kv, int32_t batch,
                                               int32_t num_heads_q, int32_t num_heads_kv, int32_t seqlen_q,
                                               int32_t head_dim_q, int32_t head_dim_kv, float softmax_scale) {
  begin_call();
  int rc = check_common(Q, K, V, O, batch, num_heads_q, num_heads_kv, seqlen_q, head_dim_q, head_dim_kv,
                        softmax_scale, false);
  if (rc != FMHA_DECODE_SUCCESS || batch == 0) return rc;
  if ((rc = split_check_workspace_args(max_seqlen_kv)) != FMHA_DECODE_SUCCESS) return rc;
  if (!cu_seqlens_kv) return reject(FMHA_DECODE_ERROR_INVALID_VALUE, "cu_seqlens_kv must be non-null");
  {
    const size_t need =
        fmha_decode_splitkv_workspace_size(batch, num_heads_q, num_heads_kv, max_seqlen_kv, head_dim_q);
    if (need > kNoAllocScratchBytes)
      return reject(FMHA_DECODE_ERROR_INVALID_VALUE,
                    "this call needs %zu bytes of scratch; fmha_decode_fwd_splitkv_noalloc has %zu (use "
                    "fmha_decode_fwd_splitkv with a workspace)",
                    need, kNoAllocScratchBytes);
  }
  void* ws = scratch_address(&rc);
  if (ws == nullptr) return rc;
  return splitkv_packed(stream, Q, K, V, O, cu_seqlens_kv, max_seqlen_kv, batch, num_heads_q, num_heads_kv,
                        seqlen_q, head_dim_q, head_dim_kv, softmax_scale, ws, kNoAllocScratchBytes, false);
}

extern "C" int fmha_decode_fwd_splitkv_strided(void* stream, const void* Q, const void* K, const void* V, void* O,
                                               const int32_t* seqlens_kv, int32_t max_seqlen_kv,
                                               int64_t kv_batch_stride, int64_t kv_row_stride,
                                               int64_t kv_head_stride, int32_t batch, int32_t num_heads_q,
                                               int32_t num_heads_kv, int32_t seqlen_q, int32_t head_dim_q,
                                               int32_t head_dim_kv, float softmax_scale, void* workspace,
                                               size_t workspace_bytes) {
  begin_call();
  int rc = split_check_workspace_args(max_seqlen_kv);
  if (rc != FMHA_DECODE_SUCCESS) return rc;
  if (max_seqlen_kv <= FMHA_DECODE_MAX_SEQLEN_KV)
    return fmha_decode_fwd_strided(stream, Q, K, V, O, seqlens_kv, max_seqlen_kv, kv_batch_stride, kv_row_stride,
                                   kv_head_stride, batch, num_heads_q, num_heads_kv, seqlen_q, head_dim_q,
                                   head_dim_kv, softmax_scale);
  rc = check_common(Q, K, V, O, batch, num_heads_q, num_heads_kv, seqlen_q, head_dim_q, head_dim_kv, softmax_scale,
                    false);
  if (rc != FMHA_DECODE_SUCCESS || batch == 0) return rc;
  if (kv_batch_stride < 0 || kv_row_stride < 0 || kv_head_stride < 0)
    return reject(FMHA_DECODE_ERROR_INVALID_VALUE, "K/V strides must be >= 0");
  if ((kv_batch_stride | kv_row_stride | kv_head_stride) & 7)
    return reject(FMHA_DECODE_ERROR_INVALID_VALUE, "K/V strides must be multiples of 8 elements (16 bytes)");
  if (seqlens_kv && (reinterpret_cast<uintptr_t>(seqlens_kv) & 3u) != 0)
    return reject(FMHA_DECODE_ERROR_INVALID_VALUE, "seqlens_kv must be 4-byte aligned");
  // One batch's rows and heads are addressed through one range.
  const int64_t extent =
      ((int64_t)(max_seqlen_kv - 1) * kv_row_stride + (int64_t)(num_heads_kv - 1) * kv_head_stride + head_dim_q) * 2;
  if (extent >= (int64_t(1) << 30))
    return reject(FMHA_DECODE_ERROR_INVALID_VALUE, "one batch's K/V span exceeds 1 GiB");
  return with_group_padding(
      stream, Q, O, batch, num_heads_q, num_heads_kv, head_dim_q, workspace, workspace_bytes,
      [&](const void* q, void* o, int32_t hq, int32_t hkv, int32_t kvg, void* ws, size_t ws_bytes) {
        SplitArgs a;
        int rc2 = split_prepare(fmha_decode::kLayoutStrided, q, K, V, o, max_seqlen_kv, batch, hq, hkv, kvg,
                                head_dim_q, softmax_scale, ws, ws_bytes, extent, a);
        if (rc2 != FMHA_DECODE_SUCCESS) return rc2;
        a.cu = seqlens_kv;
        a.len_mode = seqlens_kv ? fmha_decode::kLenArray : fmha_decode::kLenUniform;
        a.batch_stride = kv_batch_stride;
        a.row_stride = (int32_t)kv_row_stride;
        a.head_stride = (int32_t)kv_head_stride;
        return split_launch(stream, fmha_decode::kLayoutStrided, a, head_dim_q);
      });
}

extern "C" int fmha_decode_fwd_splitkv_paged(void* stream, const void* Q, const void* K_cache, const void* V_cache,
                                             void* O, const int32_t* block_table, int32_t block_table_stride,
                                             const int32_t* seqlens_kv, int32_t page_size, int32_t max_seqlen_kv,
                                             int32_t batch, int32_t num_heads_q, int32_t num_heads_kv,
                                             int32_t seqlen_q, int32_t head_dim_q, int32_t head_dim_kv,
                                             float softmax_scale, void* workspace, size_t workspace_bytes) {
  begin_call();
  int rc = split_check_workspace_args(max_seqlen_kv);
  if (rc != FMHA_DECODE_SUCCESS) return rc;
  rc = paged_checks(Q, K_cache, V_cache, O, block_table, block_table_stride, seqlens_kv, page_size, batch,
                    num_heads_q, num_heads_kv, seqlen_q, head_dim_q, head_dim_kv, softmax_scale);
  if (rc != FMHA_DECODE_SUCCESS || batch == 0) return rc;
  max_seqlen_kv = paged_capacity(block_table_stride, page_size, max_seqlen_kv);
  // Short rows take the short kernels directly: the VALU paged kernel for G
  // <= 8, the matrix-core one above where rows lie within a batch's first
  // page (paged_mfma_layout); otherwise they go through the split kernels
  // below like longer rows (one 16-row block, one chunk).  µs, B=7812 Hq/Hkv
  // 128/8 S=16 D=128 on 16-row pages: split 331.0, matrix-core short kernel
  // 147.4 (packed 149.5).
  if (max_seqlen_kv <= FMHA_DECODE_MAX_SEQLEN_KV &&
      (valu_kernel_group(num_heads_q / num_heads_kv) != 0 ||
       paged_mfma_layout(page_size, max_seqlen_kv, num_heads_kv, head_dim_q) >= 0))
    return paged_short(stream, Q, K_cache, V_cache, O, block_table, block_table_stride, seqlens_kv, page_size,
                       max_seqlen_kv, batch, num_heads_q, num_heads_kv, head_dim_q, softmax_scale);
  // A sub-block's range covers at most 16 rows of one page.
  const int64_t row_bytes = (int64_t)num_heads_kv * head_dim_q * 2;
  const int page_layout = page_size >= 16 ? fmha_decode::kLayoutPagedBlock : fmha_decode::kLayoutPaged;
  return with_group_padding(
      stream, Q, O, batch, num_heads_q, num_heads_kv, head_dim_q, workspace, workspace_bytes,
      [&](const void* q, void* o, int32_t hq, int32_t hkv, int32_t kvg, void* ws, size_t ws_bytes) {
        SplitArgs a;
        int rc2 = split_prepare(page_layout, q, K_cache, V_cache, o, max_seqlen_kv, batch, hq, hkv, kvg, head_dim_q,
                                softmax_scale, ws, ws_bytes, 16 * row_bytes, a);
        if (rc2 != FMHA_DECODE_SUCCESS) return rc2;
        a.cu = seqlens_kv;
        a.len_mode = fmha_decode::kLenArray;
        a.block_table = block_table;
        a.bt_stride = block_table_stride;
        a.page_shift = log2_pow2(page_size);
        a.batch_stride = (int64_t)page_size * num_heads_kv * head_dim_q;
        return split_launch(stream, page_layout, a, head_dim_q);
      });
}

extern "C" const char* fmha_decode_error_string(int code) {
  switch (code) {
    case FMHA_DECODE_SUCCESS: return "success";
    case FMHA_DECODE_ERROR_INVALID_VALUE: return "invalid argument";
    case FMHA_DECODE_ERROR_NOT_SUPPORTED: return "configuration not supported";
    default: return hipGetErrorString(static_cast<hipError_t>(code));
  }
}

extern "C" const char* fmha_decode_last_error_detail(void) { return g_detail; }

extern "C" const char* fmha_decode_last_plan(void) { return fmha_decode::host::g_plan; }

extern "C" int fmha_decode_version(void) { return 100; }
