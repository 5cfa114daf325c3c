// fmha_oracle.cpp -- CPU oracle for the decode-attention path.
//
// TEST INFRASTRUCTURE ONLY.  Nothing in the product (fmha_amd/, include/)
// links, loads or calls this file.  Only tests/, __graft_entry__.smoke() and
// bench.py's cpu_baseline leg use it, and only as the checker or as the timed
// CPU baseline.
//
// It restates, in new code, the arithmetic of the reference's CPU validation
// loop (fmha_host.cpp:169-245) and its length generator (fmha_host.cpp:58-82),
// with two deliberate changes:
//   * KV head = query head / (Hq / Hkv) (grouped-query attention); the
//     reference indexes K/V with the query head (fmha_host.cpp:190-192,
//     :234-236), which is only meaningful when Hq == Hkv;
//   * 64-bit sizes everywhere (the reference sizes tensors in int,
//     fmha_host.cpp:85-93).
// For Hq == Hkv and scale == 1.0f/sqrtf(D) the bf16-P mode is bit-identical to
// the reference loop; tests/test_oracle.py checks that against the
// reference's own do_validation compiled from /root/reference (oracle/_ref).
//
// Pinning (see tests/test_oracle.py): bit-exact
// against the reference do_validation (MHA); S=1 known answer O = fp16(V);
// Q=0 closed form P = bf16(1/S); one dominant key -> O = fp16(V_j); GQA equal
// to MHA on head-repeated K/V; fp64 mode against torch's float64
// scaled_dot_product_attention; fp16/bf16 rounding against numpy/torch on
// every bf16 bit pattern; seqlen generator against the reference's own
// generate_seqlens_kv.  No function is left parity-unpinned.
#include <cmath>
#include <cstdint>
#include <cstring>
#include <random>
#include <vector>

// Planted mistakes for the oracle's own mutation tests: tests/test_oracle.py
// compiles copies of this file with ORACLE_MUTANT set to 1..4 and checks
// that its long-row checks reject every one.  The oracle the tests use is
// built without it (0: no mistake).
//   1: rows 16 and beyond score against the previous row's K;
//   2: P.V drops the last row of rows longer than 16;
//   3: the max runs over the first 16 rows only;
//   4: the sum of exponentials runs over the first 16 rows only.
#ifndef ORACLE_MUTANT
#define ORACLE_MUTANT 0
#endif

namespace {

inline float bf16_to_f32(uint16_t h) {
  uint32_t u = (uint32_t)h << 16;
  float f;
  std::memcpy(&f, &u, 4);
  return f;
}

inline uint32_t f32_bits(float f) {
  uint32_t u;
  std::memcpy(&u, &f, 4);
  return u;
}

// float -> bf16, round to nearest even (what static_cast<__bf16> does for the
// reference at fmha_host.cpp:225).
inline uint16_t f32_to_bf16(float f) {
  uint32_t u = f32_bits(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x0040u);  // quiet NaN
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

// float -> IEEE binary16, round to nearest even, with subnormals and overflow
// to infinity (what static_cast<_Float16> does at fmha_host.cpp:243).
inline uint16_t f32_to_f16(float f) {
  const uint32_t u = f32_bits(f);
  const uint32_t sign = (u >> 16) & 0x8000u;
  const uint32_t au = u & 0x7fffffffu;
  if (au > 0x7f800000u) return (uint16_t)(sign | 0x7e00u | ((au >> 13) & 0x3ffu));  // NaN
  if (au >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u);  // rounds to >= 65520: inf
  const int exp = (int)(au >> 23) - 127;
  if (exp >= -14) {
    // normal half: keep 10 mantissa bits, RNE on the 13 dropped bits
    uint32_t mant = au & 0x7fffffu;
    uint32_t h = ((uint32_t)(exp + 15) << 10) | (mant >> 13);
    const uint32_t rem = mant & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) h += 1;  // carry may bump the exponent: correct
    return (uint16_t)(sign | h);
  }
  if (exp < -25) return (uint16_t)sign;  // below half of the smallest subnormal
  // subnormal half: h = round(|f| * 2^24).  With the 24-bit significand
  // M (|f| = M * 2^(exp-23)), |f| * 2^24 = M * 2^(exp+1) = M >> shift.
  const uint32_t mant = (au & 0x7fffffu) | 0x800000u;
  const int shift = -exp - 1;  // 14..24
  const uint32_t q = mant >> shift;
  const uint32_t rem = mant & ((1u << shift) - 1u);
  const uint32_t half = 1u << (shift - 1);
  uint32_t h = q;
  if (rem > half || (rem == half && (q & 1u))) h += 1;
  return (uint16_t)(sign | h);
}

// The float nearest exp(x): exp evaluated in double (within one double ulp)
// and rounded once, which gives the nearest float except when the double
// result lies within an ulp of a float rounding midpoint.
float exp_nearest(float x) { return (float)std::exp((double)x); }

// One (batch, query head) of the reference loop, fmha_host.cpp:179-244, with
// the KV head chosen by the caller.  p_mode 0: weights rounded to bf16
// (fmha_host.cpp:225); 1: weights kept in fp32 (the semantics of
// fmha_vectorized_fma_kernel.hpp:256); 2: as 0, with every exponential the
// float nearest exp(x) (evaluated in double, rounded once) in place of the
// C library's expf, which misses the nearest float on a few arguments in
// ten thousand (the loop the library's exact path restates).
void head_f32(const uint16_t* q, const uint16_t* k, const uint16_t* v, int64_t kv_stride, int S, int D, float scale,
              int p_mode, uint16_t* o, float* slack, double slack_eps) {
  // The reference sizes these arrays for 16 rows (fmha_host.cpp:164, :215);
  // longer rows extend the same loop.
  thread_local std::vector<float> scores_buf, p_buf, jump_buf;
  scores_buf.resize(S > 16 ? S : 16);
  p_buf.resize(S > 16 ? S : 16);
  jump_buf.resize(S > 16 ? S : 16);
  float* scores = scores_buf.data();
  const int S16 = S < 16 ? S : 16;
  (void)S16;
  for (int s = 0; s < S; s++) {
    float sum = 0;
    const uint16_t* kr = k + (int64_t)((ORACLE_MUTANT == 1 && s >= 16) ? s - 1 : s) * kv_stride;
    for (int d = 0; d < D; d++) sum += bf16_to_f32(q[d]) * bf16_to_f32(kr[d]);
    scores[s] = sum;
  }
  for (int s = 0; s < S; s++) scores[s] *= scale;
  float maxv = -INFINITY;
  for (int s = 0; s < (ORACLE_MUTANT == 3 ? S16 : S); s++) maxv = fmaxf(maxv, scores[s]);
  auto ex = [p_mode](float x) { return p_mode == 2 ? exp_nearest(x) : expf(x); };
  float sum_exp = 0.0f;
  for (int s = 0; s < (ORACLE_MUTANT == 4 ? S16 : S); s++) sum_exp += ex(scores[s] - maxv);
  float* p = p_buf.data();
  float* jump = jump_buf.data();
  // How far this loop's own float32 weights may sit from the exact ones:
  // the largest score error (against a float64 dot product) counts twice
  // (the weight and its normaliser), plus the relative error of the float32
  // sum of exponentials.  Another float32 implementation summing in another
  // order is uncertain by about as much, so a weight within
  // eps = max(slack_eps, 4 * that) of a bf16 rounding midpoint may round
  // either way there.
  // A negative slack_eps asks for the fixed half-width |slack_eps| instead.
  double eps = slack_eps < 0 ? -slack_eps : slack_eps;
  if (slack && slack_eps > 0) {
    double dt = 0.0, l64 = 0.0;
    for (int s = 0; s < S; s++) {
      double acc = 0.0;
      const uint16_t* kr = k + (int64_t)s * kv_stride;
      for (int d = 0; d < D; d++) acc += (double)bf16_to_f32(q[d]) * (double)bf16_to_f32(kr[d]);
      dt = fmax(dt, fabs(acc * (double)scale - (double)scores[s]));
      l64 += exp((double)scores[s] - (double)maxv);
    }
    const double dl = S > 0 ? fabs((double)sum_exp - l64) / l64 : 0.0;
    eps = fmax(slack_eps, 4.0 * (2.0 * dt + dl));
  }
  for (int s = 0; s < S; s++) {
    const float pf = ex(scores[s] - maxv) / sum_exp;
    p[s] = p_mode != 1 ? bf16_to_f32(f32_to_bf16(pf)) : pf;
    // Size of the bf16 rounding step reachable by a relative perturbation of
    // pf by eps: non-zero only near a rounding midpoint.
    if (slack) {
      const float up = bf16_to_f32(f32_to_bf16((float)(pf * (1.0 + eps))));
      const float dn = bf16_to_f32(f32_to_bf16((float)(pf * (1.0 - eps))));
      jump[s] = fabsf(up - dn);
    }
  }
  for (int d = 0; d < D; d++) {
    float sum = 0;
    float sl = 0;
    for (int s = 0; s < ((ORACLE_MUTANT == 2 && S > 16) ? S - 1 : S); s++) {
      const float vv = bf16_to_f32(v[(int64_t)s * kv_stride + d]);
      sum += p[s] * vv;
      if (slack) sl += jump[s] * fabsf(vv);
    }
    o[d] = f32_to_f16(sum);
    if (slack) slack[d] = sl;
  }
}

// Same head in float64 throughout (no intermediate rounding), for reference
// "truth" comparisons.  With bound non-null, also a per-element bound on
// |o - t| that any bf16-weight implementation in float32 meets without tie
// slack (the bf16 rounding of a weight may go either way there):
//     2^-8 * M              each weight rounded to bf16 (unit roundoff 2^-8;
//                           sum_j p_j |V_jd| <= M = max_j |V_jd|)
//   + 2 * dt * M            float32 scores: the weight and its normaliser
//                           move by at most dt relative each
//   + 2^-10 * |t|           the fp16 rounding of the output (2^-11), doubled
//   + 1e-5 * (1 + M)        float32 sums of the output and the weights
// with dt = scale * D * 2^-23 * max_j sum_d |q_d k_jd|: a float32 dot product
// of D terms, in any order, is within D * 2^-24 * sum |terms| of the exact
// one (doubled here).
void head_f64(const uint16_t* q, const uint16_t* k, const uint16_t* v, int64_t kv_stride, int S, int D, double scale,
              double* o, double* bound) {
  thread_local std::vector<double> t_buf;
  t_buf.resize(S > 16 ? S : 16);
  double* t = t_buf.data();
  double m = -INFINITY;
  for (int s = 0; s < S; s++) {
    double sum = 0;
    const uint16_t* kr = k + (int64_t)s * kv_stride;
    for (int d = 0; d < D; d++) sum += (double)bf16_to_f32(q[d]) * (double)bf16_to_f32(kr[d]);
    t[s] = sum * scale;
    m = t[s] > m ? t[s] : m;
  }
  double z = 0;
  for (int s = 0; s < S; s++) z += exp(t[s] - m);
  for (int s = 0; s < S; s++) t[s] = exp(t[s] - m) / z;  // the weights
  for (int d = 0; d < D; d++) {
    double acc = 0;
    for (int s = 0; s < S; s++) acc += t[s] * (double)bf16_to_f32(v[(int64_t)s * kv_stride + d]);
    o[d] = S > 0 ? acc : 0.0;
  }
  if (bound) {
    double dots = 0.0;
    for (int s = 0; s < S; s++) {
      double a = 0.0;
      const uint16_t* kr = k + (int64_t)s * kv_stride;
      for (int d = 0; d < D; d++) a += fabs((double)bf16_to_f32(q[d]) * (double)bf16_to_f32(kr[d]));
      dots = a > dots ? a : dots;
    }
    const double dt = scale * D * ldexp(1.0, -23) * dots;
    for (int d = 0; d < D; d++) {
      double M = 0.0;
      for (int s = 0; s < S; s++) M = fmax(M, fabs((double)bf16_to_f32(v[(int64_t)s * kv_stride + d])));
      bound[d] = ldexp(1.0, -8) * M + 2.0 * dt * M + 1e-5 * (1.0 + M) + ldexp(1.0, -10) * fabs(o[d]);
    }
  }
}

}  // namespace

extern "C" {

// The exponential of p_mode 2 over x[0..n), for its own test.
void oracle_exp_nearest(const float* x, int64_t n, float* out) {
  for (int64_t i = 0; i < n; i++) out[i] = exp_nearest(x[i]);
}

// Decode attention over a packed batch (layouts as include/fmha_decode.h).
// cu: [batch+1] row offsets.  p_mode 0 = bf16 weights (reference CPU loop),
// 1 = fp32 weights, 2 = bf16 weights from nearest-float exponentials.  o: fp16 bits [batch, hq, d].  slack: optional float
// [batch, hq, d] (see head_f32; slack_eps is its floor, or with a negative
// value the fixed half-width -slack_eps).  Returns 0, or -1
// for a length outside
// [0, max_seqlen] or bad arguments (nothing is written then).  The
// reference's bound is 16; longer rows run the same loop.
int oracle_decode(const uint16_t* q, const uint16_t* k, const uint16_t* v, const int32_t* cu, int64_t batch, int hq,
                  int hkv, int d, float scale, int p_mode, uint16_t* o, float* slack, double slack_eps,
                  int nthreads, int max_seqlen) {
  if (batch < 0 || hq <= 0 || hkv <= 0 || hq % hkv != 0 || d <= 0 || max_seqlen < 0) return -1;
  if (p_mode < 0 || p_mode > 2) return -1;
  for (int64_t b = 0; b < batch; b++) {
    const int S = cu[b + 1] - cu[b];
    if (S < 0 || S > max_seqlen) return -1;
  }
  const int g = hq / hkv;
  const int64_t kv_stride = (int64_t)hkv * d;
#pragma omp parallel for schedule(static) num_threads(nthreads > 0 ? nthreads : 1)
  for (int64_t b = 0; b < batch; b++) {
    const int S = cu[b + 1] - cu[b];
    const int64_t row0 = cu[b];
    for (int h = 0; h < hq; h++) {
      const int hk = h / g;
      const int64_t qo = ((int64_t)b * hq + h) * d;
      head_f32(q + qo, k + row0 * kv_stride + (int64_t)hk * d, v + row0 * kv_stride + (int64_t)hk * d, kv_stride, S,
               d, scale, p_mode, o + qo, slack ? slack + qo : nullptr, slack_eps);
    }
  }
  return 0;
}

// Float64 decode attention (no rounding anywhere but the bf16 inputs);
// bound (nullable, [batch, hq, d]): see head_f64.
int oracle_decode_f64(const uint16_t* q, const uint16_t* k, const uint16_t* v, const int32_t* cu, int64_t batch,
                      int hq, int hkv, int d, double scale, double* o, int nthreads, int max_seqlen, double* bound) {
  if (batch < 0 || hq <= 0 || hkv <= 0 || hq % hkv != 0 || d <= 0 || max_seqlen < 0) return -1;
  for (int64_t b = 0; b < batch; b++) {
    const int S = cu[b + 1] - cu[b];
    if (S < 0 || S > max_seqlen) return -1;
  }
  const int g = hq / hkv;
  const int64_t kv_stride = (int64_t)hkv * d;
#pragma omp parallel for schedule(static) num_threads(nthreads > 0 ? nthreads : 1)
  for (int64_t b = 0; b < batch; b++) {
    const int S = cu[b + 1] - cu[b];
    const int64_t row0 = cu[b];
    for (int h = 0; h < hq; h++) {
      const int hk = h / g;
      const int64_t qo = ((int64_t)b * hq + h) * d;
      head_f64(q + qo, k + row0 * kv_stride + (int64_t)hk * d, v + row0 * kv_stride + (int64_t)hk * d, kv_stride, S,
               d, scale, o + qo, bound ? bound + qo : nullptr);
    }
  }
  return 0;
}

// Per-element gate: element i passes if |o-r| <= atol + rtol*|r| + slack[i]
// (slack may be null).  stats[0..8] = {fails, slack-affected elements,
// max |o-r|, max |o-r|/|r| (r != 0), fails under the reference rule
// |o-r| > 1e-2 + 1e-2|r| (fmha_host.cpp:260) with the same slack, non-finite
// outputs, first failing index (or -1), count, fails under the reference
// rule without slack}.
void oracle_compare(const uint16_t* o, const uint16_t* r, const float* slack, int64_t n, double atol, double rtol,
                    double* stats) {
  int64_t fails = 0, slacked = 0, ref_fails = 0, ref_fails_raw = 0, nonfinite = 0, first = -1;
  double max_abs = 0, max_rel = 0;
  for (int64_t i = 0; i < n; i++) {
    // fp16 -> double via the bit pattern
    auto h2d = [](uint16_t h) -> double {
      const int e = (h >> 10) & 0x1f;
      const int m = h & 0x3ff;
      const double s = (h & 0x8000) ? -1.0 : 1.0;
      if (e == 0x1f) return m ? NAN : s * INFINITY;
      if (e == 0) return s * ldexp((double)m, -24);
      return s * ldexp((double)(m | 0x400), e - 25);
    };
    const double ov = h2d(o[i]);
    const double rv = h2d(r[i]);
    if (!std::isfinite(ov)) nonfinite++;
    const double err = std::fabs(ov - rv);
    const double sl = slack ? (double)slack[i] : 0.0;
    if (sl > 0) slacked++;
    const bool ok = err <= atol + rtol * std::fabs(rv) + sl;  // false for NaN
    if (!ok) {
      if (first < 0) first = i;
      fails++;
    }
    if (!(err <= 1e-2 + 1e-2 * std::fabs(rv) + sl)) ref_fails++;
    if (!(err <= 1e-2 + 1e-2 * std::fabs(rv))) ref_fails_raw++;
    if (err > max_abs || std::isnan(err)) max_abs = std::isnan(err) ? INFINITY : err;
    if (rv != 0 && err / std::fabs(rv) > max_rel) max_rel = err / std::fabs(rv);
  }
  stats[0] = (double)fails;
  stats[1] = (double)slacked;
  stats[2] = max_abs;
  stats[3] = max_rel;
  stats[4] = (double)ref_fails;
  stats[5] = (double)nonfinite;
  stats[6] = (double)first;
  stats[7] = (double)n;
  stats[8] = (double)ref_fails_raw;
}

// Poisson(lambda) lengths rejected outside [2, max_seqlen], mt19937(seed),
// as fmha_host.cpp:58-72 (libstdc++'s poisson_distribution, so the sequence
// is the reference's for the same seed).
void oracle_generate_seqlens(int64_t batch, int max_seqlen, double lambda, uint32_t seed, int32_t* out) {
  std::mt19937 gen(seed);
  std::poisson_distribution<int> dist(lambda);
  for (int64_t i = 0; i < batch; i++) {
    int len;
    do {
      len = dist(gen);
    } while (len < 2 || len > max_seqlen);
    out[i] = len;
  }
}

// Rounding helpers exposed for their own tests.
void oracle_f32_to_bf16(const float* x, int64_t n, uint16_t* out) {
  for (int64_t i = 0; i < n; i++) out[i] = f32_to_bf16(x[i]);
}
void oracle_f32_to_f16(const float* x, int64_t n, uint16_t* out) {
  for (int64_t i = 0; i < n; i++) out[i] = f32_to_f16(x[i]);
}

}  // extern "C"
