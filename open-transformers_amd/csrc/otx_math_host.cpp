// Host build of the kernels' exp / log (the same source as the device code),
// so that CPU tests can check them against the oracle without a GPU.
#include <cmath>
#include <omp.h>
#include "otx_math.h"

extern "C" float otx_host_expf(float x) { return otx_expf(x); }
extern "C" float otx_host_logf(float x) { return otx_logf(x); }
extern "C" uint16_t otx_host_f32_to_bf16(float x) { return otx_f32_to_bf16(x); }
extern "C" float otx_host_div_rn(float a, float b) { return otx_div_rn(a, b); }

extern "C" float otx_host_expf_fast(float x, int* slow) { return otx_expf_fast(x, otx_exp2_tab64, slow); }

// The biased table the softmax exp reads (the device copies the same entries into LDS).
static const struct Tab256Biased {
  double v[OTX_EXP_LE0_TAB_N];
  Tab256Biased() {
    for (int j = 0; j < OTX_EXP_LE0_TAB_N; j++) v[j] = otx_exp2_tab256_biased(j);
  }
} tab256b;

extern "C" float otx_host_expf_fast_le0(float x) { return otx_expf_fast_le0(x, tab256b.v); }
extern "C" double otx_host_exp2_tab256(int j) { return otx_exp2_tab256[j & 255]; }


// Correctly rounded binary32 exp for the exhaustive checks below: glibc's
// binary64 exp (error below one binary64 ulp) decides the rounding unless it
// lies within 2^-45 (relative) of a binary32 rounding boundary; those inputs
// take otx_expf.  An independent reference, and a fast one.
static float exp_ref(float x) {
  const double y = std::exp((double)x);
  const double e = y * 0x1p-45;
  const float lo = (float)(y - e), hi = (float)(y + e);
  if (otx_f2u(lo) == otx_f2u(hi)) return lo;
  return otx_expf(x);
}

// Both kernel exp paths over the bit patterns [lo, lo + count) in one pass:
// out[0] / out[1] = mismatches / deferred inputs of otx_expf_fast (inputs
// <= 88), out[2] = mismatches of otx_expf_fast_le0 (inputs <= 0 or -inf; it
// defers nothing) and out[3] = the number of inputs it was compared on.  NaN
// inputs are not compared.
extern "C" void otx_host_exp_paths_check(uint64_t lo, uint64_t count, uint64_t* out) {
  uint64_t bf = 0, sf = 0, bl = 0, nl = 0;
#pragma omp parallel for schedule(dynamic, 65536) reduction(+ : bf, sf, bl, nl) num_threads(omp_get_num_procs())
  for (int64_t i = 0; i < (int64_t)count; i++) {
    const float x = otx_u2f((uint32_t)(lo + (uint64_t)i));
    const bool le0 = x <= 0.0f;
    if (!(x <= 88.0f) && !(x != x)) continue;  // outside both paths' domains
    int slow_f;
    const float f = otx_expf_fast(x, otx_exp2_tab64, &slow_f);
    sf += slow_f;
    if (x != x || (slow_f && !le0)) continue;
    const uint32_t r = otx_f2u(exp_ref(x));
    if (!slow_f && otx_f2u(f) != r) bf++;
    if (le0) {
      nl++;
      if (otx_f2u(otx_expf_fast_le0(x, tab256b.v)) != r) bl++;
    }
  }
  out[0] = bf; out[1] = sf; out[2] = bl; out[3] = nl;
}

extern "C" float otx_host_rsqrtf(float x) { return otx_rsqrtf(x); }

extern "C" float otx_host_div_by_recip(float a, float b) { return otx_div_by_recip(a, otx_recip64(b)); }
extern "C" float otx_host_div_by_recip_checked(float a, float b) {
  return otx_div_by_recip_checked(a, otx_recip64(b), b);
}

// otx_div_by_recip_checked(a, otx_recip64(b), b) against otx_div_rn(a, b) on n
// pseudo-random pairs whose quotients fall below the normal range or near its
// edge: a subnormal or small normal, b in [1, 2^20) with a significand of up to
// 12 bits (so that exact subnormal midpoints occur).  Returns the number of
// differing results; out[0] counts the pairs where the unchecked form differs.
extern "C" uint64_t otx_host_div_recip_subnormal_check(uint64_t n, uint64_t seed, uint64_t* unchecked_bad) {
  uint64_t bad = 0, ubad = 0;
#pragma omp parallel for schedule(static) reduction(+ : bad, ubad) num_threads(omp_get_num_procs())
  for (int64_t i = 0; i < (int64_t)n; i++) {
    uint64_t z = seed + 0x9E3779B97F4A7C15ull * (uint64_t)(i + 1);
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    z ^= z >> 31;
    const uint32_t ua = (uint32_t)z & 0x017fffffu;  // subnormal, or normal up to 2^-124
    const float a = otx_u2f(ua | ((uint32_t)(z >> 63) << 31));
    const uint32_t bm = ((uint32_t)(z >> 32) & 0xfffu) << 11;
    const float b = otx_u2f(((uint32_t)(127 + (int)((z >> 44) % 20)) << 23) | bm);
    const uint32_t want = otx_f2u(otx_div_rn(a, b));
    if (otx_f2u(otx_div_by_recip_checked(a, otx_recip64(b), b)) != want) bad++;
    if (otx_f2u(otx_div_by_recip(a, otx_recip64(b))) != want) ubad++;
  }
  *unchecked_bad = ubad;
  return bad;
}

// otx_div_by_recip(a, OTX_RECIP64_127) against otx_div_rn(a, 127) for every finite
// binary32 a >= 0 (every +0 .. largest finite pattern).  Returns the number of
// differing results.
extern "C" uint64_t otx_host_div_127_check(void) {
  uint64_t bad = 0;
#pragma omp parallel for schedule(static) reduction(+ : bad) num_threads(omp_get_num_procs())
  for (int64_t i = 0; i < 0x7F800000LL; i++) {
    const float a = otx_u2f((uint32_t)i);
    if (otx_f2u(otx_div_by_recip(a, OTX_RECIP64_127)) != otx_f2u(otx_div_rn(a, 127.0f))) bad++;
  }
  return bad;
}

// otx_div_by_recip(a, otx_recip64(b)) against otx_div_rn(a, b) on n pseudo-random
// (a, b) pairs: a over every binade (subnormals, +-0 and the largest values
// included), b > 0 over [2^-20, 2^20) and in [1, 2^14) (the forward's row sums).
// Returns the number of differing results.
extern "C" uint64_t otx_host_div_recip_check(uint64_t n, uint64_t seed) {
  uint64_t bad = 0;
#pragma omp parallel for schedule(static) reduction(+ : bad) num_threads(omp_get_num_procs())
  for (int64_t i = 0; i < (int64_t)n; i++) {
    uint64_t z = seed + 0x9E3779B97F4A7C15ull * (uint64_t)(i + 1);
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    z ^= z >> 31;
    const uint32_t ua = (uint32_t)z;
    if ((ua & 0x7f800000u) == 0x7f800000u) continue;  // finite a only
    const float a = otx_u2f(ua);
    const uint32_t bm = (uint32_t)(z >> 32) & 0x7fffffu;
    const int be = (i & 1) ? (int)((z >> 55) % 14) : (int)((z >> 55) % 40) - 20;
    const float b = otx_u2f(((uint32_t)(127 + be) << 23) | bm);
    if (otx_f2u(otx_div_by_recip(a, otx_recip64(b))) != otx_f2u(otx_div_rn(a, b))) bad++;
  }
  return bad;
}

// Every finite positive binary32 input of otx_logf and otx_rsqrtf, split like
// the functions themselves: the binary64 evaluation either decides the
// binary32 rounding (Ziv test) or the input must be in the exception table.
// out[0] / out[1] = undecided inputs missing from the log / rsqrt table (must
// be 0); out[2] / out[3] = table hits, whose bit patterns are written to
// hits_log / hits_rsqrt (at most max_hits each) for a check of their values.
extern "C" void otx_host_log_rsqrt_tables_check(uint64_t* out, uint32_t* hits_log, uint32_t* hits_rsqrt,
                                                int max_hits) {
  uint64_t miss_l = 0, miss_r = 0, nl = 0, nr = 0;
#pragma omp parallel for schedule(dynamic, 1 << 16) reduction(+ : miss_l, miss_r) num_threads(omp_get_num_procs())
  for (int64_t i = 1; i < 0x7F800000LL; i++) {
    const uint32_t u = (uint32_t)i;
    const float x = otx_u2f(u);
    int ok;
    uint32_t v;
    if (x != 1.0f) {
      (void)otx_round_checked(otx_log_f64_core(x), 0x1p-49, &ok);
      if (!ok) {
        if (otx_table_lookup(otx_log_exc_keys, otx_log_exc_vals, OTX_LOG_EXC_N, u, &v)) {
          uint64_t k;
#pragma omp atomic capture
          k = nl++;
          if (k < (uint64_t)max_hits) hits_log[k] = u;
        } else {
          miss_l++;
        }
      }
    }
    (void)otx_round_checked(1.0 / __builtin_sqrt((double)x), 0x1p-50, &ok);
    if (!ok) {
      if (otx_table_lookup(otx_rsqrt_exc_keys, otx_rsqrt_exc_vals, OTX_RSQRT_EXC_N, u, &v)) {
        uint64_t k;
#pragma omp atomic capture
        k = nr++;
        if (k < (uint64_t)max_hits) hits_rsqrt[k] = u;
      } else {
        miss_r++;
      }
    }
  }
  out[0] = miss_l; out[1] = miss_r; out[2] = nl; out[3] = nr;
}
