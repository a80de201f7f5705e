// Host build of the kernels' exp / log (the same source as the device code),
// so that CPU tests can check them against the oracle without a GPU.
#include <omp.h>
#include "otx_math.h"

extern "C" float otx_host_expf(float x) { return otx_expf(x); }
extern "C" float otx_host_logf(float x) { return otx_logf(x); }
extern "C" uint16_t otx_host_f32_to_bf16(float x) { return otx_f32_to_bf16(x); }
extern "C" float otx_host_div_rn(float a, float b) { return otx_div_rn(a, b); }

extern "C" float otx_host_expf_fast(float x, int* slow) { return otx_expf_fast(x, otx_exp2_tab64, slow); }

// Over the binary32 bit patterns [lo, lo + count): the number of inputs where
// the fast path returns a value (slow flag clear) that differs from otx_expf,
// and (via *nslow) the number of inputs it defers to otx_expf.
extern "C" uint64_t otx_host_exp_fast_mismatches(uint64_t lo, uint64_t count, uint64_t* nslow) {
  uint64_t bad = 0, slow_n = 0;
#pragma omp parallel for schedule(static) reduction(+ : bad, slow_n)
  for (int64_t i = 0; i < (int64_t)count; i++) {
    const float x = otx_u2f((uint32_t)(lo + (uint64_t)i));
    int slow;
    const float f = otx_expf_fast(x, otx_exp2_tab64, &slow);
    if (slow) {
      slow_n++;
    } else if (otx_f2u(f) != otx_f2u(otx_expf(x))) {
      bad++;
    }
  }
  *nslow = slow_n;
  return bad;
}

extern "C" float otx_host_expf_fast_le0(float x, int* slow) { return otx_expf_fast_le0(x, otx_exp2_tab64, slow); }

// otx_expf_fast_le0 over every binary32 x <= 0 (all negative bit patterns that
// are not NaN, and +0): returns the number of inputs where it returns a value
// (slow flag clear) different from otx_expf; *nslow counts the deferred ones.
extern "C" uint64_t otx_host_exp_le0_mismatches(uint64_t* nslow) {
  uint64_t bad = 0, slow_n = 0;
#pragma omp parallel for schedule(static) reduction(+ : bad, slow_n)
  for (int64_t i = 0; i <= (int64_t)0x7F800000; i++) {  // 0x80000000 | i: -0 ... -inf
    const float x = otx_u2f(0x80000000u | (uint32_t)i);
    int slow;
    const float f = otx_expf_fast_le0(x, otx_exp2_tab64, &slow);
    if (slow) slow_n++;
    else if (otx_f2u(f) != otx_f2u(otx_expf(x))) bad++;
  }
  int slow;
  const float f0 = otx_expf_fast_le0(0.0f, otx_exp2_tab64, &slow);
  if (slow) slow_n++;
  else if (otx_f2u(f0) != otx_f2u(otx_expf(0.0f))) bad++;
  *nslow = slow_n;
  return bad;
}

extern "C" float otx_host_rsqrtf(float x) { return otx_rsqrtf(x); }
