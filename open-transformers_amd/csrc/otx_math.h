// Correctly rounded binary32 exp and log, round-to-nearest-even bf16
// conversion and correctly rounded binary32 division, written once for the
// host and the gfx950 device so that the same source can be enumerated
// exhaustively on the CPU.
//
// exp/log method (Ziv's strategy): evaluate the function in binary64 with a
// proven relative error bound E, then round the two ends of the interval
// y*(1 -/+ 2E) to binary32.  When both ends round to the same binary32 value
// that value is the correctly rounded result.  The few binary32 inputs whose
// result lies too close to a rounding boundary are listed, with their
// correctly rounded results, in otx_math_tables.h (found by enumerating every
// binary32 input against libquadmath).
//
// Every operation below is a single IEEE-754 binary64 operation (add, mul,
// fma, div, exact conversions), so the host and device evaluate bit-identical
// intermediate values.  Build with -ffp-contract=off.
#pragma once
#include <stdint.h>

#if defined(__HIPCC__)
#include <hip/hip_runtime.h>
#define OTX_HD __host__ __device__ inline
#else
#define OTX_HD static inline
#endif

#include "otx_math_tables.h"

OTX_HD uint32_t otx_f2u(float f) { return __builtin_bit_cast(uint32_t, f); }
OTX_HD float otx_u2f(uint32_t u) { return __builtin_bit_cast(float, u); }
OTX_HD uint64_t otx_d2u(double d) { return __builtin_bit_cast(uint64_t, d); }
OTX_HD double otx_u2d(uint64_t u) { return __builtin_bit_cast(double, u); }

// binary32 -> bf16 with round-to-nearest-even (NaN stays a quiet NaN: the
// high half with the quiet bit set).  On the device this is the conversion
// instruction (v_cvt_pk_bf16_f32), which gives the same bits as the host
// formula for every one of the 2^32 inputs (tests/test_gpu_selftest.py
// compares the two over the whole range); the formula took seven vector
// instructions and a branch per value.
OTX_HD uint16_t otx_f32_to_bf16(float f) {
#if defined(__HIP_DEVICE_COMPILE__)
  return __builtin_bit_cast(uint16_t, (__bf16)f);
#else
  uint32_t u = otx_f2u(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
#endif
}
OTX_HD float otx_bf16_to_f32(uint16_t h) { return otx_u2f((uint32_t)h << 16); }

// Correctly rounded binary32 quotient a/b: the binary64 quotient is rounded
// once more to binary32; double rounding is innocuous for division because
// 53 >= 2*24 + 2.
OTX_HD float otx_div_rn(float a, float b) { return (float)((double)a / (double)b); }

// The same quotient for many a over one b, through one binary64 reciprocal:
// RN32(RN64(a * RN64(1/b))), three instructions per quotient instead of a
// division.  Correctly rounded for finite a and finite nonzero b whenever the
// quotient lies in the normal range: there a quotient of two 24-bit operands is
// never closer than 2^-49 (relative) to a midpoint m between binary32 numbers
// (a = m*b would need the odd part of a's significand to hold the 25-bit odd
// part of m's; otherwise a - m*b is a nonzero multiple of the last unit of
// m*b, whose 49-bit significand bounds it), while the two binary64 roundings
// move it by at most about 2^-52, so it rounds to the same binary32.  Below the
// normal range the binary32 grid is fixed-point and a quotient can be a midpoint
// exactly (a = 294 * 2^-149, b = 196 gives 1.5 * 2^-149), where this form may
// round the wrong way: otx_div_by_recip_checked takes the division there.
OTX_HD double otx_recip64(float b) { return 1.0 / (double)b; }
OTX_HD float otx_div_by_recip(float a, double rb) { return (float)((double)a * rb); }
OTX_HD float otx_div_by_recip_checked(float a, double rb, float b) {
  const float q = otx_div_by_recip(a, rb);
  return __builtin_fabsf(q) >= 0x1p-126f ? q : otx_div_rn(a, b);  // below the normal range, zero, NaN: divide
}
// RN64(1/127), for the int8 steps RN(pmax / 127) (checked for every finite a >= 0 on the host)
#define OTX_RECIP64_127 (1.0 / 127.0)

// Binary search of a sorted exception table (keys are binary32 bit patterns
// ordered as unsigned integers).  Returns 1 and the stored result on a hit.
OTX_HD int otx_table_lookup(const uint32_t* keys, const uint32_t* vals, int n, uint32_t key, uint32_t* out) {
  int lo = 0, hi = n - 1;
  while (lo <= hi) {
    int mid = (lo + hi) >> 1;
    uint32_t k = keys[mid];
    if (k == key) { *out = vals[mid]; return 1; }
    if (k < key) lo = mid + 1; else hi = mid - 1;
  }
  return 0;
}

// Round y (known to relative error < 2^-50) to binary32 if that is
// unambiguous.  Sets *ok = 0 when the interval straddles a rounding boundary.
OTX_HD float otx_round_checked(double y, double rel, int* ok) {
  double e = y * rel;
  float lo = (float)(y - e);
  float hi = (float)(y + e);
  *ok = (otx_f2u(lo) == otx_f2u(hi));
  return lo;
}

// exp(x) in binary64 for -104 < x < 89 with relative error below 2^-51.5.
//   k = nearest integer to x*log2(e)   (one fused multiply-add, exact rounding)
//   r = x - k*ln2                      (first fma exact, second adds ln2's tail)
//   exp(r) by its degree-13 Taylor polynomial on |r| <= 0.3466
//     (truncation < 2^-57, Horner rounding < 2^-52)
//   result = exp(r) * 2^k (exact scaling by a power of two)
OTX_HD double otx_exp_f64_core(float xf) {
  const double LOG2E = 0x1.71547652b82fep+0;
  const double SHIFT = 0x1.8p52;
  const double LN2_HI = 0x1.62e42fefa39efp-1;
  const double LN2_LO = 0x1.abc9e3b39803fp-56;
  double x = (double)xf;
  double t = __builtin_fma(x, LOG2E, SHIFT);
  double kd = t - SHIFT;
  double r = __builtin_fma(-kd, LN2_HI, x);
  r = __builtin_fma(-kd, LN2_LO, r);
  double p = 0x1.6124613a86d09p-33;           // 1/13!
  p = __builtin_fma(p, r, 0x1.1eed8eff8d898p-29);  // 1/12!
  p = __builtin_fma(p, r, 0x1.ae64567f544e4p-26);  // 1/11!
  p = __builtin_fma(p, r, 0x1.27e4fb7789f5cp-22);  // 1/10!
  p = __builtin_fma(p, r, 0x1.71de3a556c734p-19);  // 1/9!
  p = __builtin_fma(p, r, 0x1.a01a01a01a01ap-16);  // 1/8!
  p = __builtin_fma(p, r, 0x1.a01a01a01a01ap-13);  // 1/7!
  p = __builtin_fma(p, r, 0x1.6c16c16c16c17p-10);  // 1/6!
  p = __builtin_fma(p, r, 0x1.1111111111111p-7);   // 1/5!
  p = __builtin_fma(p, r, 0x1.5555555555555p-5);   // 1/4!
  p = __builtin_fma(p, r, 0x1.5555555555555p-3);   // 1/3!
  p = __builtin_fma(p, r, 0x1.0p-1);               // 1/2!
  p = __builtin_fma(p, r, 1.0);
  p = __builtin_fma(p, r, 1.0);
  int k = (int)kd;
  double scale = otx_u2d((uint64_t)(int64_t)(k + 1023) << 52);
  return p * scale;
}

// Correctly rounded binary32 exp.
OTX_HD float otx_expf(float x) {
  if (x != x) return x;
  if (!(x > -104.0f)) return 0.0f;          // exp(x) < 2^-150 rounds to +0
  if (x > 89.0f) return __builtin_inff();
  double y = otx_exp_f64_core(x);
  int ok;
  float f = otx_round_checked(y, 0x1p-50, &ok);
  if (ok) return f;
  uint32_t v;
  if (otx_table_lookup(otx_exp_exc_keys, otx_exp_exc_vals, OTX_EXP_EXC_N, otx_f2u(x), &v)) return otx_u2f(v);
  return f;  // unreachable: every inconclusive input is in the table
}

// ---------------------------------------------------------------------------
// Fast path of the correctly rounded exp for the attention inner loops.
//
// Table-driven binary64 evaluation (Tang's method, ACM TOMS 15(2), 1989):
//   k = nearest integer to x * 64/ln2        (one fma against 1.5*2^52)
//   r = x - k*ln2/64                          (first fma exact, see below;
//                                              second adds ln2/64's tail)
//   exp(x) = 2^(k>>6) * T[k & 63] * p(r),     T[j] = RN64(2^(j/64)),
//   p(r) = 1 + r + r^2/2 + ... + r^5/120      (|r| <= ln2/128 + 2^-40)
// Relative error budget: T 2^-53, truncation r^6/720 < 2^-54.6, Horner
// rounding < 2^-52.9, final product 2^-53; total below 2^-51.1.  The result
// is returned only when the interval y*(1 -/+ 2^-50) rounds to a single
// binary32 value; otherwise *slow is set and the caller must use otx_expf.
// Also flagged slow: NaN and x > 88 (overflow region).  x <= -104 returns +0
// (exp(x) < 2^-150), which is exact rounding.
//
// ln2/64 is split as HI (40 significant bits) + LO.  For x >= -104, |k| <
// 2^14 so k*HI is exact, and x - k*HI is a multiple of 2^-46 below 2^-7 when
// k != 0, hence representable: the first fma is exact.
#define OTX_EXP_TAB_N 64
#define OTX_EXP2_TAB64_VALUES                                                                   \
  0x1.0000000000000p+0, 0x1.02c9a3e778061p+0, 0x1.059b0d3158574p+0, 0x1.0874518759bc8p+0,      \
      0x1.0b5586cf9890fp+0, 0x1.0e3ec32d3d1a2p+0, 0x1.11301d0125b51p+0, 0x1.1429aaea92de0p+0,  \
      0x1.172b83c7d517bp+0, 0x1.1a35beb6fcb75p+0, 0x1.1d4873168b9aap+0, 0x1.2063b88628cd6p+0,  \
      0x1.2387a6e756238p+0, 0x1.26b4565e27cddp+0, 0x1.29e9df51fdee1p+0, 0x1.2d285a6e4030bp+0,  \
      0x1.306fe0a31b715p+0, 0x1.33c08b26416ffp+0, 0x1.371a7373aa9cbp+0, 0x1.3a7db34e59ff7p+0,  \
      0x1.3dea64c123422p+0, 0x1.4160a21f72e2ap+0, 0x1.44e086061892dp+0, 0x1.486a2b5c13cd0p+0,  \
      0x1.4bfdad5362a27p+0, 0x1.4f9b2769d2ca7p+0, 0x1.5342b569d4f82p+0, 0x1.56f4736b527dap+0,  \
      0x1.5ab07dd485429p+0, 0x1.5e76f15ad2148p+0, 0x1.6247eb03a5585p+0, 0x1.6623882552225p+0,  \
      0x1.6a09e667f3bcdp+0, 0x1.6dfb23c651a2fp+0, 0x1.71f75e8ec5f74p+0, 0x1.75feb564267c9p+0,  \
      0x1.7a11473eb0187p+0, 0x1.7e2f336cf4e62p+0, 0x1.82589994cce13p+0, 0x1.868d99b4492edp+0,  \
      0x1.8ace5422aa0dbp+0, 0x1.8f1ae99157736p+0, 0x1.93737b0cdc5e5p+0, 0x1.97d829fde4e50p+0,  \
      0x1.9c49182a3f090p+0, 0x1.a0c667b5de565p+0, 0x1.a5503b23e255dp+0, 0x1.a9e6b5579fdbfp+0,  \
      0x1.ae89f995ad3adp+0, 0x1.b33a2b84f15fbp+0, 0x1.b7f76f2fb5e47p+0, 0x1.bcc1e904bc1d2p+0,  \
      0x1.c199bdd85529cp+0, 0x1.c67f12e57d14bp+0, 0x1.cb720dcef9069p+0, 0x1.d072d4a07897cp+0,  \
      0x1.d5818dcfba487p+0, 0x1.da9e603db3285p+0, 0x1.dfc97337b9b5fp+0, 0x1.e502ee78b3ff6p+0,  \
      0x1.ea4afa2a490dap+0, 0x1.efa1bee615a27p+0, 0x1.f50765b6e4540p+0, 0x1.fa7c1819e90d8p+0

static constexpr double otx_exp2_tab64[OTX_EXP_TAB_N] = {OTX_EXP2_TAB64_VALUES};

// 2^(j/256), j = 0..255, each correctly rounded to binary64: the table of the
// softmax path below (otx_exp_le0_*).
#define OTX_EXP_LE0_TAB_N 256
#define OTX_EXP2_TAB256_VALUES \
      0x1.0000000000000p+0, 0x1.00b1afa5abcbfp+0, 0x1.0163da9fb3335p+0, 0x1.02168143b0281p+0, \
      0x1.02c9a3e778061p+0, 0x1.037d42e11bbccp+0, 0x1.04315e86e7f85p+0, 0x1.04e5f72f654b1p+0, \
      0x1.059b0d3158574p+0, 0x1.0650a0e3c1f89p+0, 0x1.0706b29ddf6dep+0, 0x1.07bd42b72a836p+0, \
      0x1.0874518759bc8p+0, 0x1.092bdf66607e0p+0, 0x1.09e3ecac6f383p+0, 0x1.0a9c79b1f3919p+0, \
      0x1.0b5586cf9890fp+0, 0x1.0c0f145e46c85p+0, 0x1.0cc922b7247f7p+0, 0x1.0d83b23395decp+0, \
      0x1.0e3ec32d3d1a2p+0, 0x1.0efa55fdfa9c5p+0, 0x1.0fb66affed31bp+0, 0x1.1073028d7233ep+0, \
      0x1.11301d0125b51p+0, 0x1.11edbab5e2ab6p+0, 0x1.12abdc06c31ccp+0, 0x1.136a814f204abp+0, \
      0x1.1429aaea92de0p+0, 0x1.14e95934f312ep+0, 0x1.15a98c8a58e51p+0, 0x1.166a45471c3c2p+0, \
      0x1.172b83c7d517bp+0, 0x1.17ed48695bbc0p+0, 0x1.18af9388c8deap+0, 0x1.1972658375d2fp+0, \
      0x1.1a35beb6fcb75p+0, 0x1.1af99f8138a1cp+0, 0x1.1bbe084045cd4p+0, 0x1.1c82f95281c6bp+0, \
      0x1.1d4873168b9aap+0, 0x1.1e0e75eb44027p+0, 0x1.1ed5022fcd91dp+0, 0x1.1f9c18438ce4dp+0, \
      0x1.2063b88628cd6p+0, 0x1.212be3578a819p+0, 0x1.21f49917ddc96p+0, 0x1.22bdda27912d1p+0, \
      0x1.2387a6e756238p+0, 0x1.2451ffb82140ap+0, 0x1.251ce4fb2a63fp+0, 0x1.25e85711ece75p+0, \
      0x1.26b4565e27cddp+0, 0x1.2780e341ddf29p+0, 0x1.284dfe1f56381p+0, 0x1.291ba7591bb70p+0, \
      0x1.29e9df51fdee1p+0, 0x1.2ab8a66d10f13p+0, 0x1.2b87fd0dad990p+0, 0x1.2c57e39771b2fp+0, \
      0x1.2d285a6e4030bp+0, 0x1.2df961f641589p+0, 0x1.2ecafa93e2f56p+0, 0x1.2f9d24abd886bp+0, \
      0x1.306fe0a31b715p+0, 0x1.31432edeeb2fdp+0, 0x1.32170fc4cd831p+0, 0x1.32eb83ba8ea32p+0, \
      0x1.33c08b26416ffp+0, 0x1.3496266e3fa2dp+0, 0x1.356c55f929ff1p+0, 0x1.36431a2de883bp+0, \
      0x1.371a7373aa9cbp+0, 0x1.37f26231e754ap+0, 0x1.38cae6d05d866p+0, 0x1.39a401b7140efp+0, \
      0x1.3a7db34e59ff7p+0, 0x1.3b57fbfec6cf4p+0, 0x1.3c32dc313a8e5p+0, 0x1.3d0e544ede173p+0, \
      0x1.3dea64c123422p+0, 0x1.3ec70df1c5175p+0, 0x1.3fa4504ac801cp+0, 0x1.40822c367a024p+0, \
      0x1.4160a21f72e2ap+0, 0x1.423fb2709468ap+0, 0x1.431f5d950a897p+0, 0x1.43ffa3f84b9d4p+0, \
      0x1.44e086061892dp+0, 0x1.45c2042a7d232p+0, 0x1.46a41ed1d0057p+0, 0x1.4786d668b3237p+0, \
      0x1.486a2b5c13cd0p+0, 0x1.494e1e192aed2p+0, 0x1.4a32af0d7d3dep+0, 0x1.4b17dea6db7d7p+0, \
      0x1.4bfdad5362a27p+0, 0x1.4ce41b817c114p+0, 0x1.4dcb299fddd0dp+0, 0x1.4eb2d81d8abffp+0, \
      0x1.4f9b2769d2ca7p+0, 0x1.508417f4531eep+0, 0x1.516daa2cf6642p+0, 0x1.5257de83f4eefp+0, \
      0x1.5342b569d4f82p+0, 0x1.542e2f4f6ad27p+0, 0x1.551a4ca5d920fp+0, 0x1.56070dde910d2p+0, \
      0x1.56f4736b527dap+0, 0x1.57e27dbe2c4cfp+0, 0x1.58d12d497c7fdp+0, 0x1.59c0827ff07ccp+0, \
      0x1.5ab07dd485429p+0, 0x1.5ba11fba87a03p+0, 0x1.5c9268a5946b7p+0, 0x1.5d84590998b93p+0, \
      0x1.5e76f15ad2148p+0, 0x1.5f6a320dceb71p+0, 0x1.605e1b976dc09p+0, 0x1.6152ae6cdf6f4p+0, \
      0x1.6247eb03a5585p+0, 0x1.633dd1d1929fdp+0, 0x1.6434634ccc320p+0, 0x1.652b9febc8fb7p+0, \
      0x1.6623882552225p+0, 0x1.671c1c70833f6p+0, 0x1.68155d44ca973p+0, 0x1.690f4b19e9538p+0, \
      0x1.6a09e667f3bcdp+0, 0x1.6b052fa75173ep+0, 0x1.6c012750bdabfp+0, 0x1.6cfdcddd47645p+0, \
      0x1.6dfb23c651a2fp+0, 0x1.6ef9298593ae5p+0, 0x1.6ff7df9519484p+0, 0x1.70f7466f42e87p+0, \
      0x1.71f75e8ec5f74p+0, 0x1.72f8286ead08ap+0, 0x1.73f9a48a58174p+0, 0x1.74fbd35d7cbfdp+0, \
      0x1.75feb564267c9p+0, 0x1.77024b1ab6e09p+0, 0x1.780694fde5d3fp+0, 0x1.790b938ac1cf6p+0, \
      0x1.7a11473eb0187p+0, 0x1.7b17b0976cfdbp+0, 0x1.7c1ed0130c132p+0, 0x1.7d26a62ff86f0p+0, \
      0x1.7e2f336cf4e62p+0, 0x1.7f3878491c491p+0, 0x1.80427543e1a12p+0, 0x1.814d2add106d9p+0, \
      0x1.82589994cce13p+0, 0x1.8364c1eb941f7p+0, 0x1.8471a4623c7adp+0, 0x1.857f4179f5b21p+0, \
      0x1.868d99b4492edp+0, 0x1.879cad931a436p+0, 0x1.88ac7d98a6699p+0, 0x1.89bd0a478580fp+0, \
      0x1.8ace5422aa0dbp+0, 0x1.8be05bad61778p+0, 0x1.8cf3216b5448cp+0, 0x1.8e06a5e0866d9p+0, \
      0x1.8f1ae99157736p+0, 0x1.902fed0282c8ap+0, 0x1.9145b0b91ffc6p+0, 0x1.925c353aa2fe2p+0, \
      0x1.93737b0cdc5e5p+0, 0x1.948b82b5f98e5p+0, 0x1.95a44cbc8520fp+0, 0x1.96bdd9a7670b3p+0, \
      0x1.97d829fde4e50p+0, 0x1.98f33e47a22a2p+0, 0x1.9a0f170ca07bap+0, 0x1.9b2bb4d53fe0dp+0, \
      0x1.9c49182a3f090p+0, 0x1.9d674194bb8d5p+0, 0x1.9e86319e32323p+0, 0x1.9fa5e8d07f29ep+0, \
      0x1.a0c667b5de565p+0, 0x1.a1e7aed8eb8bbp+0, 0x1.a309bec4a2d33p+0, 0x1.a42c980460ad8p+0, \
      0x1.a5503b23e255dp+0, 0x1.a674a8af46052p+0, 0x1.a799e1330b358p+0, 0x1.a8bfe53c12e59p+0, \
      0x1.a9e6b5579fdbfp+0, 0x1.ab0e521356ebap+0, 0x1.ac36bbfd3f37ap+0, 0x1.ad5ff3a3c2774p+0, \
      0x1.ae89f995ad3adp+0, 0x1.afb4ce622f2ffp+0, 0x1.b0e07298db666p+0, 0x1.b20ce6c9a8952p+0, \
      0x1.b33a2b84f15fbp+0, 0x1.b468415b749b1p+0, 0x1.b59728de5593ap+0, 0x1.b6c6e29f1c52ap+0, \
      0x1.b7f76f2fb5e47p+0, 0x1.b928cf22749e4p+0, 0x1.ba5b030a1064ap+0, 0x1.bb8e0b79a6f1fp+0, \
      0x1.bcc1e904bc1d2p+0, 0x1.bdf69c3f3a207p+0, 0x1.bf2c25bd71e09p+0, 0x1.c06286141b33dp+0, \
      0x1.c199bdd85529cp+0, 0x1.c2d1cd9fa652cp+0, 0x1.c40ab5fffd07ap+0, 0x1.c544778fafb22p+0, \
      0x1.c67f12e57d14bp+0, 0x1.c7ba88988c933p+0, 0x1.c8f6d9406e7b5p+0, 0x1.ca3405751c4dbp+0, \
      0x1.cb720dcef9069p+0, 0x1.ccb0f2e6d1675p+0, 0x1.cdf0b555dc3fap+0, 0x1.cf3155b5bab74p+0, \
      0x1.d072d4a07897cp+0, 0x1.d1b532b08c968p+0, 0x1.d2f87080d89f2p+0, 0x1.d43c8eacaa1d6p+0, \
      0x1.d5818dcfba487p+0, 0x1.d6c76e862e6d3p+0, 0x1.d80e316c98398p+0, 0x1.d955d71ff6075p+0, \
      0x1.da9e603db3285p+0, 0x1.dbe7cd63a8315p+0, 0x1.dd321f301b460p+0, 0x1.de7d5641c0658p+0, \
      0x1.dfc97337b9b5fp+0, 0x1.e11676b197d17p+0, 0x1.e264614f5a129p+0, 0x1.e3b333b16ee12p+0, \
      0x1.e502ee78b3ff6p+0, 0x1.e653924676d76p+0, 0x1.e7a51fbc74c83p+0, 0x1.e8f7977cdb740p+0, \
      0x1.ea4afa2a490dap+0, 0x1.eb9f4867cca6ep+0, 0x1.ecf482d8e67f1p+0, 0x1.ee4aaa2188510p+0, \
      0x1.efa1bee615a27p+0, 0x1.f0f9c1cb6412ap+0, 0x1.f252b376bba97p+0, 0x1.f3ac948dd7274p+0, \
      0x1.f50765b6e4540p+0, 0x1.f6632798844f8p+0, 0x1.f7bfdad9cbe14p+0, 0x1.f91d802243c89p+0, \
      0x1.fa7c1819e90d8p+0, 0x1.fbdba3692d514p+0, 0x1.fd3c22b8f71f1p+0, 0x1.fe9d96b2a23d9p+0

static constexpr double otx_exp2_tab256[OTX_EXP_LE0_TAB_N] = {OTX_EXP2_TAB256_VALUES};

// `tab` points at the 64 table entries (LDS on the device, otx_exp2_tab64 on
// the host).  Branch-free; *slow is 0 or 1.
OTX_HD float otx_expf_fast(float x, const double* tab, int* slow) {
  const double INV_LN2_64 = 0x1.71547652b82fep+6;
  const double SHIFT = 0x1.8p52;
  const double LN2_64_HI = 0x1.62e42fefa2000p-7;
  const double LN2_64_LO = 0x1.9ef35793c7673p-47;
  const float xc = x > -104.0f ? x : -104.0f;  // also maps -inf (NaN stays NaN)
  const double xd = (double)xc;
  const double t = __builtin_fma(xd, INV_LN2_64, SHIFT);
  const double kd = t - SHIFT;
  double r = __builtin_fma(-kd, LN2_64_HI, xd);
  r = __builtin_fma(-kd, LN2_64_LO, r);
  const uint32_t kb = (uint32_t)otx_d2u(t);  // k in two's complement
  double p = __builtin_fma(r, 0x1.1111111111111p-7, 0x1.5555555555555p-5);  // 1/120, 1/24
  p = __builtin_fma(p, r, 0x1.5555555555555p-3);                             // 1/6
  p = __builtin_fma(p, r, 0.5);
  p = __builtin_fma(p, r, 1.0);
  p = __builtin_fma(p, r, 1.0);
  const double y0 = tab[kb & 63u] * p;
  const double y = otx_u2d(otx_d2u(y0) + ((uint64_t)(int64_t)((int32_t)kb >> 6) << 52));
  const double e = y * 0x1p-50;
  const float lo = (float)(y - e);
  const float hi = (float)(y + e);
  const int in_range = (x > -104.0f) & (x <= 88.0f);
  *slow = (otx_f2u(lo) != otx_f2u(hi)) & in_range;
  *slow |= (x != x) | (x > 88.0f);
  return in_range ? lo : 0.0f;
}

// The softmax arguments x <= 0 (including -inf) take a shorter evaluation,
// split into two stages so that a kernel can run the first stage (and its
// table reads) for a whole register array before the second.  `tab` points at
// the 256 entries of otx_exp2_tab256 biased by otx_exp2_tab256_biased (LDS on
// the device):
//   otx_exp_le0_reduce: x is clamped to [-104, 0] (exp(-104) < 2^-150 already
//     rounds to +0, and so does the clamped evaluation); k = round(x*256/ln2),
//     the table entry T[k & 255] and the reduced argument
//     r = x - k*ln2/256, |r| <= ln2/512 (ln2/256 split as HI, 36 significant
//     bits, + LO: |k| < 2^16, so k*HI and the first fma are exact);
//   otx_exp_le0_finish: y = (2^(k>>8) * T) * p(r), p the degree-4 Taylor
//     polynomial (truncation below 2^-54.5 relative), rounded once to binary32.
// No rounding test is needed on this domain: the binary32 rounding of y equals
// the correctly rounded exp(x) for every binary32 x <= 0 and for -inf,
// including the four inputs whose exp lies within 2^-50 of a rounding
// boundary.  That is a property of these exact binary64 operations,
// established by enumerating all 2^31 + 1 such inputs against otx_expf (the
// host build of this header runs the same operations).  NaN or positive x
// must not be passed (the kernels guarantee x <= 0 by construction, or check
// it).
OTX_HD float otx_clamp_le0(float x) {
#if defined(__HIP_DEVICE_COMPILE__)
  return __builtin_amdgcn_fmed3f(x, -104.0f, 0.0f);  // one instruction
#else
  return x < -104.0f ? -104.0f : (x > 0.0f ? 0.0f : x);
#endif
}

// Entry j of the table the evaluation reads: the bits of 2^(j/256)
// (otx_exp2_tab256[j]) with j << 12 subtracted from the high word.  Adding
// k << 12 to that high word (32-bit wrap-around, k the two's-complement low
// word of t below, j = k & 255) then adds ((k - j) / 256) << 20, i.e.
// (k >> 8) to the exponent field: one integer add gives the binary64
// 2^(k>>8) * T exactly (its exponent stays >= 1023 - 151, far from the
// binary64 subnormals), so y = RN(2^(k>>8) * T * p) = 2^(k>>8) * RN(T * p),
// the same value as scaling RN(T * p) afterwards.  A biased entry is only a
// bit pattern, never used as a number.
OTX_HD double otx_exp2_tab256_biased(int j) {
  return otx_u2d(otx_d2u(otx_exp2_tab256[j]) - ((uint64_t)(uint32_t)j << 44));
}

// The operations, stage by stage (a kernel evaluating many values runs each
// stage over all of them before the next, so that dependent binary64
// operations are not issued back to back):
//   t = fma(xd, 256/ln2, 1.5*2^52), xd = clamp(x) in binary64;
//   k = the low word of t: table index k & 255 (the scale exponent k >> 8
//   enters through the biased entry);
//   r = x - k*ln2/256 in two fmas;  p = p4(r);  y = (2^(k>>8) * T) * p.
OTX_HD double otx_exp_le0_t(float x, double* xd) {
  *xd = (double)otx_clamp_le0(x);
  return __builtin_fma(*xd, 0x1.71547652b82fep+8, 0x1.8p52);
}
OTX_HD double otx_exp_le0_r(double t, double xd) {
  const double kd = t - 0x1.8p52;
  const double r = __builtin_fma(-kd, 0x1.62e42fefa0000p-9, xd);  // ln2/256, 36 significant bits
  return __builtin_fma(-kd, 0x1.cf79abc9e3b3ap-48, r);             // the rest of ln2/256
}
OTX_HD double otx_exp_le0_p(double r) {
  double p = __builtin_fma(r, 0x1.5555555555555p-5, 0x1.5555555555555p-3);  // 1/24, 1/6
  p = __builtin_fma(p, r, 0.5);
  p = __builtin_fma(p, r, 1.0);
  return __builtin_fma(p, r, 1.0);
}
// tvb: the biased entry T[k & 255]; kb: the low word of t (k)
OTX_HD float otx_exp_le0_y(double p, double tvb, uint32_t kb) {
  const uint64_t u = otx_d2u(tvb);
  uint32_t hi = (uint32_t)(u >> 32);
#if defined(__HIP_DEVICE_COMPILE__)
  // one v_lshl_add_u32 on the high word in place (written in C, the add is
  // widened to a 64-bit shift-and-add plus moves)
  asm("v_lshl_add_u32 %0, %1, 12, %0" : "+v"(hi) : "v"(kb));
#else
  hi += kb << 12;
#endif
  const double scaled = otx_u2d(((uint64_t)hi << 32) | (u & 0xFFFFFFFFu));  // 2^(k>>8) * T
  return (float)(scaled * p);
}

OTX_HD double otx_exp_le0_reduce(float x, const double* tab, double* tvb, uint32_t* kb) {
  double xd;
  const double t = otx_exp_le0_t(x, &xd);
  *kb = (uint32_t)otx_d2u(t);
  *tvb = tab[*kb & 255u];
  return otx_exp_le0_r(t, xd);
}

OTX_HD float otx_exp_le0_finish(double r, double tvb, uint32_t kb) {
  return otx_exp_le0_y(otx_exp_le0_p(r), tvb, kb);
}

// `tab`: the 256 biased entries (otx_exp2_tab256_biased)
OTX_HD float otx_expf_fast_le0(float x, const double* tab) {
  double tvb;
  uint32_t kb;
  const double r = otx_exp_le0_reduce(x, tab, &tvb, &kb);
  return otx_exp_le0_finish(r, tvb, kb);
}

// Correctly rounded binary32 1/sqrt(x) (RMSNorm's rstd).  The binary64
// evaluation 1/sqrt(x) (correctly rounded sqrt, then a correctly rounded
// division) has relative error below 2^-52; the Ziv test at 2^-50 decides the
// binary32 rounding except on the inputs listed in otx_rsqrt_exc (enumerated
// over every positive binary32 against libquadmath).  x = +0 gives +inf,
// x < 0 or NaN gives NaN.
OTX_HD float otx_rsqrtf(float x) {
  if (!(x > 0.0f)) return x == 0.0f ? __builtin_inff() : __builtin_nanf("");
  if (x == __builtin_inff()) return 0.0f;
  const double y = 1.0 / __builtin_sqrt((double)x);
  int ok;
  const float f = otx_round_checked(y, 0x1p-50, &ok);
  if (ok) return f;
  uint32_t v;
  if (otx_table_lookup(otx_rsqrt_exc_keys, otx_rsqrt_exc_vals, OTX_RSQRT_EXC_N, otx_f2u(x), &v)) return otx_u2f(v);
  return f;  // unreachable: every inconclusive input is in the table
}

// log(x) in binary64 for finite x > 0 with relative error below 2^-51.
//   x = m * 2^e with m in [sqrt(2)/2, sqrt(2))
//   u = (m-1)/(m+1)   (m-1 and m+1 exact; one rounded division)
//   log(m) = 2 atanh(u) = 2u + u * (u^2 * sum_{k>=1} 2/(2k+1) u^(2k-2)), |u| <= 0.1716
//     (series to k = 12: truncation < 2^-60)
//   log(x) = e*ln2_hi + (e*ln2_lo + log(m))
OTX_HD double otx_log_f64_core(float xf) {
  const double LN2_HI = 0x1.62e42fefa39efp-1;
  const double LN2_LO = 0x1.abc9e3b39803fp-56;
  uint32_t u32 = otx_f2u(xf);
  int e;
  double m;
  if (u32 < 0x00800000u) {  // subnormal: scale by 2^32 exactly
    u32 = otx_f2u(xf * 0x1p32f);
    e = (int)(u32 >> 23) - 127 - 32;
  } else {
    e = (int)(u32 >> 23) - 127;
  }
  m = (double)otx_u2f((u32 & 0x007fffffu) | 0x3f800000u);
  if (m > 0x1.6a09e667f3bcdp+0) { m = m * 0.5; e += 1; }
  double u = (m - 1.0) / (m + 1.0);
  double u2 = u * u;
  double s = 0x1.47ae147ae147bp-4;            // 2/25
  s = __builtin_fma(s, u2, 0x1.642c8590b2164p-4);  // 2/23
  s = __builtin_fma(s, u2, 0x1.8618618618618p-4);  // 2/21
  s = __builtin_fma(s, u2, 0x1.af286bca1af28p-4);  // 2/19
  s = __builtin_fma(s, u2, 0x1.e1e1e1e1e1e1ep-4);  // 2/17
  s = __builtin_fma(s, u2, 0x1.1111111111111p-3);  // 2/15
  s = __builtin_fma(s, u2, 0x1.3b13b13b13b14p-3);  // 2/13
  s = __builtin_fma(s, u2, 0x1.745d1745d1746p-3);  // 2/11
  s = __builtin_fma(s, u2, 0x1.c71c71c71c71cp-3);  // 2/9
  s = __builtin_fma(s, u2, 0x1.2492492492492p-2);  // 2/7
  s = __builtin_fma(s, u2, 0x1.999999999999ap-2);  // 2/5
  s = __builtin_fma(s, u2, 0x1.5555555555555p-1);  // 2/3
  s = s * u2;
  double two_u = u + u;
  double logm = __builtin_fma(u, s, two_u);
  double ed = (double)e;
  double y = __builtin_fma(ed, LN2_LO, logm);
  return __builtin_fma(ed, LN2_HI, y);
}

// Correctly rounded binary32 natural logarithm.
OTX_HD float otx_logf(float x) {
  if (x != x) return x;
  if (x < 0.0f) return __builtin_nanf("");
  if (x == 0.0f) return -__builtin_inff();
  if (x == __builtin_inff()) return x;
  if (x == 1.0f) return 0.0f;
  double y = otx_log_f64_core(x);
  int ok;
  float f = otx_round_checked(y, 0x1p-49, &ok);
  if (ok) return f;
  uint32_t v;
  if (otx_table_lookup(otx_log_exc_keys, otx_log_exc_vals, OTX_LOG_EXC_N, otx_f2u(x), &v)) return otx_u2f(v);
  return f;  // unreachable: every inconclusive input is in the table
}
