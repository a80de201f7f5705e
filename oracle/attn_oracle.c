/*
 * CPU oracle for the deterministic causal flash attention path.  TEST
 * INFRASTRUCTURE ONLY: tests/, the smoke check and the CPU-baseline leg of the
 * benchmark may call it as the checker; the product never links or calls it.
 *
 * It restates, one scalar operation at a time, the arithmetic contract that
 * the HIP kernels must reproduce bit for bit.  The reference operator is
 * repop.nn.flash_attention.causal_flash_attention(q, k, v, dropout=0.0,
 * window=w), called at src/pretrain/model/modules/attention_repop.py:53 of
 * the reference; repop itself is closed source and absent, so the bit-level
 * rules below are this project's written contract built from the documented
 * facts (fp32 scores and online-softmax statistics, 1/sqrt(D) applied inside,
 * key blocks of 32, bf16 outputs, fp32 backward math, fixed-order
 * reductions: attention_repop.py:1-20,45-53; docs/MODEL_OP_DTYPE_TRACE.md:
 * 80,102; docs/unified-audit-results.md:71-74).
 *
 * Contract (all arithmetic IEEE-754 binary32, round to nearest even,
 * subnormals preserved; fma = one rounding; RN() = one rounding):
 *   Layout  q [B,H,S,D], k/v [B,Hkv,S,D]; query head h reads KV head
 *           h / (H/Hkv) (GQA, attention_repop.py:83,146-147).  S % 32 == 0.
 *   Mask    key j is visible to query i when j <= i and, for window w > 0,
 *           j > i - w (attention_repop.py:88-96 chooses w per layer).
 *   Blocks  keys and queries are cut into blocks of 32.  Query block I
 *           processes key blocks max(0, I - w/32) .. I (w = 0: 0 .. I), in
 *           ascending order; key block J is processed by query blocks
 *           J .. min(S/32-1, J + w/32) (w = 0: J .. S/32-1).  A processed
 *           block is dense: masked pairs take part with score -inf and
 *           probability +0.
 *   dot     dot(x, y) = serial fma over d = 0..D-1 starting from +0.
 *   scale   sigma = RN(1/sqrt(D)).
 *   Forward per row i: m = -inf, l = +0, acc[d] = +0; for each block:
 *             s_j = masked ? -inf : RN(dot(q_i, k_j) * sigma)
 *             mb = max_j s_j (ascending compare-select), m' = (mb > m) ? mb : m
 *             alpha = (m' == m) ? 1 : exp(m - m')
 *             p_j = masked ? +0 : exp(s_j - m')
 *             l = RN(l * alpha); then l = RN(l + p_j) for j ascending
 *             acc[d] = RN(acc[d] * alpha); then acc[d] = fma(p_j, v_j[d], acc[d]), j ascending
 *             m = m'
 *           O_i[d] = RN(acc[d] / l) (then RNE to bf16 for bf16 inputs),
 *           LSE_i = RN(m + log(l)).  exp and log are correctly rounded.
 *   Backward: Dsum_i = dot(dO_i, O_i) with O as stored (bf16 values for bf16).
 *           s_ij as forward, P_ij = masked ? +0 : exp(RN(s_ij - LSE_i)),
 *           dP_ij = dot(dO_i, v_j) (for every pair of a processed block),
 *           dS_ij = RN(P_ij * RN(dP_ij - Dsum_i)).
 *           dV_j[d] = serial fma of P_ij * dO_i[d] over the query heads of j's
 *           group (ascending), then the processed query blocks (ascending),
 *           then i within the block (ascending), from +0.
 *           dK_j[d] = RN(sigma * <same fold of dS_ij * q_i[d]>).
 *           dQ_i[d] = RN(sigma * <serial fma of dS_ij * k_j[d] over the
 *           processed key blocks and j ascending, from +0>).
 *           Outputs RNE to bf16 for bf16 inputs.
 *
 * Parallelism (OpenMP over rows / key columns / heads) never changes the
 * order of any reduction, so results do not depend on the thread count.
 *
 * How each rule is pinned independently of this file (every bit rule has a
 * closed-form probe that a planted one-line deviation of this file fails):
 * exp/log against libquadmath over dense and exhaustive ranges
 * (tests/test_oracle_math.py); the dot order and fma, the q = 0 and first-row
 * closed forms, float64 mathematics and the invariants
 * (tests/test_oracle_attn.py); the forward's l fold, acc rescale, LSE
 * composition, exp argument, O division and masked-block rules
 * (tests/fwd_probes.py, tests/test_oracle_fwd_probes.py); the backward's GQA
 * and query fold orders, Dsum from the stored O, sigma applied once and the dS
 * rounding (tests/bwd_probes.py, tests/test_oracle_bwd_probes.py).
 */
#include <math.h>
#include <quadmath.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#include <omp.h>

static inline uint32_t f2u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static inline float u2f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

/* Correctly rounded binary32 exp.  The binary64 libm value (error below one
 * binary64 ulp) decides the rounding unless it lies within 2^-48 (relative)
 * of a binary32 rounding boundary; those inputs are resolved with
 * libquadmath's expq (about 2^-112 relative), which no binary32 result of
 * exp comes close enough to a boundary to defeat. */
static float cr_round(double y, int* ok) {
  double e = y * 0x1p-48;
  float lo = (float)(y - e), hi = (float)(y + e);
  *ok = f2u(lo) == f2u(hi);
  return lo;
}

float orc_expf(float x) {
  if (x != x) return x;
  if (x == -INFINITY) return 0.0f;
  int ok;
  float f = cr_round(exp((double)x), &ok);
  if (ok) return f;
  return (float)expq((__float128)x);
}

float orc_logf(float x) {
  if (x != x || x < 0.0f) return NAN;
  if (x == 0.0f) return -INFINITY;
  if (x == INFINITY) return x;
  int ok;
  float f = cr_round(log((double)x), &ok);
  if (ok) return f;
  return (float)logq((__float128)x);
}

/* Reference correctly rounded values straight from libquadmath (slow). */
float orc_expf_quad(float x) { return (float)expq((__float128)x); }
float orc_logf_quad(float x) { return (float)logq((__float128)x); }
/* cos and sin of binary32 angles rounded once from libquadmath's binary128 values
 * (about 2^-112 relative): the checker of the RoPE tables, whose entries the
 * reference takes from repop's correctly rounded cos/sin (rope.py:29-31). */
void orc_cos_sin_quad_batch(const float* x, float* c, float* s, long n) {
#pragma omp parallel for schedule(static)
  for (long i = 0; i < n; i++) {
    c[i] = (float)cosq((__float128)x[i]);
    s[i] = (float)sinq((__float128)x[i]);
  }
}

/* sigma = RN(1/sqrt(D)) via binary128. */
float orc_scale(int D) { return (float)(1.0Q / sqrtq((__float128)D)); }

/* binary32 -> nearest-even bf16 value, returned as binary32. */
float orc_round_bf16(float f) {
  uint32_t u = f2u(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return u2f((u | 0x00400000u) & 0xffff0000u);
  uint32_t lsb = (u >> 16) & 1u;
  uint32_t r = u + 0x7fffu + lsb;
  return u2f(r & 0xffff0000u);
}

/* out[i] = fmaf(a[i], b[i], c[i]) (IEEE fused multiply-add, libm / FMA3). */
void orc_fmaf_batch(const float* a, const float* b, const float* c, float* out, long n) {
  for (long i = 0; i < n; i++) out[i] = fmaf(a[i], b[i], c[i]);
}

/* Order-independent checksum of (x, f(x)) over the bit patterns [lo, lo+count):
 * sum mod 2^64 of a 64-bit mix of the pair, f = orc_expf (which 0) or orc_logf
 * (which 1).  The GPU library computes the same sum with its own exp/log. */
static inline uint64_t mix64(uint32_t x, uint32_t y) {
  uint64_t h = ((uint64_t)x << 32) | y;
  h ^= h >> 33; h *= 0xff51afd7ed558ccdull; h ^= h >> 33; h *= 0xc4ceb9fe1a85ec53ull; h ^= h >> 33;
  return h;
}
uint64_t orc_math_checksum(int which, uint64_t lo, uint64_t count) {
  uint64_t s = 0;
#pragma omp parallel for reduction(+ : s) schedule(static)
  for (int64_t i = 0; i < (int64_t)count; i++) {
    uint32_t u = (uint32_t)(lo + (uint64_t)i);
    float x = u2f(u);
    float y = which == 0 ? orc_expf(x) : which == 1 ? orc_logf(x) : which == 4 ? orc_round_bf16(x) : rintf(x);
    s += mix64(u, f2u(y));
  }
  return s;
}

/* Mismatches of orc_expf / orc_logf against the quad reference on the bit
 * patterns [lo, hi) (NaNs skipped; log only for x >= 0). */
uint64_t orc_verify_math(uint32_t lo, uint32_t hi, int which) {
  uint64_t bad = 0;
#pragma omp parallel for reduction(+ : bad) schedule(static)
  for (int64_t u = lo; u < (int64_t)hi; u++) {
    float x = u2f((uint32_t)u);
    if (x != x) continue;
    if (which == 0) {
      if (f2u(orc_expf(x)) != f2u(orc_expf_quad(x))) bad++;
    } else if (x >= 0.0f) {
      if (f2u(orc_logf(x)) != f2u(orc_logf_quad(x))) bad++;
    }
  }
  return bad;
}

static inline int q_block_lo(int I, int window) {
  if (window <= 0) return 0;
  int lo = I - window / 32;
  return lo < 0 ? 0 : lo;
}
static inline int k_block_hi(int J, int window, int nb) {
  if (window <= 0) return nb - 1;
  int hi = J + window / 32;
  return hi > nb - 1 ? nb - 1 : hi;
}
static inline int masked(int i, int j, int window) {
  return j > i || (window > 0 && j <= i - window);
}
static inline float dotf(const float* x, const float* y, int D) {
  float a = 0.0f;
  for (int d = 0; d < D; d++) a = fmaf(x[d], y[d], a);
  return a;
}

static int check_shape(int B, int H, int Hkv, int S, int D, int window) {
  if (B <= 0 || H <= 0 || Hkv <= 0 || S <= 0 || D <= 0) return -1;
  if (H % Hkv) return -1;
  if (S % 32) return -1;
  if (window < 0 || window % 32) return -1;
  return 0;
}

/* Forward.  o receives RN(acc/l) (rounded to a bf16 value when out_bf16). */
int orc_attn_fwd(const float* q, const float* k, const float* v, float* o, float* lse, int B, int H,
                 int Hkv, int S, int D, int window, int out_bf16, int nthreads) {
  if (check_shape(B, H, Hkv, S, D, window)) return -1;
  const int G = H / Hkv;
  const float sigma = orc_scale(D);
  const long rows = (long)B * H * S;
  if (nthreads > 0) omp_set_num_threads(nthreads);
#pragma omp parallel
  {
    float* acc = (float*)malloc(sizeof(float) * D);
    float s[32], p[32];
#pragma omp for schedule(dynamic, 16)
    for (long row = 0; row < rows; row++) {
      const int i = (int)(row % S);
      const long bh = row / S;
      const int h = (int)(bh % H), b = (int)(bh / H);
      const int g = h / G;
      const float* qi = q + row * D;
      const float* kb = k + ((long)b * Hkv + g) * S * D;
      const float* vb = v + ((long)b * Hkv + g) * S * D;
      float m = -INFINITY, l = 0.0f;
      for (int d = 0; d < D; d++) acc[d] = 0.0f;
      const int I = i / 32;
      for (int J = q_block_lo(I, window); J <= I; J++) {
        for (int jj = 0; jj < 32; jj++) {
          const int j = 32 * J + jj;
          s[jj] = masked(i, j, window) ? -INFINITY : dotf(qi, kb + (long)j * D, D) * sigma;
        }
        float mb = s[0];
        for (int jj = 1; jj < 32; jj++)
          if (s[jj] > mb) mb = s[jj];
        const float mn = (mb > m) ? mb : m;
        const float alpha = (mn == m) ? 1.0f : orc_expf(m - mn);
        l = l * alpha;
        for (int jj = 0; jj < 32; jj++) {
          p[jj] = masked(i, 32 * J + jj, window) ? 0.0f : orc_expf(s[jj] - mn);
          l = l + p[jj];
        }
        for (int d = 0; d < D; d++) {
          float a = acc[d] * alpha;
          for (int jj = 0; jj < 32; jj++) a = fmaf(p[jj], vb[(long)(32 * J + jj) * D + d], a);
          acc[d] = a;
        }
        m = mn;
      }
      float* oi = o + row * D;
      for (int d = 0; d < D; d++) {
        float x = (float)((double)acc[d] / (double)l);
        oi[d] = out_bf16 ? orc_round_bf16(x) : x;
      }
      lse[row] = m + orc_logf(l);
    }
    free(acc);
  }
  return 0;
}

/* Backward.  o must hold the forward output as stored (bf16 values for bf16).
 * Groups (batch, KV head) are taken one at a time; inside a group the rows
 * (P, dS, dQ) and the key columns (dK, dV) are spread over the threads.  Each
 * output element is still reduced by one thread in the contract's order. */
int orc_attn_bwd(const float* q, const float* k, const float* v, const float* o, const float* lse,
                 const float* dO, float* dq, float* dk, float* dv, int B, int H, int Hkv, int S, int D,
                 int window, int out_bf16, int nthreads) {
  if (check_shape(B, H, Hkv, S, D, window)) return -1;
  const int G = H / Hkv;
  const int nb = S / 32;
  const float sigma = orc_scale(D);
  if (nthreads > 0) omp_set_num_threads(nthreads);
  /* P and dS of one group's heads, dense S x S per head (only processed blocks are filled). */
  float* P = (float*)malloc(sizeof(float) * (size_t)S * S * G);
  float* dS = (float*)malloc(sizeof(float) * (size_t)S * S * G);
  if (!P || !dS) { free(P); free(dS); return -2; }
  for (long bg = 0; bg < (long)B * Hkv; bg++) {
    const int b = (int)(bg / Hkv), g = (int)(bg % Hkv);
    const float* kb = k + ((long)b * Hkv + g) * S * D;
    const float* vb = v + ((long)b * Hkv + g) * S * D;
    for (int r = 0; r < G; r++) {
      const int h = g * G + r;
      const long base = ((long)b * H + h) * S;
      float* Pr = P + (size_t)r * S * S;
      float* dSr = dS + (size_t)r * S * S;
#pragma omp parallel for schedule(dynamic, 8)
      for (int i = 0; i < S; i++) {
        const int I = i / 32;
        const float* qi = q + (base + i) * D;
        const float* doi = dO + (base + i) * D;
        const float Li = lse[base + i];
        const float Di = dotf(doi, o + (base + i) * D, D);
        for (int j = 32 * q_block_lo(I, window); j < 32 * (I + 1); j++) {
          float pij;
          if (masked(i, j, window)) {
            pij = 0.0f;
          } else {
            const float s = dotf(qi, kb + (long)j * D, D) * sigma;
            pij = orc_expf(s - Li);
          }
          const float dp = dotf(doi, vb + (long)j * D, D);
          Pr[(size_t)i * S + j] = pij;
          dSr[(size_t)i * S + j] = pij * (dp - Di);
        }
        /* dQ row i: key blocks ascending, keys ascending. */
        float* dqi = dq + (base + i) * D;
        for (int d = 0; d < D; d++) {
          float a = 0.0f;
          for (int j = 32 * q_block_lo(I, window); j < 32 * (I + 1); j++)
            a = fmaf(dSr[(size_t)i * S + j], kb[(long)j * D + d], a);
          const float x = a * sigma;
          dqi[d] = out_bf16 ? orc_round_bf16(x) : x;
        }
      }
    }
    /* dK / dV for the group's KV head: heads ascending, query blocks ascending. */
#pragma omp parallel
    {
      float* accv = (float*)malloc(sizeof(float) * D);
      float* acck = (float*)malloc(sizeof(float) * D);
#pragma omp for schedule(dynamic, 8)
      for (int j = 0; j < S; j++) {
        const int J = j / 32;
        const int ihi = 32 * (k_block_hi(J, window, nb) + 1);
        for (int d = 0; d < D; d++) { accv[d] = 0.0f; acck[d] = 0.0f; }
        for (int r = 0; r < G; r++) {
          const int h = g * G + r;
          const long base = ((long)b * H + h) * S;
          const float* Pr = P + (size_t)r * S * S;
          const float* dSr = dS + (size_t)r * S * S;
          for (int i = 32 * J; i < ihi; i++) {
            const float pij = Pr[(size_t)i * S + j], dsij = dSr[(size_t)i * S + j];
            const float* doi = dO + (base + i) * D;
            const float* qi = q + (base + i) * D;
            for (int d = 0; d < D; d++) {
              accv[d] = fmaf(pij, doi[d], accv[d]);
              acck[d] = fmaf(dsij, qi[d], acck[d]);
            }
          }
        }
        float* dvj = dv + (((long)b * Hkv + g) * S + j) * D;
        float* dkj = dk + (((long)b * Hkv + g) * S + j) * D;
        for (int d = 0; d < D; d++) {
          const float x = acck[d] * sigma;
          dvj[d] = out_bf16 ? orc_round_bf16(accv[d]) : accv[d];
          dkj[d] = out_bf16 ? orc_round_bf16(x) : x;
        }
      }
      free(accv);
      free(acck);
    }
  }
  free(P);
  free(dS);
  return 0;
}
