/*
 * CPU oracle for the int8-PV attention forward.  TEST INFRASTRUCTURE ONLY:
 * tests/ and the benchmark's checks call it; the product never links or calls
 * it.
 *
 * Reference operator: repop.nn.flash_attention.int8pv_causal_flash_attention
 * (q, k, v, window=w), called at src/pretrain/model/modules/attention_repop.py:52
 * of the reference when ModelConfig.attn_int8_pv is set (the production
 * default: src/pretrain/config/schema.py:159-166).  The documented facts
 * (docs/MODEL_OP_DTYPE_TRACE.md:29-32,80,102): fp32 scores and online-softmax
 * statistics, P and V quantized to int8 per block, int32 P.V accumulation,
 * fp32 dequantization into an fp32 output accumulator, bf16 output; the
 * backward is the fp32 flash backward (straight-through "float shadow").  repop
 * is closed and absent, so the bit-level rules are this project's contract.
 * Everything not listed here is the binary32 forward of attn_oracle.c
 * (mask, blocks, s, mb, m', alpha, p, l, O = RN(acc / l), LSE):
 *
 *   V quantization, per (batch, KV head, key block J, column d):
 *     amax = max over the 32 keys of |v_j[d]| (NaN if any is NaN)
 *     amax = 0          -> qv_j[d] = 0, sv = 0
 *     amax not finite   -> qv_j[d] = 0, sv = NaN
 *     otherwise         inv = RN(127 / amax), sv = RN(amax / 127),
 *                       qv_j[d] = rint(RN(v_j[d] * inv))   (half-even, |qv| <= 127)
 *   P quantization, per (query row, processed key block):
 *     pmax = max_j p_j (ascending compare-select; p_j >= 0)
 *     pmax = 0          -> qp_j = 0, sp = 0
 *     otherwise         inv = RN(127 / pmax), sp = RN(pmax / 127),
 *                       qp_j = rint(RN(p_j * inv))          (0 <= qp <= 127)
 *   Accumulation, per column d:
 *     a_d    = sum_j qp_j * qv_j[d]     (exact integer, |a_d| <= 32 * 127 * 127)
 *     acc[d] = fma(RN(a_d * sv_d), sp, RN(acc[d] * alpha))
 *   l is the sum of the unquantized p, so LSE equals the binary32 forward's.
 *
 * Bound used by the clamps below: |x| * RN(127/|x|) < 127.5 for every finite x
 * with |x| >= 127 / FLT_MAX (about 3.7e-37), so the rounded quotient stays in
 * [-127, 127]; for a smaller block maximum 127/max overflows to +inf, every
 * nonzero value of the block then quantizes to +-inf and clamps to +-127, and a
 * zero value (0 * inf = NaN) quantizes to 0.
 *
 * Pinned independently of this file: the quantizer's properties, closed forms
 * on an exact grid, LSE identity with the binary32 forward and a float64 error
 * bound (tests/test_oracle_int8pv.py); the accumulate
 * fma(RN(a*sv), sp, RN(acc*alpha)) and both quantizers' multiply by
 * RN(127/max), each by a closed-form probe that a planted one-line deviation
 * of this file fails (tests/layer_probes.py, tests/test_oracle_layer_probes.py).
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#include <omp.h>

float orc_expf(float x);
float orc_logf(float x);
float orc_scale(int D);
float orc_round_bf16(float f);

static inline int masked(int i, int j, int window) { return j > i || (window > 0 && j <= i - window); }
static inline int q_block_lo(int I, int window) {
  if (window <= 0) return 0;
  int lo = I - window / 32;
  return lo < 0 ? 0 : lo;
}
static inline float dotf(const float* x, const float* y, int D) {
  float a = 0.0f;
  for (int d = 0; d < D; d++) a = fmaf(x[d], y[d], a);
  return a;
}
static inline float div_rn(float a, float b) { return (float)((double)a / (double)b); }
static inline int8_t quant(float x, float inv) {
  const float r = rintf(x * inv);
  if (r != r) return 0;
  return (int8_t)(r > 127.0f ? 127.0f : (r < -127.0f ? -127.0f : r));
}

/* qv [B,Hkv,S,D] int8 values, sv [B,Hkv,S/32,D]. */
int orc_quantize_v(const float* v, int8_t* qv, float* sv, int B, int Hkv, int S, int D) {
  if (B <= 0 || Hkv <= 0 || S <= 0 || S % 32 || D <= 0) return -1;
  const long nblk = (long)B * Hkv * (S / 32);
#pragma omp parallel for schedule(static)
  for (long blk = 0; blk < nblk; blk++) {
    const float* vb = v + blk * 32 * D;
    int8_t* qb = qv + blk * 32 * D;
    for (int d = 0; d < D; d++) {
      float amax = 0.0f;
      for (int j = 0; j < 32; j++) {
        const float a = fabsf(vb[(long)j * D + d]);
        if (a != a || a > amax) amax = a;
        if (amax != amax) break;
      }
      float s, inv;
      if (amax == 0.0f) {
        s = 0.0f, inv = 0.0f;
      } else if (!isfinite(amax)) {
        s = NAN, inv = 0.0f;
      } else {
        inv = div_rn(127.0f, amax), s = div_rn(amax, 127.0f);
      }
      sv[blk * D + d] = s;
      for (int j = 0; j < 32; j++) qb[(long)j * D + d] = inv == 0.0f ? 0 : quant(vb[(long)j * D + d], inv);
    }
  }
  return 0;
}

/* Forward with int8 P.V.  o receives RN(acc/l) (rounded to a bf16 value when out_bf16). */
int orc_attn_fwd_int8pv(const float* q, const float* k, const float* v, float* o, float* lse, int B, int H,
                        int Hkv, int S, int D, int window, int out_bf16, int nthreads) {
  if (B <= 0 || H <= 0 || Hkv <= 0 || S <= 0 || D <= 0 || H % Hkv || S % 32 || window < 0 || window % 32) return -1;
  const int G = H / Hkv;
  const float sigma = orc_scale(D);
  const long rows = (long)B * H * S;
  int8_t* qv = (int8_t*)malloc((size_t)B * Hkv * S * D);
  float* sv = (float*)malloc(sizeof(float) * (size_t)B * Hkv * (S / 32) * D);
  if (!qv || !sv) { free(qv); free(sv); return -2; }
  if (nthreads > 0) omp_set_num_threads(nthreads);
  orc_quantize_v(v, qv, sv, B, Hkv, S, D);
#pragma omp parallel
  {
    float* acc = (float*)malloc(sizeof(float) * D);
    float s[32], p[32];
    int qp[32];
#pragma omp for schedule(dynamic, 16)
    for (long row = 0; row < rows; row++) {
      const int i = (int)(row % S);
      const long bh = row / S;
      const int h = (int)(bh % H), b = (int)(bh / H);
      const long bg = (long)b * Hkv + h / G;
      const float* qi = q + row * D;
      const float* kb = k + bg * S * D;
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
        float pmax = 0.0f;
        for (int jj = 0; jj < 32; jj++) {
          p[jj] = masked(i, 32 * J + jj, window) ? 0.0f : orc_expf(s[jj] - mn);
          l = l + p[jj];
          if (p[jj] > pmax) pmax = p[jj];
        }
        float sp = 0.0f, inv = 0.0f;
        if (pmax > 0.0f) inv = div_rn(127.0f, pmax), sp = div_rn(pmax, 127.0f);
        for (int jj = 0; jj < 32; jj++) qp[jj] = inv == 0.0f ? 0 : quant(p[jj], inv);
        const int8_t* qvb = qv + (bg * S + 32L * J) * D;
        const float* svb = sv + (bg * (S / 32) + J) * D;
        for (int d = 0; d < D; d++) {
          int32_t a = 0;
          for (int jj = 0; jj < 32; jj++) a += qp[jj] * (int32_t)qvb[(long)jj * D + d];
          acc[d] = fmaf((float)a * svb[d], sp, acc[d] * alpha);
        }
        m = mn;
      }
      float* oi = o + row * D;
      for (int d = 0; d < D; d++) {
        const float x = div_rn(acc[d], l);
        oi[d] = out_bf16 ? orc_round_bf16(x) : x;
      }
      lse[row] = m + orc_logf(l);
    }
    free(acc);
  }
  free(qv);
  free(sv);
  return 0;
}
