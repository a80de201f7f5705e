/*
 * CPU oracle for the fused cross-entropy + z-loss.  TEST INFRASTRUCTURE ONLY:
 * tests/ and the benchmark's checks call it; the product never links or calls
 * it.
 *
 * Reference: pretrain.model.fused_loss.fused_ce_z_loss and _FusedCEZLoss
 * (src/pretrain/model/fused_loss.py:40-120) over _z_loss_lse
 * (src/pretrain/model/z_loss.py:53-66).  The reference is plain torch around
 * repop.ops.{exp, sum_dim, log, mean, pow}; its elementwise steps are restated
 * literally, the repop reductions get this project's order (repop is closed).
 * Binary32, RN, subnormals kept; x = the binary32 value of a logit.
 *
 *   fold(a[0..n))  recursive chunk-32 fold: partials p_c = a[32c] + ... +
 *                  a[min(32c+32, n) - 1] added serially from +0; repeat on the
 *                  partials until one value is left (n = 0 gives +0).
 *   per row n:     m = max_v x_v;  e_v = exp(RN(x_v - m));  Z = fold(e);
 *                  lse = RN(log(Z) + m);  d_n = RN(lse - x_label);  q_n = RN(lse * lse)
 *   forward:       ce = RN(fold(d) / N);  z = coeff == 0 ? +0 : RN(f32(coeff) * RN(fold(q) / N))
 *   backward:      (gce, gz = upstream gradients of ce and z)
 *                  cs = RN(gce * f32(1.0 / N));  c2 = f32(2.0 * coeff * (1.0 / N))  [binary64 host math]
 *                  coef_n = RN(RN(c2 * gz) * lse_n)
 *                  sm = RN(e_v / Z);  g = RN(sm * cs);  coeff != 0: g = RN(g + RN(sm * coef_n))
 *                  v == label: g = RN(g - cs);  stored in the logits dtype (bf16 RNE).
 * exp and log are correctly rounded.  A label outside [0, V) makes d_n NaN.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#include <omp.h>

float orc_expf(float x);
float orc_logf(float x);
float orc_round_bf16(float f);

/* Recursive chunk-32 fold; scratch must hold ceil(n/32) floats (may alias nothing). */
static float fold32t(const float* a, long n, float* scratch) {
  if (n <= 0) return 0.0f;
  const float* src = a;
  long cur = n;
  while (1) {
    const long parts = (cur + 31) / 32;
    for (long c = 0; c < parts; c++) {
      float s = 0.0f;
      const long hi = 32 * c + 32 < cur ? 32 * c + 32 : cur;
      for (long i = 32 * c; i < hi; i++) s = s + src[i];
      scratch[c] = s; /* c <= 32c: never overwrites an unread source element */
    }
    if (parts == 1) return scratch[0];
    src = scratch;
    cur = parts;
  }
}

float orc_fold32t(const float* a, long n) {
  float* s = (float*)malloc(sizeof(float) * ((n + 31) / 32 + 1));
  const float r = fold32t(a, n, s);
  free(s);
  return r;
}

static inline float div_rn(float a, float b) { return (float)((double)a / (double)b); }

/* stats [5][N]: m, Z, lse, d, q.  loss[2] = (ce, z). */
int orc_ce_zloss_fwd(const float* logits, const int64_t* labels, long N, int V, double coeff, float* stats,
                     float* loss, int nthreads) {
  if (N <= 0 || V <= 0 || N >= (1L << 24)) return -1;
  if (nthreads > 0) omp_set_num_threads(nthreads);
  float *sm = stats, *sz = stats + N, *sl = stats + 2 * N, *sd = stats + 3 * N, *sq = stats + 4 * N;
#pragma omp parallel
  {
    float* e = (float*)malloc(sizeof(float) * V);
    float* scr = (float*)malloc(sizeof(float) * ((V + 31) / 32 + 1));
#pragma omp for schedule(static)
    for (long n = 0; n < N; n++) {
      const float* x = logits + n * (long)V;
      float m = x[0];
      for (int v = 1; v < V; v++)
        if (x[v] > m) m = x[v];
      for (int v = 0; v < V; v++) e[v] = orc_expf(x[v] - m);
      const float Z = fold32t(e, V, scr);
      const float lse = orc_logf(Z) + m;
      const int64_t lab = labels[n];
      sm[n] = m;
      sz[n] = Z;
      sl[n] = lse;
      sd[n] = (lab >= 0 && lab < V) ? lse - x[lab] : NAN;
      sq[n] = lse * lse;
    }
    free(e);
    free(scr);
  }
  float* scr = (float*)malloc(sizeof(float) * ((N + 31) / 32 + 1));
  loss[0] = div_rn(fold32t(sd, N, scr), (float)N);
  loss[1] = coeff == 0.0 ? 0.0f : (float)coeff * div_rn(fold32t(sq, N, scr), (float)N);
  free(scr);
  return 0;
}

/* Rows [0, N) of a batch of n_total rows (n_total sets the 1/N scale; stats
 * holds the N rows' columns of the [5][N] layout). */
int orc_ce_zloss_bwd(const float* logits, const int64_t* labels, const float* stats, float gce, float gz, long N,
                     long n_total, int V, double coeff, float* grad, int out_bf16, int nthreads) {
  if (N <= 0 || V <= 0 || n_total < N || n_total >= (1L << 24)) return -1;
  if (nthreads > 0) omp_set_num_threads(nthreads);
  const float cs = gce * (float)(1.0 / (double)n_total);
  const float c2 = (float)(2.0 * coeff * (1.0 / (double)n_total));
  const float *sm = stats, *sz = stats + N, *sl = stats + 2 * N;
#pragma omp parallel for schedule(static)
  for (long n = 0; n < N; n++) {
    const float* x = logits + n * (long)V;
    float* g = grad + n * (long)V;
    const float coef = (c2 * gz) * sl[n];
    for (int v = 0; v < V; v++) {
      const float s = div_rn(orc_expf(x[v] - sm[n]), sz[n]);
      float t = s * cs;
      if (coeff != 0.0) t = t + s * coef;
      if (v == labels[n]) t = t - cs;
      g[v] = out_bf16 ? orc_round_bf16(t) : t;
    }
  }
  return 0;
}
