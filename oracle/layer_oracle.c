/*
 * CPU oracle for the decoder-layer operators around the attention (BASELINE
 * configuration 5): bf16 GEMM with a serial binary32 fold, RMSNorm forward /
 * backward and SiLU forward / backward.  TEST INFRASTRUCTURE ONLY: tests/ and
 * the benchmark's checks call it; the product never links or calls it.
 *
 * The reference operators are repop.nn.linear.Linear, repop.nn.rmsnorm.rms_norm
 * and repop.nn.activations.silu (src/pretrain/model/modules/_linear.py:31-65,
 * norm_repop.py:19-22, ffn_repop.py:39-54 of the reference; dtypes in
 * docs/MODEL_OP_DTYPE_TRACE.md:76-82,100-105).  repop is closed and absent, so
 * the bit-level rules are this project's contract (binary32, RN, subnormals
 * kept, fma = one rounding; bf16 outputs are RNE of the binary32 value):
 *
 *   GEMM     C[i][j] = fold over r = 0..R-1 ascending of fma(A(i,r), B(j,r), acc),
 *            acc from +0 ("strict sequential fold ... no split-K":
 *            docs/unified-audit-results.md:71-74).
 *   fold32   partial_c = serial fma over the 32 indices of chunk c from +0; the
 *            partials are added in ascending c starting from +0.
 *   RMSNorm  ss = fold32(x*x); rstd = rsqrt(RN(RN(ss/D) + eps)) correctly
 *            rounded; y = RN(RN(x*rstd)*w).
 *            backward: xh = RN(x*rstd), g = RN(dy*w), c = RN(fold32(g*xh)/D),
 *            dx = RN(rstd*RN(g - RN(xh*c))), dw = fold32 over rows of dy*xh.
 *   SiLU     d = RN(1 + exp(-x)), y = RN(x/d); backward s = RN(1/d),
 *            dx = RN(dy*RN(s*RN(1 + RN(x*RN(1 - s))))), exp correctly rounded.
 *
 * Pinned independently of this file: the GEMM's serial order and exact
 * integer products, rsqrt against libquadmath, float64 mathematics
 * (tests/test_layer_cpu.py); RMSNorm's chunk-32 folds of ss, c and dw, the
 * divisions by D, y's rounding, dx's grouping, and SiLU's division and the
 * grouping of its derivative, each by a closed-form probe that a planted
 * one-line deviation of this file fails (tests/layer_probes.py,
 * tests/test_oracle_layer_probes.py).
 */
#include <math.h>
#include <quadmath.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#include <omp.h>

float orc_expf(float x);
float orc_round_bf16(float f);

/* Correctly rounded binary32 1/sqrt(x) from libquadmath (test infrastructure). */
float orc_rsqrtf(float x) {
  if (!(x > 0.0f)) return x == 0.0f ? INFINITY : NAN;
  return (float)(1.0Q / sqrtq((__float128)x));
}

static inline float out_round(float v, int out_bf16) { return out_bf16 ? orc_round_bf16(v) : v; }

/* C[i*ldc + j] for i < M, j < N. */
int orc_gemm(const float* A, long a_i, long a_r, const float* B, long b_j, long b_r, float* C, long ldc, int M,
             int N, int R, int out_bf16, int nthreads) {
  if (M <= 0 || N <= 0 || R <= 0) return -1;
  float* Bt = (float*)malloc(sizeof(float) * (size_t)R * N); /* Bt[r][j] */
  if (!Bt) return -2;
  for (long r = 0; r < R; r++)
    for (long j = 0; j < N; j++) Bt[r * N + j] = B[j * b_j + r * b_r];
  if (nthreads > 0) omp_set_num_threads(nthreads);
#pragma omp parallel
  {
    float* acc = (float*)malloc(sizeof(float) * N);
#pragma omp for schedule(dynamic, 4)
    for (long i = 0; i < M; i++) {
      for (long j = 0; j < N; j++) acc[j] = 0.0f;
      for (long r = 0; r < R; r++) {
        const float a = A[i * a_i + r * a_r];
        const float* br = Bt + r * N;
        for (long j = 0; j < N; j++) acc[j] = fmaf(a, br[j], acc[j]); /* independent chains over j */
      }
      for (long j = 0; j < N; j++) C[i * ldc + j] = out_round(acc[j], out_bf16);
    }
    free(acc);
  }
  free(Bt);
  return 0;
}

/* fold32 of term(i) over i < n (n a multiple of 32), for one row. */
static float fold32_row(const float* a, const float* b, int n) {
  float acc = 0.0f;
  for (int c = 0; c < n / 32; c++) {
    float p = 0.0f;
    for (int i = 32 * c; i < 32 * c + 32; i++) p = fmaf(a[i], b[i], p);
    acc = acc + p;
  }
  return acc;
}

int orc_rmsnorm_fwd(const float* x, const float* w, float* y, float* rstd, long rows, int D, float eps,
                    int out_bf16, int nthreads) {
  if (rows <= 0 || D <= 0 || D % 32) return -1;
  if (nthreads > 0) omp_set_num_threads(nthreads);
#pragma omp parallel for schedule(static)
  for (long r = 0; r < rows; r++) {
    const float* xr = x + r * D;
    const float ss = fold32_row(xr, xr, D);
    const float mean = (float)((double)ss / (double)D);
    const float rs = orc_rsqrtf(mean + eps);
    rstd[r] = rs;
    for (int d = 0; d < D; d++) {
      const float xh = xr[d] * rs;
      y[r * D + d] = out_round(xh * w[d], out_bf16);
    }
  }
  return 0;
}

int orc_rmsnorm_bwd(const float* x, const float* w, const float* rstd, const float* dy, float* dx, float* dw,
                    long rows, int D, int out_bf16, int nthreads) {
  if (rows <= 0 || rows % 32 || D <= 0 || D % 32) return -1;
  if (nthreads > 0) omp_set_num_threads(nthreads);
  float* xh = (float*)malloc(sizeof(float) * (size_t)rows * D);
  if (!xh) return -2;
#pragma omp parallel
  {
    float* g = (float*)malloc(sizeof(float) * D);
#pragma omp for schedule(static)
    for (long r = 0; r < rows; r++) {
      const float rs = rstd[r];
      for (int d = 0; d < D; d++) {
        xh[r * D + d] = x[r * D + d] * rs;
        g[d] = dy[r * D + d] * w[d];
      }
      const float dot = fold32_row(g, xh + r * D, D);
      const float cc = (float)((double)dot / (double)D);
      for (int d = 0; d < D; d++) dx[r * D + d] = out_round(rs * (g[d] - xh[r * D + d] * cc), out_bf16);
    }
    free(g);
  }
  /* dw: fold over rows in chunks of 32 */
#pragma omp parallel for schedule(static)
  for (int d = 0; d < D; d++) {
    float acc = 0.0f;
    for (long c = 0; c < rows / 32; c++) {
      float p = 0.0f;
      for (long r = 32 * c; r < 32 * c + 32; r++) p = fmaf(dy[r * D + d], xh[r * D + d], p);
      acc = acc + p;
    }
    dw[d] = acc;
  }
  free(xh);
  return 0;
}

int orc_silu_fwd(const float* x, float* y, long n, int out_bf16) {
#pragma omp parallel for schedule(static)
  for (long i = 0; i < n; i++) {
    const float d = 1.0f + orc_expf(-x[i]);
    y[i] = out_round((float)((double)x[i] / (double)d), out_bf16);
  }
  return 0;
}

int orc_silu_bwd(const float* x, const float* dy, float* dx, long n, int out_bf16) {
#pragma omp parallel for schedule(static)
  for (long i = 0; i < n; i++) {
    const float d = 1.0f + orc_expf(-x[i]);
    const float s = (float)(1.0 / (double)d);
    const float g = s * (1.0f + x[i] * (1.0f - s));
    dx[i] = out_round(dy[i] * g, out_bf16);
  }
  return 0;
}

/* Embedding backward: grad_w [V][D] = for each id, the fold over positions p
 * ascending with ids[p] == id of g[p][d] (binary32 additions from +0); ids
 * outside [0, V) are skipped (repop.nn.embedding.Embedding backward,
 * docs/MODEL_OP_DTYPE_TRACE.md:106: stable sort + fixed-order segment add). */
int orc_embedding_bwd(const int64_t* ids, const float* g, float* gw, long npos, int V, int D, int out_bf16) {
  if (npos <= 0 || V <= 0 || D <= 0) return -1;
  memset(gw, 0, sizeof(float) * (size_t)V * D);
  for (long p = 0; p < npos; p++) {
    const int64_t id = ids[p];
    if (id < 0 || id >= V) continue;
    float* row = gw + id * (long)D;
    const float* gr = g + p * (long)D;
    for (int d = 0; d < D; d++) row[d] = row[d] + gr[d];
  }
  if (out_bf16)
    for (long i = 0; i < (long)V * D; i++) gw[i] = orc_round_bf16(gw[i]);
  return 0;
}
