// RMSNorm and SiLU for the decoder layer around the attention (BASELINE
// configuration 5).
//
// RMSNorm replaces repop.nn.rmsnorm.rms_norm (src/pretrain/model/modules/
// norm_repop.py:19-22; fp32 arithmetic, correctly rounded rsqrt, output in the
// input dtype, fp32 weight gradient: docs/MODEL_OP_DTYPE_TRACE.md:76-77,105).
// SiLU replaces repop.nn.activations.silu (ffn_repop.py; correctly rounded
// exp: MODEL_OP_DTYPE_TRACE.md:81,101).  Contract (binary32, RN):
//   fold32(f, n)  = partials p_c = serial fma over i = 32c .. 32c+31 from +0,
//                   then acc = +0, acc = acc + p_c for c ascending
//   RMSNorm fwd   ss = fold32(x_d * x_d), rstd = rsqrt(RN(RN(ss / D) + eps)),
//                 y_d = RN(RN(x_d * rstd) * w_d) (stored in the input dtype)
//   RMSNorm bwd   xh_d = RN(x_d * rstd), g_d = RN(dy_d * w_d),
//                 c = RN(fold32(g_d * xh_d) / D),
//                 dx_d = RN(rstd * RN(g_d - RN(xh_d * c)))
//                 dw_d = fold32 over rows r of dy_rd * xh_rd   (binary32)
//   SiLU fwd      d = RN(1 + exp(-x)), y = RN(x / d)
//   SiLU bwd      s = RN(1 / d), g = RN(s * RN(1 + RN(x * RN(1 - s)))),
//                 dx = RN(dy * g)
//   SwiGLU        gate, up = the two halves of each row of gu [rows, 2F]
//                 (ffn_repop.py:52-54: chunk(2, -1), silu(gate) * up):
//                 y = put(SiLU(gate)), h = put(RN(y * up));
//                 backward gy = put(RN(dh * up)), dgate = put(RN(gy * g)),
//                 dup = put(RN(dh * y)) into dgu [rows, 2F] (the halves of
//                 chunk's backward, which concatenates them)
// exp and rsqrt are correctly rounded; bf16 results are RNE of the binary32
// value.  One wave per row for the row reductions: lane c computes partial
// c (a serial fma chain), the partials are folded in order.
#include <initializer_list>
#include "otx_common.h"

namespace otx {

// Partials of fold32 over one row, term(d, acc) = fma(f_d..., acc): chunk c is
// computed by lane c % 64 into slot c / 64.
template <int SLOTS, typename F>
__device__ __forceinline__ void row_partials(int D, F&& term, float (&part)[SLOTS]) {
  const int L = threadIdx.x & 63;
#pragma unroll
  for (int s = 0; s < SLOTS; s++) {
    const int cidx = s * 64 + L;
    float p = 0.0f;
    if (cidx * 32 < D) {
#pragma unroll 8
      for (int i = 0; i < 32; i++) p = term(cidx * 32 + i, p);
    }
    part[s] = p;
  }
}

// Ascending fold of the partials (chunk c in lane c % 64, slot c / 64); every
// lane ends with the same value.
template <int SLOTS>
__device__ __forceinline__ float fold_all(const float (&part)[SLOTS], int nch) {
  float acc = 0.0f;
#pragma unroll
  for (int s = 0; s < SLOTS; s++) {
    const int n = nch - 64 * s < 64 ? nch - 64 * s : 64;
    for (int l = 0; l < n; ++l) acc = acc + __shfl(part[s], l);
  }
  return acc;
}

template <typename T, int SLOTS>
__global__ __launch_bounds__(256) void rmsnorm_fwd_kernel(const T* __restrict__ x, const T* __restrict__ w,
                                                          T* __restrict__ y, float* __restrict__ rstd_out, long rows,
                                                          int D, float eps) {
  const long row = (long)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= rows) return;
  const int L = threadIdx.x & 63;
  const T* xr = x + row * D;
  float part[SLOTS];
  row_partials<SLOTS>(D, [&](int d, float acc) {
    const float v = Elem<T>::ld(xr + d);
    return __builtin_fmaf(v, v, acc);
  }, part);
  const float ss = fold_all<SLOTS>(part, D / 32);
  const float mean = otx_div_rn(ss, (float)D);
  const float rstd = otx_rsqrtf(mean + eps);
  T* yr = y + row * D;
  for (int d = L; d < D; d += 64) {
    const float xh = Elem<T>::ld(xr + d) * rstd;
    yr[d] = Elem<T>::put(xh * Elem<T>::ld(w + d));
  }
  if (L == 0) rstd_out[row] = rstd;
}

template <typename T, int SLOTS>
__global__ __launch_bounds__(256) void rmsnorm_bwd_kernel(const T* __restrict__ x, const T* __restrict__ w,
                                                          const float* __restrict__ rstd_in,
                                                          const T* __restrict__ dy, T* __restrict__ dx, long rows,
                                                          int D) {
  const long row = (long)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= rows) return;
  const int L = threadIdx.x & 63;
  const T* xr = x + row * D;
  const T* dyr = dy + row * D;
  const float rstd = rstd_in[row];
  float part[SLOTS];
  row_partials<SLOTS>(D, [&](int d, float acc) {
    const float xh = Elem<T>::ld(xr + d) * rstd;
    const float g = Elem<T>::ld(dyr + d) * Elem<T>::ld(w + d);
    return __builtin_fmaf(g, xh, acc);
  }, part);
  const float cc = otx_div_rn(fold_all<SLOTS>(part, D / 32), (float)D);
  T* dxr = dx + row * D;
  for (int d = L; d < D; d += 64) {
    const float xh = Elem<T>::ld(xr + d) * rstd;
    const float g = Elem<T>::ld(dyr + d) * Elem<T>::ld(w + d);
    dxr[d] = Elem<T>::put(rstd * (g - xh * cc));
  }
}

// Row-group form for D = 32 G with G a power of two up to 64: lane L of a wave
// owns chunk c = L % G of row L / G (64 / G rows per wave) and reads its 32
// elements with 16-byte loads; the partials are folded in order with G
// shuffles inside the row's lane group.  Same arithmetic as the kernels above.
template <typename T>
struct Chunk32 {
  static constexpr int NV = 32 * (int)sizeof(T) / 16;  // 16-byte vectors per chunk
  __device__ __forceinline__ static void load(const T* p, float (&v)[32]) {
#pragma unroll
    for (int k = 0; k < NV; k++) {
      const uint4 w = reinterpret_cast<const uint4*>(p)[k];
#pragma unroll
      for (int e = 0; e < Elem<T>::VEC; e++) v[k * Elem<T>::VEC + e] = Elem<T>::get(w, e);
    }
  }
  __device__ __forceinline__ static void store(T* p, const float (&v)[32]) {
#pragma unroll
    for (int k = 0; k < NV; k++) {
      uint4 w;
      uint32_t* wp = reinterpret_cast<uint32_t*>(&w);
      if constexpr (sizeof(T) == 2) {
#pragma unroll
        for (int q = 0; q < 4; q++)
          wp[q] = (uint32_t)Elem<T>::put(v[8 * k + 2 * q]) | ((uint32_t)Elem<T>::put(v[8 * k + 2 * q + 1]) << 16);
      } else {
#pragma unroll
        for (int q = 0; q < 4; q++) wp[q] = __float_as_uint(v[4 * k + q]);
      }
      reinterpret_cast<uint4*>(p)[k] = w;
    }
  }
};

// Ascending fold of the G partials of this lane's row group (every lane of the
// group ends with the same value).
template <int G>
__device__ __forceinline__ float fold_group(float p) {
  const int base = (threadIdx.x & 63) & ~(G - 1);
  float acc = 0.0f;
#pragma unroll
  for (int k = 0; k < G; k++) acc = acc + __shfl(p, base + k);
  return acc;
}

template <typename T, int G>
__global__ __launch_bounds__(256) void rmsnorm_fwd_rows_kernel(const T* __restrict__ x, const T* __restrict__ w,
                                                               T* __restrict__ y, float* __restrict__ rstd_out,
                                                               long rows, float eps) {
  constexpr int D = 32 * G, RPW = 64 / G;
  const int L = threadIdx.x & 63, c = L % G;
  const long row = ((long)blockIdx.x * 4 + (threadIdx.x >> 6)) * RPW + L / G;
  const bool live = row < rows;
  float v[32];
  if (live) Chunk32<T>::load(x + row * D + 32 * c, v);
  else
#pragma unroll
    for (int i = 0; i < 32; i++) v[i] = 0.0f;
  float p = 0.0f;
#pragma unroll
  for (int i = 0; i < 32; i++) p = __builtin_fmaf(v[i], v[i], p);
  const float ss = fold_group<G>(p);
  const float rstd = otx_rsqrtf(otx_div_rn(ss, (float)D) + eps);
  if (!live) return;
  float wv[32];
  Chunk32<T>::load(w + 32 * c, wv);
#pragma unroll
  for (int i = 0; i < 32; i++) v[i] = (v[i] * rstd) * wv[i];
  Chunk32<T>::store(y + row * D + 32 * c, v);
  if (c == 0) rstd_out[row] = rstd;
}

template <typename T, int G>
__global__ __launch_bounds__(256) void rmsnorm_bwd_rows_kernel(const T* __restrict__ x, const T* __restrict__ w,
                                                               const float* __restrict__ rstd_in,
                                                               const T* __restrict__ dy, T* __restrict__ dx,
                                                               long rows) {
  constexpr int D = 32 * G, RPW = 64 / G;
  const int L = threadIdx.x & 63, c = L % G;
  const long row = ((long)blockIdx.x * 4 + (threadIdx.x >> 6)) * RPW + L / G;
  const bool live = row < rows;
  float xh[32], g[32];
  float rstd = 0.0f;
  if (live) {
    float wv[32];
    rstd = rstd_in[row];
    Chunk32<T>::load(x + row * D + 32 * c, xh);
    Chunk32<T>::load(dy + row * D + 32 * c, g);
    Chunk32<T>::load(w + 32 * c, wv);
#pragma unroll
    for (int i = 0; i < 32; i++) {
      xh[i] = xh[i] * rstd;
      g[i] = g[i] * wv[i];
    }
  } else {
#pragma unroll
    for (int i = 0; i < 32; i++) xh[i] = g[i] = 0.0f;
  }
  float p = 0.0f;
#pragma unroll
  for (int i = 0; i < 32; i++) p = __builtin_fmaf(g[i], xh[i], p);
  const float cc = otx_div_rn(fold_group<G>(p), (float)D);
  if (!live) return;
#pragma unroll
  for (int i = 0; i < 32; i++) g[i] = rstd * (g[i] - xh[i] * cc);
  Chunk32<T>::store(dx + row * D + 32 * c, g);
}

// dw partials: part[c][d] = serial fma over rows 32c .. 32c+31 of dy * xh.
template <typename T>
__global__ __launch_bounds__(256) void rmsnorm_dw_partial_kernel(const T* __restrict__ x,
                                                                 const float* __restrict__ rstd_in,
                                                                 const T* __restrict__ dy, float* __restrict__ part,
                                                                 long rows, int D) {
  const int d = blockIdx.x * 256 + threadIdx.x;
  const long cidx = blockIdx.y;
  if (d >= D) return;
  float acc = 0.0f;
  for (int i = 0; i < 32; i++) {
    const long r = cidx * 32 + i;
    const float xh = Elem<T>::ld(x + r * D + d) * rstd_in[r];
    acc = __builtin_fmaf(Elem<T>::ld(dy + r * D + d), xh, acc);
  }
  part[cidx * D + d] = acc;
}

// out[d] = serial fold over c ascending of part[c][d], from +0.  The chain of
// one column is inherently serial, so the work is arranged for its loads:
// a workgroup owns FC_W columns and stages FC_R partials of each through LDS
// with all 256 threads loading at once (one 16-byte load per partial row), so
// that a column of up to FC_R partials costs one memory round trip; then FC_W
// threads add them in order.
constexpr int FC_W = 4, FC_R = 4096;
__global__ __launch_bounds__(256) void fold_columns_kernel(const float* __restrict__ part, float* __restrict__ out,
                                                           long nch, int D) {
  __shared__ __align__(16) float tile[FC_R * FC_W];
  const int d0 = blockIdx.x * FC_W;
  const int t = threadIdx.x;
  float acc = 0.0f;
  for (long c0 = 0; c0 < nch; c0 += FC_R) {
    const int rows = nch - c0 < FC_R ? (int)(nch - c0) : FC_R;
    constexpr int PER = FC_R / 256;
    float4 v[PER];
#pragma unroll
    for (int k = 0; k < PER; k++) {
      const int r = t + 256 * k;
      v[k] = r < rows ? *reinterpret_cast<const float4*>(part + (c0 + r) * D + d0) : make_float4(0.f, 0.f, 0.f, 0.f);
    }
#pragma unroll
    for (int k = 0; k < PER; k++) reinterpret_cast<float4*>(tile)[t + 256 * k] = v[k];
    __syncthreads();
    if (t < FC_W) {
      int r = 0;
      for (; r + 16 <= rows; r += 16) {
        float q[16];
#pragma unroll
        for (int u = 0; u < 16; u++) q[u] = tile[(r + u) * FC_W + t];
#pragma unroll
        for (int u = 0; u < 16; u++) acc = acc + q[u];
      }
      for (; r < rows; r++) acc = acc + tile[r * FC_W + t];
    }
    __syncthreads();
  }
  if (t < FC_W) out[d0 + t] = acc;
}

__device__ __forceinline__ float silu_denominator(float x) { return 1.0f + otx_expf(-x); }

template <typename T>
__global__ __launch_bounds__(256) void silu_fwd_kernel(const T* __restrict__ x, T* __restrict__ y, long n) {
  const long i = (long)blockIdx.x * 256 + threadIdx.x;
  if (i >= n) return;
  const float v = Elem<T>::ld(x + i);
  y[i] = Elem<T>::put(otx_div_rn(v, silu_denominator(v)));
}

template <typename T>
__global__ __launch_bounds__(256) void silu_bwd_kernel(const T* __restrict__ x, const T* __restrict__ dy,
                                                       T* __restrict__ dx, long n) {
  const long i = (long)blockIdx.x * 256 + threadIdx.x;
  if (i >= n) return;
  const float v = Elem<T>::ld(x + i);
  const float s = otx_div_rn(1.0f, silu_denominator(v));
  const float g = s * (1.0f + v * (1.0f - s));
  dx[i] = Elem<T>::put(Elem<T>::ld(dy + i) * g);
}

// SwiGLU over rows of gu = [gate | up] (each F wide): one thread per 16 bytes of
// h, i.e. 8 bf16 or 4 binary32 elements of gate, up and h.
template <typename T>
struct Swiglu16 {
  static constexpr int N = 16 / sizeof(T);
  __device__ __forceinline__ static void load(const T* p, float (&v)[N]) {
    const uint4 w = *(const uint4*)p;
#pragma unroll
    for (int e = 0; e < N; e++) v[e] = Elem<T>::get(w, e);
  }
  __device__ __forceinline__ static void store(T* p, const float (&v)[N]) {
    uint4 w;
    uint32_t* wp = (uint32_t*)&w;
    if constexpr (sizeof(T) == 2) {
#pragma unroll
      for (int k = 0; k < 4; k++)
        wp[k] = (uint32_t)Elem<T>::put(v[2 * k]) | ((uint32_t)Elem<T>::put(v[2 * k + 1]) << 16);
    } else {
#pragma unroll
      for (int k = 0; k < 4; k++) wp[k] = __float_as_uint(v[k]);
    }
    *(uint4*)p = w;
  }
  __device__ __forceinline__ static float round(float v) {
    if constexpr (sizeof(T) == 2)
      return otx_bf16_to_f32(otx_f32_to_bf16(v));
    else
      return v;
  }
};

template <typename T>
__global__ __launch_bounds__(256) void swiglu_fwd_kernel(const T* __restrict__ gu, T* __restrict__ h, long rows,
                                                         int F) {
  constexpr int N = Swiglu16<T>::N;
  const int CPR = F / N;
  const long g = (long)blockIdx.x * 256 + threadIdx.x;
  if (g >= rows * CPR) return;
  const long row = g / CPR;
  const int c = (int)(g - row * CPR);
  float x[N], u[N], r[N];
  Swiglu16<T>::load(gu + row * 2 * F + c * N, x);
  Swiglu16<T>::load(gu + row * 2 * F + F + c * N, u);
#pragma unroll
  for (int e = 0; e < N; e++) {
    const float y = Swiglu16<T>::round(otx_div_rn(x[e], silu_denominator(x[e])));
    r[e] = y * u[e];
  }
  Swiglu16<T>::store(h + row * F + c * N, r);
}

template <typename T>
__global__ __launch_bounds__(256) void swiglu_bwd_kernel(const T* __restrict__ gu, const T* __restrict__ dh,
                                                         T* __restrict__ dgu, long rows, int F) {
  constexpr int N = Swiglu16<T>::N;
  const int CPR = F / N;
  const long g = (long)blockIdx.x * 256 + threadIdx.x;
  if (g >= rows * CPR) return;
  const long row = g / CPR;
  const int c = (int)(g - row * CPR);
  float x[N], u[N], d[N], dg[N], du[N];
  Swiglu16<T>::load(gu + row * 2 * F + c * N, x);
  Swiglu16<T>::load(gu + row * 2 * F + F + c * N, u);
  Swiglu16<T>::load(dh + row * F + c * N, d);
#pragma unroll
  for (int e = 0; e < N; e++) {
    const float den = silu_denominator(x[e]);
    const float y = Swiglu16<T>::round(otx_div_rn(x[e], den));
    const float s = otx_div_rn(1.0f, den);
    const float gy = Swiglu16<T>::round(d[e] * u[e]);
    const float gs = s * (1.0f + x[e] * (1.0f - s));
    dg[e] = gy * gs;
    du[e] = d[e] * y;
  }
  Swiglu16<T>::store(dgu + row * 2 * F + c * N, dg);
  Swiglu16<T>::store(dgu + row * 2 * F + F + c * N, du);
}

static bool aligned16p(const void* p) { return ((uintptr_t)p & 15u) == 0; }

// Rows of width D = 32 G (G a power of two up to 64) go to the row-group
// kernels when every row pointer is 16-byte aligned.
static int row_group(int D, std::initializer_list<const void*> ptrs) {
  if (D % 32) return 0;
  const int G = D / 32;
  if (G > 64 || (G & (G - 1))) return 0;
  for (const void* p : ptrs)
    if (!aligned16p(p)) return 0;
  return G;
}

template <typename T, int G>
static void launch_rows_fwd(const void* x, const void* w, void* y, float* rstd, long rows, float eps,
                            hipStream_t st) {
  const long per_block = 4L * (64 / G);
  hipLaunchKernelGGL((rmsnorm_fwd_rows_kernel<T, G>), dim3((unsigned)((rows + per_block - 1) / per_block)), dim3(256),
                     0, st, (const T*)x, (const T*)w, (T*)y, rstd, rows, eps);
}

template <typename T, int G>
static void launch_rows_bwd(const void* x, const void* w, const float* rstd, const void* dy, void* dx, long rows,
                            hipStream_t st) {
  const long per_block = 4L * (64 / G);
  hipLaunchKernelGGL((rmsnorm_bwd_rows_kernel<T, G>), dim3((unsigned)((rows + per_block - 1) / per_block)), dim3(256),
                     0, st, (const T*)x, (const T*)w, rstd, (const T*)dy, (T*)dx, rows);
}

template <typename T>
static bool launch_rows_fwd_any(int G, const void* x, const void* w, void* y, float* rstd, long rows, float eps,
                                hipStream_t st) {
  switch (G) {
    case 1: launch_rows_fwd<T, 1>(x, w, y, rstd, rows, eps, st); return true;
    case 2: launch_rows_fwd<T, 2>(x, w, y, rstd, rows, eps, st); return true;
    case 4: launch_rows_fwd<T, 4>(x, w, y, rstd, rows, eps, st); return true;
    case 8: launch_rows_fwd<T, 8>(x, w, y, rstd, rows, eps, st); return true;
    case 16: launch_rows_fwd<T, 16>(x, w, y, rstd, rows, eps, st); return true;
    case 32: launch_rows_fwd<T, 32>(x, w, y, rstd, rows, eps, st); return true;
    case 64: launch_rows_fwd<T, 64>(x, w, y, rstd, rows, eps, st); return true;
    default: return false;
  }
}

template <typename T>
static bool launch_rows_bwd_any(int G, const void* x, const void* w, const float* rstd, const void* dy, void* dx,
                                long rows, hipStream_t st) {
  switch (G) {
    case 1: launch_rows_bwd<T, 1>(x, w, rstd, dy, dx, rows, st); return true;
    case 2: launch_rows_bwd<T, 2>(x, w, rstd, dy, dx, rows, st); return true;
    case 4: launch_rows_bwd<T, 4>(x, w, rstd, dy, dx, rows, st); return true;
    case 8: launch_rows_bwd<T, 8>(x, w, rstd, dy, dx, rows, st); return true;
    case 16: launch_rows_bwd<T, 16>(x, w, rstd, dy, dx, rows, st); return true;
    case 32: launch_rows_bwd<T, 32>(x, w, rstd, dy, dx, rows, st); return true;
    case 64: launch_rows_bwd<T, 64>(x, w, rstd, dy, dx, rows, st); return true;
    default: return false;
  }
}

template <typename T>
static hipError_t launch_rmsnorm_fwd_t(const void* x, const void* w, void* y, float* rstd, long rows, int D,
                                       float eps, hipStream_t st) {
  if (launch_rows_fwd_any<T>(row_group(D, {x, w, y}), x, w, y, rstd, rows, eps, st)) return hipGetLastError();
  const dim3 grid((unsigned)((rows + 3) / 4)), block(256);
  if (D <= 2048)
    hipLaunchKernelGGL((rmsnorm_fwd_kernel<T, 1>), grid, block, 0, st, (const T*)x, (const T*)w, (T*)y, rstd, rows,
                       D, eps);
  else
    hipLaunchKernelGGL((rmsnorm_fwd_kernel<T, 4>), grid, block, 0, st, (const T*)x, (const T*)w, (T*)y, rstd, rows,
                       D, eps);
  return hipGetLastError();
}

hipError_t launch_rmsnorm_fwd(int dtype, const void* x, const void* w, void* y, float* rstd, long rows, int D,
                              float eps, hipStream_t st) {
  return dtype == 1 ? launch_rmsnorm_fwd_t<uint16_t>(x, w, y, rstd, rows, D, eps, st)
                    : launch_rmsnorm_fwd_t<float>(x, w, y, rstd, rows, D, eps, st);
}

template <typename T>
static hipError_t launch_rmsnorm_bwd_t(const void* x, const void* w, const float* rstd, const void* dy, void* dx,
                                       float* dw, float* part, long rows, int D, hipStream_t st) {
  const dim3 grid((unsigned)((rows + 3) / 4)), block(256);
  if (!launch_rows_bwd_any<T>(row_group(D, {x, w, dy, dx}), x, w, rstd, dy, dx, rows, st)) {
    if (D <= 2048)
      hipLaunchKernelGGL((rmsnorm_bwd_kernel<T, 1>), grid, block, 0, st, (const T*)x, (const T*)w, rstd,
                         (const T*)dy, (T*)dx, rows, D);
    else
      hipLaunchKernelGGL((rmsnorm_bwd_kernel<T, 4>), grid, block, 0, st, (const T*)x, (const T*)w, rstd,
                         (const T*)dy, (T*)dx, rows, D);
  }
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  const long nch = rows / 32;
  hipLaunchKernelGGL((rmsnorm_dw_partial_kernel<T>), dim3((unsigned)((D + 255) / 256), (unsigned)nch), dim3(256), 0,
                     st, (const T*)x, rstd, (const T*)dy, part, rows, D);
  e = hipGetLastError();
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL(fold_columns_kernel, dim3((unsigned)((D + FC_W - 1) / FC_W)), dim3(256), 0, st, part, dw, nch, D);
  return hipGetLastError();
}

hipError_t launch_rmsnorm_bwd(int dtype, const void* x, const void* w, const float* rstd, const void* dy, void* dx,
                              float* dw, float* part, long rows, int D, hipStream_t st) {
  return dtype == 1 ? launch_rmsnorm_bwd_t<uint16_t>(x, w, rstd, dy, dx, dw, part, rows, D, st)
                    : launch_rmsnorm_bwd_t<float>(x, w, rstd, dy, dx, dw, part, rows, D, st);
}

hipError_t launch_swiglu(int dtype, int backward, const void* gu, const void* dh, void* out, long rows, int F,
                         hipStream_t st) {
  const long threads = rows * (F / (dtype == 1 ? 8 : 4));
  const dim3 grid((unsigned)((threads + 255) / 256)), block(256);
  if (dtype == 1) {
    if (backward)
      hipLaunchKernelGGL((swiglu_bwd_kernel<uint16_t>), grid, block, 0, st, (const uint16_t*)gu, (const uint16_t*)dh,
                         (uint16_t*)out, rows, F);
    else
      hipLaunchKernelGGL((swiglu_fwd_kernel<uint16_t>), grid, block, 0, st, (const uint16_t*)gu, (uint16_t*)out,
                         rows, F);
  } else {
    if (backward)
      hipLaunchKernelGGL((swiglu_bwd_kernel<float>), grid, block, 0, st, (const float*)gu, (const float*)dh,
                         (float*)out, rows, F);
    else
      hipLaunchKernelGGL((swiglu_fwd_kernel<float>), grid, block, 0, st, (const float*)gu, (float*)out, rows, F);
  }
  return hipGetLastError();
}

hipError_t launch_silu(int dtype, int backward, const void* x, const void* dy, void* out, long n, hipStream_t st) {
  const dim3 grid((unsigned)((n + 255) / 256)), block(256);
  if (dtype == 1) {
    if (backward)
      hipLaunchKernelGGL((silu_bwd_kernel<uint16_t>), grid, block, 0, st, (const uint16_t*)x, (const uint16_t*)dy,
                         (uint16_t*)out, n);
    else
      hipLaunchKernelGGL((silu_fwd_kernel<uint16_t>), grid, block, 0, st, (const uint16_t*)x, (uint16_t*)out, n);
  } else {
    if (backward)
      hipLaunchKernelGGL((silu_bwd_kernel<float>), grid, block, 0, st, (const float*)x, (const float*)dy,
                         (float*)out, n);
    else
      hipLaunchKernelGGL((silu_fwd_kernel<float>), grid, block, 0, st, (const float*)x, (float*)out, n);
  }
  return hipGetLastError();
}

}  // namespace otx
