// Fused cross-entropy + z-loss for gfx950.
//
// Replaces pretrain.model.fused_loss.fused_ce_z_loss / _FusedCEZLoss
// (src/pretrain/model/fused_loss.py:40-120 of the reference) and the
// logsumexp of _z_loss_lse (src/pretrain/model/z_loss.py:53-66).  Contract
// (binary32, RN; exp and log correctly rounded):
//   fold(a[0..n))  recursive chunk-32 fold: partials of 32 consecutive values
//                  summed serially from +0, repeated on the partials until one
//                  value is left
//   per row        m = max x;  e_v = exp(RN(x_v - m));  Z = fold(e);
//                  lse = RN(log Z + m);  d = RN(lse - x_label);  q = RN(lse * lse)
//   forward        ce = RN(fold(d) / N);  z = coeff == 0 ? +0 : RN(f32(coeff) * RN(fold(q) / N))
//   backward       cs = RN(gce * f32(1/N));  c2 = f32(2 coeff / N);  coef = RN(RN(c2 * gz) * lse)
//                  sm = RN(e_v / Z);  g = RN(sm * cs);  coeff != 0: g = RN(g + RN(sm * coef));
//                  v == label: g = RN(g - cs);  stored in the logits dtype
// Layout: logits [N][V] row-major (bf16 or binary32), labels [N] int64,
// stats [5][N] binary32 = (m, Z, lse, d, q), loss [2] = (ce, z).
//
// Forward: one 1024-thread workgroup per row (chunk c of 32 logits in thread
// c % 1024): a pass for the maximum, a second pass (served by the cache) for
// exp and the chunk partials, then the fold of the partials in LDS.  The
// correctly rounded exp needs too many temporaries to also keep a 128k-logit
// row in registers.  Backward: elementwise from the stored (m, Z, lse); one
// thread per 8 logits, 16-byte loads and stores.
#include "otx_common.h"

namespace otx {

constexpr int CE_LT = 1024;           // threads per row in the forward
constexpr int CE_MAX_CHUNKS = 4096;   // 32-logit chunks per row: V <= 131072
constexpr int CE_TPB = 32;            // backward: 2048-logit tiles per workgroup

// Recursive chunk-32 fold of a[0..n) (a, b: LDS buffers, b >= ceil(n/32)).
// Every thread of the block calls it with the same n; all see the result.
__device__ float block_fold32(float* a, float* b, int n) {
  float* src = a;
  float* dst = b;
  while (n > 1) {
    const int parts = (n + 31) / 32;
    for (int c = threadIdx.x; c < parts; c += blockDim.x) {
      const int hi = 32 * c + 32 < n ? 32 * c + 32 : n;
      float s = 0.0f;
      for (int i = 32 * c; i < hi; i++) s = s + src[i];
      dst[c] = s;
    }
    __syncthreads();
    float* t = src;
    src = dst;
    dst = t;
    n = parts;
  }
  return src[0];
}

template <typename T> struct CeWords { static constexpr int W = 32 * sizeof(T) / 4; };

template <typename T>
__device__ __forceinline__ float ce_elem(const uint32_t* raw, int i) {
  if constexpr (sizeof(T) == 2) {
    const uint32_t w = raw[i >> 1];
    return __uint_as_float((i & 1) ? (w & 0xffff0000u) : (w << 16));
  } else {
    return __uint_as_float(raw[i]);
  }
}

// The 32 logits of chunk c (binary32 bit patterns; -inf past the end of the row).
template <typename T>
__device__ __forceinline__ void ce_load_chunk(const T* row, int c, int V, int vec, uint32_t (&raw)[CeWords<T>::W]) {
  constexpr int W = CeWords<T>::W;
  if (vec && 32 * c + 32 <= V) {
    const uint4* src = reinterpret_cast<const uint4*>(row + 32 * c);
#pragma unroll
    for (int x = 0; x < W / 4; x++) {
      const uint4 u = src[x];
      raw[4 * x] = u.x; raw[4 * x + 1] = u.y; raw[4 * x + 2] = u.z; raw[4 * x + 3] = u.w;
    }
    return;
  }
  const uint32_t ninf = sizeof(T) == 2 ? 0xff80ff80u : 0xff800000u;
#pragma unroll
  for (int x = 0; x < W; x++) raw[x] = ninf;
#pragma unroll
  for (int i = 0; i < 32; i++) {
    if (32 * c + i >= V) continue;
    if constexpr (sizeof(T) == 2) {
      const uint32_t bits = reinterpret_cast<const uint16_t*>(row)[32 * c + i];
      raw[i >> 1] = (i & 1) ? ((raw[i >> 1] & 0xffffu) | (bits << 16)) : ((raw[i >> 1] & 0xffff0000u) | bits);
    } else {
      raw[i] = reinterpret_cast<const uint32_t*>(row)[32 * c + i];
    }
  }
}

// One row per workgroup: the maximum (first pass over the row), then exp and
// the level-0 partials (second pass, from registers for bf16 rows, from the
// cache for binary32 ones), then the fold of the partials in LDS.
template <typename T>
__global__ __launch_bounds__(CE_LT) void ce_fwd_kernel(const T* __restrict__ logits,
                                                       const int64_t* __restrict__ labels, long N, int V, int vec,
                                                       float* __restrict__ stats) {
  constexpr int W = CeWords<T>::W;
  __shared__ double tab[OTX_EXP_LE0_TAB_N];
  __shared__ float pa[CE_MAX_CHUNKS];
  __shared__ float pb[CE_MAX_CHUNKS / 32];
  __shared__ float wmax[CE_LT / 64];
  const long n = blockIdx.x;
  const int t = threadIdx.x;
  otx_load_exp_table(tab);
  const T* row = logits + (size_t)n * V;
  const int nch = (V + 31) / 32;

  // bf16 rows stay in registers between the two passes (PER chunks of 16
  // words per thread); binary32 rows are read twice (the second pass is
  // served by the cache).
  constexpr bool KEEP = sizeof(T) == 2;
  constexpr int PER = KEEP ? CE_MAX_CHUNKS / CE_LT : 1;
  uint32_t keep[PER][W];
  float mx = -__builtin_inff();
  if constexpr (KEEP) {
#pragma unroll
    for (int k = 0; k < PER; k++) {
      const int c = t + k * CE_LT;
      if (c < nch) {
        ce_load_chunk<T>(row, c, V, vec, keep[k]);
#pragma unroll
        for (int i = 0; i < 32; i++) {
          const float x = ce_elem<T>(keep[k], i);
          mx = x > mx ? x : mx;
        }
      }
    }
  } else {
    for (int c = t; c < nch; c += CE_LT) {
      uint32_t raw[W];
      ce_load_chunk<T>(row, c, V, vec, raw);
#pragma unroll
      for (int i = 0; i < 32; i++) {
        const float x = ce_elem<T>(raw, i);
        mx = x > mx ? x : mx;
      }
    }
  }
  // block maximum (exact in any order)
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) {
    const float y = __shfl_xor(mx, o);
    mx = y > mx ? y : mx;
  }
  if ((t & 63) == 0) wmax[t >> 6] = mx;
  __syncthreads();
  float m = wmax[0];
#pragma unroll
  for (int w = 1; w < CE_LT / 64; w++) m = wmax[w] > m ? wmax[w] : m;

  // exp and the level-0 partials (chunk c of 32 logits, summed serially from +0)
  if constexpr (KEEP) {
#pragma unroll
    for (int k = 0; k < PER; k++) {
      const int c = t + k * CE_LT;
      if (c < nch) {
        float s = 0.0f;
#pragma unroll
        for (int h = 0; h < 2; h++) {  // the chunk in two halves of 16 (fewer live registers, same order)
          float e[16];
#pragma unroll
          for (int i = 0; i < 16; i++) e[i] = ce_elem<T>(keep[k], 16 * h + i) - m;
          otx_exp_n<16, true, 4>(e, tab);
#pragma unroll
          for (int i = 0; i < 16; i++) s = s + e[i];  // padding contributes +0 at the end: s + 0 == s
        }
        pa[c] = s;
      }
    }
  } else {
    for (int c = t; c < nch; c += CE_LT) {
      uint32_t raw[W];
      ce_load_chunk<T>(row, c, V, vec, raw);
      float e[32];
#pragma unroll
      for (int i = 0; i < 32; i++) e[i] = ce_elem<T>(raw, i) - m;
      otx_exp_n<32, true>(e, tab);
      float s = 0.0f;
#pragma unroll
      for (int i = 0; i < 32; i++) s = s + e[i];  // padding contributes +0 at the end: s + 0 == s
      pa[c] = s;
    }
  }
  __syncthreads();
  const float Z = block_fold32(pa, pb, nch);
  if (t == 0) {
    const float lse = otx_logf(Z) + m;
    const long lab = labels[n];
    float d;
    if (lab >= 0 && lab < V) {
      if constexpr (sizeof(T) == 2)
        d = lse - __uint_as_float((uint32_t)reinterpret_cast<const uint16_t*>(row)[lab] << 16);
      else
        d = lse - reinterpret_cast<const float*>(row)[lab];
    } else {
      d = __builtin_nanf("");
    }
    stats[n] = m;
    stats[N + n] = Z;
    stats[2 * N + n] = lse;
    stats[3 * N + n] = d;
    stats[4 * N + n] = lse * lse;
  }
}

// ce and z from the per-row d and q (one workgroup; N <= 32 * 8192).
__global__ __launch_bounds__(CE_LT) void ce_mean_kernel(const float* __restrict__ stats, long N, float coeff32,
                                                        int has_coeff, float* __restrict__ loss) {
  __shared__ float pa[8192];
  __shared__ float pb[256];
  float f[2];
#pragma unroll 1
  for (int which = 0; which < 2; which++) {
    const float* a = stats + (3 + which) * N;
    const int parts = (int)((N + 31) / 32);
    for (int c = threadIdx.x; c < parts; c += blockDim.x) {
      const long hi = 32L * c + 32 < N ? 32L * c + 32 : N;
      float s = 0.0f;
      for (long i = 32L * c; i < hi; i++) s = s + a[i];
      pa[c] = s;
    }
    __syncthreads();
    f[which] = block_fold32(pa, pb, parts);
    __syncthreads();
  }
  if (threadIdx.x == 0) {
    loss[0] = otx_div_rn(f[0], (float)N);
    loss[1] = has_coeff ? coeff32 * otx_div_rn(f[1], (float)N) : 0.0f;
  }
}

// Gradient of ce * gce + z * gz with respect to the logits (gloss = {gce, gz}).
template <typename T>
__global__ __launch_bounds__(256) void ce_bwd_kernel(const T* __restrict__ logits, const int64_t* __restrict__ labels,
                                                     const float* __restrict__ stats, const float* __restrict__ gloss,
                                                     long N, int V, int vec, int tiles, float inv_n, float c2,
                                                     int has_coeff, T* __restrict__ grad) {
  __shared__ double tab[OTX_EXP_LE0_TAB_N];
  otx_load_exp_table(tab);
  __syncthreads();
  // CE_TPB tiles of 2048 logits of one row per workgroup (one exp table load each)
  const int groups = (tiles + CE_TPB - 1) / CE_TPB;
  const long n = blockIdx.x / groups;
  const int t0 = (int)(blockIdx.x % groups) * CE_TPB;
  const float m = stats[n], Z = stats[N + n], lse = stats[2 * N + n];
  const float cs = gloss[0] * inv_n;
  const float coef = (c2 * gloss[1]) * lse;
  const long lab = labels[n];
  const double rz = otx_recip64(Z);
  for (int k = 0; k < CE_TPB && t0 + k < tiles; k++) {
    const int v0 = (t0 + k) * 2048 + threadIdx.x * 8;
    if (v0 >= V) break;
    const T* src = logits + (size_t)n * V + v0;
    T* dst = grad + (size_t)n * V + v0;
    const int cnt = V - v0 < 8 ? V - v0 : 8;
    float x[8];
    if (vec && cnt == 8) {
      if constexpr (sizeof(T) == 2) {
        const uint4 u = *reinterpret_cast<const uint4*>(src);
        const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
        for (int i = 0; i < 8; i++) x[i] = __uint_as_float((i & 1) ? (w[i >> 1] & 0xffff0000u) : (w[i >> 1] << 16));
      } else {
        const float4 a = reinterpret_cast<const float4*>(src)[0], b = reinterpret_cast<const float4*>(src)[1];
        x[0] = a.x; x[1] = a.y; x[2] = a.z; x[3] = a.w; x[4] = b.x; x[5] = b.y; x[6] = b.z; x[7] = b.w;
      }
    } else {
#pragma unroll
      for (int i = 0; i < 8; i++) x[i] = i < cnt ? Elem<T>::ld(src + i) : m;
    }
    float e[8];
#pragma unroll
    for (int i = 0; i < 8; i++) e[i] = x[i] - m;
    otx_exp_n<8, true>(e, tab);
    // sm = RN(e / Z) through one binary64 reciprocal of Z (rz), with the bytes of
    // otx_div_by_recip_checked: correctly rounded in the normal range; below it,
    // where a quotient can be a midpoint exactly, and for NaN, the division
    // itself.  The check is made wave-uniform (a ballot), so that the division
    // is only evaluated when some lane needs it.
    float smv[8];
    bool low = false;
#pragma unroll
    for (int i = 0; i < 8; i++) {
      smv[i] = otx_div_by_recip(e[i], rz);
      low = low || !(smv[i] >= 0x1p-126f);
    }
    if (__builtin_expect(__ballot(low) != 0, 0)) {
#pragma unroll
      for (int i = 0; i < 8; i++)
        if (!(smv[i] >= 0x1p-126f)) smv[i] = otx_div_rn(e[i], Z);
    }
    float g[8];
#pragma unroll
    for (int i = 0; i < 8; i++) {
      const float sm = smv[i];
      float r = sm * cs;
      if (has_coeff) r = r + sm * coef;
      if (v0 + i == lab) r = r - cs;
      g[i] = r;
    }
    if (vec && cnt == 8) {
      if constexpr (sizeof(T) == 2) {
        uint4 u;
        u.x = (uint32_t)otx_f32_to_bf16(g[0]) | ((uint32_t)otx_f32_to_bf16(g[1]) << 16);
        u.y = (uint32_t)otx_f32_to_bf16(g[2]) | ((uint32_t)otx_f32_to_bf16(g[3]) << 16);
        u.z = (uint32_t)otx_f32_to_bf16(g[4]) | ((uint32_t)otx_f32_to_bf16(g[5]) << 16);
        u.w = (uint32_t)otx_f32_to_bf16(g[6]) | ((uint32_t)otx_f32_to_bf16(g[7]) << 16);
        *reinterpret_cast<uint4*>(dst) = u;
      } else {
        reinterpret_cast<float4*>(dst)[0] = make_float4(g[0], g[1], g[2], g[3]);
        reinterpret_cast<float4*>(dst)[1] = make_float4(g[4], g[5], g[6], g[7]);
      }
    } else {
      for (int i = 0; i < cnt; i++) dst[i] = Elem<T>::put(g[i]);
    }
  }
}

// Largest vocabulary of the forward's LDS partials.
int ce_max_vocab(int) { return 32 * CE_MAX_CHUNKS; }

hipError_t launch_ce_fwd(int dtype, const void* logits, const int64_t* labels, long N, int V, int vec, float coeff32,
                         int has_coeff, float* stats, float* loss, hipStream_t st) {
  if (dtype == 1)
    hipLaunchKernelGGL((ce_fwd_kernel<uint16_t>), dim3((unsigned)N), dim3(CE_LT), 0, st,
                       (const uint16_t*)logits, labels, N, V, vec, stats);
  else
    hipLaunchKernelGGL((ce_fwd_kernel<float>), dim3((unsigned)N), dim3(CE_LT), 0, st, (const float*)logits,
                       labels, N, V, vec, stats);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL(ce_mean_kernel, dim3(1), dim3(CE_LT), 0, st, (const float*)stats, N, coeff32, has_coeff, loss);
  return hipGetLastError();
}

hipError_t launch_ce_bwd(int dtype, const void* logits, const int64_t* labels, const float* stats,
                         const float* gloss, long N, int V, int vec, float inv_n, float c2, int has_coeff, void* grad,
                         hipStream_t st) {
  const int tiles = (V + 2047) / 2048;
  const dim3 grid((unsigned)(N * ((tiles + CE_TPB - 1) / CE_TPB))), block(256);
  if (dtype == 1)
    hipLaunchKernelGGL((ce_bwd_kernel<uint16_t>), grid, block, 0, st, (const uint16_t*)logits, labels, stats, gloss, N,
                       V, vec, tiles, inv_n, c2, has_coeff, (uint16_t*)grad);
  else
    hipLaunchKernelGGL((ce_bwd_kernel<float>), grid, block, 0, st, (const float*)logits, labels, stats, gloss, N, V,
                       vec, tiles, inv_n, c2, has_coeff, (float*)grad);
  return hipGetLastError();
}

}  // namespace otx
