// Rotary position embedding fused with the attention operator's [B, H, T, D]
// layout, and the plain head-layout swaps around the attention.
//
// The reference's attention module (src/pretrain/model/modules/
// attention_repop.py:143-155) computes apply_rope (rope.py:103-125) in torch,
// then q/k/v.transpose(1, 2).contiguous(), and after the attention
// out.transpose(1, 2).contiguous().  Torch's arithmetic for that chain fixes
// the bytes (binary32, RN; put() = rounding to the tensor dtype, RNE for bf16;
// c, s = cos[t][i], sin[t][i] binary32; e, o = x[2i], x[2i+1]):
//   forward   y[2i]   = put(RN(RN(e * c) - RN(o * s)))
//             y[2i+1] = put(RN(RN(e * s) + RN(o * c)))
//   backward  (g = dy, ge = g[2i], go = g[2i+1]; autograd's products are cast
//             to x's dtype per branch, the two branches of x[..., 0::2] and of
//             x[..., 1::2] are summed in x's dtype, and the two slice gradients
//             are then summed as full tensors, each holding +0 where the other
//             slice lies, so a -0 sum becomes +0)
//             dx[2i]   = z(put(RN(put(RN(ge * c)) + put(RN(go * s)))))
//             dx[2i+1] = z(put(RN(put(RN(-ge * s)) + put(RN(go * c)))))
//             with z(v) = RN(v + +0).
// Every row is D contiguous elements; one thread moves 16 bytes (8 bf16 or 4
// binary32 elements, i.e. 4 or 2 pairs), so each row is one coalesced run of
// D/8 or D/4 threads on both sides of the transpose.
#include "otx_common.h"

namespace otx {

template <typename T>
struct Vec16 {
  static constexpr int N = 16 / sizeof(T);  // elements per 16-byte chunk
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
};

// Rounds a binary32 value to T and back (the value a T tensor holds).
template <typename T>
__device__ __forceinline__ float round_to(float v) {
  if constexpr (sizeof(T) == 2)
    return otx_bf16_to_f32(otx_f32_to_bf16(v));
  else
    return v;
}

// Thread g handles chunk g % CPR of output row g / CPR.  Rows of the output are
// ordered (b, h, t) for the forward and (b, t, h) for the backward.
template <typename T, bool BACKWARD>
__global__ __launch_bounds__(256) void rope_heads_kernel(const T* __restrict__ in, const float* __restrict__ cosv,
                                                         const float* __restrict__ sinv, T* __restrict__ out, int B,
                                                         int Tn, int H, int D) {
  constexpr int N = Vec16<T>::N;
  const int CPR = D / N;
  const long g = (long)blockIdx.x * 256 + threadIdx.x;
  const long rows = (long)B * Tn * H;
  if (g >= rows * CPR) return;
  const long row = g / CPR;
  const int c = (int)(g - row * CPR);
  long b, h, t;
  if (!BACKWARD) {  // out row (b, h, t), in row (b, t, h)
    t = row % Tn;
    h = (row / Tn) % H;
    b = row / ((long)Tn * H);
  } else {          // out row (b, t, h), in row (b, h, t)
    h = row % H;
    t = (row / H) % Tn;
    b = row / ((long)H * Tn);
  }
  const long in_row = BACKWARD ? (b * H + h) * Tn + t : (b * Tn + t) * H + h;
  float v[N], r[N];
  Vec16<T>::load(in + in_row * D + c * N, v);
  const float* cp = cosv + t * (D / 2) + c * (N / 2);
  const float* sp = sinv + t * (D / 2) + c * (N / 2);
#pragma unroll
  for (int p = 0; p < N / 2; p++) {
    const float cs = cp[p], sn = sp[p];
    const float e = v[2 * p], o = v[2 * p + 1];
    if (!BACKWARD) {
      r[2 * p] = e * cs - o * sn;
      r[2 * p + 1] = e * sn + o * cs;
    } else {
      const float a = round_to<T>(round_to<T>(e * cs) + round_to<T>(o * sn));
      const float q = round_to<T>(round_to<T>((-e) * sn) + round_to<T>(o * cs));
      r[2 * p] = a + 0.0f;
      r[2 * p + 1] = q + 0.0f;
    }
  }
  Vec16<T>::store(out + row * D + c * N, r);
}

// [B, X, Y, D] -> [B, Y, X, D], 16 bytes per thread.
template <typename T>
__global__ __launch_bounds__(256) void swap_heads_kernel(const T* __restrict__ in, T* __restrict__ out, int B, int X,
                                                         int Y, int D) {
  constexpr int N = Vec16<T>::N;
  const int CPR = D / N;
  const long g = (long)blockIdx.x * 256 + threadIdx.x;
  const long rows = (long)B * X * Y;
  if (g >= rows * CPR) return;
  const long row = g / CPR;  // output row (b, y, x)
  const int c = (int)(g - row * CPR);
  const long x = row % X, y = (row / X) % Y, b = row / ((long)X * Y);
  const long in_row = (b * X + x) * Y + y;
  *(uint4*)(out + row * D + c * N) = *(const uint4*)(in + in_row * D + c * N);
}

template <typename T>
static hipError_t launch_rope_t(int backward, const void* in, const float* cosv, const float* sinv, void* out, int B,
                                int Tn, int H, int D, hipStream_t st) {
  const long threads = (long)B * Tn * H * (D / Vec16<T>::N);
  const dim3 grid((unsigned)((threads + 255) / 256)), block(256);
  if (backward)
    hipLaunchKernelGGL((rope_heads_kernel<T, true>), grid, block, 0, st, (const T*)in, cosv, sinv, (T*)out, B, Tn, H,
                       D);
  else
    hipLaunchKernelGGL((rope_heads_kernel<T, false>), grid, block, 0, st, (const T*)in, cosv, sinv, (T*)out, B, Tn,
                       H, D);
  return hipGetLastError();
}

hipError_t launch_rope_heads(int dtype, int backward, const void* in, const float* cosv, const float* sinv, void* out,
                             int B, int Tn, int H, int D, hipStream_t st) {
  return dtype == 1 ? launch_rope_t<uint16_t>(backward, in, cosv, sinv, out, B, Tn, H, D, st)
                    : launch_rope_t<float>(backward, in, cosv, sinv, out, B, Tn, H, D, st);
}

hipError_t launch_swap_heads(int dtype, const void* in, void* out, int B, int X, int Y, int D, hipStream_t st) {
  if (dtype == 1) {
    const long threads = (long)B * X * Y * (D / Vec16<uint16_t>::N);
    hipLaunchKernelGGL((swap_heads_kernel<uint16_t>), dim3((unsigned)((threads + 255) / 256)), dim3(256), 0, st,
                       (const uint16_t*)in, (uint16_t*)out, B, X, Y, D);
  } else {
    const long threads = (long)B * X * Y * (D / Vec16<float>::N);
    hipLaunchKernelGGL((swap_heads_kernel<float>), dim3((unsigned)((threads + 255) / 256)), dim3(256), 0, st,
                       (const float*)in, (float*)out, B, X, Y, D);
  }
  return hipGetLastError();
}

}  // namespace otx
