// Token embedding with a deterministic backward, for gfx950.
//
// Replaces repop.nn.embedding.Embedding (_DeterministicEmbeddingFn), used by
// src/pretrain/model/modules/embedding_repop.py:33-40 of the reference:
// forward = plain gather of weight rows; backward = "stable-sort + fixed-order
// segment scatter-add", fp32 accumulation, result in the gradient's dtype
// (docs/MODEL_OP_DTYPE_TRACE.md:75,106).  Contract:
//   grad_w[v][d] = RN_dtype( fold over positions p ascending with ids[p] == v
//                            of g[p][d], serial binary32 additions from +0 )
//   rows of ids that do not occur are +0; ids outside [0, V) are skipped in the
//   backward and give NaN rows in the forward.
// Backward pipeline: int32 keys (the ids) and values (the positions) -> stable
// LSD radix sort of the keys with hipCUB (an integer permutation; positions of
// equal ids stay ascending) -> zero fill of grad_w -> one workgroup per segment
// head folds its segment's rows column by column in position order.
#include <hipcub/hipcub.hpp>
#include "otx_common.h"

namespace otx {

template <typename T>
__global__ __launch_bounds__(256) void emb_fwd_kernel(const int64_t* __restrict__ ids, const T* __restrict__ w,
                                                      T* __restrict__ out, long npos, int V, int D) {
  const long p = blockIdx.x;
  const int d = (blockIdx.y * 256 + threadIdx.x) * (int)(16 / sizeof(T));
  if (p >= npos || d >= D) return;
  const long id = ids[p];
  uint4 val;
  if (id >= 0 && id < V) {
    val = *reinterpret_cast<const uint4*>(w + id * (long)D + d);
  } else {
    const uint32_t nan = sizeof(T) == 2 ? 0x7fc07fc0u : 0x7fc00000u;
    val = make_uint4(nan, nan, nan, nan);
  }
  *reinterpret_cast<uint4*>(out + p * (long)D + d) = val;
}

// keys = ids (V for ids outside [0, V)), values = positions
__global__ __launch_bounds__(256) void emb_keys_kernel(const int64_t* __restrict__ ids, int* __restrict__ keys,
                                                       int* __restrict__ pos, long npos, int V) {
  const long p = (long)blockIdx.x * 256 + threadIdx.x;
  if (p >= npos) return;
  const long id = ids[p];
  keys[p] = (id >= 0 && id < V) ? (int)id : V;
  pos[p] = (int)p;
}

__global__ __launch_bounds__(256) void emb_zero_kernel(uint4* __restrict__ dst, long n16) {
  for (long i = (long)blockIdx.x * 256 + threadIdx.x; i < n16; i += (long)gridDim.x * 256)
    dst[i] = make_uint4(0u, 0u, 0u, 0u);
}

// Workgroup (i, column block): if sorted index i starts a segment of a valid id,
// fold the segment's gradient rows for 256 columns in position order.
template <typename T>
__global__ __launch_bounds__(256) void emb_fold_kernel(const int* __restrict__ skeys, const int* __restrict__ spos,
                                                       const T* __restrict__ g, T* __restrict__ gw, long npos, int V,
                                                       int D) {
  const long i = blockIdx.x;
  const int key = skeys[i];
  if (key >= V || (i > 0 && skeys[i - 1] == key)) return;
  const int d = blockIdx.y * 256 + threadIdx.x;
  if (d >= D) return;
  float acc = 0.0f;
  for (long j = i; j < npos && skeys[j] == key; j++) acc = acc + Elem<T>::ld(g + (long)spos[j] * D + d);
  gw[(long)key * D + d] = Elem<T>::put(acc);
}

static int key_bits(int V) {
  int b = 1;
  while ((1L << b) <= V) b++;  // keys are 0..V
  return b;
}

// Temporary storage of the key sort; 0 if the size query fails.
size_t emb_sort_temp_bytes(long npos, int V) {
  size_t bytes = 0;
  const hipError_t e = hipcub::DeviceRadixSort::SortPairs(nullptr, bytes, (const int*)nullptr, (int*)nullptr,
                                                          (const int*)nullptr, (int*)nullptr, (int)npos, 0, key_bits(V));
  return e == hipSuccess ? bytes : 0;
}

hipError_t launch_emb_fwd(int dtype, const int64_t* ids, const void* w, void* out, long npos, int V, int D,
                          hipStream_t st) {
  const int per = dtype == 1 ? 8 : 4;
  const dim3 grid((unsigned)npos, (unsigned)((D / per + 255) / 256)), block(256);
  if (dtype == 1)
    hipLaunchKernelGGL((emb_fwd_kernel<uint16_t>), grid, block, 0, st, ids, (const uint16_t*)w, (uint16_t*)out, npos,
                       V, D);
  else
    hipLaunchKernelGGL((emb_fwd_kernel<float>), grid, block, 0, st, ids, (const float*)w, (float*)out, npos, V, D);
  return hipGetLastError();
}

// ws: keys, pos, sorted keys, sorted pos (npos int32 each, 256-byte aligned), then hipCUB temp storage.
hipError_t launch_emb_bwd(int dtype, const int64_t* ids, const void* g, void* gw, long npos, int V, int D, char* ws,
                          size_t temp_bytes, hipStream_t st) {
  const size_t arr = ((size_t)npos * 4 + 255) / 256 * 256;
  int* keys = (int*)ws;
  int* pos = (int*)(ws + arr);
  int* skeys = (int*)(ws + 2 * arr);
  int* spos = (int*)(ws + 3 * arr);
  void* temp = ws + 4 * arr;
  hipLaunchKernelGGL(emb_keys_kernel, dim3((unsigned)((npos + 255) / 256)), dim3(256), 0, st, ids, keys, pos, npos, V);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  e = hipcub::DeviceRadixSort::SortPairs(temp, temp_bytes, keys, skeys, pos, spos, (int)npos, 0, key_bits(V), st);
  if (e != hipSuccess) return e;
  const long n16 = (long)V * D * (dtype == 1 ? 2 : 4) / 16;
  hipLaunchKernelGGL(emb_zero_kernel, dim3(2048), dim3(256), 0, st, (uint4*)gw, n16);
  e = hipGetLastError();
  if (e != hipSuccess) return e;
  const dim3 grid((unsigned)npos, (unsigned)((D + 255) / 256)), block(256);
  if (dtype == 1)
    hipLaunchKernelGGL((emb_fold_kernel<uint16_t>), grid, block, 0, st, skeys, spos, (const uint16_t*)g,
                       (uint16_t*)gw, npos, V, D);
  else
    hipLaunchKernelGGL((emb_fold_kernel<float>), grid, block, 0, st, skeys, spos, (const float*)g, (float*)gw, npos,
                       V, D);
  return hipGetLastError();
}

}  // namespace otx
