// bf16 GEMM with a serial binary32 fold, for the projections around the
// attention (Q/K/V/O, SwiGLU gate/up/down) and their backward.
//
// Replaces repop.nn.linear.Linear (src/pretrain/model/modules/_linear.py:31-65
// of the reference; bf16 operands, fp32 accumulate, bf16 result:
// docs/MODEL_OP_DTYPE_TRACE.md:82,100,165-167).  Contract:
//   C[i][j] = RN_out( acc ),  acc = +0; for r = 0 .. R-1 ascending:
//             acc = fma(A(i, r), B(j, r), acc)
// with A(i, r) = A[i*a_i + r*a_r] and B(j, r) = B[j*b_j + r*b_r] (element
// strides), bf16 values, RN_out = round-to-nearest-even bf16 (or none for a
// binary32 output).  bf16 x bf16 products are exact in binary32, so every
// step is one rounded addition and the order is the whole contract
// (docs/unified-audit-results.md:71-74: "strict sequential ... fold ... no
// split-K").  Each fma is one lane of a v_mfma_f32_32x32x1_2b_f32, whose
// chain over r is that serial fold.
//
// Tiling: a workgroup of 4 waves owns a 128 x 128 block of C, each wave a
// 64 x 64 quarter (two MFMAs per r: i-blocks {0,1} x j-block 0, then x
// j-block 1), or, in the narrow form, a 128 x 64 block with 64 x 32 per wave
// (one MFMA per r).  r advances in chunks of 32; the A and B chunks are staged
// in LDS as binary32 (see GemmOperand for the layouts) with the next chunk's
// global loads issued before the current chunk's MFMAs.  Either operand may be
// r-contiguous (a_r == 1) or i-contiguous (a_i == 1); the loads are 16-byte
// vectors along the contiguous axis.  Every output is one lane's serial chain
// whatever the tile, so both forms give the same bytes.
#include "otx_common.h"

namespace otx {

constexpr int GT = 128;   // workgroup tile (i and j)
constexpr int GRC = 32;   // r chunk
constexpr int GP = GT + 4;  // LDS pitch (floats) of one r row of a staged tile

// One operand's chunk: ROWS rows (i; 128, or 64 for the narrow form's B) x 32 r
// = ROWS * 4 vectors of 8 bf16, NV per thread.  An r-contiguous operand is
// staged [i][r] (pitch GRC + 4 floats: the 16-byte reads of 16 consecutive rows
// start in 16 distinct 4-bank groups), so both its commit and its reads are
// 16-byte vectors along r; an i-contiguous operand is staged [r][i] (pitch
// ROWS + 4), read one r at a time with the lanes on consecutive i.
template <bool RCONT, int ROWS>
struct GemmOperand {
  static constexpr int NV = ROWS * GRC / 8 / 256;  // 16-byte vectors per thread
  static constexpr int IV = ROWS / 8;              // vectors per r of an i-contiguous operand
  static constexpr int PITCH = RCONT ? GRC + 4 : ROWS + 4;
  static constexpr int FLOATS = RCONT ? ROWS * (GRC + 4) : GRC * (ROWS + 4);
  static_assert(NV >= 1 && NV * 256 * 8 == ROWS * GRC, "the chunk must split evenly over 256 threads");
  uint4 v[NV];
  __device__ __forceinline__ void issue(const uint16_t* base, long s_i, long s_r, int i0, int r0) {
#pragma unroll
    for (int x = 0; x < NV; x++) {
      const int idx = threadIdx.x + 256 * x;
      if constexpr (RCONT) {  // 8 consecutive r of one row i
        const int i = idx >> 2, rv = (idx & 3) * 8;
        v[x] = *reinterpret_cast<const uint4*>(base + (long)(i0 + i) * s_i + (r0 + rv));
      } else {  // 8 consecutive i of one r
        const int r = idx / IV, iv = (idx % IV) * 8;
        v[x] = *reinterpret_cast<const uint4*>(base + (long)(r0 + r) * s_r + (i0 + iv));
      }
    }
  }
  __device__ __forceinline__ void commit(float* tile) const {
#pragma unroll
    for (int x = 0; x < NV; x++) {
      const int idx = threadIdx.x + 256 * x;
      float* d;
      if constexpr (RCONT) {
        const int i = idx >> 2, rv = (idx & 3) * 8;
        d = tile + i * PITCH + rv;
      } else {
        const int r = idx / IV, iv = (idx % IV) * 8;
        d = tile + r * PITCH + iv;
      }
      *reinterpret_cast<float4*>(d) = make_float4(Elem<uint16_t>::get(v[x], 0), Elem<uint16_t>::get(v[x], 1),
                                                  Elem<uint16_t>::get(v[x], 2), Elem<uint16_t>::get(v[x], 3));
      *reinterpret_cast<float4*>(d + 4) = make_float4(Elem<uint16_t>::get(v[x], 4), Elem<uint16_t>::get(v[x], 5),
                                                      Elem<uint16_t>::get(v[x], 6), Elem<uint16_t>::get(v[x], 7));
    }
  }
  // Staged values (i, r0 .. r0 + 3).
  __device__ __forceinline__ static void load4(const float* tile, int i, int r0, float (&o)[4]) {
    if constexpr (RCONT) {
      const float4 t = *reinterpret_cast<const float4*>(tile + i * PITCH + r0);
      o[0] = t.x; o[1] = t.y; o[2] = t.z; o[3] = t.w;
    } else {
#pragma unroll
      for (int e = 0; e < 4; e++) o[e] = tile[(r0 + e) * PITCH + i];
    }
  }
};

// WJ: the columns of C per wave (64, or 32 in the narrow form); the workgroup
// tile is 128 x 2 WJ.
template <bool ARC, bool BRC, bool OUT_F32, int WJ>
__global__ __launch_bounds__(256, 2) void gemm_bf16_kernel(const uint16_t* __restrict__ A, long a_i, long a_r,
                                                            const uint16_t* __restrict__ B, long b_j, long b_r,
                                                            void* __restrict__ C, long ldc, int M, int N, int R) {
  constexpr int GTJ = 2 * WJ;
  __shared__ __align__(16) float As[GemmOperand<ARC, GT>::FLOATS];
  __shared__ __align__(16) float Bs[GemmOperand<BRC, GTJ>::FLOATS];
  const int tiles_j = N / GTJ;
  const int i0 = (blockIdx.x / tiles_j) * GT, j0 = (blockIdx.x % tiles_j) * GTJ;
  const int wave = threadIdx.x >> 6, L = threadIdx.x & 63, hh = L >> 5, c = L & 31;
  const int wi = (wave >> 1) * 64, wj = (wave & 1) * WJ;  // wave quarter inside the tile

  GemmOperand<ARC, GT> ga;
  GemmOperand<BRC, GTJ> gb;
  f32x32 acc0 = f32x32{}, acc1 = f32x32{};
  const int nch = R / GRC;
  ga.issue(A, a_i, a_r, i0, 0);
  gb.issue(B, b_j, b_r, j0, 0);
  for (int ch = 0; ch < nch; ++ch) {
    __syncthreads();  // previous chunk fully consumed
    ga.commit(As);
    gb.commit(Bs);
    __syncthreads();
    if (ch + 1 < nch) {
      ga.issue(A, a_i, a_r, i0, (ch + 1) * GRC);
      gb.issue(B, b_j, b_r, j0, (ch + 1) * GRC);
    }
    const int ai = wi + hh * 32 + c, bj = wj + c;
#pragma unroll
    for (int r0 = 0; r0 < GRC; r0 += 4) {
      float a[4], b0[4], b1[4];
      GemmOperand<ARC, GT>::load4(As, ai, r0, a);
      GemmOperand<BRC, GTJ>::load4(Bs, bj, r0, b0);
      if constexpr (WJ == 64) GemmOperand<BRC, GTJ>::load4(Bs, bj + 32, r0, b1);
#pragma unroll
      for (int e = 0; e < 4; e++) {
        acc0 = otx_mfma(a[e], b0[e], acc0);
        if constexpr (WJ == 64) acc1 = otx_mfma(a[e], b1[e], acc1);
      }
    }
  }
  // acc0: rows wi + blk*32 + R(r%16, hh), column wj + c; acc1: column wj + 32 + c.
#pragma unroll
  for (int r = 0; r < 32; r++) {
    const int i = i0 + wi + 32 * (r >> 4) + otx_row(r, hh);
    const long o0 = (long)i * ldc + j0 + wj + c;
    if constexpr (OUT_F32) {
      static_cast<float*>(C)[o0] = acc0[r];
      if constexpr (WJ == 64) static_cast<float*>(C)[o0 + 32] = acc1[r];
    } else {
      static_cast<uint16_t*>(C)[o0] = otx_f32_to_bf16(acc0[r]);
      if constexpr (WJ == 64) static_cast<uint16_t*>(C)[o0 + 32] = otx_f32_to_bf16(acc1[r]);
    }
  }
}

template <bool ARC, bool BRC, int WJ>
static hipError_t launch_gemm_w(const void* A, long a_i, long a_r, const void* B, long b_j, long b_r, void* C,
                                long ldc, int M, int N, int R, bool out_f32, hipStream_t st) {
  const dim3 grid((unsigned)((M / GT) * (N / (2 * WJ)))), block(256);
  if (out_f32)
    hipLaunchKernelGGL((gemm_bf16_kernel<ARC, BRC, true, WJ>), grid, block, 0, st, (const uint16_t*)A, a_i, a_r,
                       (const uint16_t*)B, b_j, b_r, C, ldc, M, N, R);
  else
    hipLaunchKernelGGL((gemm_bf16_kernel<ARC, BRC, false, WJ>), grid, block, 0, st, (const uint16_t*)A, a_i, a_r,
                       (const uint16_t*)B, b_j, b_r, C, ldc, M, N, R);
  return hipGetLastError();
}

template <bool ARC, bool BRC>
static hipError_t launch_gemm_t(const void* A, long a_i, long a_r, const void* B, long b_j, long b_r, void* C,
                                long ldc, int M, int N, int R, bool out_f32, bool narrow, hipStream_t st) {
  if (narrow) return launch_gemm_w<ARC, BRC, 32>(A, a_i, a_r, B, b_j, b_r, C, ldc, M, N, R, out_f32, st);
  return launch_gemm_w<ARC, BRC, 64>(A, a_i, a_r, B, b_j, b_r, C, ldc, M, N, R, out_f32, st);
}

// Tile choice (both forms give the same bytes).  With t tiles of 128 x 128 on
// n CUs, the busiest CU works through ceil(t / n) of them, or ceil(2t / n)
// narrow ones of half the work each.  The narrow form costs 3-5 % more per
// unit of work (one MFMA per operand read of A instead of two), so it is taken
// when its busiest CU still comes out at least 4 % ahead: t = 5.5 n (the
// OPEN-1B gate/up weight gradient, 1408 tiles) puts six wide tiles or eleven
// narrow ones (5.5 wide tiles' work) on the busiest CU; measured -3.2 %.  At
// 256 tiles (one per CU) the two forms are equal.  variant 1 forces the wide
// form, 2 the narrow one.
static bool gemm_narrow(int M, int N, int variant) {
  if (variant == 1) return false;
  if (variant == 2) return true;
  const long t = (long)(M / GT) * (N / GT), n = otx_cu_count();
  const long wide = (t + n - 1) / n, narrow2 = (2 * t + n - 1) / n;  // narrow2 / 2 wide tiles' work
  return 104 * narrow2 < 200 * wide;
}

hipError_t launch_gemm(const void* A, long a_i, long a_r, const void* B, long b_j, long b_r, void* C, long ldc, int M,
                       int N, int R, bool out_f32, int variant, hipStream_t st) {
  const bool arc = a_r == 1, brc = b_r == 1, nw = gemm_narrow(M, N, variant);
  if (arc && brc) return launch_gemm_t<true, true>(A, a_i, a_r, B, b_j, b_r, C, ldc, M, N, R, out_f32, nw, st);
  if (arc) return launch_gemm_t<true, false>(A, a_i, a_r, B, b_j, b_r, C, ldc, M, N, R, out_f32, nw, st);
  if (brc) return launch_gemm_t<false, true>(A, a_i, a_r, B, b_j, b_r, C, ldc, M, N, R, out_f32, nw, st);
  return launch_gemm_t<false, false>(A, a_i, a_r, B, b_j, b_r, C, ldc, M, N, R, out_f32, nw, st);
}

}  // namespace otx
