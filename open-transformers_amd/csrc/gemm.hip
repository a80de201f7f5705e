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
// (one MFMA per r), or, in the small form, a 64 x 64 block with 32 x 32 per
// wave (one v_mfma_f32_16x16x1_4b_f32 per r, also one fma per output).  r
// advances in chunks of 32.  The wide and narrow forms (gemm_bf16_v2_kernel)
// keep each chunk in LDS as bf16 in two slots, one barrier per chunk: an
// i-contiguous operand is copied straight from global memory into LDS, an
// r-contiguous one loaded into registers and stored transposed, and the MFMA
// operands are read with ds_read_u16_d16_hi, which yields the binary32 value of
// a bf16 with no conversion instruction (see GemmTile16).  The narrow form of
// dx = dy w and the small form stage their chunks as binary32 (GemmOperand),
// converted once per element, with the next chunk's global loads issued before
// the current chunk's MFMAs.  Either operand may be r-contiguous (a_r == 1) or
// i-contiguous (a_i == 1); the loads are 16-byte vectors along the contiguous
// axis.  Every output is one lane's serial chain whatever the tile, so every
// form gives the same bytes.
#include "otx_common.h"

namespace otx {

constexpr int GT = 128;   // workgroup tile (i and j)
constexpr int GRC = 32;   // r chunk
constexpr int GP = GT + 4;  // LDS pitch (floats) of one r row of a staged tile
#ifndef OTX_GEMM_SMALL_PF
#define OTX_GEMM_SMALL_PF 3  // chunks of global loads in flight in the small form
#endif

// Tile of workgroup `bid` among ntiles = tiles_i x tiles_j.  Workgroups are
// dealt to the 8 XCDs round-robin (workgroup b runs on XCD b % 8, each XCD with
// its own L2), so the tiles are renumbered to give every XCD a contiguous band,
// walked in groups of GM tile rows with the rows fastest: the workgroups that
// an XCD runs at once then share their A rows and B columns in its L2.  For the
// lm-head logits (64 x 1002 tiles) the B operand (the 128256-row weight, larger
// than the last-level cache) is streamed from HBM once per XCD instead of once
// per tile row: -4 %.  Any order gives the same bytes.
__device__ __forceinline__ void gemm_tile(int bid, int ntiles, int tiles_j, int* ti, int* tj) {
  constexpr int GM = 4;
  int s = bid;
  if ((ntiles & 7) == 0) s = (bid & 7) * (ntiles >> 3) + (bid >> 3);
  const int tiles_i = ntiles / tiles_j;
  const int first = (s / (GM * tiles_j)) * GM;
  const int gm = tiles_i - first < GM ? tiles_i - first : GM;
  const int within = s - first * tiles_j;
  *ti = first + within % gm;
  *tj = within / gm;
}

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
  int ti, tj;
  gemm_tile(blockIdx.x, (M / GT) * tiles_j, tiles_j, &ti, &tj);
  const int i0 = ti * GT, j0 = tj * GTJ;
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

// One operand's chunk of 32 r held in LDS as bf16, [r][row] with a pitch of PB
// bytes per r, read by ds_read_u16_d16_hi straight into the binary32 operand
// registers (no conversion instruction).  An i-contiguous operand is copied
// straight from global memory (global_load_lds_dwordx4: each r row of the chunk
// is ROWS contiguous bf16, 1 KB per instruction); an r-contiguous one is loaded
// into registers (8 consecutive r of one row per 16-byte load) and written
// transposed with 2-byte stores, its pitch padded by 8 bytes so that the four r
// rows a wave writes at once fall in distinct banks.
template <bool RCONT, int ROWS>
struct GemmTile16 {
  static constexpr int PB = RCONT ? ROWS * 2 + 8 : ROWS * 2;
  static constexpr int BYTES = GRC * PB;
  static constexpr int NV = ROWS * GRC / 8 / 256;  // 16-byte loads per thread (r-contiguous)
  static constexpr int RPI = 1024 / (ROWS * 2);    // r rows per direct copy instruction
  static constexpr int NI = GRC / RPI / 4;         // direct copy instructions per wave
  static_assert(NV >= 1 && NI >= 1, "tile shape");
  uint4 v[RCONT ? NV : 1];
  __device__ __forceinline__ void issue(const uint16_t* base, long s_i, long s_r, int i0, int r0, unsigned char* slot,
                                        int wave_u, int L) {
    if constexpr (RCONT) {
#pragma unroll
      for (int x = 0; x < NV; x++) {
        const int idx = threadIdx.x + 256 * x;
        const int i = idx >> 2, rv = (idx & 3) * 8;
        v[x] = *reinterpret_cast<const uint4*>(base + (long)(i0 + i) * s_i + (r0 + rv));
      }
    } else {
#pragma unroll
      for (int x = 0; x < NI; x++) {
        const int rb = (wave_u + 4 * x) * RPI;
        const int r = rb + L / (ROWS / 8), iv = (L % (ROWS / 8)) * 8;
        otx_dma16(base + (long)(r0 + r) * s_r + (i0 + iv), slot + rb * PB);
      }
    }
  }
  __device__ __forceinline__ void commit(unsigned char* slot) const {
    if constexpr (RCONT) {
#pragma unroll
      for (int x = 0; x < NV; x++) {
        const int idx = threadIdx.x + 256 * x;
        const int i = idx >> 2, rv = (idx & 3) * 8;
        unsigned char* p = slot + rv * PB + i * 2;
        const uint32_t* w = reinterpret_cast<const uint32_t*>(&v[x]);
#pragma unroll
        for (int k = 0; k < 4; k++) {
          *reinterpret_cast<uint16_t*>(p + (2 * k) * PB) = (uint16_t)w[k];
          *reinterpret_cast<uint16_t*>(p + (2 * k + 1) * PB) = (uint16_t)(w[k] >> 16);
        }
      }
    }
  }
};

template <int N>
__device__ __forceinline__ void gemm_lds_wait6(float (&r)[6]) {
  asm volatile("s_waitcnt lgkmcnt(%6)"
               : "+v"(r[0]), "+v"(r[1]), "+v"(r[2]), "+v"(r[3]), "+v"(r[4]), "+v"(r[5])
               : "i"(N));
}

// The wide and narrow forms with bf16 LDS tiles, two slots and one barrier per
// chunk: chunk ch is read from slot ch & 1 while the copies of chunk ch + 1
// (issued one chunk earlier) land in the other slot.  The operands are read one
// group of two r ahead with hand-kept lgkmcnt accounting (six or four reads per
// group, at most twelve outstanding); the accumulators stay in the
// accumulation registers, so 64 vector registers remain and four workgroups
// share a CU (launch bound: four waves per SIMD).  No vector instruction
// converts or stages an i-contiguous operand, and an r-contiguous one costs
// only its 2-byte stores.
template <bool ARC, bool BRC, bool OUT_F32, int WJ>
__global__ __launch_bounds__(256, 4) void gemm_bf16_v2_kernel(const uint16_t* __restrict__ A, long a_i, long a_r,
                                                               const uint16_t* __restrict__ B, long b_j, long b_r,
                                                               void* __restrict__ C, long ldc, int M, int N, int R) {
  constexpr int GTJ = 2 * WJ;
  using TA = GemmTile16<ARC, GT>;
  using TB = GemmTile16<BRC, GTJ>;
  constexpr int SLOT = TA::BYTES + TB::BYTES;
  __shared__ __align__(16) unsigned char smem[2 * SLOT];
  const int tiles_j = N / GTJ;
  int ti, tj;
  gemm_tile(blockIdx.x, (M / GT) * tiles_j, tiles_j, &ti, &tj);
  const int i0 = ti * GT, j0 = tj * GTJ;
  const int wave = threadIdx.x >> 6, L = threadIdx.x & 63, hh = L >> 5, c = L & 31;
  const int wave_u = __builtin_amdgcn_readfirstlane(wave);
  const int wi = (wave >> 1) * 64, wj = (wave & 1) * WJ;
  constexpr int NRD = WJ == 64 ? 6 : 4;  // reads per group of two r
  TA ta;
  TB tb;
  f32x32 acc0 = f32x32{}, acc1 = f32x32{};
  const int nch = R / GRC;
  auto slot_a = [&](int s) { return smem + s * SLOT; };
  auto slot_b = [&](int s) { return smem + s * SLOT + TA::BYTES; };
  ta.issue(A, a_i, a_r, i0, 0, slot_a(0), wave_u, L);
  tb.issue(B, b_j, b_r, j0, 0, slot_b(0), wave_u, L);
  ta.commit(slot_a(0));
  tb.commit(slot_b(0));
  if (nch > 1) {
    ta.issue(A, a_i, a_r, i0, GRC, slot_a(1), wave_u, L);
    tb.issue(B, b_j, b_r, j0, GRC, slot_b(1), wave_u, L);
  }
  asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)" ::: "memory");
  __syncthreads();
  float opr[2][6] = {};
  for (int ch = 0; ch < nch; ++ch) {
    const int s = ch & 1;
    const uint32_t aA = otx_lds_addr(slot_a(s)) + (wi + hh * 32 + c) * 2;
    const uint32_t aB = otx_lds_addr(slot_b(s)) + (wj + c) * 2;
    auto rd = [&](auto gc) {
      constexpr int G = decltype(gc)::value, BK = G & 1;
      OtxUnroll<0, 2>::run([&](auto ec) {
        constexpr int E = decltype(ec)::value, RR = 2 * G + E;
        otx_lds_bf16<RR * TA::PB>(opr[BK][E], aA);
        otx_lds_bf16<RR * TB::PB>(opr[BK][2 + E], aB);
        if constexpr (WJ == 64) otx_lds_bf16<RR * TB::PB + 64>(opr[BK][4 + E], aB);
      });
    };
    rd(std::integral_constant<int, 0>{});
    OtxUnroll<0, GRC / 2>::run([&](auto gc) {
      constexpr int G = decltype(gc)::value, BK = G & 1;
      if constexpr (G + 1 < GRC / 2) {
        rd(std::integral_constant<int, G + 1>{});
        gemm_lds_wait6<NRD>(opr[BK]);
      } else {
        gemm_lds_wait6<0>(opr[BK]);
      }
      OtxUnroll<0, 2>::run([&](auto ec) {
        constexpr int E = decltype(ec)::value;
        acc0 = otx_mfma(opr[BK][E], opr[BK][2 + E], acc0);
        if constexpr (WJ == 64) acc1 = otx_mfma(opr[BK][E], opr[BK][4 + E], acc1);
      });
      // bank BK is consumed before it is read again
      if constexpr (WJ == 64)
        asm volatile("" : "+a"(acc0), "+a"(acc1));
      else
        asm volatile("" : "+a"(acc0));
    });
    if (ch + 1 < nch) {
      ta.commit(slot_a(s ^ 1));
      tb.commit(slot_b(s ^ 1));
    }
    asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)" ::: "memory");  // this thread's copies of chunk ch + 1 have landed
    __syncthreads();  // chunk ch + 1 is visible, and slot s is no longer read
    if (ch + 2 < nch) {
      ta.issue(A, a_i, a_r, i0, (ch + 2) * GRC, slot_a(s), wave_u, L);
      tb.issue(B, b_j, b_r, j0, (ch + 2) * GRC, slot_b(s), wave_u, L);
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

// Small form: a workgroup of 4 waves owns a 64 x 64 block of C, each wave a
// 32 x 32 quarter as the four 16 x 16 blocks of one v_mfma_f32_16x16x1_4b_f32
// per r (lane L supplies A row wi + 16 (b & 1) + L % 16 and B column
// wj + 16 (b >> 1) + L % 16 of block b = L / 16).  For grids of far fewer
// 128 x 128 tiles than CUs, where the other forms would leave CUs idle.
template <bool ARC, bool BRC, bool OUT_F32>
__global__ __launch_bounds__(256, 2) void gemm_bf16_small_kernel(const uint16_t* __restrict__ A, long a_i, long a_r,
                                                                  const uint16_t* __restrict__ B, long b_j, long b_r,
                                                                  void* __restrict__ C, long ldc, int M, int N,
                                                                  int R) {
  constexpr int GS = 64;
  __shared__ __align__(16) float As[GemmOperand<ARC, GS>::FLOATS];
  __shared__ __align__(16) float Bs[GemmOperand<BRC, GS>::FLOATS];
  const int tiles_j = N / GS;
  int ti, tj;
  gemm_tile(blockIdx.x, (M / GS) * tiles_j, tiles_j, &ti, &tj);
  const int i0 = ti * GS, j0 = tj * GS;
  const int wave = threadIdx.x >> 6, L = threadIdx.x & 63, blk = L >> 4, c = L & 15;
  const int wi = (wave >> 1) * 32, wj = (wave & 1) * 32;

  // A chunk's MFMAs take a quarter of the wide form's time, less than a global
  // load's latency, so the loads run PF chunks ahead (a ring of PF register
  // sets, indexed statically by unrolling over the ring).
  constexpr int PF = OTX_GEMM_SMALL_PF;
  GemmOperand<ARC, GS> ga[PF];
  GemmOperand<BRC, GS> gb[PF];
  f32x16 acc = f32x16{};
  const int nch = R / GRC;
#pragma unroll
  for (int k = 0; k < PF; k++)
    if (k < nch) {
      ga[k].issue(A, a_i, a_r, i0, k * GRC);
      gb[k].issue(B, b_j, b_r, j0, k * GRC);
    }
  const int ai = wi + 16 * (blk & 1) + c, bj = wj + 16 * (blk >> 1) + c;
  for (int ch0 = 0; ch0 < nch; ch0 += PF) {
#pragma unroll
    for (int k = 0; k < PF; k++) {
      const int ch = ch0 + k;
      if (ch < nch) {
        __syncthreads();  // previous chunk fully consumed
        ga[k].commit(As);
        gb[k].commit(Bs);
        __syncthreads();
        if (ch + PF < nch) {
          ga[k].issue(A, a_i, a_r, i0, (ch + PF) * GRC);
          gb[k].issue(B, b_j, b_r, j0, (ch + PF) * GRC);
        }
#pragma unroll
        for (int r0 = 0; r0 < GRC; r0 += 4) {
          float a[4], b[4];
          GemmOperand<ARC, GS>::load4(As, ai, r0, a);
          GemmOperand<BRC, GS>::load4(Bs, bj, r0, b);
#pragma unroll
          for (int e = 0; e < 4; e++) acc = otx_mfma16(a[e], b[e], acc);
        }
      }
    }
  }
  // acc[r]: block r / 4 (i-block (r / 4) & 1, j-block (r / 4) >> 1), row 4 (L / 16) + r % 4, column L % 16.
#pragma unroll
  for (int r = 0; r < 16; r++) {
    const int bb = r >> 2;
    const int i = i0 + wi + 16 * (bb & 1) + 4 * blk + (r & 3);
    const long o = (long)i * ldc + j0 + wj + 16 * (bb >> 1) + c;
    if constexpr (OUT_F32)
      static_cast<float*>(C)[o] = acc[r];
    else
      static_cast<uint16_t*>(C)[o] = otx_f32_to_bf16(acc[r]);
  }
}

// The bf16-tile kernel serves both forms, except the narrow form of an
// r-contiguous A with an i-contiguous B (dx = dy w), where the binary32-tile
// kernel measured 11-14 % faster (its A commit is shared by half as many
// MFMAs there as in the wide form).
template <bool ARC, bool BRC, int WJ>
static hipError_t launch_gemm_w(const void* A, long a_i, long a_r, const void* B, long b_j, long b_r, void* C,
                                long ldc, int M, int N, int R, bool out_f32, hipStream_t st) {
  const dim3 grid((unsigned)((M / GT) * (N / (2 * WJ)))), block(256);
  if constexpr (!(WJ == 32 && ARC && !BRC)) {
    if (out_f32)
      hipLaunchKernelGGL((gemm_bf16_v2_kernel<ARC, BRC, true, WJ>), grid, block, 0, st, (const uint16_t*)A, a_i, a_r,
                         (const uint16_t*)B, b_j, b_r, C, ldc, M, N, R);
    else
      hipLaunchKernelGGL((gemm_bf16_v2_kernel<ARC, BRC, false, WJ>), grid, block, 0, st, (const uint16_t*)A, a_i,
                         a_r, (const uint16_t*)B, b_j, b_r, C, ldc, M, N, R);
  } else {
    if (out_f32)
      hipLaunchKernelGGL((gemm_bf16_kernel<ARC, BRC, true, WJ>), grid, block, 0, st, (const uint16_t*)A, a_i, a_r,
                         (const uint16_t*)B, b_j, b_r, C, ldc, M, N, R);
    else
      hipLaunchKernelGGL((gemm_bf16_kernel<ARC, BRC, false, WJ>), grid, block, 0, st, (const uint16_t*)A, a_i, a_r,
                         (const uint16_t*)B, b_j, b_r, C, ldc, M, N, R);
  }
  return hipGetLastError();
}

template <bool ARC, bool BRC>
static hipError_t launch_gemm_small(const void* A, long a_i, long a_r, const void* B, long b_j, long b_r, void* C,
                                    long ldc, int M, int N, int R, bool out_f32, hipStream_t st) {
  const dim3 grid((unsigned)((M / 64) * (N / 64))), block(256);
  if (out_f32)
    hipLaunchKernelGGL((gemm_bf16_small_kernel<ARC, BRC, true>), grid, block, 0, st, (const uint16_t*)A, a_i, a_r,
                       (const uint16_t*)B, b_j, b_r, C, ldc, M, N, R);
  else
    hipLaunchKernelGGL((gemm_bf16_small_kernel<ARC, BRC, false>), grid, block, 0, st, (const uint16_t*)A, a_i, a_r,
                       (const uint16_t*)B, b_j, b_r, C, ldc, M, N, R);
  return hipGetLastError();
}

// form: 0 wide (128 x 128), 1 narrow (128 x 64), 2 small (64 x 64).
template <bool ARC, bool BRC>
static hipError_t launch_gemm_t(const void* A, long a_i, long a_r, const void* B, long b_j, long b_r, void* C,
                                long ldc, int M, int N, int R, bool out_f32, int form, hipStream_t st) {
  if (form == 2) return launch_gemm_small<ARC, BRC>(A, a_i, a_r, B, b_j, b_r, C, ldc, M, N, R, out_f32, st);
  if (form == 1) return launch_gemm_w<ARC, BRC, 32>(A, a_i, a_r, B, b_j, b_r, C, ldc, M, N, R, out_f32, st);
  return launch_gemm_w<ARC, BRC, 64>(A, a_i, a_r, B, b_j, b_r, C, ldc, M, N, R, out_f32, st);
}

// Tile choice (every form gives the same bytes).  With t tiles of 128 x 128 on
// n CUs, the busiest CU works through ceil(t / n) wide tiles, ceil(2t / n)
// narrow ones (half the work each) or ceil(4t / n) small ones (a quarter).
// Per unit of work the narrow form costs 2-6 % more than the wide one (one
// MFMA per operand read of A instead of two) and the small form about 10 %
// more (a quarter of the work per chunk for the same barriers and staging), so
// the launcher takes the form whose busiest CU does the least weighted work:
// t = 5.5 n (the OPEN-1B gate/up weight gradient, 1408 tiles) gives six wide,
// eleven narrow or 22 small tiles (5.5 wide tiles' work), and the narrow form
// wins (-3.2 % with binary32 tiles, -6 to -9 % with bf16 tiles); t = n / 4 (the
// k and v weight gradients, 64 tiles) leaves three quarters of the CUs idle in
// the wide form, half of them in the narrow one and none in the small one (-23 %
// against narrow with binary32 tiles, -10 % against the bf16-tile narrow form).  At t = n (one tile per
// CU) the wide and narrow forms are equal.  variant 1, 2, 3 force the wide,
// narrow and small form.
static int gemm_form(int M, int N, int variant) {
  if (variant >= 1) return variant - 1;
  const long t = (long)(M / GT) * (N / GT), n = otx_cu_count();
  const long wide = 400 * ((t + n - 1) / n), narrow = 208 * ((2 * t + n - 1) / n),
             small = 110 * ((4 * t + n - 1) / n);  // in 1/400 of a wide tile's work
  if (small < wide && small < narrow) return 2;
  return narrow < wide ? 1 : 0;
}

hipError_t launch_gemm(const void* A, long a_i, long a_r, const void* B, long b_j, long b_r, void* C, long ldc, int M,
                       int N, int R, bool out_f32, int variant, hipStream_t st) {
  const bool arc = a_r == 1, brc = b_r == 1;
  const int f = gemm_form(M, N, variant);
  if (arc && brc) return launch_gemm_t<true, true>(A, a_i, a_r, B, b_j, b_r, C, ldc, M, N, R, out_f32, f, st);
  if (arc) return launch_gemm_t<true, false>(A, a_i, a_r, B, b_j, b_r, C, ldc, M, N, R, out_f32, f, st);
  if (brc) return launch_gemm_t<false, true>(A, a_i, a_r, B, b_j, b_r, C, ldc, M, N, R, out_f32, f, st);
  return launch_gemm_t<false, false>(A, a_i, a_r, B, b_j, b_r, C, ldc, M, N, R, out_f32, f, st);
}

}  // namespace otx
