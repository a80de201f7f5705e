// Shared device helpers for the gfx950 attention kernels.
//
// Matrix-core primitive.  Every GEMM-shaped step uses
// v_mfma_f32_32x32x1_2b_f32: two independent 32x32 rank-1 updates
//   D[blk][row][col] = fma(A[blk][row], B[blk][col], C[blk][row][col])
// with one IEEE fma per output (measured on gfx950: bit-identical to fmaf for
// normal, subnormal, signed-zero and tie inputs).  A chain of these
// instructions over k = 0..K-1 is therefore exactly the serial ascending fma
// fold the arithmetic contract prescribes.
//
// Operand/result layout of one instruction (lane L = 32*h + c, h = L/32):
//   A: lane L supplies row c of block h;  B: lane L supplies column c of block h.
//   result register r (0..31) of lane L holds block r/16, column c,
//   row R(r%16, h) = 8*((r%16)/4) + 4*h + (r%4).
// v_permlane32_swap(x, y) exchanges the upper half of x with the lower half of y.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <type_traits>
#include "otx_math.h"

typedef float f32x32 __attribute__((ext_vector_type(32)));

#define OTX_BLK 32  // contract block size (keys / queries)

__device__ __forceinline__ f32x32 otx_mfma(float a, float b, f32x32 c) {
  return __builtin_amdgcn_mfma_f32_32x32x1f32(a, b, c, 0, 0, 0);
}
// The same with the B operand of one half-wave broadcast to both (BLGP 1: lanes
// 0..31 supply B for all 64 lanes; BLGP 2: lanes 32..63 do).
template <int HALF>
__device__ __forceinline__ f32x32 otx_mfma_bhalf(float a, float b, f32x32 c) {
  return __builtin_amdgcn_mfma_f32_32x32x1f32(a, b, c, 0, 0, HALF ? 2 : 1);
}

// v_mfma_f32_16x16x1_4b_f32: four independent 16x16 rank-1 updates, one IEEE
// fma per output (checked on the GPU like the 32x32 form).  Lane L supplies A
// of block L/16, row L%16 and B of block L/16, column L%16; result register r
// (0..15) of lane L holds block r/4, row 4*(L/16) + r%4, column L%16.
typedef float f32x16 __attribute__((ext_vector_type(16)));
__device__ __forceinline__ f32x16 otx_mfma16(float a, float b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_16x16x1f32(a, b, c, 0, 0, 0);
}

// (x, y) <- (x.lo | y.lo, x.hi | y.hi)   [lo = lanes 0..31, hi = lanes 32..63]
__device__ __forceinline__ void otx_swap_halves(float& x, float& y) {
  auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(y), false, false);
  x = __uint_as_float(r[0]);
  y = __uint_as_float(r[1]);
}

// Broadcast both halves: returns lo-half value in all lanes via *lo and the
// hi-half value in all lanes via *hi.
__device__ __forceinline__ void otx_bcast_halves(float v, float* lo, float* hi) {
  float x = v, y = v;
  otx_swap_halves(x, y);
  *lo = x;
  *hi = y;
}

// ---- correctly rounded exp over register arrays ----
// Copies the biased 2^(j/256) table (otx_exp2_tab256_biased) into LDS (every
// thread of the block calls it; the caller's next __syncthreads publishes it).
__device__ __forceinline__ void otx_load_exp_table(double* tab) {
  for (int i = threadIdx.x; i < OTX_EXP_LE0_TAB_N; i += blockDim.x) tab[i] = otx_exp2_tab256_biased(i);
}

// otx_expf out of line, for the rarely taken fallback below: inlined, its
// series constants would be materialised once per kernel and held in
// registers across the kernels' main loops.
__device__ __attribute__((noinline)) inline float otx_expf_call(float x) { return otx_expf(x); }

// v[j] = exp(v[j]) correctly rounded, in place, for softmax arguments
// v[j] <= 0 (or -inf), j < N <= 32.  The table-driven path (otx_exp_le0_*,
// correctly rounded on that whole domain with no rounding test) runs in chunks
// of NB values, two passes per chunk: first every reduction and table read (so
// the LDS reads of the chunk are in flight together), then every polynomial.
// NB trades latency hiding against live registers.  With CHECKED the inputs
// may be anything (a caller-supplied LSE can make them positive, or NaN): if
// any lane has an input outside [-inf, -0], the whole wave's array is
// evaluated by otx_expf instead, which is correctly rounded for every input
// (and equals the table-driven path wherever that applies).
// Byte offset 8 * (k & 255) of table entry k & 255 in one instruction: a shift
// whose operand select takes byte 0 of k (SDWA).  With the table at LDS address
// 0 the offset is the read's address, so a table read costs one vector
// instruction rather than a mask and a shift-add.
__device__ __forceinline__ uint32_t otx_tab_off(uint32_t k) {
  uint32_t off;
  asm("v_lshlrev_b32_sdwa %0, 3, %1 dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:DWORD src1_sel:BYTE_0"
      : "=v"(off)
      : "v"(k));
  return off;
}

template <int N, bool CHECKED = false, int NB = 8>
__device__ __forceinline__ void otx_exp_n(float (&v)[N], const double* tab) {
  static_assert(N % NB == 0 || N < NB, "chunk size must divide the array");
  constexpr int B = N < NB ? N : NB;
  uint64_t outside = 0;
  if constexpr (CHECKED) {
    // Every input is -0, negative or -inf exactly when every bit pattern, read as a
    // signed integer, is <= 0xFF800000 (-inf): -0 is INT_MIN and the negative values
    // lie between, while negative NaNs (0xFF800001 .. 0xFFFFFFFF: -8388607 .. -1), +0,
    // positive values and positive NaNs (>= 0) all lie above.  So one maximum over the
    // array decides it instead of a comparison per element.  +0 takes the fallback too
    // (rare: s = LSE happens when a row has a single non-negligible probability).
    // (a tree of three-input maxima, so that the wave does not wait on a chain)
    int32_t t[N];
#pragma unroll
    for (int j = 0; j < N; j++) t[j] = (int32_t)otx_f2u(v[j]);
#pragma unroll
    for (int n = N; n > 1; n = (n + 2) / 3) {
#pragma unroll
      for (int i = 0; i < (n + 2) / 3; i++) {
        int32_t m = t[3 * i];
        if (3 * i + 1 < n) m = m > t[3 * i + 1] ? m : t[3 * i + 1];
        if (3 * i + 2 < n) m = m > t[3 * i + 2] ? m : t[3 * i + 2];
        t[i] = m;
      }
    }
    outside = __ballot(t[0] > (int32_t)0xFF800000u);
  }
  if constexpr (CHECKED) {
    // The fallback is decided before the evaluation, so that the inputs need not
    // stay live beside it: each path rewrites the array in place.
    // The fallback takes v[0] and rotates the array by one, N times, so that it
    // needs no per-element selection masks (which would hold scalar registers
    // across the whole kernel).
    if (__builtin_expect(outside != 0, 0)) {
#pragma unroll 1
      for (int j = 0; j < N; j++) {
        const float e = otx_expf_call(v[0]);
#pragma unroll
        for (int i = 0; i + 1 < N; i++) v[i] = v[i + 1];
        v[N - 1] = e;
      }
      return;
    }
  }
#pragma unroll
  for (int c = 0; c < N; c += B) {
    double xd[B], d[B], tv[B];
    uint32_t kb[B];
    // stage by stage over the chunk (the operations of otx_exp_le0_reduce / _finish)
#pragma unroll
    for (int j = 0; j < B; j++) d[j] = otx_exp_le0_t(v[c + j], &xd[j]);
#pragma unroll
    for (int j = 0; j < B; j++) {
      kb[j] = (uint32_t)otx_d2u(d[j]);
      tv[j] = *reinterpret_cast<const double*>(reinterpret_cast<const unsigned char*>(tab) + otx_tab_off(kb[j]));
    }
#pragma unroll
    for (int j = 0; j < B; j++) d[j] = otx_exp_le0_r(d[j], xd[j]);
#pragma unroll
    for (int j = 0; j < B; j++) d[j] = otx_exp_le0_p(d[j]);
#pragma unroll
    for (int j = 0; j < B; j++) v[c + j] = otx_exp_le0_y(d[j], tv[j], kb[j]);
  }
}

__device__ __forceinline__ float otx_exp1(float x, const double* tab) {
  float v[1] = {x};
  otx_exp_n<1>(v, tab);
  return v[0];
}

// Maximum of 32 values by a tree grouped in threes, so that each inner maximum is one v_maximum3_f32 (16
// instructions rather than 31 two-input ones).  NaN-propagating (IEEE maximum): any NaN among the values
// gives NaN, so that a NaN score reaches the row statistics instead of being passed over.  Exact
// otherwise; only the sign of a zero maximum can depend on the grouping.
__device__ __forceinline__ float otx_max2p(float a, float b) { return __builtin_elementwise_maximum(a, b); }
__device__ __forceinline__ float otx_max32(const float (&v)[32]) {
  float t[10];
#pragma unroll
  for (int i = 0; i < 10; i++) t[i] = otx_max2p(otx_max2p(v[3 * i], v[3 * i + 1]), v[3 * i + 2]);
  const float u0 = otx_max2p(otx_max2p(t[0], t[1]), t[2]);
  const float u1 = otx_max2p(otx_max2p(t[3], t[4]), t[5]);
  const float u2 = otx_max2p(otx_max2p(t[6], t[7]), t[8]);
  const float u3 = otx_max2p(otx_max2p(t[9], v[30]), v[31]);
  return otx_max2p(otx_max2p(otx_max2p(u0, u1), u2), u3);
}

// The running maximum's update m' = (mb > m) ? mb : m of the contract, with a NaN block maximum taken
// over (a NaN m then stays NaN: nothing compares greater).  With m NaN every later exp argument s - m
// is NaN and the row ends with O and LSE NaN, as in the contract, where the NaN reaches l through p.
__device__ __forceinline__ float otx_max_update(float mb, float m) { return (mb > m || mb != mb) ? mb : m; }

// Row of result register r held by a lane in half h.
__host__ __device__ constexpr int otx_row(int r, int h) { return 8 * ((r & 15) >> 2) + 4 * h + (r & 3); }

// Direct global -> LDS copy of 16 bytes per lane (global_load_lds_dwordx4):
// lane l of the wave writes lds_base + 16 l (lds_base wave-uniform), from its
// own global address.  Completion is tracked by vmcnt.
__device__ __forceinline__ void otx_dma16(const void* gsrc, void* lds_base) {
  __builtin_amdgcn_global_load_lds(gsrc, (void __attribute__((address_space(3)))*)lds_base, 16, 0, 0);
}
// The same with 4 bytes per lane (global_load_lds_dword): lane l writes lds_base + 4 l.
__device__ __forceinline__ void otx_dma4(const void* gsrc, void* lds_base) {
  __builtin_amdgcn_global_load_lds(gsrc, (void __attribute__((address_space(3)))*)lds_base, 4, 0, 0);
}

// Compute units of the current device, cached per device (256 on MI355X).
inline int otx_cu_count() {
  static int cache[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  if (cache[dev] == 0) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
    cache[dev] = n;
  }
  return cache[dev];
}

// Kernel-level grid order of the forward and dQ kernels: the C ABI's order 0
// (longest chunks first) becomes OTX_ORDER_PAIRED, two chunks per workgroup,
// when the unpaired grid fills at least two rounds of the device's workgroup
// slots (per_cu workgroups per CU); with fewer workgroups pairing would leave
// CUs idle, and order 0 stays one chunk per workgroup (OTX_ORDER_LONGEST).
enum { OTX_ORDER_PAIRED = 0, OTX_ORDER_HEAD = 1, OTX_ORDER_LONGEST = 2 };
inline int otx_chunk_order(int order, long wgs, int per_cu) {
  if (order != 0) return OTX_ORDER_HEAD;
  return wgs >= 2L * per_cu * otx_cu_count() ? OTX_ORDER_PAIRED : OTX_ORDER_LONGEST;
}

// Byte address of an LDS location (the offset ds_* instructions take).
__device__ __forceinline__ uint32_t otx_lds_addr(const void* p) {
  return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void*)p;
}

// ds_read_u16_d16_hi: the bf16 at LDS byte address addr + OFF goes to the high
// half of r and the low half reads as zero, so r becomes the binary32 value of
// that bf16 with no conversion instruction.  On gfx950 (SRAM ECC on) the
// instruction writes zero to the low half (checked on the GPU); the registers
// used with it are also zeroed once and only ever written by it, so the result
// is the same where the low half is preserved instead.  The compiler
// does not track these reads: otx_lds_wait<N> (lgkmcnt(N)) must precede any
// use, tied to the registers it releases.  N counts only reads issued by this
// helper after the ones waited for; LDS requests complete in order, so other
// outstanding LGKM requests only make the wait longer, never shorter.
// Because the compiler takes the destination as written when the read is
// issued, it may copy that register before the wait (it did, when it moved a
// chain's products past the next read of their operand bank): the copy then
// holds the register's old contents whenever the load is slow.  Chains keep
// each bank's consumers ahead of its next read (an empty asm on the
// accumulators after the group's products), and build.py disassembles the
// library and refuses it if any instruction touches a register whose LDS load
// is still in flight (isa_check.py).
template <int OFF>
__device__ __forceinline__ void otx_lds_bf16(float& r, uint32_t addr) {
  static_assert(OFF >= 0 && OFF < 65536, "ds offset is 16 bits");
  asm volatile("ds_read_u16_d16_hi %0, %1 offset:%2" : "+v"(r) : "v"(addr), "i"(OFF));
}
template <int N>
__device__ __forceinline__ void otx_lds_wait(float (&r)[4]) {
  asm volatile("s_waitcnt lgkmcnt(%4)" : "+v"(r[0]), "+v"(r[1]), "+v"(r[2]), "+v"(r[3]) : "i"(N));
}

// lgkmcnt is a 4-bit counter: callers keep at most 15 of these reads outstanding.
// 8-byte LDS read (binary32 x 2) under the same accounting.
typedef float otx_f2 __attribute__((ext_vector_type(2)));
template <int OFF>
__device__ __forceinline__ void otx_lds_f2(otx_f2& r, uint32_t addr) {
  static_assert(OFF >= 0 && OFF < 65536 && OFF % 8 == 0, "ds offset is 16 bits");
  asm volatile("ds_read_b64 %0, %1 offset:%2" : "=v"(r) : "v"(addr), "i"(OFF));
}
template <int N>
__device__ __forceinline__ void otx_lds_wait(float (&r)[2]) {
  asm volatile("s_waitcnt lgkmcnt(%2)" : "+v"(r[0]), "+v"(r[1]) : "i"(N));
}
template <int N>
__device__ __forceinline__ void otx_lds_wait(float (&r)[8]) {
  asm volatile("s_waitcnt lgkmcnt(%8)"
               : "+v"(r[0]), "+v"(r[1]), "+v"(r[2]), "+v"(r[3]), "+v"(r[4]), "+v"(r[5]), "+v"(r[6]), "+v"(r[7])
               : "i"(N));
}
// 4-byte LDS read (one binary32) under the same accounting.
template <int OFF>
__device__ __forceinline__ void otx_lds_b32(float& r, uint32_t addr) {
  static_assert(OFF >= 0 && OFF < 65536 && OFF % 4 == 0, "ds offset is 16 bits");
  asm volatile("ds_read_b32 %0, %1 offset:%2" : "=v"(r) : "v"(addr), "i"(OFF));
}
template <int N>
__device__ __forceinline__ void otx_lds_wait(float (&r)[6]) {
  asm volatile("s_waitcnt lgkmcnt(%6)"
               : "+v"(r[0]), "+v"(r[1]), "+v"(r[2]), "+v"(r[3]), "+v"(r[4]), "+v"(r[5])
               : "i"(N));
}
// 16-byte LDS read (four 32-bit values, 16-byte aligned address) under the same accounting.
typedef float otx_f4 __attribute__((ext_vector_type(4)));
template <int OFF>
__device__ __forceinline__ void otx_lds_f4(otx_f4& r, uint32_t addr) {
  static_assert(OFF >= 0 && OFF < 65536 && OFF % 16 == 0, "ds offset is 16 bits");
  asm volatile("ds_read_b128 %0, %1 offset:%2" : "=v"(r) : "v"(addr), "i"(OFF));
}
template <int N>
__device__ __forceinline__ void otx_lds_wait(otx_f4& a, otx_f4 (&b)[4]) {
  asm volatile("s_waitcnt lgkmcnt(%5)" : "+v"(a), "+v"(b[0]), "+v"(b[1]), "+v"(b[2]), "+v"(b[3]) : "i"(N));
}
template <int N>
__device__ __forceinline__ void otx_lds_wait(otx_f2 (&a)[2], otx_f2 (&b)[2]) {
  asm volatile("s_waitcnt lgkmcnt(%4)" : "+v"(a[0]), "+v"(a[1]), "+v"(b[0]), "+v"(b[1]) : "i"(N));
}
template <int N>
__device__ __forceinline__ void otx_lds_wait(float (&r)[4], otx_f2& a) {
  asm volatile("s_waitcnt lgkmcnt(%5)" : "+v"(r[0]), "+v"(r[1]), "+v"(r[2]), "+v"(r[3]), "+v"(a) : "i"(N));
}
template <int N>
__device__ __forceinline__ void otx_lds_wait(float (&r)[4], otx_f2& a, otx_f2& b) {
  asm volatile("s_waitcnt lgkmcnt(%6)" : "+v"(r[0]), "+v"(r[1]), "+v"(r[2]), "+v"(r[3]), "+v"(a), "+v"(b) : "i"(N));
}

// Compile-time loop: f(std::integral_constant<int, I>) for I = B .. E-1.
template <int B, int E>
struct OtxUnroll {
  template <class F>
  __device__ __forceinline__ static void run(F&& f) {
    if constexpr (B < E) {
      f(std::integral_constant<int, B>{});
      OtxUnroll<B + 1, E>::run(f);
    }
  }
};

// Chains whose A operand of lane L is the element pair (2L, 2L+1) of a row
// (D = 128; for D = 64 lane L takes element 2c + hh): row index d of result
// register r of chain n for a lane in half hh.
template <int D>
__device__ __forceinline__ int dpair_row(int n, int r, int hh) {
  const int rho = otx_row(r, hh), bb = r >> 4;
  if constexpr (D == 128) return 64 * bb + 2 * rho + n;
  else return 2 * rho + bb;
}

// ---- contract block ranges (identical on host and device) ----
__host__ __device__ inline int otx_kblock_lo(int qb, int window) {
  if (window <= 0) return 0;
  int lo = qb - window / OTX_BLK;
  return lo < 0 ? 0 : lo;
}
__host__ __device__ inline int otx_qblock_hi(int kb, int window, int nb) {
  if (window <= 0) return nb - 1;
  int hi = kb + window / OTX_BLK;
  return hi > nb - 1 ? nb - 1 : hi;
}
__host__ __device__ inline bool otx_masked(int i, int j, int window) {
  return j > i || (window > 0 && j <= i - window);
}
// Number of processed (query block, key block) pairs before query block qb.
__host__ __device__ inline long otx_tile_offset(int qb, int window) {
  if (window <= 0) return (long)qb * (qb + 1) / 2;
  long c = window / OTX_BLK;  // a query block qb processes min(qb, c) + 1 key blocks
  if (qb <= c + 1) return (long)qb * (qb + 1) / 2;
  return (c + 1) * (c + 2) / 2 + (long)(qb - c - 1) * (c + 1);
}

// ---- element access for the two storage types ----
// bf16 tensors are handled as raw uint16_t; fp32 as float.
template <typename T> struct Elem;
template <> struct Elem<uint16_t> {
  static constexpr int VEC = 8;  // elements per 16-byte vector
  __device__ __forceinline__ static float get(const uint4& v, int e) {
    uint32_t w = (e >> 1) == 0 ? v.x : (e >> 1) == 1 ? v.y : (e >> 1) == 2 ? v.z : v.w;
    return __uint_as_float((e & 1) ? (w & 0xffff0000u) : (w << 16));
  }
  __device__ __forceinline__ static float ld(const uint16_t* p) { return __uint_as_float((uint32_t)*p << 16); }
  // Two consecutive elements from one 32-bit load.
  __device__ __forceinline__ static void ld2(const uint16_t* p, float* a, float* b) {
    uint32_t w = *(const uint32_t*)p;
    *a = __uint_as_float(w << 16);
    *b = __uint_as_float(w & 0xffff0000u);
  }
  __device__ __forceinline__ static uint16_t put(float f) { return otx_f32_to_bf16(f); }
};
template <> struct Elem<float> {
  static constexpr int VEC = 4;
  __device__ __forceinline__ static float get(const uint4& v, int e) {
    uint32_t w = e == 0 ? v.x : e == 1 ? v.y : e == 2 ? v.z : v.w;
    return __uint_as_float(w);
  }
  __device__ __forceinline__ static float ld(const float* p) { return *p; }
  __device__ __forceinline__ static void ld2(const float* p, float* a, float* b) {
    float2 w = *(const float2*)p;
    *a = w.x;
    *b = w.y;
  }
  __device__ __forceinline__ static float put(float f) { return f; }
};
