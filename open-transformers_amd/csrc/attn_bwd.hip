// Deterministic flash attention backward for gfx950 (no atomics).
//
// Replaces causal_flash_attention_bwd of repop (the backward of the operator
// called at src/pretrain/model/modules/attention_repop.py:53 of the
// reference; fp32 math, bf16 dq/dk/dv: docs/MODEL_OP_DTYPE_TRACE.md:102).
//
// Three kernels, all ordered by the arithmetic contract restated by the CPU
// oracle:
//   dsum : Dsum_i = serial fma of dO_i[d] * O_i[d] over d.
//   dkdv : one wave per 32-key block; walks the processed query blocks of its
//          keys in ascending pairs (query heads of the GQA group outermost).
//          S = Q K^T and dP = dO V^T are 32x32x1 MFMA chains over d; after a
//          half-wave swap each lane owns one key and 32 queries, computes
//          P = exp(RN(s*sigma) - LSE) and dS = RN(P * RN(dP - Dsum)), writes
//          its dS row segment to the workspace and feeds P / dS (broadcast to
//          both half-waves) into the dV^T and dK^T chains over queries.
//          A second bf16 form (attn_dkdv_bf16_kb2_kernel) gives two key blocks
//          to a workgroup of four waves and splits each tile into a dP/softmax
//          phase per (query block, key block) pair and a dV/dK fold phase; the
//          launcher takes it when the one-wave-per-key-block grid would fill
//          the device only once (its long chunks would then set the time).
//   dq   : one wave per 32-query block; dQ^T chain over the processed keys
//          reading the stored dS tiles, scaled by sigma at the end.
// Every output element is produced by a single lane in a single fixed order.
#include "otx_common.h"


namespace otx {

// Rows of O and dO per Dsum workgroup (one lane per row): the two padded row
// blocks take about 70 KB of LDS, so two workgroups share a CU.
template <typename T>
constexpr int dsum_rows() { return sizeof(T) == 2 ? 128 : 64; }

// Dsum_i = fold over d of fma(dO_i[d], O_i[d]) from +0, one lane per row.  The
// workgroup's rows of O and dO are first copied straight into LDS with
// coalesced 16-byte copies (rows padded by 16 bytes: copy unit x is row
// x / U, slot x % U; the pad slot and rows past the end copy an in-bounds
// chunk that is never read), then each lane folds its own row from LDS.
template <typename T, int D>
__global__ __launch_bounds__(dsum_rows<T>()) void attn_dsum_kernel(const T* __restrict__ o, const T* __restrict__ dO,
                                                                  float* __restrict__ dsum, long rows) {
  constexpr int VEC = Elem<T>::VEC;
  constexpr int CH = D / VEC;              // 16-byte chunks per row
  constexpr int RB = D * (int)sizeof(T);   // row bytes in global memory
  constexpr int RP = RB + 16;              // padded pitch in LDS
  constexpr int U = RP / 16;               // copy units per padded row
  constexpr int ROWS = dsum_rows<T>();
  constexpr int NW = ROWS / 64;
  static_assert((ROWS * U) % 64 == 0, "the copy units must fill whole copy instructions");
  __shared__ __align__(16) unsigned char so[ROWS * RP];
  __shared__ __align__(16) unsigned char sd[ROWS * RP];
  const int wave = threadIdx.x >> 6, L = threadIdx.x & 63;
  const long r0 = (long)blockIdx.x * ROWS;
  const int nr = rows - r0 < ROWS ? (int)(rows - r0) : ROWS;
  const unsigned char* go = reinterpret_cast<const unsigned char*>(o + r0 * D);
  const unsigned char* gd = reinterpret_cast<const unsigned char*>(dO + r0 * D);
  for (int i = wave; i < ROWS * U / 64; i += NW) {
    const int x = 64 * i + L, row = x / U, su = x % U;
    const int off = row < nr ? row * RB + 16 * (su < CH ? su : 0) : 0;
    otx_dma16(go + off, so + 64 * i * 16);
    otx_dma16(gd + off, sd + 64 * i * 16);
  }
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // this lane's copies have landed
  __syncthreads();                                   // everyone's copies are visible
  const int row = threadIdx.x;
  if (row >= nr) return;
  const uint4* po = reinterpret_cast<const uint4*>(so + row * RP);
  const uint4* pd = reinterpret_cast<const uint4*>(sd + row * RP);
  float a = 0.0f;
#pragma unroll
  for (int x = 0; x < CH; x++) {
    const uint4 vo = po[x], vd = pd[x];
#pragma unroll
    for (int e = 0; e < VEC; e++) a = __builtin_fmaf(Elem<T>::get(vd, e), Elem<T>::get(vo, e), a);
  }
  dsum[r0 + row] = a;
}

// A-operand pair for the dV/dK/dQ chains: with D = 128 lane L supplies
// d = 2L (instruction 0) and d = 2L+1 (instruction 1); with D = 64 one
// instruction where lane L = 32h + c supplies d = 2c + h.
template <typename T, int D>
__device__ __forceinline__ void load_dpair(const T* row, int L, float* a0, float* a1) {
  if constexpr (D == 128) {
    Elem<T>::ld2(row + 2 * L, a0, a1);
  } else {
    float x, y;
    Elem<T>::ld2(row + 2 * (L & 31), &x, &y);
    *a0 = (L >> 5) ? y : x;
    *a1 = *a0;
  }
}

template <typename T, int D, int NWK>
__global__ __launch_bounds__(64 * NWK) void attn_dkdv_kernel(
    const T* __restrict__ q, const T* __restrict__ k, const T* __restrict__ v, const T* __restrict__ dO,
    const float* __restrict__ lse, const float* __restrict__ dsum, T* __restrict__ dk, T* __restrict__ dv,
    float* __restrict__ ws_ds, int B, int H, int Hkv, int S, int window, float sigma, int order) {
  constexpr int ES = sizeof(T);
  constexpr int VEC = Elem<T>::VEC;
  constexpr int PADE = 16 / ES;
  constexpr int KP = D + PADE;
  constexpr int CH = D * ES / 16;
  constexpr int NI = D / 64;
  constexpr int KV_ELEMS = 2 * NWK * 32 * KP;
  constexpr int QD_ELEMS = 2 * 64 * KP;
  __shared__ __align__(16) T smem_t[KV_ELEMS + QD_ELEMS];
  __shared__ float Ls[64], Ds[64];
  __shared__ double tab[OTX_EXP_LE0_TAB_N];
  T* Ks = smem_t;
  T* Vs = Ks + NWK * 32 * KP;
  T* Qs = Vs + NWK * 32 * KP;
  T* dOs = Qs + 64 * KP;

  const int nkt = S / OTX_BLK;
  const int nchunk = (nkt + NWK - 1) / NWK;
  const int BG = B * Hkv;
  const int G = H / Hkv;
  const int bid = blockIdx.x;
  int chunk, bg;
  if (order == 0) {  // low key chunks see the most query blocks: launch them first
    chunk = bid / BG;
    bg = bid % BG;
  } else {
    chunk = nchunk - 1 - bid % nchunk;
    bg = bid / nchunk;
  }
  const int b = bg / Hkv, g = bg % Hkv;
  const int wave = threadIdx.x >> 6, L = threadIdx.x & 63, hh = L >> 5, c = L & 31;
  const int kt = chunk * NWK + wave;
  const bool wactive = kt < nkt;
  const int kt0 = chunk * NWK;
  const int ktl = (kt0 + NWK < nkt ? kt0 + NWK : nkt) - 1;
  const T* kg = k + (size_t)bg * S * D;
  const T* vg = v + (size_t)bg * S * D;
  const long tiles_per_head = otx_tile_offset(nkt, window);

  otx_load_exp_table(tab);
  // K and V rows of the workgroup's key blocks.
  for (int idx = threadIdx.x; idx < NWK * 32 * CH; idx += 64 * NWK) {
    const int row = idx / CH, ch = idx % CH;
    const int key = kt0 * OTX_BLK + row;
    if (key < S) {
      *reinterpret_cast<uint4*>(Ks + row * KP + ch * VEC) =
          *reinterpret_cast<const uint4*>(kg + (size_t)key * D + ch * VEC);
      *reinterpret_cast<uint4*>(Vs + row * KP + ch * VEC) =
          *reinterpret_cast<const uint4*>(vg + (size_t)key * D + ch * VEC);
    }
  }

  f32x32 accV[NI], accK[NI];
#pragma unroll
  for (int n = 0; n < NI; n++) { accV[n] = f32x32{}; accK[n] = f32x32{}; }

  const int qhi = wactive ? otx_qblock_hi(kt, window, nkt) : -1;
  const int u_begin = kt0 >> 1;
  const int u_end = otx_qblock_hi(ktl, window, nkt) >> 1;
  const int key = kt * OTX_BLK + c;
  const T* krow = Ks + (wave * 32 + c) * KP;
  const T* vrow = Vs + (wave * 32 + c) * KP;

  for (int r = 0; r < G; r++) {
    const int h = g * G + r;
    const size_t bh = (size_t)b * H + h;
    const T* qg = q + bh * S * D;
    const T* dog = dO + bh * S * D;
    for (int u = u_begin; u <= u_end; u++) {
      __syncthreads();
      for (int idx = threadIdx.x; idx < 64 * CH; idx += 64 * NWK) {
        const int row = idx / CH, ch = idx % CH;
        const int qrow = 64 * u + row;
        if (qrow < S) {
          *reinterpret_cast<uint4*>(Qs + row * KP + ch * VEC) =
              *reinterpret_cast<const uint4*>(qg + (size_t)qrow * D + ch * VEC);
          *reinterpret_cast<uint4*>(dOs + row * KP + ch * VEC) =
              *reinterpret_cast<const uint4*>(dog + (size_t)qrow * D + ch * VEC);
        }
      }
      for (int idx = threadIdx.x; idx < 64; idx += 64 * NWK) {
        const int qrow = 64 * u + idx;
        if (qrow < S) {
          Ls[idx] = lse[bh * S + qrow];
          Ds[idx] = dsum[bh * S + qrow];
        }
      }
      __syncthreads();
      const int qa = 2 * u, qb = 2 * u + 1;
      const bool doA = wactive && qa >= kt && qa <= qhi;
      const bool doB = wactive && qb >= kt && qb <= qhi;
      if (!(doA || doB)) continue;

      // ---- S = Q K^T and dP = dO V^T (two interleaved chains over d) ----
      f32x32 sacc = f32x32{}, pacc = f32x32{};
      const T* qrow = Qs + (hh * 32 + c) * KP;
      const T* drow = dOs + (hh * 32 + c) * KP;
#pragma unroll
      for (int d0 = 0; d0 < D; d0 += VEC) {
        const uint4 qv = *reinterpret_cast<const uint4*>(qrow + d0);
        const uint4 kv = *reinterpret_cast<const uint4*>(krow + d0);
        const uint4 dv4 = *reinterpret_cast<const uint4*>(drow + d0);
        const uint4 vv = *reinterpret_cast<const uint4*>(vrow + d0);
#pragma unroll
        for (int e = 0; e < VEC; e++) {
          sacc = otx_mfma(Elem<T>::get(qv, e), Elem<T>::get(kv, e), sacc);
          pacc = otx_mfma(Elem<T>::get(dv4, e), Elem<T>::get(vv, e), pacc);
        }
      }
      float P[32], dS[32];
#pragma unroll
      for (int rr = 0; rr < 16; rr++) {
        float x = sacc[rr], y = sacc[16 + rr];
        otx_swap_halves(x, y);
        P[otx_row(rr, 0)] = x;
        P[otx_row(rr, 1)] = y;
        float x2 = pacc[rr], y2 = pacc[16 + rr];
        otx_swap_halves(x2, y2);
        dS[otx_row(rr, 0)] = x2;
        dS[otx_row(rr, 1)] = y2;
      }
      // lane (hh, c): key `key`, queries (qa + hh) * 32 + i for i = 0..31
      const int qbase = (qa + hh) * OTX_BLK;
      const bool hact = hh ? doB : doA;
      float ex[32];
#pragma unroll
      for (int i = 0; i < 32; i++) {
        const bool msk = !hact || otx_masked(qbase + i, key, window);
        const float sv = P[i] * sigma;
        ex[i] = msk ? -__builtin_inff() : sv - Ls[hh * 32 + i];  // exp(-inf) = +0 for masked pairs
      }
      otx_exp_n<32, true, 16>(ex, tab);
#pragma unroll
      for (int i = 0; i < 32; i++) {
        P[i] = ex[i];
        dS[i] = P[i] * (dS[i] - Ds[hh * 32 + i]);
      }
      // ---- export dS for the dQ kernel: tile (query block, key block), row-major ----
      if ((hh == 0 && doA) || (hh == 1 && doB)) {
        const int qblk = qa + hh;
        float* tile = ws_ds + ((long)bh * tiles_per_head + otx_tile_offset(qblk, window) +
                               (kt - otx_kblock_lo(qblk, window))) * (OTX_BLK * OTX_BLK);
#pragma unroll
        for (int i = 0; i < 32; i++) tile[i * 32 + c] = dS[i];
      }
      // ---- dV^T += dO^T P, dK^T += Q^T dS (serial over queries) ----
      if (doA) {
#pragma unroll
        for (int i = 0; i < 32; i++) {
          float plo, phi, slo, shi;
          otx_bcast_halves(P[i], &plo, &phi);
          otx_bcast_halves(dS[i], &slo, &shi);
          P[i] = phi;
          dS[i] = shi;
          float a0, a1, b0, b1;
          load_dpair<T, D>(dOs + i * KP, L, &a0, &a1);
          load_dpair<T, D>(Qs + i * KP, L, &b0, &b1);
          accV[0] = otx_mfma(a0, plo, accV[0]);
          accK[0] = otx_mfma(b0, slo, accK[0]);
          if constexpr (NI == 2) {
            accV[1] = otx_mfma(a1, plo, accV[1]);
            accK[1] = otx_mfma(b1, slo, accK[1]);
          }
        }
      } else {
#pragma unroll
        for (int i = 0; i < 32; i++) {
          float plo, phi, slo, shi;
          otx_bcast_halves(P[i], &plo, &phi);
          otx_bcast_halves(dS[i], &slo, &shi);
          P[i] = phi;
          dS[i] = shi;
        }
      }
      if (doB) {
#pragma unroll
        for (int i = 0; i < 32; i++) {
          float a0, a1, b0, b1;
          load_dpair<T, D>(dOs + (32 + i) * KP, L, &a0, &a1);
          load_dpair<T, D>(Qs + (32 + i) * KP, L, &b0, &b1);
          accV[0] = otx_mfma(a0, P[i], accV[0]);
          accK[0] = otx_mfma(b0, dS[i], accK[0]);
          if constexpr (NI == 2) {
            accV[1] = otx_mfma(a1, P[i], accV[1]);
            accK[1] = otx_mfma(b1, dS[i], accK[1]);
          }
        }
      }
    }
  }

  // ---- epilogue: dV as is, dK = RN(acc * sigma); transpose through LDS ----
  __syncthreads();
  T* Vo = smem_t + wave * 2 * 32 * KP;
  T* Ko = Vo + 32 * KP;
  if (wactive) {
#pragma unroll
    for (int n = 0; n < NI; n++)
#pragma unroll
      for (int r = 0; r < 32; r++) {
        const int d = dpair_row<D>(n, r, hh);
        Vo[c * KP + d] = Elem<T>::put(accV[n][r]);
        Ko[c * KP + d] = Elem<T>::put(accK[n][r] * sigma);
      }
  }
  __syncthreads();
  if (wactive) {
    for (int idx = L; idx < 32 * CH; idx += 64) {
      const int row = idx / CH, ch = idx % CH;
      const size_t off = ((size_t)bg * S + kt * OTX_BLK + row) * D + ch * VEC;
      *reinterpret_cast<uint4*>(dv + off) = *reinterpret_cast<const uint4*>(Vo + row * KP + ch * VEC);
      *reinterpret_cast<uint4*>(dk + off) = *reinterpret_cast<const uint4*>(Ko + row * KP + ch * VEC);
    }
  }
}

// bf16 dK/dV kernel.  One wave (and one SIMD) per 32-key block, NWK waves
// per workgroup, one workgroup per CU.  LDS holds the workgroup's own K and V
// rows for the whole kernel and two slots of the streamed query side: 64-row
// tiles of Q and dO with their LSE and Dsum, copied straight from global
// memory one tile ahead (global_load_lds, no staging registers).  All rows are
// bf16, padded to 2D + 16 bytes.  Every chain operand is read with
// ds_read_u16_d16_hi (binary32 value of a bf16, no conversion instruction)
// under hand-kept lgkmcnt accounting: groups of 4 reads, two groups ahead (at
// most 12 outstanding).  Arithmetic order is the same as in attn_dkdv_kernel.
template <int D, int NWK, bool SC>
__global__ __launch_bounds__(64 * NWK, 1) void attn_dkdv_bf16_kernel(
    const uint16_t* __restrict__ q, const uint16_t* __restrict__ k, const uint16_t* __restrict__ v,
    const uint16_t* __restrict__ dO, const float* __restrict__ lse, const float* __restrict__ dsum,
    uint16_t* __restrict__ dk, uint16_t* __restrict__ dv, float* __restrict__ ws_ds, int B, int H, int Hkv, int S,
    int window, float sigma, int order, const float* __restrict__ scache) {
  constexpr int NI = D / 64;                 // dV / dK chains per operand
  constexpr int CH = D / 8;                  // 16-byte chunks per global row
  constexpr int RPB = 2 * D + 16;            // padded row pitch in LDS (bytes)
  constexpr int KPH = RPB / 2;               // the same pitch in bf16 elements
  constexpr int UK = RPB / 16;               // 16-byte units per padded row
  constexpr int QT_BYTES = 64 * RPB;         // one 64-row tile of Q (or dO)
  constexpr int SLOT = 2 * QT_BYTES + 2 * 64 * 4;  // Q, dO, LSE, Dsum
  constexpr int KV_BYTES = NWK * 32 * RPB;   // K (or V) rows of the workgroup
  constexpr int IN_BYTES = 2 * SLOT + 2 * KV_BYTES;
  constexpr int OPE = D + 8;                 // bf16 pitch of the epilogue staging (reuses the whole buffer)
  constexpr int OS_BYTES = NWK * 2 * 32 * OPE * 2;
  constexpr int SMEM = IN_BYTES > OS_BYTES ? IN_BYTES : OS_BYTES;
  constexpr int RG = 2 / NI;                 // query rows per dV/dK read group
  // the exp table at LDS address 0 (a table read then needs no base add), the buffers after it
  __shared__ __align__(16) unsigned char lds[OTX_EXP_LE0_TAB_N * 8 + SMEM];
  double* tab = reinterpret_cast<double*>(lds);
  unsigned char* smem = lds + OTX_EXP_LE0_TAB_N * 8;
  uint16_t* Ks = reinterpret_cast<uint16_t*>(smem + 2 * SLOT);
  uint16_t* Vs = reinterpret_cast<uint16_t*>(smem + 2 * SLOT + KV_BYTES);
  auto slot = [&](int sl) { return smem + sl * SLOT; };

  const int nkt = S / OTX_BLK;
  const int nchunk = (nkt + NWK - 1) / NWK;
  const int BG = B * Hkv;
  const int G = H / Hkv;
  const int bid = blockIdx.x;
  int chunk, bg;
  if (order == 0) {  // low key chunks see the most query blocks: launch them first
    chunk = bid / BG;
    bg = bid % BG;
  } else {
    chunk = nchunk - 1 - bid % nchunk;
    bg = bid / nchunk;
  }
  const int b = bg / Hkv, g = bg % Hkv;
  const int wave = threadIdx.x >> 6, L = threadIdx.x & 63, hh = L >> 5, c = L & 31;
  const int kt = chunk * NWK + wave;
  const int kt_u = __builtin_amdgcn_readfirstlane(kt);  // the same value, known to be wave-uniform
  const bool wactive = kt < nkt;
  const int kt0 = chunk * NWK;
  const int ktl = (kt0 + NWK < nkt ? kt0 + NWK : nkt) - 1;
  const long tiles_per_head = otx_tile_offset(nkt, window);
  const int key = kt * OTX_BLK + c;

  // K and V rows of the workgroup's key blocks (V only with the score cache),
  // copied straight into LDS in padded rows (copy unit x is row x / UK, slot x % UK; the pad slot and rows
  // past S copy an in-bounds chunk that is never read).  The loop's first
  // wait and barrier make them visible.
  {
    static_assert((NWK * UK) % 2 == 0, "the K/V copy units must fill whole copy instructions");
    const size_t row0 = (size_t)bg * S + (size_t)kt0 * OTX_BLK;
    const unsigned char* kg = reinterpret_cast<const unsigned char*>(k + row0 * D);
    const unsigned char* vg = reinterpret_cast<const unsigned char*>(v + row0 * D);
    const int rows = S - kt0 * OTX_BLK < NWK * OTX_BLK ? S - kt0 * OTX_BLK : NWK * OTX_BLK;
    for (int i = wave; i < NWK * UK / 2; i += NWK) {
      const int x = 64 * i + L, row = x / UK, su = x % UK;
      const int off = row < rows ? row * (2 * D) + 16 * (su < CH ? su : 0) : 0;
      if constexpr (!SC) otx_dma16(kg + off, reinterpret_cast<unsigned char*>(Ks) + 64 * i * 16);  // the cache replaces Q K^T
      otx_dma16(vg + off, reinterpret_cast<unsigned char*>(Vs) + 64 * i * 16);
    }
  }
  const uint32_t kaddr = otx_lds_addr(Ks + (wave * 32 + c) * KPH);
  const uint32_t vaddr = otx_lds_addr(Vs + (wave * 32 + c) * KPH);
  // operand registers of the d16 reads: three banks of 4, low halves zero
  float opr[3][4];
#pragma unroll
  for (int x = 0; x < 4; x++) { opr[0][x] = 0.0f; opr[1][x] = 0.0f; opr[2][x] = 0.0f; }
  // the score-cache dP chain's operands: four banks of 4, low halves zero
  float opr4[4][4];
#pragma unroll
  for (int x = 0; x < 4; x++) { opr4[x][0] = 0.0f; opr4[x][1] = 0.0f; opr4[x][2] = 0.0f; opr4[x][3] = 0.0f; }

  f32x32 accV[NI], accK[NI];
#pragma unroll
  for (int n = 0; n < NI; n++) { accV[n] = f32x32{}; accK[n] = f32x32{}; }

  const int qhi = wactive ? otx_qblock_hi(kt, window, nkt) : -1;
  const int u_begin = kt0 >> 1;
  const int u_end = otx_qblock_hi(ktl, window, nkt) >> 1;
  const int nu = u_end - u_begin + 1;
  const int n_it = G * nu;

  // ---- tile copies: Q and dO rows [64u, 64u + 64) of head r of the group, LSE, Dsum ----
  // Copy unit x of a padded tile is row x / UK, slot x % UK; the pad slot (and
  // rows past S) copy an in-bounds chunk that is never read.  The source
  // offsets of this wave's units (i = wave + NWK m) are the same for every
  // tile and are formed once; an offset at or past rows * 2D is a row past S.
  constexpr int UPW = (UK + NWK - 1) / NWK;
  const int wave_u = __builtin_amdgcn_readfirstlane(wave);
  int uoff[UPW];
#pragma unroll
  for (int m = 0; m < UPW; m++) {
    const int x = 64 * (wave_u + NWK * m) + L, row = x / UK, su = x % UK;
    uoff[m] = row * (2 * D) + 16 * (su < CH ? su : 0);
  }
  auto issue = [&](int it, int sl) {
    const int r = it / nu, u = u_begin + it % nu;
    const size_t bh = (size_t)b * H + g * G + r;
    const unsigned char* qg = reinterpret_cast<const unsigned char*>(q + (bh * S + 64 * u) * D);
    const unsigned char* dg = reinterpret_cast<const unsigned char*>(dO + (bh * S + 64 * u) * D);
    const int rows = S - 64 * u < 64 ? S - 64 * u : 64;
    const int lim = rows * (2 * D);
    unsigned char* base = slot(sl);
#pragma unroll
    for (int m = 0; m < UPW; m++) {
      const int i = wave_u + NWK * m;
      if (i < UK) {
        const int off = uoff[m] < lim ? uoff[m] : 0;
        otx_dma16(qg + off, base + 64 * i * 16);
        otx_dma16(dg + off, base + QT_BYTES + 64 * i * 16);
      }
    }
    if (wave_u == 0) {
      const size_t row = bh * S + 64 * u + (L < rows ? L : 0);
      otx_dma4(lse + row, base + 2 * QT_BYTES);
      otx_dma4(dsum + row, base + 2 * QT_BYTES + 256);
    }
  };

  if (n_it > 0) issue(0, 0);
  otx_load_exp_table(tab);
  // With the score cache the dP chain's B operand, row `key` of V, is the same
  // for every tile: its first half is read into registers once (as the
  // binary32 value of each bf16), so over that half of d the chain reads only
  // its dO operand from LDS.  Measured (A/B in one process, bytes equal):
  // half of the row -0.3 to -1.0 % on the dK/dV launch; the whole row +2 to
  // +4 % (the compiler then parks registers in the accumulation file around
  // the exp and copies them back every tile).
  constexpr int VR = SC ? D / 2 : 1;
  float vreg[VR];
  if constexpr (SC) {
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // this lane's copies of V (and of tile 0) have landed
    __syncthreads();                                   // every V copy is visible
    const uint16_t* vr = Vs + (wave * 32 + c) * KPH;
#pragma unroll
    for (int d = 0; d < VR; d++) vreg[d] = __uint_as_float((uint32_t)vr[d] << 16);
  }
  for (int it = 0; it < n_it; ++it) {
    const int sl = it & 1;
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // this lane's copies of tile it (and of K, V) have landed
    __syncthreads();  // every copy of tile it is visible; slot sl ^ 1 is no longer read
    if (it + 1 < n_it) issue(it + 1, sl ^ 1);
    const int r = it / nu, u = u_begin + it % nu;
    const size_t bh = (size_t)b * H + g * G + r;
    const int qa = 2 * u, qb = 2 * u + 1;
    const bool doA = wactive && qa >= kt && qa <= qhi;
    const bool doB = wactive && qb >= kt && qb <= qhi;
    if (!(doA || doB)) continue;
    const uint32_t qt_a = otx_lds_addr(slot(sl)), dt_a = qt_a + QT_BYTES;
    const float* Lb = reinterpret_cast<const float*>(slot(sl) + 2 * QT_BYTES);
    const float* Db = Lb + 64;
    if constexpr (SC) {
      // the dV / dK accumulators stay in the accumulation registers (the chains read and write them
      // there), which leaves the vector registers to the half row of V
#pragma unroll
      for (int n = 0; n < NI; n++) asm volatile("" : "+a"(accV[n]), "+a"(accK[n]));
    }

    float P[32], dS[32];
    if constexpr (SC) {
      // ---- scores from the forward's cache: lane (hh, c) reads row c (key) of the transposed tile
      // (query block qa + hh, key block kt); an inactive half reads the active half's tile and
      // discards it (its arguments become -inf below) ----
      // (tile (qb, kt) lies qb - lo(qb) tiles after tile (qa, kt): a wave-uniform base and a 32-bit lane offset)
      const bool selb = (hh ? doB : doA) ? hh != 0 : !doA;
      const float* t0 =
          scache + (((long)bh * tiles_per_head + otx_tile_offset(qa, window) + (kt_u - otx_kblock_lo(qa, window))) << 10);
      const float4* src = reinterpret_cast<const float4*>(
          reinterpret_cast<const unsigned char*>(t0) +
          ((selb ? (uint32_t)(qb - otx_kblock_lo(qb, window)) << 12 : 0u) + 128u * (uint32_t)c));
#pragma unroll
      for (int x = 0; x < 8; x++) {
        const float4 t4 = src[x];
        P[4 * x] = t4.x;
        P[4 * x + 1] = t4.y;
        P[4 * x + 2] = t4.z;
        P[4 * x + 3] = t4.w;
      }
      // ---- dP = dO V^T (chain over d); group G = d 2G, 2G + 1: the dO reads, and the V reads past
      // the first VR elements (held in registers); three groups ahead ----
      f32x32 pacc = f32x32{};
      const uint32_t drow = dt_a + (hh * 32 + c) * RPB;
      constexpr int NG = D / 2, NGR = VR / 2;
      auto nrd = [](int Gd) { return Gd < NGR ? 2 : 4; };  // reads of group Gd
      auto rd = [&](auto gc) {
        constexpr int Gd = decltype(gc)::value, BK = Gd % 4;
        otx_lds_bf16<4 * Gd>(opr4[BK][0], drow);
        if constexpr (Gd >= NGR) otx_lds_bf16<4 * Gd>(opr4[BK][1], vaddr);
        otx_lds_bf16<4 * Gd + 2>(opr4[BK][2], drow);
        if constexpr (Gd >= NGR) otx_lds_bf16<4 * Gd + 2>(opr4[BK][3], vaddr);
      };
      rd(std::integral_constant<int, 0>{});
      rd(std::integral_constant<int, 1>{});
      rd(std::integral_constant<int, 2>{});
      OtxUnroll<0, NG>::run([&](auto gc) {
        constexpr int Gd = decltype(gc)::value, BK = Gd % 4;
        if constexpr (Gd + 3 < NG) {
          rd(std::integral_constant<int, Gd + 3>{});
          otx_lds_wait<nrd(Gd + 1) + nrd(Gd + 2) + nrd(Gd + 3)>(opr4[BK]);
        } else if constexpr (Gd + 2 < NG) {
          otx_lds_wait<nrd(Gd + 1) + nrd(Gd + 2)>(opr4[BK]);
        } else if constexpr (Gd + 1 < NG) {
          otx_lds_wait<nrd(Gd + 1)>(opr4[BK]);
        } else {
          otx_lds_wait<0>(opr4[BK]);
        }
        if constexpr (Gd < NGR) {
          pacc = otx_mfma(opr4[BK][0], vreg[2 * Gd], pacc);
          pacc = otx_mfma(opr4[BK][2], vreg[2 * Gd + 1], pacc);
        } else {
          pacc = otx_mfma(opr4[BK][0], opr4[BK][1], pacc);
          pacc = otx_mfma(opr4[BK][2], opr4[BK][3], pacc);
        }
      });
#pragma unroll
      for (int rr = 0; rr < 16; rr++) {
        float x2 = pacc[rr], y2 = pacc[16 + rr];
        otx_swap_halves(x2, y2);
        dS[otx_row(rr, 0)] = x2;
        dS[otx_row(rr, 1)] = y2;
      }
    } else {
      // ---- S = Q K^T and dP = dO V^T (two interleaved chains over d); group G = one d ----
      f32x32 sacc = f32x32{}, pacc = f32x32{};
      const uint32_t qrow = qt_a + (hh * 32 + c) * RPB, drow = dt_a + (hh * 32 + c) * RPB;
      auto rd = [&](auto gc) {
        constexpr int Gd = decltype(gc)::value, BK = Gd % 3;
        otx_lds_bf16<2 * Gd>(opr[BK][0], qrow);
        otx_lds_bf16<2 * Gd>(opr[BK][1], kaddr);
        otx_lds_bf16<2 * Gd>(opr[BK][2], drow);
        otx_lds_bf16<2 * Gd>(opr[BK][3], vaddr);
      };
      rd(std::integral_constant<int, 0>{});
      rd(std::integral_constant<int, 1>{});
      OtxUnroll<0, D>::run([&](auto gc) {
        constexpr int Gd = decltype(gc)::value, BK = Gd % 3;
        if constexpr (Gd + 2 < D) {
          rd(std::integral_constant<int, Gd + 2>{});
          otx_lds_wait<8>(opr[BK]);
        } else if constexpr (Gd + 1 < D) {
          otx_lds_wait<4>(opr[BK]);
        } else {
          otx_lds_wait<0>(opr[BK]);
        }
        sacc = otx_mfma(opr[BK][0], opr[BK][1], sacc);
        pacc = otx_mfma(opr[BK][2], opr[BK][3], pacc);
      });
      // s = RN(dot * sigma), the contract's score
#pragma unroll
      for (int rr = 0; rr < 16; rr++) {
        float x = sacc[rr], y = sacc[16 + rr];
        otx_swap_halves(x, y);
        P[otx_row(rr, 0)] = x * sigma;
        P[otx_row(rr, 1)] = y * sigma;
        float x2 = pacc[rr], y2 = pacc[16 + rr];
        otx_swap_halves(x2, y2);
        dS[otx_row(rr, 0)] = x2;
        dS[otx_row(rr, 1)] = y2;
      }
    }
    // lane (hh, c): key `key`, queries (qa + hh) * 32 + i for i = 0..31
    const int qbase = (qa + hh) * OTX_BLK;
    const bool hact = hh ? doB : doA;
    const bool need_mask = (qa + hh) == kt || (window > 0 && (qa + hh) == qhi);
    float ex[32];
#pragma unroll
    for (int i = 0; i < 32; i++) ex[i] = P[i] - Lb[hh * 32 + i];
    if (__any(need_mask || !hact)) {
#pragma unroll
      for (int i = 0; i < 32; i++)  // exp(-inf) = +0 for masked pairs
        ex[i] = (!hact || otx_masked(qbase + i, key, window)) ? -__builtin_inff() : ex[i];
    }
    otx_exp_n<32, true, 16>(ex, tab);
#pragma unroll
    for (int i = 0; i < 32; i++) {
      P[i] = ex[i];
      dS[i] = P[i] * (dS[i] - Db[hh * 32 + i]);
    }
    // ---- export dS for the dQ kernel: tile (query block, key block), row-major ----
    if (hact) {
      // Non-temporal stores: the tiles (as large as the score cache) are read once, by the dQ kernel after
      // this kernel ends, so they are not kept in the caches (measured: dK/dV -0.8 to -1.4 % at B4 H16 S2048, within
      // +-0.8 % at the other shapes).  Tiles (qa, kt) and (qb, kt) lie qb - lo(qb) tiles apart, so a lane adds a 32-bit byte offset to
      // the wave-uniform address of tile (qa, kt): the stores take the scalar-base form, one 32-bit
      // address register per lane.
      float* t0 = ws_ds + ((long)bh * tiles_per_head + otx_tile_offset(qa, window) + (kt_u - otx_kblock_lo(qa, window))) *
                              (OTX_BLK * OTX_BLK);
      const uint32_t loff = (hh ? (uint32_t)(qb - otx_kblock_lo(qb, window)) << 12 : 0u) + 4u * (uint32_t)c;
      float* tile = reinterpret_cast<float*>(reinterpret_cast<unsigned char*>(t0) + loff);
#pragma unroll
      for (int i = 0; i < 32; i++) __builtin_nontemporal_store(dS[i], &tile[i * 32]);
    }
    // ---- dV^T += dO^T P, dK^T += Q^T dS (serial over queries) ----
    // Lane L's A operands of query row i: elements 2L, 2L + 1 of dO and Q rows
    // (D = 128), or element 2c + hh (D = 64); RG rows per read group of 4.
    const uint32_t lane_off = D == 128 ? 4 * L : 4 * c + 2 * hh;
    const uint32_t do_l = dt_a + lane_off, q_l = qt_a + lane_off;
    auto half_chain = [&](auto half_c) {
      constexpr int R0 = decltype(half_c)::value * 32;
      constexpr int NG = 32 / RG;
      auto rd = [&](auto gc) {
        constexpr int Gd = decltype(gc)::value, BK = Gd % 3;
        OtxUnroll<0, RG>::run([&](auto e) {
          constexpr int E = decltype(e)::value, ROW = R0 + RG * Gd + E;
          OtxUnroll<0, NI>::run([&](auto nc) {
            constexpr int Nn = decltype(nc)::value;
            otx_lds_bf16<ROW * RPB + 2 * Nn>(opr[BK][E * 2 * NI + Nn], do_l);
            otx_lds_bf16<ROW * RPB + 2 * Nn>(opr[BK][E * 2 * NI + NI + Nn], q_l);
          });
        });
      };
      rd(std::integral_constant<int, 0>{});
      rd(std::integral_constant<int, 1>{});
      OtxUnroll<0, NG>::run([&](auto gc) {
        constexpr int Gd = decltype(gc)::value, BK = Gd % 3;
        if constexpr (Gd + 2 < NG) {
          rd(std::integral_constant<int, Gd + 2>{});
          otx_lds_wait<8>(opr[BK]);
        } else if constexpr (Gd + 1 < NG) {
          otx_lds_wait<4>(opr[BK]);
        } else {
          otx_lds_wait<0>(opr[BK]);
        }
        OtxUnroll<0, RG>::run([&](auto e) {
          constexpr int E = decltype(e)::value, I = RG * Gd + E;
          constexpr int HALF = R0 / 32;  // block A's P and dS in lanes 0..31, block B's in 32..63
          OtxUnroll<0, NI>::run([&](auto nc) {
            constexpr int Nn = decltype(nc)::value;
            accV[Nn] = otx_mfma_bhalf<HALF>(opr[BK][E * 2 * NI + Nn], P[I], accV[Nn]);
            accK[Nn] = otx_mfma_bhalf<HALF>(opr[BK][E * 2 * NI + NI + Nn], dS[I], accK[Nn]);
          });
        });
      });
    };
    if (doA) half_chain(std::integral_constant<int, 0>{});
    if (doB) half_chain(std::integral_constant<int, 1>{});
  }

  // ---- epilogue: dV as is, dK = RN(acc * sigma); transpose through LDS ----
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // no copy into LDS is still in flight
  __syncthreads();
  uint16_t* Vo = reinterpret_cast<uint16_t*>(smem) + wave * 2 * 32 * OPE;
  uint16_t* Ko = Vo + 32 * OPE;
  if (wactive) {
#pragma unroll
    for (int n = 0; n < NI; n++)
#pragma unroll
      for (int r = 0; r < 32; r++) {
        const int d = dpair_row<D>(n, r, hh);
        Vo[c * OPE + d] = otx_f32_to_bf16(accV[n][r]);
        Ko[c * OPE + d] = otx_f32_to_bf16(accK[n][r] * sigma);
      }
  }
  __syncthreads();
  if (wactive) {
    for (int idx = L; idx < 32 * CH; idx += 64) {
      const int row = idx / CH, ch = idx % CH;
      const size_t off = ((size_t)bg * S + kt * OTX_BLK + row) * D + ch * 8;
      *reinterpret_cast<uint4*>(dv + off) = *reinterpret_cast<const uint4*>(Vo + row * OPE + ch * 8);
      *reinterpret_cast<uint4*>(dk + off) = *reinterpret_cast<const uint4*>(Ko + row * OPE + ch * 8);
    }
  }
}

// bf16 dK/dV kernel with two key blocks per workgroup of four waves.  Each
// 64-query tile of a head runs in two phases separated by a barrier:
//   A: wave w takes one (query block, key block) pair, qa + (w & 1) against
//      kt0 + (w >> 1): its dP (and, without the score cache, its scores) are
//      one v_mfma_f32_16x16x1_4b_f32 chain over d (one fma per output and step,
//      the contract's serial fold), then P = exp(RN(s - LSE)) and
//      dS = RN(P * RN(dP - Dsum)) lane-locally; P and dS go to LDS (and dS to
//      the workspace for the dQ kernel).  With the score cache the chain's V
//      operand is held in registers for most of d (it is the same for every
//      tile), since four d16 reads per two 16x16 products saturate the LDS,
//      and each remaining read serves a pair of d (CBSZ / ABID and BLGP
//      broadcasts between the blocks that share rows or columns).
//   B: wave w folds two of the eight dV / dK accumulators over the tile's
//      queries: key block kt0 + (w >> 1), dV (w even) or dK (w odd), the A
//      operands (dO or Q rows) by ds_read_u16_d16_hi and the B operand (P or
//      dS of query i, key c) by ds_read_b32 from phase A's tiles, one read per
//      pair of queries (half-wave hh holds query 2G + hh, broadcast by BLGP).
// The arithmetic and its order are those of attn_dkdv_bf16_kernel; only the
// split of work between waves differs.  With half the key blocks per
// workgroup the grid has twice the workgroups, so the causal triangle's long
// chunks no longer set the time of a grid that fills the device only once.
template <int D, bool SC>
__global__ __launch_bounds__(256, 1) void attn_dkdv_bf16_kb2_kernel(
    const uint16_t* __restrict__ q, const uint16_t* __restrict__ k, const uint16_t* __restrict__ v,
    const uint16_t* __restrict__ dO, const float* __restrict__ lse, const float* __restrict__ dsum,
    uint16_t* __restrict__ dk, uint16_t* __restrict__ dv, float* __restrict__ ws_ds, int B, int H, int Hkv, int S,
    int window, float sigma, int order, const float* __restrict__ scache) {
  constexpr int KB = 2;                      // key blocks per workgroup
  constexpr int NI = D / 64;                 // dV / dK chains per accumulator kind
  constexpr int CH = D / 8;                  // 16-byte chunks per global row
  constexpr int RPB = 2 * D + 16;            // padded row pitch in LDS (bytes)
  constexpr int KPH = RPB / 2;               // the same pitch in bf16 elements
  constexpr int UK = RPB / 16;               // 16-byte units per padded row
  constexpr int QT_BYTES = 64 * RPB;         // one 64-row tile of Q (or dO)
  constexpr int SLOT = 2 * QT_BYTES + 2 * 64 * 4;  // Q, dO, LSE, Dsum
  constexpr int KV_BYTES = KB * 32 * RPB;    // K (or V) rows of the workgroup
  constexpr int XPB = 36 * 4;                // row pitch of an exchanged 32x32 tile (bytes)
  constexpr int XT_BYTES = 32 * XPB;
  constexpr int X_BYTES = 2 * KB * 2 * XT_BYTES;  // P and dS of the four pairs
  constexpr int IN_BYTES = 2 * SLOT + (SC ? 1 : 2) * KV_BYTES + X_BYTES;
  constexpr int OPE = D + 8;                 // bf16 pitch of the epilogue staging (reuses the buffer)
  constexpr int OS_BYTES = KB * 2 * 32 * OPE * 2;
  constexpr int SMEM = IN_BYTES > OS_BYTES ? IN_BYTES : OS_BYTES;
  // the exp table at LDS address 0 (a table read then needs no base add), the buffers after it
  __shared__ __align__(16) unsigned char lds[OTX_EXP_LE0_TAB_N * 8 + SMEM];
  double* tab = reinterpret_cast<double*>(lds);
  unsigned char* smem = lds + OTX_EXP_LE0_TAB_N * 8;
  unsigned char* Xs = smem + 2 * SLOT;
  uint16_t* Vs = reinterpret_cast<uint16_t*>(Xs + X_BYTES);
  uint16_t* Ks = Vs + KB * 32 * KPH;         // without the score cache only
  auto slot = [&](int sl) { return smem + sl * SLOT; };

  const int nkt = S / OTX_BLK;
  const int nchunk = (nkt + KB - 1) / KB;
  const int BG = B * Hkv;
  const int G = H / Hkv;
  const int bid = blockIdx.x;
  int chunk, bg;
  if (order == 0) {  // low key chunks see the most query blocks: launch them first
    chunk = bid / BG;
    bg = bid % BG;
  } else {
    chunk = nchunk - 1 - bid % nchunk;
    bg = bid / nchunk;
  }
  const int b = bg / Hkv, g = bg % Hkv;
  const int wave = threadIdx.x >> 6, L = threadIdx.x & 63, hh = L >> 5, c = L & 31;
  const int kt0 = chunk * KB;
  const int ktl = (kt0 + KB < nkt ? kt0 + KB : nkt) - 1;
  const long tiles_per_head = otx_tile_offset(nkt, window);

  // K and V rows of the workgroup's key blocks (V only with the score cache),
  // copied straight into LDS in padded rows (copy unit x is row x / UK, slot
  // x % UK; the pad slot and rows past S copy an in-bounds chunk that is never
  // read).  The loop's first wait and barrier make them visible.
  {
    static_assert((KB * 32 * UK) % 64 == 0, "the K/V copy units must fill whole copy instructions");
    const size_t row0 = (size_t)bg * S + (size_t)kt0 * OTX_BLK;
    const unsigned char* kg = reinterpret_cast<const unsigned char*>(k + row0 * D);
    const unsigned char* vg = reinterpret_cast<const unsigned char*>(v + row0 * D);
    const int rows = S - kt0 * OTX_BLK < KB * OTX_BLK ? S - kt0 * OTX_BLK : KB * OTX_BLK;
    for (int i = wave; i < KB * 32 * UK / 64; i += 4) {
      const int x = 64 * i + L, row = x / UK, su = x % UK;
      const int off = row < rows ? row * (2 * D) + 16 * (su < CH ? su : 0) : 0;
      if constexpr (!SC) otx_dma16(kg + off, reinterpret_cast<unsigned char*>(Ks) + 64 * i * 16);
      otx_dma16(vg + off, reinterpret_cast<unsigned char*>(Vs) + 64 * i * 16);
    }
  }

  // ---- phase A roles: pair (query block qa + aq, key block ka) ----
  const int aq = wave & 1, akb = wave >> 1, ka = kt0 + akb;
  const int ka_qhi = ka < nkt ? otx_qblock_hi(ka, window, nkt) : -1;
  // lane L: A rows of the 16x16 chains are queries qsub, B columns keys ksub
  const int qsub = (L >> 5) * 16 + (L & 15), ksub = ((L >> 4) & 1) * 16 + (L & 15);
  const uint32_t va_addr = otx_lds_addr(Vs + (akb * 32 + ksub) * KPH);
  const uint32_t ka_addr = otx_lds_addr(Ks + (akb * 32 + ksub) * KPH);
  // ---- phase B roles: key block kb, dV (role 0) or dK (role 1) ----
  const int bkb = wave >> 1, role = wave & 1, kb = kt0 + bkb;
  const int kb_qhi = kb < nkt ? otx_qblock_hi(kb, window, nkt) : -1;

  float opr[4][4];  // phase A operand banks (d16 reads: low halves zero)
  float opb[3][6];  // phase B operand banks
#pragma unroll
  for (int x = 0; x < 4; x++) { opr[0][x] = 0.0f; opr[1][x] = 0.0f; opr[2][x] = 0.0f; opr[3][x] = 0.0f; }
#pragma unroll
  for (int x = 0; x < 6; x++) { opb[0][x] = 0.0f; opb[1][x] = 0.0f; opb[2][x] = 0.0f; }

  f32x32 acc[NI];
#pragma unroll
  for (int n = 0; n < NI; n++) acc[n] = f32x32{};

  const int u_begin = kt0 >> 1;
  const int u_end = otx_qblock_hi(ktl, window, nkt) >> 1;
  const int nu = u_end - u_begin + 1;
  const int n_it = G * nu;

  // Source offsets of this wave's copy units of a tile (i = wave + 4 m), formed
  // once; an offset at or past rows * 2D is a row past S.
  constexpr int UPW = (UK + 3) / 4;
  const int wave_u = __builtin_amdgcn_readfirstlane(wave);
  int uoff[UPW];
#pragma unroll
  for (int m = 0; m < UPW; m++) {
    const int x = 64 * (wave_u + 4 * m) + L, row = x / UK, su = x % UK;
    uoff[m] = row * (2 * D) + 16 * (su < CH ? su : 0);
  }
  auto issue = [&](int it, int sl) {
    const int r = it / nu, u = u_begin + it % nu;
    const size_t bh = (size_t)b * H + g * G + r;
    const unsigned char* qg = reinterpret_cast<const unsigned char*>(q + (bh * S + 64 * u) * D);
    const unsigned char* dg = reinterpret_cast<const unsigned char*>(dO + (bh * S + 64 * u) * D);
    const int rows = S - 64 * u < 64 ? S - 64 * u : 64;
    const int lim = rows * (2 * D);
    unsigned char* base = slot(sl);
#pragma unroll
    for (int m = 0; m < UPW; m++) {
      const int i = wave_u + 4 * m;
      if (i < UK) {
        const int off = uoff[m] < lim ? uoff[m] : 0;
        otx_dma16(qg + off, base + 64 * i * 16);
        otx_dma16(dg + off, base + QT_BYTES + 64 * i * 16);
      }
    }
    if (wave_u == 0) {
      const size_t row = bh * S + 64 * u + (L < rows ? L : 0);
      otx_dma4(lse + row, base + 2 * QT_BYTES);
      otx_dma4(dsum + row, base + 2 * QT_BYTES + 256);
    }
  };
  auto pair_active = [&](int qblk, int kblk) {
    return kblk < nkt && qblk >= kblk && qblk <= otx_qblock_hi(kblk, window, nkt);
  };

  if (n_it > 0) issue(0, 0);
  otx_load_exp_table(tab);
  // With the score cache, phase A's B operand (V row ksub of key block akb) is
  // the same for every tile.  Its first VR elements are read into registers
  // once, which takes the V reads off the chain's first VR / 2 groups (four
  // d16 reads per two 16x16 products keep the LDS saturated).  7/8 of the row
  // fit beside the exp's registers when the exp runs in chunks of 4.
  constexpr int VR = SC ? 7 * D / 8 : 1;
  float vreg[VR];
  if constexpr (SC) {
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // this lane's copies of V (and of tile 0) have landed
    __syncthreads();                                   // every V copy is visible
    const uint16_t* vr = Vs + (akb * 32 + ksub) * KPH;
#pragma unroll
    for (int d = 0; d < VR; d++) vreg[d] = __uint_as_float((uint32_t)vr[d] << 16);
  }
  for (int it = 0; it < n_it; ++it) {
    const int sl = it & 1;
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // this lane's copies of tile it (and of K, V) have landed
    __syncthreads();  // tile it is visible; slot sl ^ 1 and the exchange tiles are no longer read
    if (it + 1 < n_it) issue(it + 1, sl ^ 1);
    const int r = it / nu, u = u_begin + it % nu;
    const size_t bh = (size_t)b * H + g * G + r;
    const int qa = 2 * u;
    // workgroup-uniform: skip tiles where no pair is processed
    if (!(pair_active(qa, kt0) || pair_active(qa + 1, kt0) || pair_active(qa, kt0 + 1) ||
          pair_active(qa + 1, kt0 + 1)))
      continue;
    const uint32_t qt_a = otx_lds_addr(slot(sl)), dt_a = qt_a + QT_BYTES;
    const float* Lb = reinterpret_cast<const float*>(slot(sl) + 2 * QT_BYTES);
    const float* Db = Lb + 64;

    // ================= phase A =================
    const int qw = qa + aq;
    if (ka < nkt && qw >= ka && qw <= ka_qhi) {
      // the pair's tile, formed from wave-uniform values so that its address stays in scalar registers
      // (the cache loads and dS stores then take the scalar-base form with 32-bit lane offsets)
      const int qw_u = __builtin_amdgcn_readfirstlane(qw), ka_u = __builtin_amdgcn_readfirstlane(ka);
      const long tile = (long)bh * tiles_per_head + otx_tile_offset(qw_u, window) + (ka_u - otx_kblock_lo(qw_u, window));
      float s[16];
      if constexpr (SC) {
        // the forward's cached scores of this pair, stored [key][query]
        const float* src = scache + (tile << 10);
#pragma unroll
        for (int qs = 0; qs < 2; qs++)
#pragma unroll
          for (int ks = 0; ks < 2; ks++) {
            const float4 t4 = *reinterpret_cast<const float4*>(src + (ks * 16 + (L & 15)) * 32 + qs * 16 +
                                                               4 * (L >> 4));
            s[qs * 8 + ks * 4 + 0] = t4.x;
            s[qs * 8 + ks * 4 + 1] = t4.y;
            s[qs * 8 + ks * 4 + 2] = t4.z;
            s[qs * 8 + ks * 4 + 3] = t4.w;
          }
      }
      f32x16 pacc = f32x16{}, sacc = f32x16{};
      const uint32_t drow = dt_a + (aq * 32 + qsub) * RPB;
      if constexpr (SC) {
        // dP = dO V^T, one chain over d; read group G = d 2G, 2G + 1, three groups ahead.  Blocks 2j and
        // 2j + 1 of the 16x16 instruction share their A rows (the same 16 queries): one d16 read serves the
        // pair of d (blocks 2j read element 2G, blocks 2j + 1 element 2G + 1), and each product takes its
        // element from one block of the two by the CBSZ / ABID broadcast.  Likewise blocks j and j + 2 share
        // their B columns (the same 16 keys): past the first VR elements one read of V serves the pair (the
        // lower half-wave reads 2G, the upper 2G + 1), broadcast by BLGP.  (Measured: this kernel 0 to -0.9 %,
        // bytes equal.)
        const uint32_t drow_p = drow + 2 * ((L >> 4) & 1), va_p = va_addr + 2 * (L >> 5);
        constexpr int NG = D / 2, NGR = VR / 2;
        auto nrd = [](int Gd) { return Gd < NGR ? 1 : 2; };  // reads of group Gd
        auto rd = [&](auto gc) {
          constexpr int Gd = decltype(gc)::value, BK = Gd % 4;
          otx_lds_bf16<4 * Gd>(opr[BK][0], drow_p);
          if constexpr (Gd >= NGR) otx_lds_bf16<4 * Gd>(opr[BK][1], va_p);
        };
        rd(std::integral_constant<int, 0>{});
        rd(std::integral_constant<int, 1>{});
        rd(std::integral_constant<int, 2>{});
        OtxUnroll<0, NG>::run([&](auto gc) {
          constexpr int Gd = decltype(gc)::value, BK = Gd % 4;
          if constexpr (Gd + 3 < NG) {
            rd(std::integral_constant<int, Gd + 3>{});
            otx_lds_wait<nrd(Gd + 1) + nrd(Gd + 2) + nrd(Gd + 3)>(opr[BK]);
          } else if constexpr (Gd + 2 < NG) {
            otx_lds_wait<nrd(Gd + 1) + nrd(Gd + 2)>(opr[BK]);
          } else if constexpr (Gd + 1 < NG) {
            otx_lds_wait<nrd(Gd + 1)>(opr[BK]);
          } else {
            otx_lds_wait<0>(opr[BK]);
          }
          if constexpr (Gd < NGR) {
            pacc = __builtin_amdgcn_mfma_f32_16x16x1f32(opr[BK][0], vreg[2 * Gd], pacc, 1, 0, 0);
            pacc = __builtin_amdgcn_mfma_f32_16x16x1f32(opr[BK][0], vreg[2 * Gd + 1], pacc, 1, 1, 0);
          } else {
            pacc = __builtin_amdgcn_mfma_f32_16x16x1f32(opr[BK][0], opr[BK][1], pacc, 1, 0, 1);
            pacc = __builtin_amdgcn_mfma_f32_16x16x1f32(opr[BK][0], opr[BK][1], pacc, 1, 1, 2);
          }
          asm volatile("" : "+a"(pacc));  // bank BK is consumed before it is read again
        });
      } else {
        // S = Q K^T and dP = dO V^T, two interleaved chains over d; group G = one d
        const uint32_t qrow = qt_a + (aq * 32 + qsub) * RPB;
        auto rd = [&](auto gc) {
          constexpr int Gd = decltype(gc)::value, BK = Gd % 4;
          otx_lds_bf16<2 * Gd>(opr[BK][0], qrow);
          otx_lds_bf16<2 * Gd>(opr[BK][1], ka_addr);
          otx_lds_bf16<2 * Gd>(opr[BK][2], drow);
          otx_lds_bf16<2 * Gd>(opr[BK][3], va_addr);
        };
        rd(std::integral_constant<int, 0>{});
        rd(std::integral_constant<int, 1>{});
        rd(std::integral_constant<int, 2>{});
        OtxUnroll<0, D>::run([&](auto gc) {
          constexpr int Gd = decltype(gc)::value, BK = Gd % 4;
          if constexpr (Gd + 3 < D) {
            rd(std::integral_constant<int, Gd + 3>{});
            otx_lds_wait<12>(opr[BK]);
          } else {
            otx_lds_wait<4 * (D - 1 - Gd)>(opr[BK]);
          }
          sacc = otx_mfma16(opr[BK][0], opr[BK][1], sacc);
          pacc = otx_mfma16(opr[BK][2], opr[BK][3], pacc);
          // Both products of this group stay ahead of the next group's reads, so
          // bank BK is consumed before it is read again and never copied while
          // its loads are in flight.
          asm volatile("" : "+a"(sacc), "+a"(pacc));
        });
#pragma unroll
        for (int x = 0; x < 16; x++) s[x] = sacc[x] * sigma;  // s = RN(dot * sigma), the contract's score
      }
      // lane L, register x: query qw*32 + qi(x), key ka*32 + kj(x)
      float lq[16], dsq[16];
#pragma unroll
      for (int qs = 0; qs < 2; qs++) {
        const float4 l4 = *reinterpret_cast<const float4*>(Lb + aq * 32 + qs * 16 + 4 * (L >> 4));
        const float4 d4 = *reinterpret_cast<const float4*>(Db + aq * 32 + qs * 16 + 4 * (L >> 4));
#pragma unroll
        for (int ks = 0; ks < 2; ks++) {
          lq[qs * 8 + ks * 4 + 0] = l4.x; lq[qs * 8 + ks * 4 + 1] = l4.y;
          lq[qs * 8 + ks * 4 + 2] = l4.z; lq[qs * 8 + ks * 4 + 3] = l4.w;
          dsq[qs * 8 + ks * 4 + 0] = d4.x; dsq[qs * 8 + ks * 4 + 1] = d4.y;
          dsq[qs * 8 + ks * 4 + 2] = d4.z; dsq[qs * 8 + ks * 4 + 3] = d4.w;
        }
      }
      float ex[16];
#pragma unroll
      for (int x = 0; x < 16; x++) ex[x] = s[x] - lq[x];
      const bool need_mask = qw == ka || (window > 0 && qw == ka_qhi);
      if (__any(need_mask)) {
#pragma unroll
        for (int x = 0; x < 16; x++) {
          const int qi = (x >> 3) * 16 + 4 * (L >> 4) + (x & 3), kj = ((x >> 2) & 1) * 16 + (L & 15);
          ex[x] = otx_masked(qw * OTX_BLK + qi, ka * OTX_BLK + kj, window) ? -__builtin_inff() : ex[x];
        }
      }
      otx_exp_n<16, true, 4>(ex, tab);  // chunks of 4: registers for V (above)
      float* tds = ws_ds + (tile << 10);
      unsigned char* xp = Xs + (2 * wave) * XT_BYTES;  // P of this pair; dS follows
#pragma unroll
      for (int x = 0; x < 16; x++) {
        const int qi = (x >> 3) * 16 + 4 * (L >> 4) + (x & 3), kj = ((x >> 2) & 1) * 16 + (L & 15);
        const float p = ex[x];
        const float ds = p * (pacc[x] - dsq[x]);
        *reinterpret_cast<float*>(xp + qi * XPB + 4 * kj) = p;
        *reinterpret_cast<float*>(xp + XT_BYTES + qi * XPB + 4 * kj) = ds;
        __builtin_nontemporal_store(ds, &tds[qi * 32 + kj]);  // the dQ kernel's tile, row-major
      }
    }
    __syncthreads();  // phase A's P and dS are visible

    // ================= phase B =================
    // dV^T += dO^T P or dK^T += Q^T dS over the tile's queries (serial)
    const uint32_t lane_off = D == 128 ? 4 * L : 4 * c + 2 * hh;
    const uint32_t a_l = (role ? qt_a : dt_a) + lane_off;
    auto half_chain = [&](auto half_c) {
      constexpr int HB = decltype(half_c)::value;
      constexpr int R0 = HB * 32;
      // The B operand (P or dS of query i, key c) is the same in both half-waves: half hh reads row
      // 2G + hh of the group's pair, and each row's products take it from one half by the BLGP
      // broadcast (measured: this kernel -0.1 to -1.4 %, bytes equal).
      constexpr int RPG = 2 * NI + 1;  // reads per group of two query rows
      constexpr int NG = 16;
      const uint32_t x_l = otx_lds_addr(Xs + (2 * (2 * bkb + HB) + role) * XT_BYTES) + 4 * c + hh * XPB;
      auto rd = [&](auto gc) {
        constexpr int Gd = decltype(gc)::value, BK = Gd % 3;
        OtxUnroll<0, 2>::run([&](auto e) {
          constexpr int E = decltype(e)::value, I = 2 * Gd + E;
          OtxUnroll<0, NI>::run([&](auto nc) {
            constexpr int Nn = decltype(nc)::value;
            otx_lds_bf16<(R0 + I) * RPB + 2 * Nn>(opb[BK][E * (NI + 1) + Nn], a_l);
          });
        });
        otx_lds_b32<2 * Gd * XPB>(opb[BK][NI], x_l);
      };
      rd(std::integral_constant<int, 0>{});
      rd(std::integral_constant<int, 1>{});
      OtxUnroll<0, NG>::run([&](auto gc) {
        constexpr int Gd = decltype(gc)::value, BK = Gd % 3;
        if constexpr (Gd + 2 < NG) {
          rd(std::integral_constant<int, Gd + 2>{});
          otx_lds_wait<2 * RPG>(opb[BK]);
        } else if constexpr (Gd + 1 < NG) {
          otx_lds_wait<RPG>(opb[BK]);
        } else {
          otx_lds_wait<0>(opb[BK]);
        }
        OtxUnroll<0, 2>::run([&](auto e) {
          constexpr int E = decltype(e)::value;
          OtxUnroll<0, NI>::run([&](auto nc) {
            constexpr int Nn = decltype(nc)::value;
            acc[Nn] = otx_mfma_bhalf<E>(opb[BK][E * (NI + 1) + Nn], opb[BK][NI], acc[Nn]);
          });
        });
      });
    };
    if (kb < nkt && qa >= kb && qa <= kb_qhi) half_chain(std::integral_constant<int, 0>{});
    if (kb < nkt && qa + 1 >= kb && qa + 1 <= kb_qhi) half_chain(std::integral_constant<int, 1>{});
  }

  // ---- epilogue: dV as is, dK = RN(acc * sigma); transpose through LDS ----
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // no copy into LDS is still in flight
  __syncthreads();
  uint16_t* Os = reinterpret_cast<uint16_t*>(smem) + wave * 32 * OPE;
  if (kb < nkt) {
#pragma unroll
    for (int n = 0; n < NI; n++)
#pragma unroll
      for (int rr = 0; rr < 32; rr++) {
        const int d = dpair_row<D>(n, rr, hh);
        Os[c * OPE + d] = otx_f32_to_bf16(role ? acc[n][rr] * sigma : acc[n][rr]);
      }
  }
  __syncthreads();
  if (kb < nkt) {
    uint16_t* out = role ? dk : dv;
    for (int idx = L; idx < 32 * CH; idx += 64) {
      const int row = idx / CH, ch = idx % CH;
      const size_t off = ((size_t)bg * S + kb * OTX_BLK + row) * D + ch * 8;
      *reinterpret_cast<uint4*>(out + off) = *reinterpret_cast<const uint4*>(Os + row * OPE + ch * 8);
    }
  }
}

// dQ = RN(sigma * fold over key blocks and keys of dS_ij k_j), one wave per
// 32-query block, NWQ waves per workgroup sharing each key block's K rows.
// The K rows of a key block and each wave's dS tile travel straight from
// global memory into LDS (16 bytes per lane per instruction, no registers),
// double-buffered one key block ahead of the matrix chains.  The dS tile is
// stored with its 16-byte chunks XOR-swizzled by row, so that the row reads of
// the 32 lanes (one row each) fall into distinct LDS banks.
template <typename T, int D, int NWQ>
__global__ __launch_bounds__(64 * NWQ) void attn_dq_kernel(const T* __restrict__ k, const float* __restrict__ ws_ds,
                                                           T* __restrict__ dq, int B, int H, int Hkv, int S,
                                                           int window, float sigma, int order, int hg) {
  constexpr int ES = sizeof(T);
  constexpr int VEC = Elem<T>::VEC;
  constexpr int PADE = 16 / ES;
  constexpr int KP = D + PADE;             // epilogue staging pitch (elements)
  constexpr int CH = D * ES / 16;
  constexpr int NI = D / 64;
  constexpr int KB_BYTES = 32 * D * ES;    // K rows of one key block (unpadded)
  constexpr int KB_CH = KB_BYTES / 16;     // 16-byte chunks of them
  constexpr int ST_BYTES = 32 * 32 * 4;    // one dS tile
  constexpr int BUF_BYTES = 2 * KB_BYTES + 2 * NWQ * ST_BYTES;
  constexpr int O_BYTES = NWQ * 32 * KP * ES;
  constexpr int SMEM = BUF_BYTES > O_BYTES ? BUF_BYTES : O_BYTES;
  static_assert(KB_CH % (64 * NWQ) == 0 || (64 * NWQ) % KB_CH == 0, "K chunks must split evenly over the lanes");
  __shared__ __align__(128) unsigned char smem[SMEM];  // 128-aligned: dS rows are addressed by XOR

  const int nqt = S / OTX_BLK;
  const int G = H / Hkv;
  // A workgroup's NWQ waves take NWQ consecutive query blocks of one head, or,
  // with hg (GQA, NWQ dividing the group), NWQ query heads of one KV head on one
  // query block, so that every wave has the same key range (dQ of different
  // heads are independent).  A chunk is the workgroup's unit along the query
  // axis, a head unit its unit along the head axis.
  const int nchunk = hg ? nqt : (nqt + NWQ - 1) / NWQ;
  const int BU = hg ? B * Hkv * (G / NWQ) : B * H;
  const int bid = blockIdx.x;
  // OTX_ORDER_PAIRED: workgroup (j, u) runs chunk nchunk-1-j and then chunk j of head unit u, so that under
  // the causal mask every workgroup carries about the same work and the grid drains together (several
  // workgroups share a CU, so the hardware's dispatch order cannot balance unequal ones).
  // OTX_ORDER_LONGEST: one chunk per workgroup, longest first.  OTX_ORDER_HEAD: one chunk each, head-major.
  const int ntask = (order == OTX_ORDER_PAIRED && nchunk - 1 - bid / BU != bid / BU) ? 2 : 1;
  for (int task = 0; task < ntask; ++task) {
  int chunk, bu;
  if (order == OTX_ORDER_PAIRED) {
    chunk = task == 0 ? nchunk - 1 - bid / BU : bid / BU;
    bu = bid % BU;
  } else if (order == OTX_ORDER_LONGEST) {
    chunk = nchunk - 1 - bid / BU;
    bu = bid % BU;
  } else {
    chunk = bid % nchunk;
    bu = bid / nchunk;
  }
  const int wave = threadIdx.x >> 6, L = threadIdx.x & 63, hh = L >> 5, c = L & 31;
  int b, g, bh, qt, qt0, qtl;
  if (hg) {
    const int bgk = bu / (G / NWQ);
    b = bgk / Hkv;
    g = bgk % Hkv;
    bh = b * H + g * G + (bu % (G / NWQ)) * NWQ + wave;
    qt = qt0 = qtl = chunk;
  } else {
    bh = bu;
    b = bh / H;
    g = (bh % H) / G;
    qt = chunk * NWQ + wave;
    qt0 = chunk * NWQ;
    qtl = (qt0 + NWQ < nqt ? qt0 + NWQ : nqt) - 1;
  }
  const bool wactive = qt < nqt;
  const T* kg = k + ((size_t)b * Hkv + g) * S * D;
  const long tiles_per_head = otx_tile_offset(nqt, window);
  const int lo = wactive ? otx_kblock_lo(qt, window) : 0;
  const int kt_begin = otx_kblock_lo(qt0, window);
  auto kbuf = [&](int sl) { return smem + sl * KB_BYTES; };
  auto sbuf = [&](int sl) { return smem + 2 * KB_BYTES + (sl * NWQ + wave) * ST_BYTES; };

  // Copies of key block kt into buffer slot sl: its K rows (all waves share
  // the work) and, for an active wave that processes (qt, kt), its dS tile.
  auto issue = [&](int kt, int sl) {
    const unsigned char* ksrc = reinterpret_cast<const unsigned char*>(kg + (size_t)kt * OTX_BLK * D);
    for (int base = wave * 64; base < KB_CH; base += 64 * NWQ)
      otx_dma16(ksrc + (size_t)(base + L) * 16, kbuf(sl) + base * 16);
    if (wactive && kt >= lo && kt <= qt) {
      const float* tile =
          ws_ds + ((long)bh * tiles_per_head + otx_tile_offset(qt, window) + (kt - lo)) * (OTX_BLK * OTX_BLK);
#pragma unroll
      for (int i = 0; i < 4; i++) {
        const int slot = 64 * i + L, row = slot >> 3, x = slot & 7;  // slot (row, x) holds chunk x ^ (row & 7)
        otx_dma16(tile + row * 32 + 4 * (x ^ (row & 7)), sbuf(sl) + 64 * i * 16);
      }
    }
  };

  f32x32 acc[NI];
#pragma unroll
  for (int n = 0; n < NI; n++) acc[n] = f32x32{};
  // operand registers of the d16 reads (bf16 K), low halves zero
  float opr[2][4];
#pragma unroll
  for (int x = 0; x < 4; x++) { opr[0][x] = 0.0f; opr[1][x] = 0.0f; }

  // Every wave takes part in the copies and barriers of every key block of the
  // workgroup, but accumulates only over its own key blocks [a_lo, a_hi]: three
  // loops, so that the accumulators stay in the matrix registers across the
  // active one.
  auto sync = [&](int kt) {
    const int sl = (kt - kt_begin) & 1;
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // this lane's copies of key block kt have landed
    __syncthreads();  // everyone's copies are visible, and slot sl ^ 1 is no longer read
    if (kt + 1 <= qtl) issue(kt + 1, sl ^ 1);
    return sl;
  };
  auto compute = [&](int sl) {
    if constexpr (sizeof(T) == 2) {
      // Per group of 2 keys: the K elements by d16 reads and the two dS values by
      // an 8-byte read, one group ahead with hand-kept lgkmcnt accounting (at
      // most 10 reads outstanding).
      constexpr int RPK = D == 128 ? 2 : 1;  // K reads per key
      const uint32_t kaddr = otx_lds_addr(kbuf(sl)) + (D == 128 ? 4 * L : 4 * c + 2 * hh);
      const uint32_t srow = otx_lds_addr(sbuf(sl)) + c * 128 + ((c & 7) << 4);  // chunk x sits at slot x ^ (c & 7)
      otx_f2 gs[2];
      auto rd = [&](auto gc) {
        constexpr int G = decltype(gc)::value, BK = G & 1;
        OtxUnroll<0, 2 * RPK>::run([&](auto e) {
          constexpr int E = decltype(e)::value;
          otx_lds_bf16<(2 * G + E / RPK) * (2 * D) + 2 * (E % RPK)>(opr[BK][E], kaddr);
        });
        otx_lds_f2<8 * (G & 1)>(gs[BK], srow ^ ((G >> 1) << 4));
      };
      rd(std::integral_constant<int, 0>{});
      OtxUnroll<0, 16>::run([&](auto gc) {
        constexpr int G = decltype(gc)::value, BK = G & 1;
        if constexpr (G + 1 < 16) {
          rd(std::integral_constant<int, G + 1>{});
          otx_lds_wait<2 * RPK + 1>(opr[BK], gs[BK]);
        } else {
          otx_lds_wait<0>(opr[BK], gs[BK]);
        }
        OtxUnroll<0, 2>::run([&](auto e) {
          constexpr int E = decltype(e)::value;
          acc[0] = otx_mfma(opr[BK][E * RPK], gs[BK][E], acc[0]);
          if constexpr (NI == 2) acc[1] = otx_mfma(opr[BK][E * RPK + 1], gs[BK][E], acc[1]);
        });
      });
      return;
    }
    const T* Ks = reinterpret_cast<const T*>(kbuf(sl));
    const float4* st = reinterpret_cast<const float4*>(sbuf(sl));
#pragma unroll
    for (int j0 = 0; j0 < 32; j0 += 4) {
      const float4 sv = st[c * 8 + ((j0 >> 2) ^ (c & 7))];  // dS[query c][j0 .. j0 + 3]
      const float bvals[4] = {sv.x, sv.y, sv.z, sv.w};
#pragma unroll
      for (int e = 0; e < 4; e++) {
        float a0, a1;
        load_dpair<T, D>(Ks + (j0 + e) * D, L, &a0, &a1);
        acc[0] = otx_mfma(a0, bvals[e], acc[0]);
        if constexpr (NI == 2) acc[1] = otx_mfma(a1, bvals[e], acc[1]);
      }
    }
  };
  const int a_lo = wactive ? lo : qtl + 1;
  const int a_hi = wactive ? qt : qtl;
  if (kt_begin <= qtl) issue(kt_begin, 0);
  int kt = kt_begin;
  for (; kt < a_lo; kt++) sync(kt);
  for (; kt <= a_hi; kt++) compute(sync(kt));
  for (; kt <= qtl; kt++) sync(kt);

  __syncthreads();
  T* Os = reinterpret_cast<T*>(smem) + wave * 32 * KP;
  if (wactive) {
#pragma unroll
    for (int n = 0; n < NI; n++)
#pragma unroll
      for (int r = 0; r < 32; r++) Os[c * KP + dpair_row<D>(n, r, hh)] = Elem<T>::put(acc[n][r] * sigma);
  }
  __syncthreads();
  if (wactive) {
    for (int idx = L; idx < 32 * CH; idx += 64) {
      const int row = idx / CH, ch = idx % CH;
      *reinterpret_cast<uint4*>(dq + ((size_t)bh * S + qt * OTX_BLK + row) * D + ch * VEC) =
          *reinterpret_cast<const uint4*>(Os + row * KP + ch * VEC);
    }
  }
  __syncthreads();  // the next task's copies overwrite the output staging
  }
}

template <typename T, int D>
static hipError_t launch_bwd_t(int nw, const void* q, const void* k, const void* v, const void* o, const float* lse,
                               const void* dO, void* dq, void* dk, void* dv, float* dsum, float* ds, int B, int H,
                               int Hkv, int S, int window, float sigma, int order, int stages, const float* scache,
                               hipStream_t st) {
  const long rows = (long)B * H * S;
  hipError_t e = hipSuccess;
  if (stages & 1) {
    constexpr int DR = dsum_rows<T>();
    hipLaunchKernelGGL((attn_dsum_kernel<T, D>), dim3((unsigned)((rows + DR - 1) / DR)), dim3(DR), 0, st,
                       (const T*)o, (const T*)dO, dsum, rows);
    e = hipGetLastError();
    if (e != hipSuccess) return e;
  }
  const int nt = S / OTX_BLK;
#define OTX_LAUNCH_DKDV(NW)                                                                                      \
  hipLaunchKernelGGL((attn_dkdv_kernel<T, D, NW>), dim3((unsigned)(((nt + NW - 1) / NW) * B * Hkv)),            \
                     dim3(64 * NW), 0, st, (const T*)q, (const T*)k, (const T*)v, (const T*)dO, lse, dsum,      \
                     (T*)dk, (T*)dv, ds, B, H, Hkv, S, window, sigma, order)
  // dQ workgroups: head-grouped (see attn_dq_kernel) for GQA in the default launch order.
  auto dq_hg = [&](int nw) { return (nw > 1 && (H / Hkv) % nw == 0 && order == 0) ? 1 : 0; };
  auto dq_nu = [&](int nw) { return (long)(dq_hg(nw) ? nt : (nt + nw - 1) / nw); };
  auto dq_bu = [&](int nw) { return dq_hg(nw) ? (long)B * Hkv * ((H / Hkv) / nw) : (long)B * H; };
  auto dq_order = [&](int nw) { return otx_chunk_order(order, dq_nu(nw) * dq_bu(nw), 2); };
#define OTX_LAUNCH_DQ(NW)                                                                                        \
  hipLaunchKernelGGL((attn_dq_kernel<T, D, NW>),                                                                 \
                     dim3((unsigned)((dq_order(NW) == OTX_ORDER_PAIRED ? (dq_nu(NW) + 1) / 2 : dq_nu(NW)) *        \
                                     dq_bu(NW))),                                                                \
                     dim3(64 * NW), 0, st, (const T*)k, ds, (T*)dq, B, H, Hkv, S, window, sigma, dq_order(NW),     \
                     dq_hg(NW))
  if (!(stages & 2)) {
  } else if constexpr (sizeof(T) == 2) {
#define OTX_LAUNCH_DKDV_BF16(NW, SC)                                                                         \
  hipLaunchKernelGGL((attn_dkdv_bf16_kernel<D, NW, SC>), dim3((unsigned)(((nt + NW - 1) / NW) * B * Hkv)),    \
                     dim3(64 * NW), 0, st, (const uint16_t*)q, (const uint16_t*)k, (const uint16_t*)v,         \
                     (const uint16_t*)dO, lse, dsum, (uint16_t*)dk, (uint16_t*)dv, ds, B, H, Hkv, S, window,   \
                     sigma, order, scache)
#define OTX_LAUNCH_DKDV_KB2(SC)                                                                              \
  hipLaunchKernelGGL((attn_dkdv_bf16_kb2_kernel<D, SC>), dim3((unsigned)(((nt + 1) / 2) * B * Hkv)), dim3(256), \
                     0, st, (const uint16_t*)q, (const uint16_t*)k, (const uint16_t*)v, (const uint16_t*)dO, lse,  \
                     dsum, (uint16_t*)dk, (uint16_t*)dv, ds, B, H, Hkv, S, window, sigma, order, scache)
    // Kernel choice (every choice gives the same bits).  Four key blocks per
    // workgroup, one wave each, costs least per key block under a full causal
    // mask; when that grid fills the device's workgroup slots (one per CU) at
    // most once, the longest chunks set the time, and two key blocks per
    // workgroup (phases A/B, twice the workgroups) balance it.  Under a sliding
    // window with the score cache the two-key-block form wins at any grid size:
    // its query range per workgroup is two blocks narrower, so fewer tiles have
    // idle waves at the band's edges.  nw 4 (the default variant) takes that
    // choice, nw 1 the other one, nw 2 two key blocks with one wave each.
    const bool one_round = (long)((nt + 3) / 4) * B * Hkv <= otx_cu_count();
    const bool prefer_kb2 = one_round || (window > 0 && scache != nullptr);
    const bool kb2 = nw == 4 ? prefer_kb2 : (nw == 1 ? !prefer_kb2 : false);
    if (scache != nullptr) {
      if (kb2) OTX_LAUNCH_DKDV_KB2(true); else if (nw == 2) OTX_LAUNCH_DKDV_BF16(2, true); else OTX_LAUNCH_DKDV_BF16(4, true);
    } else {
      if (kb2) OTX_LAUNCH_DKDV_KB2(false); else if (nw == 2) OTX_LAUNCH_DKDV_BF16(2, false); else OTX_LAUNCH_DKDV_BF16(4, false);
    }
#undef OTX_LAUNCH_DKDV_BF16
#undef OTX_LAUNCH_DKDV_KB2
  } else {
    if (scache != nullptr) return hipErrorInvalidValue;  // the score cache is a bf16-path feature
    // fp32 with D = 128 holds twice the LDS per key block: at most 2 key blocks per workgroup.
    constexpr bool kWide = D != 128;
    switch (nw) {
      case 4:
        if constexpr (kWide) OTX_LAUNCH_DKDV(4); else OTX_LAUNCH_DKDV(2);
        break;
      case 2: OTX_LAUNCH_DKDV(2); break;
      default: OTX_LAUNCH_DKDV(1); break;
    }
  }
  e = hipGetLastError();
  if (e != hipSuccess) return e;
  if (stages & 4) {
    switch (nw) {
      case 4: OTX_LAUNCH_DQ(4); break;
      case 2: OTX_LAUNCH_DQ(2); break;
      default: OTX_LAUNCH_DQ(1); break;
    }
  }
#undef OTX_LAUNCH_DKDV
#undef OTX_LAUNCH_DQ
  return hipGetLastError();
}

// scache (bf16 only, may be null): the forward's score cache, read by dK/dV instead of recomputing Q K^T.
hipError_t launch_bwd(int dtype, int D, int nw, const void* q, const void* k, const void* v, const void* o,
                      const float* lse, const void* dO, void* dq, void* dk, void* dv, float* dsum, float* ds, int B,
                      int H, int Hkv, int S, int window, float sigma, int order, int stages, const float* scache,
                      hipStream_t st) {
  if (dtype == 1) {
    if (D == 128)
      return launch_bwd_t<uint16_t, 128>(nw, q, k, v, o, lse, dO, dq, dk, dv, dsum, ds, B, H, Hkv, S, window, sigma,
                                         order, stages, scache, st);
    return launch_bwd_t<uint16_t, 64>(nw, q, k, v, o, lse, dO, dq, dk, dv, dsum, ds, B, H, Hkv, S, window, sigma,
                                      order, stages, scache, st);
  }
  if (D == 128)
    return launch_bwd_t<float, 128>(nw, q, k, v, o, lse, dO, dq, dk, dv, dsum, ds, B, H, Hkv, S, window, sigma, order, stages,
                                    scache, st);
  return launch_bwd_t<float, 64>(nw, q, k, v, o, lse, dO, dq, dk, dv, dsum, ds, B, H, Hkv, S, window, sigma, order, stages,
                                 scache, st);
}

}  // namespace otx
