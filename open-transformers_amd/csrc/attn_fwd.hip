// Deterministic causal / sliding-window flash attention forward for gfx950.
//
// Replaces the forward of repop.nn.flash_attention.causal_flash_attention
// (called at src/pretrain/model/modules/attention_repop.py:53 of the
// reference).  Output bits follow the arithmetic contract restated by the CPU
// oracle: serial ascending fma folds, online softmax per 32-key block with
// fp32 running max/sum, correctly rounded exp/log/division.
//
// Work decomposition.  A workgroup of NWQ waves owns NWQ consecutive 32-query
// blocks of one (batch, head).  It walks the key blocks in ascending pairs
// (64 keys), staging K (row-major) and V^T into LDS once per pair for all its
// waves.  Each wave owns one query block:
//   S^T = K Q^T : 32x32x1 MFMA chain over d, block 0 = first key block of the
//                 pair, block 1 = second; A = K rows (LDS), B = Q row (VGPRs).
//   one v_permlane32_swap per register pair gives every lane all 32 scores of
//   one (query, key block): lanes 0..31 the first block, lanes 32..63 the second.
//   softmax bookkeeping is then lane-local (plus two half-wave broadcasts).
//   O^T += V^T P^T : chain over keys, blocks = two 32-wide d ranges; A = V^T
//                 rows (LDS), B = the probability broadcast to both halves.
// No atomics; every output element is produced by one lane in one fixed order.
#include "otx_common.h"

namespace otx {

template <typename T, int D, int NWQ>
__global__ __launch_bounds__(64 * NWQ) void attn_fwd_kernel(const T* __restrict__ q, const T* __restrict__ k,
                                                            const T* __restrict__ v, T* __restrict__ o,
                                                            float* __restrict__ lse, int B, int H, int Hkv, int S,
                                                            int window, float sigma, int order) {
  constexpr int ES = sizeof(T);
  constexpr int VEC = Elem<T>::VEC;   // elements per 16-byte vector
  constexpr int PADE = 16 / ES;       // row padding (one vector) against LDS bank conflicts
  constexpr int KP = D + PADE;        // K tile / output staging pitch (elements)
  constexpr int VP = 64 + PADE;       // V^T tile pitch (elements)
  constexpr int NI = D / 64;          // PV instructions per key
  constexpr int QW = D * ES / 4;      // 32-bit words of one Q row
  constexpr int CH = D * ES / 16;     // 16-byte vectors per row
  constexpr int KV_BYTES = (64 * KP + D * VP) * ES;
  constexpr int OS_BYTES = NWQ * 32 * KP * ES;
  constexpr int SMEM = KV_BYTES > OS_BYTES ? KV_BYTES : OS_BYTES;
  __shared__ __align__(16) unsigned char smem[SMEM];
  T* Ks = reinterpret_cast<T*>(smem);
  T* Vt = Ks + 64 * KP;

  const int nqt = S / OTX_BLK;
  const int nchunk = (nqt + NWQ - 1) / NWQ;
  const int BH = B * H;
  const int bid = blockIdx.x;
  int chunk, bh;
  if (order == 0) {  // heaviest query chunks first; heads fastest (same head -> same XCD when BH % 8 == 0)
    chunk = nchunk - 1 - bid / BH;
    bh = bid % BH;
  } else {  // alternative launch order used by the launch-invariance tests
    chunk = bid % nchunk;
    bh = bid / nchunk;
  }
  const int b = bh / H, h = bh % H, g = h / (H / Hkv);
  const int wave = threadIdx.x >> 6, L = threadIdx.x & 63, hh = L >> 5, c = L & 31;
  const int qt = chunk * NWQ + wave;
  const bool wactive = qt < nqt;
  const int qt0 = chunk * NWQ;
  const int qtl = (qt0 + NWQ < nqt ? qt0 + NWQ : nqt) - 1;
  const T* kg = k + ((size_t)b * Hkv + g) * S * D;
  const T* vg = v + ((size_t)b * Hkv + g) * S * D;
  const int qi = qt * OTX_BLK + c;

  // Q row of this lane's query in registers (raw words).
  uint32_t qw[QW];
  if (wactive) {
    const uint4* src = reinterpret_cast<const uint4*>(q + ((size_t)bh * S + qi) * D);
#pragma unroll
    for (int x = 0; x < QW / 4; x++) {
      uint4 t = src[x];
      qw[4 * x] = t.x; qw[4 * x + 1] = t.y; qw[4 * x + 2] = t.z; qw[4 * x + 3] = t.w;
    }
  } else {
#pragma unroll
    for (int x = 0; x < QW; x++) qw[x] = 0;
  }
  auto qelem = [&](int d) -> float {
    if constexpr (ES == 2) {
      uint32_t w = qw[d >> 1];
      return __uint_as_float((d & 1) ? (w & 0xffff0000u) : (w << 16));
    } else {
      return __uint_as_float(qw[d]);
    }
  };

  float m = -__builtin_inff(), l = 0.0f;
  f32x32 acc[NI];
#pragma unroll
  for (int n = 0; n < NI; n++) acc[n] = f32x32{};

  const int lo = otx_kblock_lo(qt, window), hi = qt;
  const int p_begin = otx_kblock_lo(qt0, window) >> 1, p_end = qtl >> 1;
  for (int p = p_begin; p <= p_end; ++p) {
    __syncthreads();
    // ---- stage K rows [64p, 64p+64) and V^T into LDS ----
    for (int idx = threadIdx.x; idx < 64 * CH; idx += 64 * NWQ) {
      const int row = idx / CH, ch = idx % CH;
      const int key = 64 * p + row;
      if (key < S) {
        const uint4 kv = *reinterpret_cast<const uint4*>(kg + (size_t)key * D + ch * VEC);
        *reinterpret_cast<uint4*>(Ks + row * KP + ch * VEC) = kv;
        const uint4 vv = *reinterpret_cast<const uint4*>(vg + (size_t)key * D + ch * VEC);
        if constexpr (ES == 2) {
          const uint32_t w[4] = {vv.x, vv.y, vv.z, vv.w};
#pragma unroll
          for (int e = 0; e < VEC; e++)
            Vt[(ch * VEC + e) * VP + row] = (uint16_t)((e & 1) ? (w[e >> 1] >> 16) : (w[e >> 1] & 0xffffu));
        } else {
          const float w[4] = {__uint_as_float(vv.x), __uint_as_float(vv.y), __uint_as_float(vv.z),
                              __uint_as_float(vv.w)};
#pragma unroll
          for (int e = 0; e < VEC; e++) Vt[(ch * VEC + e) * VP + row] = w[e];
        }
      }
    }
    __syncthreads();
    const int ka = 2 * p, kb = 2 * p + 1;
    const bool doA = wactive && ka >= lo && ka <= hi;
    const bool doB = wactive && kb >= lo && kb <= hi;
    if (!(doA || doB)) continue;

    // ---- S^T = K Q^T over d (serial fma chain) ----
    f32x32 sacc = f32x32{};
    const T* krow = Ks + (hh * 32 + c) * KP;
#pragma unroll
    for (int d0 = 0; d0 < D; d0 += VEC) {
      const uint4 kv = *reinterpret_cast<const uint4*>(krow + d0);
#pragma unroll
      for (int e = 0; e < VEC; e++) sacc = otx_mfma(Elem<T>::get(kv, e), qelem(d0 + e), sacc);
    }
    // ---- gather the 32 scores of (query c, key block ka+hh) into this lane ----
    float s[32];
#pragma unroll
    for (int rr = 0; rr < 16; rr++) {
      float x = sacc[rr], y = sacc[16 + rr];
      otx_swap_halves(x, y);
      s[otx_row(rr, 0)] = x;
      s[otx_row(rr, 1)] = y;
    }
    const int kbase = (2 * p + hh) * OTX_BLK;
    float mb = -__builtin_inff();
#pragma unroll
    for (int j = 0; j < 32; j++) {
      const bool msk = otx_masked(qi, kbase + j, window);
      s[j] = msk ? -__builtin_inff() : s[j] * sigma;
      mb = (s[j] > mb) ? s[j] : mb;
    }
    float mbA, mbB;
    otx_bcast_halves(mb, &mbA, &mbB);
    float ma = m, alpha_a = 1.0f;
    if (doA) {
      ma = (mbA > m) ? mbA : m;
      alpha_a = (ma == m) ? 1.0f : otx_expf(m - ma);
    }
    float mbn = ma, alpha_b = 1.0f;
    if (doB) {
      mbn = (mbB > ma) ? mbB : ma;
      alpha_b = (mbn == ma) ? 1.0f : otx_expf(ma - mbn);
    }
    const float mref = hh ? mbn : ma;
#pragma unroll
    for (int j = 0; j < 32; j++) s[j] = otx_masked(qi, kbase + j, window) ? 0.0f : otx_expf(s[j] - mref);
    // running sum: l = RN(l*alpha), then + p_j ascending (first block in lanes 0..31, second in 32..63)
    if (doA) {
      float t = l * alpha_a;
#pragma unroll
      for (int j = 0; j < 32; j++) t = t + s[j];
      float tlo, thi;
      otx_bcast_halves(t, &tlo, &thi);
      l = tlo;
    }
    if (doB) {
      float t = l * alpha_b;
#pragma unroll
      for (int j = 0; j < 32; j++) t = t + s[j];
      float tlo, thi;
      otx_bcast_halves(t, &tlo, &thi);
      l = thi;
    }
    // ---- O^T = O^T * alpha, then += V^T P^T (serial over keys) ----
    if (doA) {
      if (__any(alpha_a != 1.0f)) {
#pragma unroll
        for (int n = 0; n < NI; n++)
#pragma unroll
          for (int r = 0; r < 32; r++) acc[n][r] = acc[n][r] * alpha_a;
      }
#pragma unroll
      for (int j0 = 0; j0 < 32; j0 += VEC) {
        uint4 va[NI];
#pragma unroll
        for (int n = 0; n < NI; n++) va[n] = *reinterpret_cast<const uint4*>(Vt + (64 * n + L) * VP + j0);
#pragma unroll
        for (int e = 0; e < VEC; e++) {
          float plo, phi;
          otx_bcast_halves(s[j0 + e], &plo, &phi);
          s[j0 + e] = phi;
#pragma unroll
          for (int n = 0; n < NI; n++) acc[n] = otx_mfma(Elem<T>::get(va[n], e), plo, acc[n]);
        }
      }
    } else {
#pragma unroll
      for (int j = 0; j < 32; j++) {
        float plo, phi;
        otx_bcast_halves(s[j], &plo, &phi);
        s[j] = phi;
      }
    }
    if (doB) {
      if (__any(alpha_b != 1.0f)) {
#pragma unroll
        for (int n = 0; n < NI; n++)
#pragma unroll
          for (int r = 0; r < 32; r++) acc[n][r] = acc[n][r] * alpha_b;
      }
#pragma unroll
      for (int j0 = 0; j0 < 32; j0 += VEC) {
        uint4 va[NI];
#pragma unroll
        for (int n = 0; n < NI; n++)
          va[n] = *reinterpret_cast<const uint4*>(Vt + (64 * n + L) * VP + 32 + j0);
#pragma unroll
        for (int e = 0; e < VEC; e++)
#pragma unroll
          for (int n = 0; n < NI; n++) acc[n] = otx_mfma(Elem<T>::get(va[n], e), s[j0 + e], acc[n]);
      }
    }
    m = mbn;
  }

  // ---- epilogue: O = RN(acc / l) in the storage type, LSE = RN(m + log l) ----
  __syncthreads();
  T* Os = reinterpret_cast<T*>(smem) + wave * 32 * KP;
  if (wactive) {
#pragma unroll
    for (int n = 0; n < NI; n++)
#pragma unroll
      for (int r = 0; r < 32; r++) {
        const int d = 64 * n + 32 * (r >> 4) + otx_row(r, hh);
        Os[c * KP + d] = Elem<T>::put(otx_div_rn(acc[n][r], l));
      }
  }
  __syncthreads();
  if (wactive) {
    for (int idx = L; idx < 32 * CH; idx += 64) {
      const int row = idx / CH, ch = idx % CH;
      *reinterpret_cast<uint4*>(o + ((size_t)bh * S + qt * OTX_BLK + row) * D + ch * VEC) =
          *reinterpret_cast<const uint4*>(Os + row * KP + ch * VEC);
    }
    if (hh == 0) lse[(size_t)bh * S + qi] = m + otx_logf(l);
  }
}

template <typename T, int D, int NWQ>
static hipError_t launch_fwd_t(const void* q, const void* k, const void* v, void* o, float* lse, int B, int H,
                               int Hkv, int S, int window, float sigma, int order, hipStream_t stream) {
  const int nqt = S / OTX_BLK;
  const int nchunk = (nqt + NWQ - 1) / NWQ;
  dim3 grid((unsigned)(nchunk * B * H)), block(64 * NWQ);
  hipLaunchKernelGGL((attn_fwd_kernel<T, D, NWQ>), grid, block, 0, stream, (const T*)q, (const T*)k, (const T*)v,
                     (T*)o, lse, B, H, Hkv, S, window, sigma, order);
  return hipGetLastError();
}

template <typename T, int D>
static hipError_t launch_fwd_d(int nwq, const void* q, const void* k, const void* v, void* o, float* lse, int B,
                               int H, int Hkv, int S, int window, float sigma, int order, hipStream_t st) {
  switch (nwq) {
    case 4: return launch_fwd_t<T, D, 4>(q, k, v, o, lse, B, H, Hkv, S, window, sigma, order, st);
    case 2: return launch_fwd_t<T, D, 2>(q, k, v, o, lse, B, H, Hkv, S, window, sigma, order, st);
    default: return launch_fwd_t<T, D, 1>(q, k, v, o, lse, B, H, Hkv, S, window, sigma, order, st);
  }
}

hipError_t launch_fwd(int dtype, int D, int nwq, const void* q, const void* k, const void* v, void* o, float* lse,
                      int B, int H, int Hkv, int S, int window, float sigma, int order, hipStream_t st) {
  if (dtype == 1) {
    if (D == 128) return launch_fwd_d<uint16_t, 128>(nwq, q, k, v, o, lse, B, H, Hkv, S, window, sigma, order, st);
    return launch_fwd_d<uint16_t, 64>(nwq, q, k, v, o, lse, B, H, Hkv, S, window, sigma, order, st);
  }
  if (D == 128) return launch_fwd_d<float, 128>(nwq, q, k, v, o, lse, B, H, Hkv, S, window, sigma, order, st);
  return launch_fwd_d<float, 64>(nwq, q, k, v, o, lse, B, H, Hkv, S, window, sigma, order, st);
}

}  // namespace otx
