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
// (64 keys), staging K and V (converted to binary32, row-major) into LDS once
// per pair for all its waves, so that every MFMA operand read from LDS is
// ready to use.  Each wave owns one query block:
//   S^T = K Q^T : 32x32x1 MFMA chain over d, block 0 = first key block of the
//                 pair, block 1 = second; A = K rows (LDS), B = Q row (VGPRs).
//   one v_permlane32_swap per register pair gives every lane all 32 scores of
//   one (query, key block): lanes 0..31 the first block, lanes 32..63 the second.
//   softmax bookkeeping is then lane-local (plus two half-wave broadcasts).
//   O^T += V^T P^T : chain over keys, blocks = two 32-wide d ranges; A = V row
//                 segment (LDS, 64 consecutive d per key), B = the probability
//                 broadcast to both halves.
// Masking is only evaluated on the diagonal block and on the block at the
// window's lower edge; other blocks are dense.
// No atomics; every output element is produced by one lane in one fixed order.
#include "otx_common.h"

namespace otx {

template <typename T, int D, int NWQ>
// bf16 fits two waves per SIMD (the register budget that lets one wave's
// softmax overlap the other's MFMA chains); fp32 keeps D raw Q words and runs one.
__global__ __launch_bounds__(64 * NWQ) __attribute__((amdgpu_waves_per_eu(sizeof(T) == 2 ? 2 : 1)))
void attn_fwd_kernel(const T* __restrict__ q, const T* __restrict__ k,
                                                            const T* __restrict__ v, T* __restrict__ o,
                                                            float* __restrict__ lse, int B, int H, int Hkv, int S,
                                                            int window, float sigma, int order) {
  constexpr int ES = sizeof(T);
  constexpr int VEC = Elem<T>::VEC;   // elements per 16-byte global vector
  constexpr int KPF = D + 4;          // K tile pitch in floats (16-byte pad against bank conflicts)
  constexpr int NI = D / 64;          // PV instructions per key
  constexpr int QW = D * ES / 4;      // 32-bit words of one Q row
  constexpr int CH = D * ES / 16;     // 16-byte vectors per global row
  constexpr int OPE = D + 16 / ES;    // output staging pitch (elements)
  constexpr int KS_BYTES = 64 * KPF * 4;
  constexpr int VS_BYTES = 64 * D * 4;
  constexpr int TAB_BYTES = OTX_EXP_TAB_N * 8;
  constexpr int KV_BYTES = KS_BYTES + VS_BYTES;
  constexpr int OS_BYTES = NWQ * 32 * OPE * ES;
  constexpr int SMEM = (KV_BYTES > OS_BYTES ? KV_BYTES : OS_BYTES) + TAB_BYTES;
  __shared__ __align__(16) unsigned char smem[SMEM];
  float* Ks = reinterpret_cast<float*>(smem);
  float* Vs = reinterpret_cast<float*>(smem + KS_BYTES);
  double* tab = reinterpret_cast<double*>(smem + SMEM - TAB_BYTES);

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

  otx_load_exp_table(tab);

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
  const int edge = window > 0 ? qt - window / OTX_BLK : -1;  // key block at the window's lower edge
  const int p_begin = otx_kblock_lo(qt0, window) >> 1, p_end = qtl >> 1;
  for (int p = p_begin; p <= p_end; ++p) {
    __syncthreads();
    // ---- stage keys [64p, 64p+64) of K and V into LDS as binary32 ----
    for (int idx = threadIdx.x; idx < 64 * CH; idx += 64 * NWQ) {
      const int row = idx / CH, ch = idx % CH;
      const int key = 64 * p + row;
      if (key < S) {
        const uint4 kv = *reinterpret_cast<const uint4*>(kg + (size_t)key * D + ch * VEC);
        const uint4 vv = *reinterpret_cast<const uint4*>(vg + (size_t)key * D + ch * VEC);
#pragma unroll
        for (int e0 = 0; e0 < VEC; e0 += 4) {
          *reinterpret_cast<float4*>(Ks + row * KPF + ch * VEC + e0) =
              make_float4(Elem<T>::get(kv, e0), Elem<T>::get(kv, e0 + 1), Elem<T>::get(kv, e0 + 2),
                          Elem<T>::get(kv, e0 + 3));
          *reinterpret_cast<float4*>(Vs + row * D + ch * VEC + e0) =
              make_float4(Elem<T>::get(vv, e0), Elem<T>::get(vv, e0 + 1), Elem<T>::get(vv, e0 + 2),
                          Elem<T>::get(vv, e0 + 3));
        }
      }
    }
    __syncthreads();
    const int ka = 2 * p, kb = 2 * p + 1;
    const bool doA = wactive && ka >= lo && ka <= hi;
    const bool doB = wactive && kb >= lo && kb <= hi;
    if (!(doA || doB)) continue;

    // ---- S^T = K Q^T over d (serial fma chain) ----
    // The empty asm marks the packed Q words as redefined here, which keeps the
    // compiler from hoisting all D unpacked Q values out of the loop (D live
    // registers); each value is unpacked right before its MFMA instead.
#pragma unroll
    for (int x = 0; x < QW; x++) asm volatile("" : "+v"(qw[x]));
    f32x32 sacc = f32x32{};
    const float* krow = Ks + (hh * 32 + c) * KPF;
#pragma unroll
    for (int d0 = 0; d0 < D; d0 += 4) {
      const float4 kv = *reinterpret_cast<const float4*>(krow + d0);
      sacc = otx_mfma(kv.x, qelem(d0), sacc);
      sacc = otx_mfma(kv.y, qelem(d0 + 1), sacc);
      sacc = otx_mfma(kv.z, qelem(d0 + 2), sacc);
      sacc = otx_mfma(kv.w, qelem(d0 + 3), sacc);
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
    const int kblk = 2 * p + hh;
    const int kbase = kblk * OTX_BLK;
    const bool need_mask = kblk == qt || kblk == edge;
    float mb = -__builtin_inff();
    if (__any(need_mask)) {
#pragma unroll
      for (int j = 0; j < 32; j++) {
        const bool msk = otx_masked(qi, kbase + j, window);
        s[j] = msk ? -__builtin_inff() : s[j] * sigma;
        mb = (s[j] > mb) ? s[j] : mb;
      }
    } else {
#pragma unroll
      for (int j = 0; j < 32; j++) {
        s[j] = s[j] * sigma;
        mb = (s[j] > mb) ? s[j] : mb;
      }
    }
    float mbA, mbB;
    otx_bcast_halves(mb, &mbA, &mbB);
    const float ma = doA ? ((mbA > m) ? mbA : m) : m;
    const float mbn = doB ? ((mbB > ma) ? mbB : ma) : ma;
    // (arguments of unused exps are kept finite or -inf so they never reach the slow path)
    float al[2] = {(ma == m) ? 0.0f : m - ma, (mbn == ma) ? 0.0f : ma - mbn};
    otx_exp_n<2>(al, tab);
    const float alpha_a = (ma == m) ? 1.0f : al[0];
    const float alpha_b = (mbn == ma) ? 1.0f : al[1];
    const float mref = hh ? mbn : ma;
    const bool hact = hh ? doB : doA;
    // exp arguments: masked keys carry -inf (probability +0)
#pragma unroll
    for (int j = 0; j < 32; j++) s[j] = (s[j] == -__builtin_inff() || !hact) ? -__builtin_inff() : s[j] - mref;
    otx_exp_n<32>(s, tab);
    float (&pr)[32] = s;  // probabilities
    // running sum: l = RN(l*alpha), then + p_j ascending (first block in lanes 0..31, second in 32..63)
    if (doA) {
      float t = l * alpha_a;
#pragma unroll
      for (int j = 0; j < 32; j++) t = t + pr[j];
      float tlo, thi;
      otx_bcast_halves(t, &tlo, &thi);
      l = tlo;
    }
    if (doB) {
      float t = l * alpha_b;
#pragma unroll
      for (int j = 0; j < 32; j++) t = t + pr[j];
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
      for (int j = 0; j < 32; j++) {
        float plo, phi;
        otx_bcast_halves(pr[j], &plo, &phi);
        pr[j] = phi;
#pragma unroll
        for (int n = 0; n < NI; n++) acc[n] = otx_mfma(Vs[j * D + 64 * n + L], plo, acc[n]);
      }
    } else {
#pragma unroll
      for (int j = 0; j < 32; j++) {
        float plo, phi;
        otx_bcast_halves(pr[j], &plo, &phi);
        pr[j] = phi;
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
      for (int j = 0; j < 32; j++)
#pragma unroll
        for (int n = 0; n < NI; n++) acc[n] = otx_mfma(Vs[(32 + j) * D + 64 * n + L], pr[j], acc[n]);
    }
    m = mbn;
  }

  // ---- epilogue: O = RN(acc / l) in the storage type, LSE = RN(m + log l) ----
  __syncthreads();
  T* Os = reinterpret_cast<T*>(smem) + wave * 32 * OPE;
  if (wactive) {
#pragma unroll
    for (int n = 0; n < NI; n++)
#pragma unroll
      for (int r = 0; r < 32; r++) {
        const int d = 64 * n + 32 * (r >> 4) + otx_row(r, hh);
        Os[c * OPE + d] = Elem<T>::put(otx_div_rn(acc[n][r], l));
      }
  }
  __syncthreads();
  if (wactive) {
    for (int idx = L; idx < 32 * CH; idx += 64) {
      const int row = idx / CH, ch = idx % CH;
      *reinterpret_cast<uint4*>(o + ((size_t)bh * S + qt * OTX_BLK + row) * D + ch * VEC) =
          *reinterpret_cast<const uint4*>(Os + row * OPE + ch * VEC);
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
