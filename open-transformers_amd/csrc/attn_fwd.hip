// Deterministic causal / sliding-window flash attention forward for gfx950.
//
// Replaces the forward of repop.nn.flash_attention.causal_flash_attention
// (called at src/pretrain/model/modules/attention_repop.py:53 of the
// reference).  Output bits follow the arithmetic contract restated by the CPU
// oracle: serial ascending fma folds, online softmax per 32-key block with
// fp32 running max/sum, correctly rounded exp/log/division.
//
// Work decomposition.  A workgroup of NWQ waves owns NWQ consecutive 32-query
// blocks of one (batch, head), or, under GQA in the default launch, one query
// block of NWQ query heads that share a KV head (every wave then has the same
// key range).  It walks the key blocks in ascending pairs (64 keys), with K and
// V of the pair in LDS for all its waves.  Each wave owns one query block of one
// head:
//   S^T = K Q^T : 32x32x1 MFMA chain over d, block 0 = first key block of the
//                 pair, block 1 = second; A = K rows, B = the lane's Q row.
//   one v_permlane32_swap per register pair gives every lane all 32 scores of
//   one (query, key block): lanes 0..31 the first block, lanes 32..63 the second.
//   softmax bookkeeping is then lane-local (plus two half-wave broadcasts).
//   O^T += V^T P^T : chain over keys, blocks = two 32-wide d ranges; A = V row
//                 segment (64 consecutive d per key), B = the probability
//                 broadcast to both halves.
// bf16 inputs (attn_fwd_bf16_kernel) keep Q, K and V as bf16 in LDS, copied
// straight from global memory (no staging registers; the next step's K and V
// copies overlap the current step's PV and S chains), and read every chain
// operand with ds_read_u16_d16_hi, which yields the binary32 value of a bf16
// without a conversion instruction.  binary32 inputs (attn_fwd_kernel) stage K
// and V as binary32 and keep Q in registers.
// Masking is only evaluated on the diagonal block and on the block at the
// window's lower edge; other blocks are dense.
// No atomics; every output element is produced by one lane in one fixed order.
//
// int8-PV (attn_fwd_bf16_kernel with I8; replaces repop's
// int8pv_causal_flash_attention, attention_repop.py:52).  V is quantized once
// per (key block, column) by attn_quant_v_kernel into a workspace, already
// transposed to the A-operand order of v_mfma_i32_32x32x32_i8 ([block][d][32
// keys] int8) with one binary32 step per (block, d); the kernel copies those
// instead of V.  The scores and the softmax statistics are those of the
// binary32 path; each lane quantizes the 32 probabilities of its (query, key
// block) with their own maximum, one v_permlane32_swap per packed word moves
// them to the B-operand order, and O^T += dequant(V^T P^T) takes D/32 int8
// instructions per key block instead of D matrix instructions per 32 keys.
#include "otx_common.h"


namespace otx {

typedef int i32x4 __attribute__((ext_vector_type(4)));
typedef int i32x16 __attribute__((ext_vector_type(16)));

// V quantization of the int8-PV contract, one thread per (key block, column d):
//   amax = max_j |v_j[d]| over the block's 32 keys; amax = 0 -> step 0, values 0;
//   any Inf/NaN -> step NaN, values 0; else inv = RN(127/amax), step = RN(amax/127),
//   q_j = rint(RN(v_j[d] * inv)) clamped to [-127, 127], NaN -> 0.  The clamp only
//   acts when 127/amax overflows (amax < 127 / FLT_MAX, about 3.7e-37): inv is then
//   +inf and v * inv is +-inf (or NaN for v = 0); otherwise |v * inv| < 127.5.
// Output qvt[blk][d][j] (int8, keys contiguous) and step[blk][d].
template <int D>
__global__ __launch_bounds__(256) void attn_quant_v_kernel(const uint16_t* __restrict__ v, int8_t* __restrict__ qvt,
                                                           float* __restrict__ step, long nblk) {
  constexpr int BPW = 256 / D;  // key blocks per workgroup
  const long blk = (long)blockIdx.x * BPW + threadIdx.x / D;
  const int d = threadIdx.x % D;
  if (blk >= nblk) return;
  const uint16_t* vb = v + blk * 32 * D + d;
  float x[32];
  float amax = 0.0f;
  bool bad = false;
#pragma unroll
  for (int j = 0; j < 32; j++) {
    x[j] = __uint_as_float((uint32_t)vb[j * D] << 16);
    const float a = __builtin_fabsf(x[j]);
    bad |= !(a <= 3.402823466e38f);
    amax = a > amax ? a : amax;
  }
  float inv = 0.0f, st = 0.0f;
  if (bad) {
    st = __builtin_nanf("");
  } else if (amax > 0.0f) {
    inv = otx_div_rn(127.0f, amax);
    st = otx_div_rn(amax, 127.0f);
  }
  uint32_t w[8];
#pragma unroll
  for (int g = 0; g < 8; g++) {
    uint32_t word = 0;
#pragma unroll
    for (int e = 0; e < 4; e++) {
      float r = __builtin_rintf(x[4 * g + e] * inv);
      r = r != r ? 0.0f : (r > 127.0f ? 127.0f : (r < -127.0f ? -127.0f : r));
      const int qv = inv == 0.0f ? 0 : (int)r;
      word |= ((uint32_t)qv & 0xffu) << (8 * e);
    }
    w[g] = word;
  }
  uint4* dst = reinterpret_cast<uint4*>(qvt + (blk * D + d) * 32);
  dst[0] = make_uint4(w[0], w[1], w[2], w[3]);
  dst[1] = make_uint4(w[4], w[5], w[6], w[7]);
  step[blk * D + d] = st;
}

// Generic forward (binary32 inputs; bf16 inputs run attn_fwd_bf16_kernel).
// K and V are staged in LDS as binary32; Q stays in registers (D raw words),
// which leaves room for one wave per SIMD.
template <typename T, int D, int NWQ>
__global__ __launch_bounds__(64 * NWQ) __attribute__((amdgpu_waves_per_eu(1)))
void attn_fwd_kernel(const T* __restrict__ q, const T* __restrict__ k, const T* __restrict__ v, T* __restrict__ o,
                     float* __restrict__ lse, int B, int H, int Hkv, int S, int window, float sigma, int order) {
  constexpr int ES = sizeof(T);
  constexpr int VEC = Elem<T>::VEC;   // elements per 16-byte global vector
  constexpr int KPF = D + 4;          // K tile pitch in floats (16-byte pad against bank conflicts)
  constexpr int NI = D / 64;          // PV instructions per key
  constexpr int QW = D * ES / 4;      // 32-bit words of one Q row
  constexpr int CH = D * ES / 16;     // 16-byte vectors per global row
  constexpr int OPE = D + 16 / ES;    // output staging pitch (elements)
  constexpr int KS_BYTES = 64 * KPF * 4;
  constexpr int VS_BYTES = 64 * D * 4;
  constexpr int TAB_BYTES = OTX_EXP_LE0_TAB_N * 8;
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
#pragma unroll
        for (int e0 = 0; e0 < VEC; e0 += 4)
          *reinterpret_cast<float4*>(Ks + row * KPF + ch * VEC + e0) =
              make_float4(Elem<T>::get(kv, e0), Elem<T>::get(kv, e0 + 1), Elem<T>::get(kv, e0 + 2),
                          Elem<T>::get(kv, e0 + 3));
        const uint4 vv = *reinterpret_cast<const uint4*>(vg + (size_t)key * D + ch * VEC);
#pragma unroll
        for (int e0 = 0; e0 < VEC; e0 += 4)
          *reinterpret_cast<float4*>(Vs + row * D + ch * VEC + e0) =
              make_float4(Elem<T>::get(vv, e0), Elem<T>::get(vv, e0 + 1), Elem<T>::get(vv, e0 + 2),
                          Elem<T>::get(vv, e0 + 3));
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
        mb = otx_max_update(s[j], mb);
      }
    } else {
#pragma unroll
      for (int j = 0; j < 32; j++) {
        s[j] = s[j] * sigma;
        mb = otx_max_update(s[j], mb);
      }
    }
    float mbA, mbB;
    otx_bcast_halves(mb, &mbA, &mbB);
    const float ma = doA ? otx_max_update(mbA, m) : m;
    const float mbn = doB ? otx_max_update(mbB, ma) : ma;
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

// bf16 forward with Q, K and V kept as bf16 in LDS and every chain operand read
// with ds_read_u16_d16_hi (binary32 value of a bf16, no conversion
// instruction), under hand-kept lgkmcnt accounting (groups of 4 reads, two
// groups ahead: at most 12 outstanding).  K and V of a 64-key step are copied
// straight from global memory into single LDS buffers (global_load_lds_dwordx4):
// the next step's K once every wave has finished its S chain, the next V once
// every wave has finished its PV chain, so each copy runs under the other
// half of the step.  Q rows of each wave are copied once.  K and Q rows are
// padded to 2D + 16 bytes (the rows one chain step reads spread over the
// banks); V rows are unpadded (a PV step reads 64 consecutive elements of one
// row).  Arithmetic order is the same as in attn_fwd_kernel.
// The LSE's log in a function of its own: inlined into the forward, its series
// constants were materialised once per kernel and held in registers across the
// key loop.  One call per lane and task.
__device__ __attribute__((noinline)) float otx_logf_call(float x) { return otx_logf(x); }

template <int D, int NWQ, bool I8>
__global__ __launch_bounds__(64 * NWQ) __attribute__((amdgpu_waves_per_eu(2)))
void attn_fwd_bf16_kernel(const uint16_t* __restrict__ q, const uint16_t* __restrict__ k,
                          const uint16_t* __restrict__ v, uint16_t* __restrict__ o, float* __restrict__ lse, int B,
                          int H, int Hkv, int S, int window, float sigma, int order,
                          const int8_t* __restrict__ qvt, const float* __restrict__ vstep,
                          float* __restrict__ scache, int hg) {
  constexpr int NI = D / 64;        // PV instructions per key
  constexpr int CH = D / 8;         // 16-byte vectors per global row
  constexpr int OPE = D + 8;        // output staging pitch (elements)
  constexpr int KPB = 2 * D + 16;   // K and Q row pitch in LDS (bytes)
  constexpr int UK = KPB / 16;      // 16-byte units per padded row (CH data + 1 pad)
  constexpr int VPB = 2 * D;        // V row pitch in LDS (bytes)
  constexpr int KT_BYTES = 64 * KPB;
  constexpr int QV_BYTES = 2 * D * 32;  // int8 V^T of two key blocks ([blk][d][32 keys])
  constexpr int VT_BYTES = I8 ? QV_BYTES + 2 * D * 4 : 64 * VPB;  // + binary32 steps [blk][d]
  constexpr int NQI = (32 * UK + 63) / 64;  // Q copy instructions per wave
  constexpr int QW_BYTES = NQI * 64 * 16;   // one wave's Q region (32 padded rows, rounded up)
  constexpr int OS_BYTES = NWQ * 32 * OPE * 2;
  constexpr int IN_BYTES = KT_BYTES + VT_BYTES + NWQ * QW_BYTES;
  constexpr int BUF = IN_BYTES > OS_BYTES ? IN_BYTES : OS_BYTES;
  constexpr int SMEM = BUF + OTX_EXP_LE0_TAB_N * 8;
  constexpr int NKI = (UK + NWQ - 1) / NWQ;  // K copy instructions per wave (upper bound)
  constexpr int KPG = 4 / NI;                // keys per PV read group of 4
  // the exp table at LDS address 0 (a table read then needs no base add), the buffers after it
  __shared__ __align__(16) unsigned char lds[SMEM];
  double* tab = reinterpret_cast<double*>(lds);
  unsigned char* smem = lds + OTX_EXP_LE0_TAB_N * 8;
  unsigned char* Kt = smem;
  unsigned char* Vt = smem + KT_BYTES;

  const int nqt = S / OTX_BLK;
  const int G = H / Hkv;
  // A workgroup's NWQ waves take NWQ consecutive query blocks of one head, or,
  // with hg (GQA, NWQ dividing the group), NWQ query heads of one KV head on one
  // query block: then every wave has the same key range, so no wave idles at
  // the causal diagonal or at a sliding window's edges.  K and V rows are shared
  // by the workgroup either way.  A chunk is the workgroup's unit along the
  // query axis (NWQ query blocks, or one), a head unit its unit along the head
  // axis (a head, or NWQ heads of a KV group).
  const int nchunk = hg ? nqt : (nqt + NWQ - 1) / NWQ;
  const int BU = hg ? B * Hkv * (G / NWQ) : B * H;
  const int bid = blockIdx.x;
  // OTX_ORDER_PAIRED: workgroup (j, u) runs chunk nchunk-1-j and then chunk j of head unit u, so that under the
  // causal mask every workgroup carries about the same work and the grid drains together (two workgroups
  // share a CU, so the hardware's dispatch order cannot balance unequal ones).  OTX_ORDER_LONGEST: one chunk
  // per workgroup, longest first.  OTX_ORDER_HEAD: one chunk per workgroup, head-major.
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
  const unsigned char* kg = reinterpret_cast<const unsigned char*>(k + ((size_t)b * Hkv + g) * S * D);
  const unsigned char* vg = reinterpret_cast<const unsigned char*>(v + ((size_t)b * Hkv + g) * S * D);
  unsigned char* Qw = smem + KT_BYTES + VT_BYTES + wave * QW_BYTES;
  const int qi = qt * OTX_BLK + c;

  otx_load_exp_table(tab);

  // Copy unit u of a padded row block is row u / UK, slot u % UK; the pad slot
  // (and units past the last row) copy an in-bounds chunk that is never read.
  auto padded_off = [&](int u, int rows) {
    const int row = u / UK, su = u % UK;
    return row < rows ? row * (2 * D) + 16 * (su < CH ? su : 0) : 0;
  };
  // Source offsets of this wave's K copy units (i = wave + NWQ x) for a full
  // 64-row step, formed once; an offset at or past rows * 2D is a row past S.
  const int wave_u = __builtin_amdgcn_readfirstlane(wave);
  int koff[NKI];
#pragma unroll
  for (int x = 0; x < NKI; x++) koff[x] = padded_off(64 * (wave_u + NWQ * x) + L, 64);
  auto issue_k = [&](int p) {
    const unsigned char* kt = kg + (size_t)64 * p * (2 * D);
    const int rows = S - 64 * p;  // rows of this step inside the sequence (>= 32)
    const int lim = (rows < 64 ? rows : 64) * (2 * D);
#pragma unroll
    for (int x = 0; x < NKI; x++) {
      const int i = wave_u + NWQ * x;
      if (i < UK) otx_dma16(kt + (koff[x] < lim ? koff[x] : 0), Kt + 64 * i * 16);
    }
  };
  auto issue_v = [&](int p) {
    if constexpr (I8) {
      // quantized V^T and steps of key blocks 2p, 2p+1 (the second is absent at the end of an odd S / 32)
      const size_t gblk = ((size_t)b * Hkv + g) * nqt + 2 * p;
      const int nb_here = 2 * p + 1 < nqt ? 2 : 1;
      const unsigned char* qsrc = reinterpret_cast<const unsigned char*>(qvt + gblk * D * 32);
      for (int i = wave_u; i < QV_BYTES / 1024; i += NWQ) {
        const int u = 64 * i + L;
        otx_dma16(qsrc + (u < nb_here * D * 2 ? 16 * u : 16 * (u - D * 2)), Vt + 64 * i * 16);
      }
      const unsigned char* ssrc = reinterpret_cast<const unsigned char*>(vstep + gblk * D);
      constexpr int SU = 2 * D * 4 / 16;  // 16-byte units of the steps
      if (wave_u == NWQ - 1 && L < SU) {
        const int u = L;
        otx_dma16(ssrc + (u < nb_here * D / 4 ? 16 * u : 16 * (u - D / 4)), Vt + QV_BYTES);
      }
    } else {
      const unsigned char* vt = vg + (size_t)64 * p * (2 * D);
      const int rows = S - 64 * p;
      for (int i = wave_u; i < CH; i += NWQ) {
        const int u = 64 * i + L;
        otx_dma16(vt + (u < rows * CH ? 16 * u : 0), Vt + 64 * i * 16);
      }
    }
  };
  if (wactive) {
    const unsigned char* qg = reinterpret_cast<const unsigned char*>(q + ((size_t)bh * S + qt * OTX_BLK) * D);
#pragma unroll
    for (int i = 0; i < NQI; i++) otx_dma16(qg + padded_off(64 * i + L, 32), Qw + 64 * i * 16);
  }

  // operand registers of the d16 reads: three banks of 4, low halves zero
  float opr[3][4];
#pragma unroll
  for (int x = 0; x < 4; x++) { opr[0][x] = 0.0f; opr[1][x] = 0.0f; opr[2][x] = 0.0f; }

  float m = -__builtin_inff(), l = 0.0f;
  f32x32 acc[NI];
#pragma unroll
  for (int n = 0; n < NI; n++) acc[n] = f32x32{};

  const int lo = otx_kblock_lo(qt, window), hi = qt;
  const int edge = window > 0 ? qt - window / OTX_BLK : -1;
  const int p_begin = otx_kblock_lo(qt0, window) >> 1, p_end = qtl >> 1;
  if (p_begin <= p_end) {
    issue_k(p_begin);
    issue_v(p_begin);
  }
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __syncthreads();
  const uint32_t krow = otx_lds_addr(Kt) + (hh * 32 + c) * KPB;
  // The S chain's B operand, element d of query c's row, is the same in both half-waves: one read
  // serves a pair of d (half hh reads element 2G + hh), and each product of the pair takes it from
  // one half by the BLGP broadcast (measured: forward -0.1 to -1.0 %, bf16 and int8-PV).
  const uint32_t qrow = otx_lds_addr(Qw) + c * KPB + 2 * hh;
  const uint32_t vrow = otx_lds_addr(Vt) + 2 * L;
  for (int p = p_begin; p <= p_end; ++p) {
    const int ka = 2 * p, kb = 2 * p + 1;
    const bool doA = wactive && ka >= lo && ka <= hi;
    const bool doB = wactive && kb >= lo && kb <= hi;
    const bool act = doA || doB;

    // ---- S^T = K Q^T over d (serial fma chain); group G = d 2G, 2G+1 ----
    f32x32 sacc = f32x32{};
    if (act) {
      constexpr int NG = D / 2;
      constexpr int RPG = 3;  // LDS reads per group: K at d = 2G and 2G + 1, the Q pair
      auto rd = [&](auto gc) {
        constexpr int G = decltype(gc)::value, BK = G % 3;
        otx_lds_bf16<4 * G>(opr[BK][0], krow);
        otx_lds_bf16<4 * G>(opr[BK][1], qrow);
        otx_lds_bf16<4 * G + 2>(opr[BK][2], krow);
      };
      rd(std::integral_constant<int, 0>{});
      rd(std::integral_constant<int, 1>{});
      OtxUnroll<0, NG>::run([&](auto gc) {
        constexpr int G = decltype(gc)::value, BK = G % 3;
        if constexpr (G + 2 < NG) {
          rd(std::integral_constant<int, G + 2>{});
          otx_lds_wait<2 * RPG>(opr[BK]);
        } else if constexpr (G + 1 < NG) {
          otx_lds_wait<RPG>(opr[BK]);
        } else {
          otx_lds_wait<0>(opr[BK]);
        }
        sacc = otx_mfma_bhalf<0>(opr[BK][0], opr[BK][1], sacc);
        sacc = otx_mfma_bhalf<1>(opr[BK][2], opr[BK][1], sacc);
      });
    }
    // The softmax (vector work) runs at wave priority 1 and the matrix chains at
    // 0: of the two waves on a SIMD, the one in its softmax issues first, and the
    // other wave's chain fills the gaps (measured: forward -1 to -2 %).  Wave
    // priority orders issue only; results are unchanged.
    __builtin_amdgcn_s_setprio(1);
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // this lane's copy of V for step p has landed
    __syncthreads();  // K of step p is no longer read; V of step p is visible
    if (p + 1 <= p_end) issue_k(p + 1);

    if (act) {
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
#pragma unroll
      for (int j = 0; j < 32; j++) s[j] = s[j] * sigma;
      if (__any(need_mask)) {
#pragma unroll
        for (int j = 0; j < 32; j++) s[j] = otx_masked(qi, kbase + j, window) ? -__builtin_inff() : s[j];
      }
      // block maximum as a tree of max instructions: exact and independent of the order for scores that
      // are finite or -inf, NaN if any score is NaN (finite inputs never make one); the only
      // order-dependent detail, the sign of a zero maximum, changes no result (it enters only s - m,
      // compared to m, and m + log l with log l >= 0)
      const float mb = otx_max32(s);
      // ---- score cache: the scaled scores s (-inf where masked) of this (query block, key block) as
      // the transposed tile [key j][query c], for a backward that reads them instead of recomputing ----
      if (scache != nullptr && (hh ? doB : doA)) {
        float* tile = scache + (((long)bh * otx_tile_offset(nqt, window) + otx_tile_offset(qt, window) +
                                 (kblk - otx_kblock_lo(qt, window))) << 10);
#pragma unroll
        for (int j = 0; j < 32; j++) tile[j * 32 + c] = s[j];
      }
      float mbA, mbB;
      otx_bcast_halves(mb, &mbA, &mbB);
      const float ma = doA ? otx_max_update(mbA, m) : m;
      const float mbn = doB ? otx_max_update(mbB, ma) : ma;
      float al[2] = {(ma == m) ? 0.0f : m - ma, (mbn == ma) ? 0.0f : ma - mbn};
      if (__any(ma != m || mbn != ma)) otx_exp_n<2>(al, tab);  // otherwise every alpha below is 1
      const float alpha_a = (ma == m) ? 1.0f : al[0];
      const float alpha_b = (mbn == ma) ? 1.0f : al[1];
      const float mref = hh ? mbn : ma;
      const bool hact = hh ? doB : doA;
      // exp arguments: s - mref, -inf for masked keys; a half-wave without a
      // live block (or whose block so far has no unmasked key) gets -inf from
      // subtracting +inf, which it never reads back.
      const float moff = (hact && mref != -__builtin_inff()) ? mref : __builtin_inff();
#pragma unroll
      for (int j = 0; j < 32; j++) s[j] = s[j] - moff;
      otx_exp_n<32>(s, tab);
      float (&pr)[32] = s;
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
      if constexpr (I8) {
        // ---- int8 P: per (query, key block) step pmax/127, values rint(p * 127/pmax) ----
        // pmax by a tree of max instructions: the probabilities are +0 or positive (never NaN: the table
        // exp gives +0 for a NaN argument), so the maximum is exact and independent of the order.
        const float pmax = otx_max32(pr);
        float inv = 0.0f, sp = 0.0f;
        if (pmax > 0.0f) {
          inv = otx_div_rn(127.0f, pmax);
          sp = otx_div_by_recip(pmax, OTX_RECIP64_127);  // = RN(pmax / 127), one multiply
        }
        // rint(p * 127/pmax) into byte e of the word by one v_cvt_pk_u8_f32 per value: it rounds to
        // nearest even exactly as rint on [+0, 128) (every bit pattern, tests/test_gpu_selftest.py), and
        // p * inv lies there (p <= pmax, inv = RN(127/pmax); +0 when pmax is 0).
        // When 127/pmax overflows (pmax < 127 / FLT_MAX, about 3.7e-37) inv is +inf and
        // p * inv is +inf (contract: 127) or NaN for p = 0 (contract: 0), which the
        // conversion makes 255 and 0; every other byte is at most 127, so clearing
        // bit 7 of each byte gives the contract in all cases.
        uint32_t qp[8];
#pragma unroll
        for (int w = 0; w < 8; w++) {
          uint32_t word = 0;
#pragma unroll
          for (int e = 0; e < 4; e++) word = __builtin_amdgcn_cvt_pk_u8_f32(pr[4 * w + e] * inv, e, word);
          qp[w] = word & 0x7f7f7f7fu;
        }
        // B operand: lane (h, c) needs keys 16h..16h+15 of query c; block A lives in
        // lanes 0..31, block B in lanes 32..63.
#pragma unroll
        for (int w = 0; w < 4; w++) {
          float x = __uint_as_float(qp[w]), y = __uint_as_float(qp[4 + w]);
          otx_swap_halves(x, y);
          qp[w] = __float_as_uint(x);
          qp[4 + w] = __float_as_uint(y);
        }
        float spA, spB;
        otx_bcast_halves(sp, &spA, &spB);
        // The int8 V^T tile and the steps are read by hand-kept LDS reads (five per
        // 32-row group: the A operand and four steps vectors, one group ahead), not by
        // compiler-visible loads: the compiler would put a wait for every outstanding
        // global operation (the next step's K copy, the score-cache stores) before them.
        __builtin_amdgcn_s_setprio(0);
        const uint32_t qv_l = otx_lds_addr(Vt) + c * 32 + 16 * hh;
        const uint32_t vs_l = otx_lds_addr(Vt) + QV_BYTES + 16 * hh;
        OtxUnroll<0, 2>::run([&](auto half_c) {
          constexpr int HALF = decltype(half_c)::value;
          const bool hdo = HALF ? doB : doA;
          if (!hdo) return;
          const float alpha = HALF ? alpha_b : alpha_a;
          const float spx = HALF ? spB : spA;
          if (__any(alpha != 1.0f)) {
#pragma unroll
            for (int n = 0; n < NI; n++)
#pragma unroll
              for (int r = 0; r < 32; r++) acc[n][r] = acc[n][r] * alpha;
          }
          const i32x4 bop = {(int)qp[4 * HALF], (int)qp[4 * HALF + 1], (int)qp[4 * HALF + 2], (int)qp[4 * HALF + 3]};
          constexpr int NT = D / 32;
          otx_f4 aop[2], stv[2][4];
          auto rd = [&](auto tc) {
            constexpr int T = decltype(tc)::value, BK = T % 2;
            otx_lds_f4<(HALF * D + 32 * T) * 32>(aop[BK], qv_l);
            OtxUnroll<0, 4>::run([&](auto kc) {
              constexpr int K4 = decltype(kc)::value;
              otx_lds_f4<4 * (HALF * D + 32 * T + 8 * K4)>(stv[BK][K4], vs_l);
            });
          };
          rd(std::integral_constant<int, 0>{});
          OtxUnroll<0, NT>::run([&](auto tc) {
            constexpr int T = decltype(tc)::value, BK = T % 2;
            if constexpr (T + 1 < NT) {
              rd(std::integral_constant<int, T + 1>{});
              otx_lds_wait<5>(aop[BK], stv[BK]);
            } else {
              otx_lds_wait<0>(aop[BK], stv[BK]);
            }
            const i32x16 pv = __builtin_amdgcn_mfma_i32_32x32x32_i8(__builtin_bit_cast(i32x4, aop[BK]), bop,
                                                                   i32x16{}, 0, 0, 0);
#pragma unroll
            for (int k4 = 0; k4 < 4; k4++)
#pragma unroll
              for (int e = 0; e < 4; e++) {
                const int rr = 4 * k4 + e, r2 = 16 * (T & 1) + rr;
                acc[T >> 1][r2] = __builtin_fmaf((float)pv[rr] * stv[BK][k4][e], spx, acc[T >> 1][r2]);
              }
          });
        });
        m = mbn;
      } else {
      __builtin_amdgcn_s_setprio(0);
      // ---- O^T = O^T * alpha, then += V^T P^T (serial over keys); KPG keys per group ----
      auto pv_half = [&](auto half_c) {
        constexpr int HB = decltype(half_c)::value * 32 * VPB;  // byte offset of the half's first key
        constexpr int NG = 32 / KPG;
        auto rd = [&](auto gc) {
          constexpr int G = decltype(gc)::value, BK = G % 3;
          OtxUnroll<0, 4>::run([&](auto e) {
            constexpr int E = decltype(e)::value;
            otx_lds_bf16<HB + (KPG * G + E / NI) * VPB + 128 * (E % NI)>(opr[BK][E], vrow);
          });
        };
        rd(std::integral_constant<int, 0>{});
        rd(std::integral_constant<int, 1>{});
        OtxUnroll<0, NG>::run([&](auto gc) {
          constexpr int G = decltype(gc)::value, BK = G % 3;
          if constexpr (G + 2 < NG) {
            rd(std::integral_constant<int, G + 2>{});
            otx_lds_wait<8>(opr[BK]);
          } else if constexpr (G + 1 < NG) {
            otx_lds_wait<4>(opr[BK]);
          } else {
            otx_lds_wait<0>(opr[BK]);
          }
          OtxUnroll<0, KPG>::run([&](auto jj) {
            constexpr int J = KPG * G + decltype(jj)::value;
            constexpr int HALF = decltype(half_c)::value;  // block A's P in lanes 0..31, block B's in 32..63
#pragma unroll
            for (int n = 0; n < NI; n++)
              acc[n] = otx_mfma_bhalf<HALF>(opr[BK][decltype(jj)::value * NI + n], pr[J], acc[n]);
          });
        });
      };
      if (doA) {
        if (__any(alpha_a != 1.0f)) {
#pragma unroll
          for (int n = 0; n < NI; n++)
#pragma unroll
            for (int r = 0; r < 32; r++) acc[n][r] = acc[n][r] * alpha_a;
        }
        pv_half(std::integral_constant<int, 0>{});
      }
      if (doB) {
        if (__any(alpha_b != 1.0f)) {
#pragma unroll
          for (int n = 0; n < NI; n++)
#pragma unroll
            for (int r = 0; r < 32; r++) acc[n][r] = acc[n][r] * alpha_b;
        }
        pv_half(std::integral_constant<int, 1>{});
      }
      m = mbn;
      }
    }
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // this lane's copy of K for step p + 1 has landed
    __syncthreads();  // V of step p is no longer read; K of step p + 1 is visible
    if (p + 1 <= p_end) issue_v(p + 1);
  }

  // ---- epilogue: O = RN(acc / l) as bf16, LSE = RN(m + log l) ----
  __syncthreads();
  uint16_t* Os = reinterpret_cast<uint16_t*>(smem) + wave * 32 * OPE;
  if (wactive) {
    // RN(acc / l) through one binary64 reciprocal per lane, with the bytes of
    // otx_div_by_recip_checked: quotients below the normal range take the
    // division, behind a wave-uniform branch (a ballot) so that the division is
    // only evaluated when some lane needs it.
    const double rl = otx_recip64(l);
    float oq[NI][32];
    bool low = false;
#pragma unroll
    for (int n = 0; n < NI; n++)
#pragma unroll
      for (int r = 0; r < 32; r++) {
        oq[n][r] = otx_div_by_recip(acc[n][r], rl);
        low = low || !(__builtin_fabsf(oq[n][r]) >= 0x1p-126f);
      }
    if (__builtin_expect(__ballot(low) != 0, 0)) {
#pragma unroll
      for (int n = 0; n < NI; n++)
#pragma unroll
        for (int r = 0; r < 32; r++) oq[n][r] = otx_div_by_recip_checked(acc[n][r], rl, l);
    }
#pragma unroll
    for (int n = 0; n < NI; n++)
#pragma unroll
      for (int r = 0; r < 32; r++) {
        const int d = 64 * n + 32 * (r >> 4) + otx_row(r, hh);
        Os[c * OPE + d] = otx_f32_to_bf16(oq[n][r]);
      }
  }
  __syncthreads();
  if (wactive) {
    // The output addresses are formed here, from a lane index the compiler cannot see through, so that
    // they are not computed at the start of the task and held (or spilled) across the key loop.
    int Le = L;
    asm volatile("" : "+v"(Le));
    for (int idx = Le; idx < 32 * CH; idx += 64) {
      const int row = idx / CH, ch = idx % CH;
      *reinterpret_cast<uint4*>(o + ((size_t)bh * S + qt * OTX_BLK + row) * D + ch * 8) =
          *reinterpret_cast<const uint4*>(Os + row * OPE + ch * 8);
    }
    if (hh == 0) lse[(size_t)bh * S + qt * OTX_BLK + (Le & 31)] = m + otx_logf_call(l);
  }
  __syncthreads();  // the next task's copies overwrite the output staging
  }
}

template <typename T, int D, int NWQ, bool I8 = false>
static hipError_t launch_fwd_t(const void* q, const void* k, const void* v, void* o, float* lse, int B, int H,
                               int Hkv, int S, int window, float sigma, int order, hipStream_t stream,
                               const int8_t* qvt = nullptr, const float* vstep = nullptr, float* scache = nullptr) {
  const int nqt = S / OTX_BLK;
  const int nchunk = (nqt + NWQ - 1) / NWQ;
  dim3 grid((unsigned)(nchunk * B * H)), block(64 * NWQ);
  if constexpr (sizeof(T) == 2) {
    // Head-grouped workgroups (see the kernel) for GQA in the default launch
    // order; the other launch variants keep one head per workgroup, so the
    // parity tests compare both mappings byte for byte.
    const int G = H / Hkv;
    const int hg = (NWQ > 1 && G % NWQ == 0 && order == 0) ? 1 : 0;
    const long nu = hg ? nqt : nchunk, bu = hg ? (long)B * Hkv * (G / NWQ) : (long)B * H;
    const int korder = otx_chunk_order(order, nu * bu, 2);
    grid.x = (unsigned)((korder == OTX_ORDER_PAIRED ? (nu + 1) / 2 : nu) * bu);
    hipLaunchKernelGGL((attn_fwd_bf16_kernel<D, NWQ, I8>), grid, block, 0, stream, (const uint16_t*)q,
                       (const uint16_t*)k, (const uint16_t*)v, (uint16_t*)o, lse, B, H, Hkv, S, window, sigma, korder,
                       qvt, vstep, scache, hg);
  } else {
    static_assert(!I8, "int8-PV is defined for bf16 inputs");
    if (scache != nullptr) return hipErrorInvalidValue;  // the score cache is a bf16-path feature
    hipLaunchKernelGGL((attn_fwd_kernel<T, D, NWQ>), grid, block, 0, stream, (const T*)q, (const T*)k,
                       (const T*)v, (T*)o, lse, B, H, Hkv, S, window, sigma, order);
  }
  return hipGetLastError();
}

template <int D>
static hipError_t launch_fwd_i8_d(int nwq, const void* q, const void* k, const void* v, void* o, float* lse, int B,
                                  int H, int Hkv, int S, int window, float sigma, int order, int8_t* qvt,
                                  float* vstep, float* scache, hipStream_t st) {
  const long nblk = (long)B * Hkv * (S / OTX_BLK);
  constexpr int BPW = 256 / D;
  hipLaunchKernelGGL((attn_quant_v_kernel<D>), dim3((unsigned)((nblk + BPW - 1) / BPW)), dim3(256), 0, st,
                     (const uint16_t*)v, qvt, vstep, nblk);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  switch (nwq) {
    case 4: return launch_fwd_t<uint16_t, D, 4, true>(q, k, v, o, lse, B, H, Hkv, S, window, sigma, order, st, qvt, vstep, scache);
    case 2: return launch_fwd_t<uint16_t, D, 2, true>(q, k, v, o, lse, B, H, Hkv, S, window, sigma, order, st, qvt, vstep, scache);
    default: return launch_fwd_t<uint16_t, D, 1, true>(q, k, v, o, lse, B, H, Hkv, S, window, sigma, order, st, qvt, vstep, scache);
  }
}

// int8-PV forward (bf16 inputs): quantizes V into qvt / vstep, then runs the forward.
hipError_t launch_fwd_int8pv(int D, int nwq, const void* q, const void* k, const void* v, void* o, float* lse, int B,
                             int H, int Hkv, int S, int window, float sigma, int order, int8_t* qvt, float* vstep,
                             float* scache, hipStream_t st) {
  if (D == 128)
    return launch_fwd_i8_d<128>(nwq, q, k, v, o, lse, B, H, Hkv, S, window, sigma, order, qvt, vstep, scache, st);
  return launch_fwd_i8_d<64>(nwq, q, k, v, o, lse, B, H, Hkv, S, window, sigma, order, qvt, vstep, scache, st);
}

template <typename T, int D>
static hipError_t launch_fwd_d(int nwq, const void* q, const void* k, const void* v, void* o, float* lse, int B,
                               int H, int Hkv, int S, int window, float sigma, int order, float* scache,
                               hipStream_t st) {
  switch (nwq) {
    case 4: return launch_fwd_t<T, D, 4>(q, k, v, o, lse, B, H, Hkv, S, window, sigma, order, st, nullptr, nullptr, scache);
    case 2: return launch_fwd_t<T, D, 2>(q, k, v, o, lse, B, H, Hkv, S, window, sigma, order, st, nullptr, nullptr, scache);
    default: return launch_fwd_t<T, D, 1>(q, k, v, o, lse, B, H, Hkv, S, window, sigma, order, st, nullptr, nullptr, scache);
  }
}

// scache (bf16 only, may be null): also write the score cache.
hipError_t launch_fwd(int dtype, int D, int nwq, const void* q, const void* k, const void* v, void* o, float* lse,
                      int B, int H, int Hkv, int S, int window, float sigma, int order, float* scache,
                      hipStream_t st) {
  if (dtype == 1) {
    if (D == 128)
      return launch_fwd_d<uint16_t, 128>(nwq, q, k, v, o, lse, B, H, Hkv, S, window, sigma, order, scache, st);
    return launch_fwd_d<uint16_t, 64>(nwq, q, k, v, o, lse, B, H, Hkv, S, window, sigma, order, scache, st);
  }
  if (D == 128) return launch_fwd_d<float, 128>(nwq, q, k, v, o, lse, B, H, Hkv, S, window, sigma, order, scache, st);
  return launch_fwd_d<float, 64>(nwq, q, k, v, o, lse, B, H, Hkv, S, window, sigma, order, scache, st);
}

}  // namespace otx
