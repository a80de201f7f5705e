// C-ABI of the MI355X attention library: argument validation, workspace
// sizing, kernel dispatch and two hardware self-checks.  Declared in
// include/otx_attn.h.  No function allocates device memory or synchronises
// the host.  The only mutable global state is the thread-local last-error text
// and, for the allocation-free int8-PV forward, the per-device address of its
// fixed device scratch array.
#include <cmath>
#include <cstdio>
#include <cstdarg>
#include <cstring>
#include <mutex>
#include "otx_common.h"
#include "../../include/otx_attn.h"

namespace otx {
hipError_t launch_fwd(int dtype, int D, int nwq, const void* q, const void* k, const void* v, void* o, float* lse,
                      int B, int H, int Hkv, int S, int window, float sigma, int order, float* scache,
                      hipStream_t st);
hipError_t launch_fwd_int8pv(int D, int nwq, const void* q, const void* k, const void* v, void* o, float* lse, int B,
                             int H, int Hkv, int S, int window, float sigma, int order, int8_t* qvt, float* vstep,
                             float* scache, hipStream_t st);
hipError_t launch_bwd(int dtype, int D, int nw, const void* q, const void* k, const void* v, const void* o,
                      const float* lse, const void* dO, void* dq, void* dk, void* dv, float* dsum, float* ds, int B,
                      int H, int Hkv, int S, int window, float sigma, int order, int stages, const float* scache,
                      hipStream_t st);
hipError_t launch_gemm(const void* A, long a_i, long a_r, const void* B, long b_j, long b_r, void* C, long ldc, int M,
                       int N, int R, bool out_f32, int variant, hipStream_t st);
hipError_t launch_rmsnorm_fwd(int dtype, const void* x, const void* w, void* y, float* rstd, long rows, int D,
                              float eps, hipStream_t st);
hipError_t launch_rmsnorm_bwd(int dtype, const void* x, const void* w, const float* rstd, const void* dy, void* dx,
                              float* dw, float* part, long rows, int D, hipStream_t st);
int ce_max_vocab(int dtype);
hipError_t launch_ce_fwd(int dtype, const void* logits, const int64_t* labels, long N, int V, int vec, float coeff32,
                         int has_coeff, float* stats, float* loss, hipStream_t st);
hipError_t launch_ce_bwd(int dtype, const void* logits, const int64_t* labels, const float* stats,
                         const float* gloss, long N, int V, int vec, float inv_n, float c2, int has_coeff, void* grad,
                         hipStream_t st);
size_t emb_sort_temp_bytes(long npos, int V);
hipError_t launch_emb_fwd(int dtype, const int64_t* ids, const void* w, void* out, long npos, int V, int D,
                          hipStream_t st);
hipError_t launch_emb_bwd(int dtype, const int64_t* ids, const void* g, void* gw, long npos, int V, int D, char* ws,
                          size_t temp_bytes, hipStream_t st);
hipError_t launch_silu(int dtype, int backward, const void* x, const void* dy, void* out, long n, hipStream_t st);
hipError_t launch_swiglu(int dtype, int backward, const void* gu, const void* dh, void* out, long rows, int F,
                         hipStream_t st);
hipError_t launch_rope_heads(int dtype, int backward, const void* in, const float* cosv, const float* sinv, void* out,
                             int B, int Tn, int H, int D, hipStream_t st);
hipError_t launch_swap_heads(int dtype, const void* in, void* out, int B, int X, int Y, int D, hipStream_t st);
}  // namespace otx

static thread_local char g_err[512];

static int fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
  return code;
}

static int check_shape(int B, int H, int Hkv, int S, int D, int window, int dtype) {
  if (B <= 0 || H <= 0 || Hkv <= 0 || S <= 0) return fail(OTX_EINVAL, "B, H, Hkv and S must be positive");
  if (H % Hkv != 0) return fail(OTX_EINVAL, "H (%d) must be a multiple of Hkv (%d)", H, Hkv);
  if (S % 32 != 0) return fail(OTX_EINVAL, "sequence length %d is not a multiple of 32", S);
  if (D != 64 && D != 128) return fail(OTX_EINVAL, "head_dim %d not supported (64 or 128)", D);
  if (window < 0 || window % 32 != 0) return fail(OTX_EINVAL, "window %d must be 0 or a positive multiple of 32", window);
  if (dtype != OTX_DTYPE_F32 && dtype != OTX_DTYPE_BF16) return fail(OTX_EINVAL, "dtype code %d not supported", dtype);
  if ((long long)B * H * S * D >= (1LL << 40)) return fail(OTX_EINVAL, "tensor too large");
  return OTX_OK;
}

static void launch_variant(int variant, int* nw, int* order) {
  switch (variant) {
    case 1: *nw = 2; *order = 1; break;
    case 2: *nw = 1; *order = 0; break;
    default: *nw = 4; *order = 0; break;
  }
}

static bool aligned16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

extern "C" {

const char* otx_last_error(void) { return g_err; }

float otx_softmax_scale(int D) { return (float)(1.0 / std::sqrt((double)D)); }

size_t otx_attn_bwd_workspace_bytes(int B, int H, int Hkv, int S, int D, int window) {
  if (check_shape(B, H, Hkv, S, D, window, OTX_DTYPE_BF16) != OTX_OK) return 0;
  const size_t rows = (size_t)B * H * S;
  const size_t dsum_bytes = ((rows * sizeof(float) + 255) / 256) * 256;
  const size_t tiles = (size_t)B * H * (size_t)otx_tile_offset(S / 32, window);
  return dsum_bytes + tiles * 32 * 32 * sizeof(float);
}

int otx_attn_fwd_ex(const void* q, const void* k, const void* v, void* o, float* lse, int B, int H, int Hkv, int S,
                    int D, int window, int dtype, int variant, void* stream) {
  int rc = check_shape(B, H, Hkv, S, D, window, dtype);
  if (rc) return rc;
  if (!q || !k || !v || !o || !lse) return fail(OTX_EINVAL, "null pointer argument");
  if (!aligned16(q) || !aligned16(k) || !aligned16(v) || !aligned16(o))
    return fail(OTX_EINVAL, "q, k, v and o must be 16-byte aligned");
  int nw, order;
  launch_variant(variant, &nw, &order);
  hipError_t e = otx::launch_fwd(dtype, D, nw, q, k, v, o, lse, B, H, Hkv, S, window, otx_softmax_scale(D), order,
                                 nullptr, (hipStream_t)stream);
  if (e != hipSuccess) return fail(OTX_EHIP, "forward launch failed: %s", hipGetErrorString(e));
  return OTX_OK;
}

int otx_attn_fwd(const void* q, const void* k, const void* v, void* o, float* lse, int B, int H, int Hkv, int S, int D,
                 int window, int dtype, void* stream) {
  return otx_attn_fwd_ex(q, k, v, o, lse, B, H, Hkv, S, D, window, dtype, 0, stream);
}

static size_t int8pv_qv_bytes(int B, int Hkv, int S, int D) {
  return (((size_t)B * Hkv * S * D + 255) / 256) * 256;
}

size_t otx_attn_fwd_int8pv_workspace_bytes(int B, int H, int Hkv, int S, int D) {
  if (check_shape(B, H, Hkv, S, D, 0, OTX_DTYPE_BF16) != OTX_OK) return 0;
  return int8pv_qv_bytes(B, Hkv, S, D) + (size_t)B * Hkv * (S / 32) * D * sizeof(float);
}

int otx_attn_fwd_int8pv_ex(const void* q, const void* k, const void* v, void* o, float* lse, int B, int H, int Hkv,
                           int S, int D, int window, int dtype, void* workspace, size_t workspace_bytes, int variant,
                           void* stream) {
  int rc = check_shape(B, H, Hkv, S, D, window, dtype);
  if (rc) return rc;
  if (dtype != OTX_DTYPE_BF16) return fail(OTX_EINVAL, "the int8-PV forward takes bf16 inputs (dtype code %d)", dtype);
  if (!q || !k || !v || !o || !lse || !workspace) return fail(OTX_EINVAL, "null pointer argument");
  if (!aligned16(q) || !aligned16(k) || !aligned16(v) || !aligned16(o) || ((uintptr_t)workspace & 255u))
    return fail(OTX_EINVAL, "q, k, v and o must be 16-byte aligned and the workspace 256-byte aligned");
  const size_t need = otx_attn_fwd_int8pv_workspace_bytes(B, H, Hkv, S, D);
  if (workspace_bytes < need)
    return fail(OTX_EINVAL, "workspace too small: %zu bytes given, %zu needed", workspace_bytes, need);
  int8_t* qvt = (int8_t*)workspace;
  float* vstep = (float*)((char*)workspace + int8pv_qv_bytes(B, Hkv, S, D));
  int nw, order;
  launch_variant(variant, &nw, &order);
  hipError_t e = otx::launch_fwd_int8pv(D, nw, q, k, v, o, lse, B, H, Hkv, S, window, otx_softmax_scale(D), order,
                                        qvt, vstep, nullptr, (hipStream_t)stream);
  if (e != hipSuccess) return fail(OTX_EHIP, "int8-PV forward launch failed: %s", hipGetErrorString(e));
  return OTX_OK;
}

int otx_attn_fwd_int8pv(const void* q, const void* k, const void* v, void* o, float* lse, int B, int H, int Hkv, int S,
                        int D, int window, int dtype, void* workspace, size_t workspace_bytes, void* stream) {
  return otx_attn_fwd_int8pv_ex(q, k, v, o, lse, B, H, Hkv, S, D, window, dtype, workspace, workspace_bytes, 0,
                                stream);
}

}  // extern "C"

// ---------------------------------------------------------------------------
// The allocation-free int8-PV forward: its quantized-V workspace lives in this
// file-scope device array instead of caller or library allocations.  Each GPU
// holds its own copy for the life of the process.  Host code never passes the
// array's name to a kernel (on the host it is only a stand-in symbol): the
// device address is resolved once per device with hipGetSymbolAddress, with
// that device current, and kept in g_scratch_dev.
static __device__ __align__(256) unsigned char scratch[OTX_NOALLOC_SCRATCH_BYTES];

static constexpr int kMaxDevices = 64;
static std::mutex g_scratch_mu;
static void* g_scratch_dev[kMaxDevices];

// Device address of `scratch` on the current device (resolved on the first call there).
static int scratch_on_current_device(void** out) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return fail(OTX_EHIP, "hipGetDevice failed: %s", hipGetErrorString(e));
  if (dev < 0 || dev >= kMaxDevices) return fail(OTX_EINVAL, "device index %d outside [0, %d)", dev, kMaxDevices);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_dev[dev] == nullptr) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || p == nullptr)
      return fail(OTX_EHIP, "hipGetSymbolAddress(scratch) failed on device %d: %s", dev, hipGetErrorString(e));
    g_scratch_dev[dev] = p;
  }
  *out = g_scratch_dev[dev];
  return OTX_OK;
}

extern "C" {

int otx_attn_fwd_int8pv_noalloc(const void* q, const void* k, const void* v, void* o, float* lse, int B, int H,
                                int Hkv, int S, int D, int window, int dtype, int variant, void* stream) {
  int rc = check_shape(B, H, Hkv, S, D, window, dtype);
  if (rc) return rc;
  if (dtype != OTX_DTYPE_BF16) return fail(OTX_EINVAL, "the int8-PV forward takes bf16 inputs (dtype code %d)", dtype);
  if (!q || !k || !v || !o || !lse) return fail(OTX_EINVAL, "null pointer argument");
  if (!aligned16(q) || !aligned16(k) || !aligned16(v) || !aligned16(o))
    return fail(OTX_EINVAL, "q, k, v and o must be 16-byte aligned");
  const size_t need = otx_attn_fwd_int8pv_workspace_bytes(B, H, Hkv, S, D);
  if (need > OTX_NOALLOC_SCRATCH_BYTES)
    return fail(OTX_EINVAL,
                "shape too large for the allocation-free int8-PV forward: it needs %zu bytes of scratch "
                "(B*Hkv*S*D int8 values and B*Hkv*(S/32)*D steps), the fixed scratch holds %zu; call "
                "otx_attn_fwd_int8pv with a workspace instead",
                need, (size_t)OTX_NOALLOC_SCRATCH_BYTES);
  void* base = nullptr;
  rc = scratch_on_current_device(&base);
  if (rc) return rc;
  // The quantize-V kernel writes every int8 value and step the forward reads, so
  // nothing left in the scratch by an earlier call is ever read.
  int8_t* qvt = (int8_t*)base;
  float* vstep = (float*)((char*)base + int8pv_qv_bytes(B, Hkv, S, D));
  int nw, order;
  launch_variant(variant, &nw, &order);
  hipError_t e = otx::launch_fwd_int8pv(D, nw, q, k, v, o, lse, B, H, Hkv, S, window, otx_softmax_scale(D), order,
                                        qvt, vstep, nullptr, (hipStream_t)stream);
  if (e != hipSuccess) return fail(OTX_EHIP, "int8-PV forward launch failed: %s", hipGetErrorString(e));
  return OTX_OK;
}

int otx_attn_bwd_stages(const void* q, const void* k, const void* v, const void* o, const float* lse,
                        const void* dout, void* dq, void* dk, void* dv, int B, int H, int Hkv, int S, int D, int window,
                        int dtype, void* workspace, size_t workspace_bytes, int variant, int stages, void* stream) {
  int rc = check_shape(B, H, Hkv, S, D, window, dtype);
  if (rc) return rc;
  if (stages <= 0 || stages > 7) return fail(OTX_EINVAL, "stage mask %d must be in 1..7", stages);
  if (!q || !k || !v || !o || !lse || !dout || !dq || !dk || !dv || !workspace)
    return fail(OTX_EINVAL, "null pointer argument");
  if (!aligned16(q) || !aligned16(k) || !aligned16(v) || !aligned16(o) || !aligned16(dout) || !aligned16(dq) ||
      !aligned16(dk) || !aligned16(dv) || ((uintptr_t)workspace & 255u))
    return fail(OTX_EINVAL, "tensors must be 16-byte aligned and the workspace 256-byte aligned");
  const size_t need = otx_attn_bwd_workspace_bytes(B, H, Hkv, S, D, window);
  if (workspace_bytes < need)
    return fail(OTX_EINVAL, "workspace too small: %zu bytes given, %zu needed", workspace_bytes, need);
  const size_t rows = (size_t)B * H * S;
  float* dsum = (float*)workspace;
  float* ds = (float*)((char*)workspace + ((rows * sizeof(float) + 255) / 256) * 256);
  int nw, order;
  launch_variant(variant, &nw, &order);
  hipError_t e = otx::launch_bwd(dtype, D, nw, q, k, v, o, lse, dout, dq, dk, dv, dsum, ds, B, H, Hkv, S, window,
                                 otx_softmax_scale(D), order, stages, nullptr, (hipStream_t)stream);
  if (e != hipSuccess) return fail(OTX_EHIP, "backward launch failed: %s", hipGetErrorString(e));
  return OTX_OK;
}

int otx_attn_bwd_ex(const void* q, const void* k, const void* v, const void* o, const float* lse, const void* dout,
                    void* dq, void* dk, void* dv, int B, int H, int Hkv, int S, int D, int window, int dtype,
                    void* workspace, size_t workspace_bytes, int variant, void* stream) {
  return otx_attn_bwd_stages(q, k, v, o, lse, dout, dq, dk, dv, B, H, Hkv, S, D, window, dtype, workspace,
                             workspace_bytes, variant, 7, stream);
}

int otx_attn_bwd(const void* q, const void* k, const void* v, const void* o, const float* lse, const void* dout,
                 void* dq, void* dk, void* dv, int B, int H, int Hkv, int S, int D, int window, int dtype,
                 void* workspace, size_t workspace_bytes, void* stream) {
  return otx_attn_bwd_ex(q, k, v, o, lse, dout, dq, dk, dv, B, H, Hkv, S, D, window, dtype, workspace,
                         workspace_bytes, 0, stream);
}

// ---- score cache ----

size_t otx_attn_score_cache_bytes(int B, int H, int S, int window) {
  if (B <= 0 || H <= 0 || S <= 0 || S % 32 != 0 || window < 0 || window % 32 != 0) return 0;
  return (size_t)B * H * (size_t)otx_tile_offset(S / 32, window) * 32 * 32 * sizeof(float);
}

static int check_scache(const float* scache, size_t scache_bytes, int B, int H, int S, int window, int dtype) {
  if (dtype != OTX_DTYPE_BF16) return fail(OTX_EINVAL, "the score cache is defined for bf16 inputs (dtype code %d)", dtype);
  if (!scache) return fail(OTX_EINVAL, "null score cache");
  if (!aligned16(scache)) return fail(OTX_EINVAL, "the score cache must be 16-byte aligned");
  const size_t need = otx_attn_score_cache_bytes(B, H, S, window);
  if (scache_bytes < need)
    return fail(OTX_EINVAL, "score cache too small: %zu bytes given, %zu needed", scache_bytes, need);
  return OTX_OK;
}

int otx_attn_fwd_sc(const void* q, const void* k, const void* v, void* o, float* lse, float* scache,
                    size_t scache_bytes, int B, int H, int Hkv, int S, int D, int window, int dtype, int variant,
                    void* stream) {
  int rc = check_shape(B, H, Hkv, S, D, window, dtype);
  if (rc) return rc;
  if ((rc = check_scache(scache, scache_bytes, B, H, S, window, dtype))) return rc;
  if (!q || !k || !v || !o || !lse) return fail(OTX_EINVAL, "null pointer argument");
  if (!aligned16(q) || !aligned16(k) || !aligned16(v) || !aligned16(o))
    return fail(OTX_EINVAL, "q, k, v and o must be 16-byte aligned");
  int nw, order;
  launch_variant(variant, &nw, &order);
  hipError_t e = otx::launch_fwd(dtype, D, nw, q, k, v, o, lse, B, H, Hkv, S, window, otx_softmax_scale(D), order,
                                 scache, (hipStream_t)stream);
  if (e != hipSuccess) return fail(OTX_EHIP, "forward launch failed: %s", hipGetErrorString(e));
  return OTX_OK;
}

int otx_attn_fwd_int8pv_sc(const void* q, const void* k, const void* v, void* o, float* lse, float* scache,
                           size_t scache_bytes, int B, int H, int Hkv, int S, int D, int window, int dtype,
                           void* workspace, size_t workspace_bytes, int variant, void* stream) {
  int rc = check_shape(B, H, Hkv, S, D, window, dtype);
  if (rc) return rc;
  if ((rc = check_scache(scache, scache_bytes, B, H, S, window, dtype))) return rc;
  if (!q || !k || !v || !o || !lse || !workspace) return fail(OTX_EINVAL, "null pointer argument");
  if (!aligned16(q) || !aligned16(k) || !aligned16(v) || !aligned16(o) || ((uintptr_t)workspace & 255u))
    return fail(OTX_EINVAL, "q, k, v and o must be 16-byte aligned and the workspace 256-byte aligned");
  const size_t need = otx_attn_fwd_int8pv_workspace_bytes(B, H, Hkv, S, D);
  if (workspace_bytes < need)
    return fail(OTX_EINVAL, "workspace too small: %zu bytes given, %zu needed", workspace_bytes, need);
  int8_t* qvt = (int8_t*)workspace;
  float* vstep = (float*)((char*)workspace + int8pv_qv_bytes(B, Hkv, S, D));
  int nw, order;
  launch_variant(variant, &nw, &order);
  hipError_t e = otx::launch_fwd_int8pv(D, nw, q, k, v, o, lse, B, H, Hkv, S, window, otx_softmax_scale(D), order,
                                        qvt, vstep, scache, (hipStream_t)stream);
  if (e != hipSuccess) return fail(OTX_EHIP, "int8-PV forward launch failed: %s", hipGetErrorString(e));
  return OTX_OK;
}

int otx_attn_bwd_sc(const void* q, const void* k, const void* v, const void* o, const float* lse, const void* dout,
                    void* dq, void* dk, void* dv, const float* scache, size_t scache_bytes, int B, int H, int Hkv,
                    int S, int D, int window, int dtype, void* workspace, size_t workspace_bytes, int variant,
                    int stages, void* stream) {
  int rc = check_shape(B, H, Hkv, S, D, window, dtype);
  if (rc) return rc;
  if ((rc = check_scache(scache, scache_bytes, B, H, S, window, dtype))) return rc;
  if (stages <= 0 || stages > 7) return fail(OTX_EINVAL, "stage mask %d must be in 1..7", stages);
  if (!q || !k || !v || !o || !lse || !dout || !dq || !dk || !dv || !workspace)
    return fail(OTX_EINVAL, "null pointer argument");
  if (!aligned16(q) || !aligned16(k) || !aligned16(v) || !aligned16(o) || !aligned16(dout) || !aligned16(dq) ||
      !aligned16(dk) || !aligned16(dv) || ((uintptr_t)workspace & 255u))
    return fail(OTX_EINVAL, "tensors must be 16-byte aligned and the workspace 256-byte aligned");
  const size_t need = otx_attn_bwd_workspace_bytes(B, H, Hkv, S, D, window);
  if (workspace_bytes < need)
    return fail(OTX_EINVAL, "workspace too small: %zu bytes given, %zu needed", workspace_bytes, need);
  const size_t rows = (size_t)B * H * S;
  float* dsum = (float*)workspace;
  float* ds = (float*)((char*)workspace + ((rows * sizeof(float) + 255) / 256) * 256);
  int nw, order;
  launch_variant(variant, &nw, &order);
  hipError_t e = otx::launch_bwd(dtype, D, nw, q, k, v, o, lse, dout, dq, dk, dv, dsum, ds, B, H, Hkv, S, window,
                                 otx_softmax_scale(D), order, stages, scache, (hipStream_t)stream);
  if (e != hipSuccess) return fail(OTX_EHIP, "backward launch failed: %s", hipGetErrorString(e));
  return OTX_OK;
}

// ---------------------------------------------------------------------------
// Decoder-layer operators (GEMM, RMSNorm, SiLU).

int otx_gemm_bf16(const void* A, long a_i, long a_r, const void* B, long b_j, long b_r, void* C, long ldc, int M,
                  int N, int R, int out_dtype, void* stream) {
  return otx_gemm_bf16_ex(A, a_i, a_r, B, b_j, b_r, C, ldc, M, N, R, out_dtype, 0, stream);
}

int otx_gemm_bf16_ex(const void* A, long a_i, long a_r, const void* B, long b_j, long b_r, void* C, long ldc, int M,
                     int N, int R, int out_dtype, int variant, void* stream) {
  if (!A || !B || !C) return fail(OTX_EINVAL, "null pointer argument");
  if (variant < 0 || variant > 3) return fail(OTX_EINVAL, "GEMM variant %d (0, 1, 2 or 3)", variant);
  if (M <= 0 || N <= 0 || R <= 0 || M % 128 || N % 128 || R % 32)
    return fail(OTX_EINVAL, "GEMM shape %d x %d x %d: M and N must be multiples of 128, R of 32", M, N, R);
  if (!((a_r == 1 && a_i % 8 == 0) || (a_i == 1 && a_r % 8 == 0)))
    return fail(OTX_EINVAL, "A strides (%ld, %ld): one must be 1 and the other a multiple of 8", a_i, a_r);
  if (!((b_r == 1 && b_j % 8 == 0) || (b_j == 1 && b_r % 8 == 0)))
    return fail(OTX_EINVAL, "B strides (%ld, %ld): one must be 1 and the other a multiple of 8", b_j, b_r);
  if (ldc < N) return fail(OTX_EINVAL, "ldc %ld is smaller than N %d", ldc, N);
  if (out_dtype != OTX_DTYPE_F32 && out_dtype != OTX_DTYPE_BF16) return fail(OTX_EINVAL, "bad output dtype");
  if (!aligned16(A) || !aligned16(B)) return fail(OTX_EINVAL, "A and B must be 16-byte aligned");
  hipError_t e = otx::launch_gemm(A, a_i, a_r, B, b_j, b_r, C, ldc, M, N, R, out_dtype == OTX_DTYPE_F32, variant,
                                  (hipStream_t)stream);
  return e == hipSuccess ? OTX_OK : fail(OTX_EHIP, "GEMM launch failed: %s", hipGetErrorString(e));
}

static int check_norm(long rows, int D, int dtype) {
  if (rows <= 0 || D <= 0 || D % 32 || D > 8192)
    return fail(OTX_EINVAL, "RMSNorm width %d must be a positive multiple of 32 up to 8192", D);
  if (dtype != OTX_DTYPE_F32 && dtype != OTX_DTYPE_BF16) return fail(OTX_EINVAL, "dtype code %d not supported", dtype);
  return OTX_OK;
}

int otx_rmsnorm_fwd(const void* x, const void* w, void* y, float* rstd, long rows, int D, float eps, int dtype,
                    void* stream) {
  int rc = check_norm(rows, D, dtype);
  if (rc) return rc;
  if (!x || !w || !y || !rstd) return fail(OTX_EINVAL, "null pointer argument");
  hipError_t e = otx::launch_rmsnorm_fwd(dtype, x, w, y, rstd, rows, D, eps, (hipStream_t)stream);
  return e == hipSuccess ? OTX_OK : fail(OTX_EHIP, "RMSNorm launch failed: %s", hipGetErrorString(e));
}

size_t otx_rmsnorm_bwd_workspace_bytes(long rows, int D) {
  if (rows <= 0 || rows % 32 || D <= 0) return 0;
  return (size_t)(rows / 32) * D * sizeof(float);
}

int otx_rmsnorm_bwd(const void* x, const void* w, const float* rstd, const void* dy, void* dx, float* dw, long rows,
                    int D, int dtype, void* workspace, size_t workspace_bytes, void* stream) {
  int rc = check_norm(rows, D, dtype);
  if (rc) return rc;
  if (rows % 32) return fail(OTX_EINVAL, "RMSNorm backward needs a row count that is a multiple of 32 (got %ld)", rows);
  if (!x || !w || !rstd || !dy || !dx || !dw || !workspace) return fail(OTX_EINVAL, "null pointer argument");
  if (!aligned16(workspace)) return fail(OTX_EINVAL, "RMSNorm backward workspace must be 16-byte aligned");
  const size_t need = otx_rmsnorm_bwd_workspace_bytes(rows, D);
  if (workspace_bytes < need)
    return fail(OTX_EINVAL, "workspace too small: %zu bytes given, %zu needed", workspace_bytes, need);
  hipError_t e = otx::launch_rmsnorm_bwd(dtype, x, w, rstd, dy, dx, dw, (float*)workspace, rows, D,
                                         (hipStream_t)stream);
  return e == hipSuccess ? OTX_OK : fail(OTX_EHIP, "RMSNorm backward launch failed: %s", hipGetErrorString(e));
}

int otx_silu_fwd(const void* x, void* y, long n, int dtype, void* stream) {
  if (!x || !y || n <= 0) return fail(OTX_EINVAL, "bad SiLU arguments");
  if (dtype != OTX_DTYPE_F32 && dtype != OTX_DTYPE_BF16) return fail(OTX_EINVAL, "dtype code %d not supported", dtype);
  hipError_t e = otx::launch_silu(dtype, 0, x, nullptr, y, n, (hipStream_t)stream);
  return e == hipSuccess ? OTX_OK : fail(OTX_EHIP, "SiLU launch failed: %s", hipGetErrorString(e));
}

int otx_silu_bwd(const void* x, const void* dy, void* dx, long n, int dtype, void* stream) {
  if (!x || !dy || !dx || n <= 0) return fail(OTX_EINVAL, "bad SiLU arguments");
  if (dtype != OTX_DTYPE_F32 && dtype != OTX_DTYPE_BF16) return fail(OTX_EINVAL, "dtype code %d not supported", dtype);
  hipError_t e = otx::launch_silu(dtype, 1, x, dy, dx, n, (hipStream_t)stream);
  return e == hipSuccess ? OTX_OK : fail(OTX_EHIP, "SiLU backward launch failed: %s", hipGetErrorString(e));
}

static int check_rows16(long rows, int W, int dtype, const char* what) {
  if (dtype != OTX_DTYPE_F32 && dtype != OTX_DTYPE_BF16) return fail(OTX_EINVAL, "dtype code %d not supported", dtype);
  if (rows <= 0 || W <= 0) return fail(OTX_EINVAL, "%s: sizes must be positive", what);
  if (W % 8 != 0) return fail(OTX_EINVAL, "%s: row width %d is not a multiple of 8", what, W);
  if (rows * (long long)W >= (1LL << 40)) return fail(OTX_EINVAL, "%s: tensor too large", what);
  return OTX_OK;
}

int otx_swiglu_fwd(const void* gu, void* h, long rows, int F, int dtype, void* stream) {
  int rc = check_rows16(rows, F, dtype, "SwiGLU");
  if (rc) return rc;
  if (!gu || !h || !aligned16(gu) || !aligned16(h)) return fail(OTX_EINVAL, "SwiGLU: null or unaligned pointer");
  hipError_t e = otx::launch_swiglu(dtype, 0, gu, nullptr, h, rows, F, (hipStream_t)stream);
  return e == hipSuccess ? OTX_OK : fail(OTX_EHIP, "SwiGLU launch failed: %s", hipGetErrorString(e));
}

int otx_swiglu_bwd(const void* gu, const void* dh, void* dgu, long rows, int F, int dtype, void* stream) {
  int rc = check_rows16(rows, F, dtype, "SwiGLU backward");
  if (rc) return rc;
  if (!gu || !dh || !dgu || !aligned16(gu) || !aligned16(dh) || !aligned16(dgu))
    return fail(OTX_EINVAL, "SwiGLU backward: null or unaligned pointer");
  if (dgu == gu) return fail(OTX_EINVAL, "SwiGLU backward: dgu must not alias gu");
  hipError_t e = otx::launch_swiglu(dtype, 1, gu, dh, dgu, rows, F, (hipStream_t)stream);
  return e == hipSuccess ? OTX_OK : fail(OTX_EHIP, "SwiGLU backward launch failed: %s", hipGetErrorString(e));
}

static int rope_args(const void* in, const float* cosv, const float* sinv, const void* out, int B, int T, int H, int D,
                     int dtype) {
  if (B <= 0 || T <= 0 || H <= 0) return fail(OTX_EINVAL, "RoPE: B, T and H must be positive");
  int rc = check_rows16((long)B * T * H, D, dtype, "RoPE");
  if (rc) return rc;
  if (!in || !cosv || !sinv || !out || !aligned16(in) || !aligned16(out) || ((uintptr_t)cosv & 7u) ||
      ((uintptr_t)sinv & 7u))
    return fail(OTX_EINVAL, "RoPE: null or unaligned pointer");
  if (in == out) return fail(OTX_EINVAL, "RoPE: the output must not alias the input");
  return OTX_OK;
}

int otx_rope_heads_fwd(const void* x, const float* cosv, const float* sinv, void* y, int B, int T, int H, int D,
                       int dtype, void* stream) {
  int rc = rope_args(x, cosv, sinv, y, B, T, H, D, dtype);
  if (rc) return rc;
  hipError_t e = otx::launch_rope_heads(dtype, 0, x, cosv, sinv, y, B, T, H, D, (hipStream_t)stream);
  return e == hipSuccess ? OTX_OK : fail(OTX_EHIP, "RoPE launch failed: %s", hipGetErrorString(e));
}

int otx_rope_heads_bwd(const void* dy, const float* cosv, const float* sinv, void* dx, int B, int T, int H, int D,
                       int dtype, void* stream) {
  int rc = rope_args(dy, cosv, sinv, dx, B, T, H, D, dtype);
  if (rc) return rc;
  hipError_t e = otx::launch_rope_heads(dtype, 1, dy, cosv, sinv, dx, B, T, H, D, (hipStream_t)stream);
  return e == hipSuccess ? OTX_OK : fail(OTX_EHIP, "RoPE backward launch failed: %s", hipGetErrorString(e));
}

int otx_swap_heads(const void* x, void* y, int B, int X, int Y, int D, int dtype, void* stream) {
  if (B <= 0 || X <= 0 || Y <= 0) return fail(OTX_EINVAL, "swap_heads: B, X and Y must be positive");
  int rc = check_rows16((long)B * X * Y, D, dtype, "swap_heads");
  if (rc) return rc;
  if (!x || !y || !aligned16(x) || !aligned16(y)) return fail(OTX_EINVAL, "swap_heads: null or unaligned pointer");
  if (x == y) return fail(OTX_EINVAL, "swap_heads: the output must not alias the input");
  hipError_t e = otx::launch_swap_heads(dtype, x, y, B, X, Y, D, (hipStream_t)stream);
  return e == hipSuccess ? OTX_OK : fail(OTX_EHIP, "swap_heads launch failed: %s", hipGetErrorString(e));
}

// otx_build_info() is defined in otx_stamp.cpp, stamped by the build script.

}  // extern "C"

// ---------------------------------------------------------------------------
// Self-checks of the two hardware facts the kernels rely on.

__global__ void otx_selftest_mfma_kernel(const float* a, const float* b, const float* c, float* out, int groups) {
  const int l = threadIdx.x;
  for (int t = blockIdx.x; t < groups; t += gridDim.x) {
    f32x32 acc;
#pragma unroll
    for (int r = 0; r < 32; r++) acc[r] = c[((size_t)t * 32 + r) * 64 + l];
    acc = otx_mfma(a[t * 64 + l], b[t * 64 + l], acc);
#pragma unroll
    for (int r = 0; r < 32; r++) out[((size_t)t * 32 + r) * 64 + l] = acc[r];
  }
}

// One v_mfma_f32_16x16x1_4b_f32 per group: a/b one binary32 per lane, c/out 16
// registers per lane ([group][register][lane], as above).
typedef float otx_f32x16 __attribute__((ext_vector_type(16)));
__global__ void otx_selftest_mfma16_kernel(const float* a, const float* b, const float* c, float* out, int groups) {
  const int l = threadIdx.x;
  for (int t = blockIdx.x; t < groups; t += gridDim.x) {
    otx_f32x16 acc;
#pragma unroll
    for (int r = 0; r < 16; r++) acc[r] = c[((size_t)t * 16 + r) * 64 + l];
    acc = __builtin_amdgcn_mfma_f32_16x16x1f32(a[t * 64 + l], b[t * 64 + l], acc, 0, 0, 0);
#pragma unroll
    for (int r = 0; r < 16; r++) out[((size_t)t * 16 + r) * 64 + l] = acc[r];
  }
}

// One bf16 MFMA per group with raw operand registers read from memory in the
// instruction's own lane order: a/b hold AW bf16 per lane, c/out CR floats per
// lane.  kind 0: 32x32x4_2b (AW 4, CR 32), 1: 32x32x8 (4, 16), 2: 32x32x16
// (8, 16), 3: 16x16x16 (4, 4), 4: 16x16x32 (8, 4).
typedef short otx_s4 __attribute__((ext_vector_type(4)));
typedef __bf16 otx_bf8 __attribute__((ext_vector_type(8)));
template <int KIND>
__global__ void otx_selftest_mfma_bf16_kernel(const uint16_t* a, const uint16_t* b, const float* c, float* out,
                                              int groups) {
  constexpr int AW = (KIND == 2 || KIND == 4) ? 8 : 4;
  constexpr int CR = KIND == 0 ? 32 : (KIND <= 2 ? 16 : 4);
  typedef float cvec __attribute__((ext_vector_type(CR)));
  const int l = threadIdx.x;
  for (int t = blockIdx.x; t < groups; t += gridDim.x) {
    const uint16_t* pa = a + ((size_t)t * 64 + l) * AW;
    const uint16_t* pb = b + ((size_t)t * 64 + l) * AW;
    cvec acc;
#pragma unroll
    for (int r = 0; r < CR; r++) acc[r] = c[((size_t)t * 64 + l) * CR + r];
    if constexpr (AW == 4) {
      otx_s4 va, vb;
#pragma unroll
      for (int e = 0; e < 4; e++) { va[e] = (short)pa[e]; vb[e] = (short)pb[e]; }
      if constexpr (KIND == 0) acc = __builtin_amdgcn_mfma_f32_32x32x4bf16_1k(va, vb, acc, 0, 0, 0);
      else if constexpr (KIND == 1) acc = __builtin_amdgcn_mfma_f32_32x32x8bf16_1k(va, vb, acc, 0, 0, 0);
      else acc = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(va, vb, acc, 0, 0, 0);
    } else {
      otx_bf8 va, vb;
#pragma unroll
      for (int e = 0; e < 8; e++) {
        va[e] = __builtin_bit_cast(__bf16, pa[e]);
        vb[e] = __builtin_bit_cast(__bf16, pb[e]);
      }
      if constexpr (KIND == 2) acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(va, vb, acc, 0, 0, 0);
      else acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(va, vb, acc, 0, 0, 0);
    }
#pragma unroll
    for (int r = 0; r < CR; r++) out[((size_t)t * 64 + l) * CR + r] = acc[r];
  }
}

// One v_mfma_i32_32x32x32_i8 per group with raw operand registers in the
// instruction's lane order: a/b [g][64][16] int8, c/out [g][64][16] int32.
typedef int otx_i32x4 __attribute__((ext_vector_type(4)));
typedef int otx_i32x16 __attribute__((ext_vector_type(16)));
__global__ void otx_selftest_mfma_i8_kernel(const int8_t* a, const int8_t* b, const int* c, int* out, int groups) {
  const int l = threadIdx.x;
  for (int t = blockIdx.x; t < groups; t += gridDim.x) {
    const otx_i32x4 va = *reinterpret_cast<const otx_i32x4*>(a + ((size_t)t * 64 + l) * 16);
    const otx_i32x4 vb = *reinterpret_cast<const otx_i32x4*>(b + ((size_t)t * 64 + l) * 16);
    otx_i32x16 acc;
#pragma unroll
    for (int r = 0; r < 16; r++) acc[r] = c[((size_t)t * 64 + l) * 16 + r];
    acc = __builtin_amdgcn_mfma_i32_32x32x32_i8(va, vb, acc, 0, 0, 0);
#pragma unroll
    for (int r = 0; r < 16; r++) out[((size_t)t * 64 + l) * 16 + r] = acc[r];
  }
}

__device__ inline uint64_t otx_mix64(uint32_t x, uint32_t y) {
  uint64_t h = ((uint64_t)x << 32) | y;
  h ^= h >> 33;
  h *= 0xff51afd7ed558ccdull;
  h ^= h >> 33;
  h *= 0xc4ceb9fe1a85ec53ull;
  h ^= h >> 33;
  return h;
}

// Sum (mod 2^64) of mix(x, f(x)) over the bit patterns [lo, lo + count).
// which: 0 = otx_expf, 1 = otx_logf, one input per thread; 2 / 3 = the kernels'
// batched exp (otx_exp_n as dK/dV calls it: CHECKED, chunks of 16; as the
// forward calls it: x <= 0 only, chunks of 8) on 32 consecutive inputs per
// thread, so that the fallback for undecided inputs runs on the device.
__global__ void otx_selftest_math_kernel(int which, uint64_t lo, uint64_t count, uint64_t* partial) {
  __shared__ uint64_t red[256];
  __shared__ double tab[OTX_EXP_LE0_TAB_N];
  otx_load_exp_table(tab);
  __syncthreads();
  uint64_t s = 0;
  const uint64_t stride = (uint64_t)gridDim.x * blockDim.x;
  if (which == 2 || which == 3) {
    for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < count / 32; i += stride) {
      float v[32];
#pragma unroll
      for (int j = 0; j < 32; j++) v[j] = __uint_as_float((uint32_t)(lo + 32 * i + j));
      if (which == 2)
        otx_exp_n<32, true, 16>(v, tab);
      else
        otx_exp_n<32, false, 8>(v, tab);
#pragma unroll
      for (int j = 0; j < 32; j++) s += otx_mix64((uint32_t)(lo + 32 * i + j), __float_as_uint(v[j]));
    }
  }
  for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; which < 2 && i < count; i += stride) {
    const uint32_t u = (uint32_t)(lo + i);
    const float x = __uint_as_float(u);
    const float y = which == 0 ? otx_expf(x) : otx_logf(x);
    s += otx_mix64(u, __float_as_uint(y));
  }
  for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; which == 4 && i < count; i += stride) {
    const uint32_t u = (uint32_t)(lo + i);
    s += otx_mix64(u, (uint32_t)otx_f32_to_bf16(__uint_as_float(u)) << 16);
  }
  for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; which == 5 && i < count; i += stride) {
    const uint32_t u = (uint32_t)(lo + i);
    const uint32_t b = __builtin_amdgcn_cvt_pk_u8_f32(__uint_as_float(u), 2u, 0u) >> 16;  // the int8-PV quantizer
    s += otx_mix64(u, __float_as_uint((float)b));
  }
  red[threadIdx.x] = s;
  __syncthreads();
  for (int w = 128; w > 0; w >>= 1) {
    if ((int)threadIdx.x < w) red[threadIdx.x] += red[threadIdx.x + w];
    __syncthreads();
  }
  if (threadIdx.x == 0) partial[blockIdx.x] = red[0];
}

extern "C" {

int otx_selftest_mfma(const float* a, const float* b, const float* c, float* out, int groups, void* stream) {
  if (groups <= 0 || !a || !b || !c || !out) return fail(OTX_EINVAL, "bad selftest arguments");
  hipLaunchKernelGGL(otx_selftest_mfma_kernel, dim3(groups < 1024 ? groups : 1024), dim3(64), 0, (hipStream_t)stream,
                     a, b, c, out, groups);
  hipError_t e = hipGetLastError();
  return e == hipSuccess ? OTX_OK : fail(OTX_EHIP, "selftest launch failed: %s", hipGetErrorString(e));
}

int otx_selftest_mfma16(const float* a, const float* b, const float* c, float* out, int groups, void* stream) {
  if (groups <= 0 || !a || !b || !c || !out) return fail(OTX_EINVAL, "bad selftest arguments");
  hipLaunchKernelGGL(otx_selftest_mfma16_kernel, dim3(groups < 1024 ? groups : 1024), dim3(64), 0,
                     (hipStream_t)stream, a, b, c, out, groups);
  hipError_t e = hipGetLastError();
  return e == hipSuccess ? OTX_OK : fail(OTX_EHIP, "selftest launch failed: %s", hipGetErrorString(e));
}

int otx_selftest_mfma_bf16(int kind, const uint16_t* a, const uint16_t* b, const float* c, float* out, int groups,
                           void* stream) {
  if (groups <= 0 || !a || !b || !c || !out || kind < 0 || kind > 4) return fail(OTX_EINVAL, "bad selftest arguments");
  const dim3 grid(groups < 1024 ? groups : 1024), block(64);
  hipStream_t st = (hipStream_t)stream;
  switch (kind) {
    case 0: hipLaunchKernelGGL(otx_selftest_mfma_bf16_kernel<0>, grid, block, 0, st, a, b, c, out, groups); break;
    case 1: hipLaunchKernelGGL(otx_selftest_mfma_bf16_kernel<1>, grid, block, 0, st, a, b, c, out, groups); break;
    case 2: hipLaunchKernelGGL(otx_selftest_mfma_bf16_kernel<2>, grid, block, 0, st, a, b, c, out, groups); break;
    case 3: hipLaunchKernelGGL(otx_selftest_mfma_bf16_kernel<3>, grid, block, 0, st, a, b, c, out, groups); break;
    default: hipLaunchKernelGGL(otx_selftest_mfma_bf16_kernel<4>, grid, block, 0, st, a, b, c, out, groups); break;
  }
  hipError_t e = hipGetLastError();
  return e == hipSuccess ? OTX_OK : fail(OTX_EHIP, "selftest launch failed: %s", hipGetErrorString(e));
}

int otx_selftest_mfma_i8(const int8_t* a, const int8_t* b, const int* c, int* out, int groups, void* stream) {
  if (groups <= 0 || !a || !b || !c || !out) return fail(OTX_EINVAL, "bad selftest arguments");
  hipLaunchKernelGGL(otx_selftest_mfma_i8_kernel, dim3(groups < 1024 ? groups : 1024), dim3(64), 0,
                     (hipStream_t)stream, a, b, c, out, groups);
  hipError_t e = hipGetLastError();
  return e == hipSuccess ? OTX_OK : fail(OTX_EHIP, "selftest launch failed: %s", hipGetErrorString(e));
}

int otx_selftest_math(int which, uint64_t lo, uint64_t count, uint64_t* partial, int nblocks, void* stream) {
  if (which < 0 || which > 5 || !partial || nblocks <= 0 || lo + count > (1ull << 32) ||
      (which >= 2 && count % 32 != 0))
    return fail(OTX_EINVAL, "bad selftest arguments");
  hipLaunchKernelGGL(otx_selftest_math_kernel, dim3(nblocks), dim3(256), 0, (hipStream_t)stream, which, lo, count,
                     partial);
  hipError_t e = hipGetLastError();
  return e == hipSuccess ? OTX_OK : fail(OTX_EHIP, "selftest launch failed: %s", hipGetErrorString(e));
}

static int check_ce(const void* logits, const int64_t* labels, long N, int V, int dtype, double coeff) {
  if (!logits || !labels) return fail(OTX_EINVAL, "null pointer argument");
  if (dtype != OTX_DTYPE_F32 && dtype != OTX_DTYPE_BF16) return fail(OTX_EINVAL, "dtype code %d not supported", dtype);
  if (N <= 0 || N > 32L * 8192) return fail(OTX_EINVAL, "row count %ld outside 1..262144", N);
  if (V <= 0 || V > otx::ce_max_vocab(dtype))
    return fail(OTX_EINVAL, "vocabulary %d outside 1..%d for this dtype", V, otx::ce_max_vocab(dtype));
  if (!std::isfinite(coeff)) return fail(OTX_EINVAL, "z-loss coefficient must be finite");
  return OTX_OK;
}

static int ce_vec(const void* p, int V, int dtype) {
  const int es = dtype == OTX_DTYPE_BF16 ? 2 : 4;
  return ((long)V * es) % 16 == 0 && aligned16(p);
}

int otx_ce_zloss_fwd(const void* logits, const int64_t* labels, long N, int V, int dtype, double coeff, float* stats,
                     float* loss, void* stream) {
  int rc = check_ce(logits, labels, N, V, dtype, coeff);
  if (rc) return rc;
  if (!stats || !loss) return fail(OTX_EINVAL, "null pointer argument");
  hipError_t e = otx::launch_ce_fwd(dtype, logits, labels, N, V, ce_vec(logits, V, dtype), (float)coeff,
                                    coeff != 0.0, stats, loss, (hipStream_t)stream);
  if (e != hipSuccess) return fail(OTX_EHIP, "loss forward launch failed: %s", hipGetErrorString(e));
  return OTX_OK;
}

int otx_ce_zloss_bwd(const void* logits, const int64_t* labels, const float* stats, const float* grad_loss, long N,
                     int V, int dtype, double coeff, void* grad_logits, void* stream) {
  int rc = check_ce(logits, labels, N, V, dtype, coeff);
  if (rc) return rc;
  if (!stats || !grad_loss || !grad_logits) return fail(OTX_EINVAL, "null pointer argument");
  const int vec = ce_vec(logits, V, dtype) && aligned16(grad_logits);
  const float inv_n = (float)(1.0 / (double)N);
  const float c2 = (float)(2.0 * coeff * (1.0 / (double)N));
  hipError_t e = otx::launch_ce_bwd(dtype, logits, labels, stats, grad_loss, N, V, vec, inv_n, c2, coeff != 0.0,
                                    grad_logits, (hipStream_t)stream);
  if (e != hipSuccess) return fail(OTX_EHIP, "loss backward launch failed: %s", hipGetErrorString(e));
  return OTX_OK;
}

static int check_emb(const int64_t* ids, long npos, int V, int D, int dtype) {
  if (!ids) return fail(OTX_EINVAL, "null pointer argument");
  if (dtype != OTX_DTYPE_F32 && dtype != OTX_DTYPE_BF16) return fail(OTX_EINVAL, "dtype code %d not supported", dtype);
  if (npos <= 0 || npos > 0x7fffffffL) return fail(OTX_EINVAL, "position count %ld outside 1..2^31-1", npos);
  if (V <= 0 || V >= (1 << 30)) return fail(OTX_EINVAL, "vocabulary %d outside 1..2^30-1", V);
  if (D <= 0 || D % (dtype == OTX_DTYPE_BF16 ? 8 : 4) != 0 || D > 65535 * 256)
    return fail(OTX_EINVAL, "embedding width %d must be a positive multiple of %d", D, dtype == OTX_DTYPE_BF16 ? 8 : 4);
  return OTX_OK;
}

static size_t emb_arrays_bytes(long npos) { return 4 * (((size_t)npos * 4 + 255) / 256 * 256); }

size_t otx_embedding_bwd_workspace_bytes(long npos, int V) {
  if (npos <= 0 || npos > 0x7fffffffL || V <= 0 || V >= (1 << 30)) return 0;
  const size_t temp = otx::emb_sort_temp_bytes(npos, V);
  return temp ? emb_arrays_bytes(npos) + temp : 0;
}

int otx_embedding_fwd(const int64_t* ids, const void* weight, void* out, long npos, int V, int D, int dtype,
                      void* stream) {
  int rc = check_emb(ids, npos, V, D, dtype);
  if (rc) return rc;
  if (!weight || !out) return fail(OTX_EINVAL, "null pointer argument");
  if (!aligned16(weight) || !aligned16(out)) return fail(OTX_EINVAL, "weight and out must be 16-byte aligned");
  hipError_t e = otx::launch_emb_fwd(dtype, ids, weight, out, npos, V, D, (hipStream_t)stream);
  if (e != hipSuccess) return fail(OTX_EHIP, "embedding forward launch failed: %s", hipGetErrorString(e));
  return OTX_OK;
}

int otx_embedding_bwd(const int64_t* ids, const void* grad_out, void* grad_weight, long npos, int V, int D, int dtype,
                      void* workspace, size_t workspace_bytes, void* stream) {
  int rc = check_emb(ids, npos, V, D, dtype);
  if (rc) return rc;
  if (!grad_out || !grad_weight || !workspace) return fail(OTX_EINVAL, "null pointer argument");
  if (!aligned16(grad_weight) || ((uintptr_t)workspace & 255u))
    return fail(OTX_EINVAL, "grad_weight must be 16-byte aligned and the workspace 256-byte aligned");
  const size_t need = otx_embedding_bwd_workspace_bytes(npos, V);
  if (workspace_bytes < need)
    return fail(OTX_EINVAL, "workspace too small: %zu bytes given, %zu needed", workspace_bytes, need);
  hipError_t e = otx::launch_emb_bwd(dtype, ids, grad_out, grad_weight, npos, V, D, (char*)workspace,
                                     workspace_bytes - emb_arrays_bytes(npos), (hipStream_t)stream);
  if (e != hipSuccess) return fail(OTX_EHIP, "embedding backward launch failed: %s", hipGetErrorString(e));
  return OTX_OK;
}

}  // extern "C"
