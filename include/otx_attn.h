/*
 * otx_attn.h -- C ABI of the MI355X (gfx950) deterministic causal flash
 * attention library (libotx_attn.so).
 *
 * The library replaces the native layer behind
 *   repop.nn.flash_attention.causal_flash_attention(q, k, v, dropout=0.0, window=w)
 * which the reference calls at src/pretrain/model/modules/attention_repop.py:53
 * (GQA-native, 1/sqrt(D) scale applied inside, sliding window in keys,
 * attention_repop.py:1-20,38-53).  repop's own native entry points are closed
 * source; these functions are what a ctypes / C-extension binding of that
 * operator binds to on ROCm.
 *
 * Conventions for every entry point:
 *   - Tensors are contiguous, row-major, in device memory:
 *       q, o, dq            [B, H,   S, D]
 *       k, v, dk, dv        [B, Hkv, S, D]   (query head h reads KV head h / (H/Hkv))
 *       lse                 [B, H,   S]      float32 natural-log logsumexp
 *     with dtype OTX_DTYPE_BF16 (raw bf16) or OTX_DTYPE_F32; every tensor of a
 *     call has the same dtype except lse (always float32).  Pointers other than
 *     lse must be 16-byte aligned.
 *   - S % 32 == 0 (the reference's T % 32 rule, tests/test_model_repop.py:34),
 *     D in {64, 128}, H % Hkv == 0, window == 0 (full causal) or a positive
 *     multiple of 32 (ModelConfig.swa_window rule, config/schema.py:196-200).
 *   - Work is enqueued on `stream` (a hipStream_t; NULL = default stream).  No
 *     call synchronises the host, allocates device memory or keeps global state.
 *   - Return OTX_OK, or an error code with a message from otx_last_error().
 *   - Results are bit-identical to the project's arithmetic contract (serial
 *     ascending fma folds, online softmax per 32-key block, correctly rounded
 *     exp / log / division) for every launch variant, batch size and repeat.
 */
#ifndef OTX_ATTN_H
#define OTX_ATTN_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define OTX_OK 0
#define OTX_EINVAL 1 /* precondition violated (shape, dtype, alignment, size) */
#define OTX_EHIP 2   /* HIP runtime reported an error */

#define OTX_DTYPE_F32 0
#define OTX_DTYPE_BF16 1

/* Forward: o = softmax(q k^T / sqrt(D), causal[/window]) v and lse.
 * Replaces the forward of causal_flash_attention (attention_repop.py:53). */
int otx_attn_fwd(const void* q, const void* k, const void* v, void* o, float* lse, int B, int H, int Hkv, int S, int D,
                 int window, int dtype, void* stream);

/* Same as otx_attn_fwd with an explicit launch variant (0 = default; 1 and 2 use
 * other workgroup shapes and grid orders).  Every variant produces identical bits;
 * the variants exist so that launch-configuration invariance can be tested. */
int otx_attn_fwd_ex(const void* q, const void* k, const void* v, void* o, float* lse, int B, int H, int Hkv, int S,
                    int D, int window, int dtype, int variant, void* stream);

/* Device workspace (bytes) that otx_attn_bwd needs: per-row Dsum plus the fp32 dS
 * tiles of every processed 32x32 block (the atomic-free dQ reads them).  Returns 0
 * for invalid shapes.  The caller allocates it (256-byte aligned). */
size_t otx_attn_bwd_workspace_bytes(int B, int H, int Hkv, int S, int D, int window);

/* Backward: dq, dk, dv from q, k, v, the stored forward output o, lse and the
 * upstream gradient dout.  Replaces causal_flash_attention's backward
 * (causal_flash_attention_bwd_bf16_32_256, docs/MODEL_OP_DTYPE_TRACE.md:102). */
int otx_attn_bwd(const void* q, const void* k, const void* v, const void* o, const float* lse, const void* dout,
                 void* dq, void* dk, void* dv, int B, int H, int Hkv, int S, int D, int window, int dtype,
                 void* workspace, size_t workspace_bytes, void* stream);

/* otx_attn_bwd with an explicit launch variant (see otx_attn_fwd_ex).  For bf16
 * inputs the dK/dV launch of variant 0 picks one of two kernel forms by shape
 * (two key blocks per workgroup when the four-key-block grid would fill the
 * device only once) and variant 2 picks the other form, so that comparing
 * variants 0 and 2 compares both forms on every shape. */
int otx_attn_bwd_ex(const void* q, const void* k, const void* v, const void* o, const float* lse, const void* dout,
                    void* dq, void* dk, void* dv, int B, int H, int Hkv, int S, int D, int window, int dtype,
                    void* workspace, size_t workspace_bytes, int variant, void* stream);

/* otx_attn_bwd_ex split into its launches, for per-kernel timing: `stages` is a
 * bit mask of 1 = Dsum (reads o, dout), 2 = dK/dV (reads Dsum, writes the dS
 * tiles), 4 = dQ (reads the dS tiles).  Masks 1, 2, 4 issued in that order on
 * one stream (same workspace) produce exactly the result of mask 7. */
int otx_attn_bwd_stages(const void* q, const void* k, const void* v, const void* o, const float* lse,
                        const void* dout, void* dq, void* dk, void* dv, int B, int H, int Hkv, int S, int D, int window,
                        int dtype, void* workspace, size_t workspace_bytes, int variant, int stages, void* stream);

/* ---- int8-PV forward ----
 * Replaces repop.nn.flash_attention.int8pv_causal_flash_attention(q, k, v,
 * window=w) (src/pretrain/model/modules/attention_repop.py:52; kernel
 * causal_int8pv_flash_attention_fwd_bf16_32_256, docs/MODEL_OP_DTYPE_TRACE.md:80).
 * Scores and softmax statistics as otx_attn_fwd (so lse is bit-identical to
 * it); P quantized to int8 per (query, key block) with step pmax/127, V per
 * (key block, column) with step amax/127; int32 P.V; binary32 dequantization
 * into the binary32 accumulator:
 *   acc[d] = fma(RN(a_d * step_v[d]), step_p, RN(acc[d] * alpha)).
 * bf16 inputs only.  Its backward is otx_attn_bwd on the same q, k, v with this
 * forward's o and lse (the straight-through binary32 backward,
 * docs/MODEL_OP_DTYPE_TRACE.md:102). */

/* Device workspace (bytes) for the quantized V: B*Hkv*S*D int8 values (padded to
 * 256 bytes) followed by B*Hkv*(S/32)*D binary32 steps.  0 for invalid shapes. */
size_t otx_attn_fwd_int8pv_workspace_bytes(int B, int H, int Hkv, int S, int D);

int otx_attn_fwd_int8pv(const void* q, const void* k, const void* v, void* o, float* lse, int B, int H, int Hkv, int S,
                        int D, int window, int dtype, void* workspace, size_t workspace_bytes, void* stream);

/* otx_attn_fwd_int8pv with an explicit launch variant (see otx_attn_fwd_ex). */
int otx_attn_fwd_int8pv_ex(const void* q, const void* k, const void* v, void* o, float* lse, int B, int H, int Hkv,
                           int S, int D, int window, int dtype, void* workspace, size_t workspace_bytes, int variant,
                           void* stream);

/* ---- Allocation-free int8-PV forward ----
 * No counterpart in the reference: an entry point for callers that cannot
 * allocate device memory (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc).  Same operator and same bits as
 * otx_attn_fwd_int8pv_ex, but the quantized-V workspace is a fixed device array
 * inside the library (OTX_NOALLOC_SCRATCH_BYTES per GPU, held until the process
 * ends), so the call takes no workspace and allocates nothing.  Shapes whose
 * otx_attn_fwd_int8pv_workspace_bytes exceeds that size are refused with
 * OTX_EINVAL (32 MiB holds B*Hkv*S*D up to about 29.8M elements: B4 Hkv4 S4096
 * D128 needs 9 MiB).  Every call on one GPU shares that GPU's array: calls that
 * overlap on one GPU (other streams, other threads) race and must be ordered by
 * the caller.  Nothing in the array needs to start at zero (each call rewrites
 * every value it reads).  Under HIP graph capture, make one call on each device
 * before capturing: the first call on a device resolves the array's device
 * address (hipGetSymbolAddress); captured calls after it launch kernels only. */
#define OTX_NOALLOC_SCRATCH_BYTES (32u << 20)
int otx_attn_fwd_int8pv_noalloc(const void* q, const void* k, const void* v, void* o, float* lse, int B, int H,
                                int Hkv, int S, int D, int window, int dtype, int variant, void* stream);

/* ---- Score cache (bf16 inputs) ----
 * The forward can also store every score it computes, s = RN(dot(q_i, k_j) *
 * sigma) (-inf where masked), and the backward can then read them instead of
 * recomputing Q K^T: the dK/dV kernel does 6*D instead of 8*D matrix FLOPs per
 * causal pair.  Results are bit-identical to the recomputing path (the cache
 * holds exactly the scores the backward would recompute).  The cache is one
 * binary32 32x32 tile, transposed ([key][query]), per processed (query block,
 * key block) pair: B*H*sum over query blocks of the key blocks they see, 4 KiB
 * each (520 MiB at B4 H16 S2048).  The caller allocates it (16-byte aligned)
 * and keeps it from the forward to the backward, as it keeps lse.  These
 * entry points are the same operator as otx_attn_fwd / otx_attn_fwd_int8pv /
 * otx_attn_bwd (attention_repop.py:52-53, MODEL_OP_DTYPE_TRACE.md:80,102) with
 * the cache as one more saved tensor; they trade that memory for time. */
size_t otx_attn_score_cache_bytes(int B, int H, int S, int window);

/* otx_attn_fwd_ex that also writes the score cache (bf16 only). */
int otx_attn_fwd_sc(const void* q, const void* k, const void* v, void* o, float* lse, float* scache,
                    size_t scache_bytes, int B, int H, int Hkv, int S, int D, int window, int dtype, int variant,
                    void* stream);

/* otx_attn_fwd_int8pv_ex that also writes the score cache (bf16 only; the scores are
 * those of the binary32 forward, so the cache is the same). */
int otx_attn_fwd_int8pv_sc(const void* q, const void* k, const void* v, void* o, float* lse, float* scache,
                           size_t scache_bytes, int B, int H, int Hkv, int S, int D, int window, int dtype,
                           void* workspace, size_t workspace_bytes, int variant, void* stream);

/* otx_attn_bwd_stages reading the forward's score cache (bf16 only); `stages` as
 * in otx_attn_bwd_stages (7 = the whole backward). */
int otx_attn_bwd_sc(const void* q, const void* k, const void* v, const void* o, const float* lse, const void* dout,
                    void* dq, void* dk, void* dv, const float* scache, size_t scache_bytes, int B, int H, int Hkv,
                    int S, int D, int window, int dtype, void* workspace, size_t workspace_bytes, int variant,
                    int stages, void* stream);

/* ---- Token embedding ----
 * Replaces repop.nn.embedding.Embedding (src/pretrain/model/modules/
 * embedding_repop.py:33-40; docs/MODEL_OP_DTYPE_TRACE.md:75,106).  Forward:
 * out[p] = weight[ids[p]] (NaN rows for ids outside [0, V)).  Backward:
 * grad_weight[v][d] = fold over positions p ascending with ids[p] == v of
 * grad_out[p][d] (binary32 additions from +0), in the weight dtype; rows of
 * absent ids are +0, ids outside [0, V) are skipped.  weight / grad_weight are
 * [V][D], out / grad_out [npos][D], ids int64 [npos]; D a multiple of 8 (bf16)
 * or 4 (binary32).  The backward's workspace (256-byte aligned) holds the sort;
 * its size query needs a visible device. */
size_t otx_embedding_bwd_workspace_bytes(long npos, int V);
int otx_embedding_fwd(const int64_t* ids, const void* weight, void* out, long npos, int V, int D, int dtype,
                      void* stream);
int otx_embedding_bwd(const int64_t* ids, const void* grad_out, void* grad_weight, long npos, int V, int D, int dtype,
                      void* workspace, size_t workspace_bytes, void* stream);

/* ---- Fused cross-entropy + z-loss ----
 * Replaces pretrain.model.fused_loss.fused_ce_z_loss / _FusedCEZLoss
 * (src/pretrain/model/fused_loss.py:40-120) and the logsumexp of _z_loss_lse
 * (src/pretrain/model/z_loss.py:53-66): ce = mean(lse - logit[label]),
 * z = coeff * mean(lse^2) over N rows of V logits (bf16 or binary32, row-major),
 * labels int64.  Reductions are the recursive chunk-32 fold; exp/log correctly
 * rounded; the backward follows fused_loss.py:70-104 operation by operation.
 * Limits: N <= 262144; V <= 131072.  A label outside
 * [0, V) makes ce NaN.  stats is [5][N] binary32 (m, Z, lse, d, q) written by
 * the forward and read by the backward; loss is [2] (ce, z) on the device. */
int otx_ce_zloss_fwd(const void* logits, const int64_t* labels, long N, int V, int dtype, double coeff, float* stats,
                     float* loss, void* stream);

/* grad_logits = d(gce * ce + gz * z) / d logits in the logits dtype; grad_loss is
 * the device pair (gce, gz). */
int otx_ce_zloss_bwd(const void* logits, const int64_t* labels, const float* stats, const float* grad_loss, long N,
                     int V, int dtype, double coeff, void* grad_logits, void* stream);

/* ---- Decoder-layer operators (BASELINE configuration 5 around the attention) ----
 *
 * bf16 GEMM with a serial binary32 fold: C[i][j] = RN(fold_r fma(A(i,r), B(j,r))),
 * r ascending from +0, A(i,r) = A[i*a_i + r*a_r], B(j,r) = B[j*b_j + r*b_r]
 * (element strides; for each operand one stride is 1 and the other a multiple of
 * 8), C[i*ldc + j] as bf16 (out_dtype OTX_DTYPE_BF16, RNE) or binary32.  M and N
 * multiples of 128, R of 32.  Replaces repop.nn.linear.Linear forward and
 * backward (src/pretrain/model/modules/_linear.py:31-65;
 * docs/MODEL_OP_DTYPE_TRACE.md:82,100). */
int otx_gemm_bf16(const void* A, long a_i, long a_r, const void* B, long b_j, long b_r, void* C, long ldc, int M,
                  int N, int R, int out_dtype, void* stream);

/* The same GEMM with an explicit tile form: variant 0 chooses (as
 * otx_gemm_bf16 does), 1 takes 128 x 128 workgroup tiles, 2 takes 128 x 64,
 * 3 takes 64 x 64.  The bytes are identical for every variant (each output is
 * one serial fold); the variants exist so that tests can compare the forms. */
int otx_gemm_bf16_ex(const void* A, long a_i, long a_r, const void* B, long b_j, long b_r, void* C, long ldc, int M,
                     int N, int R, int out_dtype, int variant, void* stream);

/* RMSNorm over the last dimension D (multiple of 32, <= 8192) of `rows` rows:
 * y = RN(RN(x * rstd) * w), rstd[row] = rsqrt(RN(RN(ss / D) + eps)) with ss the
 * chunk-32 fold of x*x.  Replaces repop.nn.rmsnorm.rms_norm
 * (src/pretrain/model/modules/norm_repop.py:19-22). */
int otx_rmsnorm_fwd(const void* x, const void* w, void* y, float* rstd, long rows, int D, float eps, int dtype,
                    void* stream);
/* Workspace of otx_rmsnorm_bwd: the per-32-row partials of dw (0 if rows % 32);
 * 16-byte aligned. */
size_t otx_rmsnorm_bwd_workspace_bytes(long rows, int D);
/* RMSNorm backward: dx (dtype) and dw (binary32, fold over rows in chunks of 32). */
int otx_rmsnorm_bwd(const void* x, const void* w, const float* rstd, const void* dy, void* dx, float* dw, long rows,
                    int D, int dtype, void* workspace, size_t workspace_bytes, void* stream);

/* SiLU y = RN(x / RN(1 + exp(-x))) with correctly rounded exp, and its backward
 * dx = RN(dy * RN(s * RN(1 + RN(x * RN(1 - s))))), s = RN(1 / RN(1 + exp(-x))).
 * Replaces repop.nn.activations.silu (src/pretrain/model/modules/ffn_repop.py). */
int otx_silu_fwd(const void* x, void* y, long n, int dtype, void* stream);
int otx_silu_bwd(const void* x, const void* dy, void* dx, long n, int dtype, void* stream);

/* SwiGLU over rows of gu = [gate | up] (each half F wide, F a multiple of 8,
 * 16-byte aligned rows): h = RN(put(SiLU(gate)) * up), SiLU as in otx_silu_fwd,
 * put() the rounding to dtype.  Backward: dgu = [put(RN(put(RN(dh * up)) * g)) |
 * put(RN(dh * put(SiLU(gate))))] with g the SiLU derivative of otx_silu_bwd.
 * Replaces the composition `gate, up = w_gate_up(x).chunk(2, dim=-1);
 * silu(gate) * up` of src/pretrain/model/modules/ffn_repop.py:52-54 (torch's
 * elementwise product and chunk/cat backward) with one pass each way. */
int otx_swiglu_fwd(const void* gu, void* h, long rows, int F, int dtype, void* stream);
int otx_swiglu_bwd(const void* gu, const void* dh, void* dgu, long rows, int F, int dtype, void* stream);

/* Rotary embedding into the attention layout: x [B, T, H, D] -> y [B, H, T, D]
 * with y[2i] = put(RN(RN(e c) - RN(o s))), y[2i+1] = put(RN(RN(e s) + RN(o c))),
 * (e, o) = x[2i], x[2i+1], (c, s) = cos/sin[t][i] (binary32 [T, D/2]).  The
 * backward maps dy [B, H, T, D] to dx [B, T, H, D] with torch autograd's bytes
 * for that chain (each branch's product rounded to dtype, the two branches of
 * a slice summed in dtype, a -0 sum stored as +0).  D a multiple of 8.
 * Replaces apply_rope (src/pretrain/model/modules/rope.py:103-125) followed by
 * transpose(1, 2).contiguous() (attention_repop.py:143-149). */
int otx_rope_heads_fwd(const void* x, const float* cos, const float* sin, void* y, int B, int T, int H, int D,
                       int dtype, void* stream);
int otx_rope_heads_bwd(const void* dy, const float* cos, const float* sin, void* dx, int B, int T, int H, int D,
                       int dtype, void* stream);
/* x [B, X, Y, D] -> y [B, Y, X, D] (D a multiple of 8): the v transpose and the
 * output's transpose(1, 2).contiguous() of attention_repop.py:150,155, and
 * their backward. */
int otx_swap_heads(const void* x, void* y, int B, int X, int Y, int D, int dtype, void* stream);

/* Softmax scale used by the kernels: RN_binary32(1 / sqrt(D)). */
float otx_softmax_scale(int D);

/* JSON description of the build ({"backends": ["rocm"], ...}); the analogue of
 * repop.build_info() consulted by the audit-replay backend guard
 * (src/pretrain/cli/audit_replay.py:1114-1141,1508-1511). */
const char* otx_build_info(void);

/* Message of the last failed call on this thread. */
const char* otx_last_error(void);

/* Diagnostics without a reference counterpart: checks of the hardware facts the
 * kernels depend on.
 * otx_selftest_mfma: one v_mfma_f32_32x32x1_2b_f32 per group of inputs
 *   a[g][64], b[g][64], c[g][32][64] -> out[g][32][64] (device pointers).
 * otx_selftest_math: partial[blk] = sum mod 2^64 over the blocks' share of the
 *   binary32 bit patterns [lo, lo+count) of mix(x, f(x)), f = exp (which 0) or
 *   log (which 1), evaluated by the kernels' own exp / log, the kernels' batched
 *   exp (2: checked, 3: arguments <= 0), the kernels' binary32 -> bf16
 *   rounding (4, f(x) = the bf16 value as a binary32 bit pattern), or the
 *   int8-PV quantizer's rounding to an unsigned byte (5, f(x) = that byte as a
 *   binary32; meaningful on [+0, 128)). */
int otx_selftest_mfma(const float* a, const float* b, const float* c, float* out, int groups, void* stream);
/* otx_selftest_mfma16: one v_mfma_f32_16x16x1_4b_f32 per group (the dK/dV kernel's
 * score and dP chains on 32x32 tiles): a, b [groups][64]; c, out [groups][16][64]. */
int otx_selftest_mfma16(const float* a, const float* b, const float* c, float* out, int groups, void* stream);
int otx_selftest_math(int which, uint64_t lo, uint64_t count, uint64_t* partial, int nblocks, void* stream);
/* otx_selftest_mfma_bf16: one bf16 matrix instruction per group with raw
 *   operand registers in the instruction's lane order (kind 0: 32x32x4_2b,
 *   1: 32x32x8, 2: 32x32x16, 3: 16x16x16, 4: 16x16x32); a/b [g][64][4 or 8] bf16
 *   bits, c/out [g][64][32, 16 or 4] floats.  Used to establish whether a
 *   multi-product instruction accumulates like a serial fma chain. */
int otx_selftest_mfma_bf16(int kind, const uint16_t* a, const uint16_t* b, const float* c, float* out, int groups,
                           void* stream);
/* otx_selftest_mfma_i8: one v_mfma_i32_32x32x32_i8 per group, raw registers:
 *   a/b [g][64][16] int8, c/out [g][64][16] int32 (the int8-PV operand layout). */
int otx_selftest_mfma_i8(const int8_t* a, const int8_t* b, const int* c, int* out, int groups, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* OTX_ATTN_H */
