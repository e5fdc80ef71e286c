/*
 * kernelforge_amd C ABI.
 *
 * Plain C entry points for the three operator hot paths of KernelForge
 * (RMSNorm, SANA ReLU linear attention with its rotary embedding,
 * FlashAttention forward / JVP / backward), implemented as hand-written HIP
 * kernels for gfx950 (MI355X).
 *
 * Conventions shared by every entry point:
 *   - Pointers are device pointers owned by the caller.  The library never
 *     allocates device memory; SANA's cross-split partials and the FA
 *     backward's per-row statistics live in caller-supplied workspaces whose
 *     sizes are given by kf_linattn_workspace_bytes and
 *     kf_fa_bwd_workspace_bytes.
 *   - Tensors are dense and row-major (the innermost dimension is contiguous)
 *     in the layouts documented per function.
 *   - `stream` is a hipStream_t (NULL = the default stream).  Launches are
 *     asynchronous, never synchronise the device and never call hipMalloc,
 *     so every entry point may be captured into a HIP graph.
 *   - The return value is KF_OK (0) on success or a kf_status code;
 *     kf_last_error() then returns a message for the calling thread.
 */
#ifndef KERNELFORGE_AMD_H
#define KERNELFORGE_AMD_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define KF_ABI_VERSION 1

typedef void* kf_stream_t; /* hipStream_t */

typedef enum kf_dtype {
    KF_F32 = 0,
    KF_F16 = 1,
    KF_BF16 = 2
} kf_dtype;

typedef enum kf_status {
    KF_OK = 0,
    KF_E_INVALID = 1,     /* bad shape, dtype, pointer or argument value */
    KF_E_UNSUPPORTED = 2, /* a valid request this build has no kernel for */
    KF_E_WORKSPACE = 3,   /* workspace missing or too small */
    KF_E_HIP = 4,         /* a HIP runtime call or kernel launch failed */
    KF_E_INCOMPLETE = 5   /* a finished launch reported an incomplete result (kf_linattn_check) */
} kf_status;

/* ABI version of the loaded library (KF_ABI_VERSION at build time). */
int kf_abi_version(void);

/* Static name of a kf_status value. */
const char* kf_status_string(int status);

/* Message describing the most recent failure on the calling thread. */
const char* kf_last_error(void);

/* ------------------------------------------------------------------ */
/* RMSNorm                                                             */
/* ------------------------------------------------------------------ */

/*
 * y[r, :] = dt( float(dt(x[r, :] * inv)) * float(weight[:]) ),
 * inv = 1 / sqrt(sum_c x[r, c]^2 / dim + eps), accumulated in fp32,
 * where dt() rounds to the storage dtype (round-to-nearest-even).
 *
 * Replaces the compiled callable returned by
 *   rms_norm(batch, seq_len, dim, eps, dtype)   rmsnorm/custom.py:15-73
 * whose rounding points follow RMSNorm.forward   rmsnorm/original.py:38,51-52.
 *
 * x, y: [rows, dim]; weight: [dim]; all of `dtype`.  rows >= 0, dim >= 1.
 */
int kf_rmsnorm_fwd(const void* x, const void* weight, void* y,
                   int64_t rows, int64_t dim, float eps, int dtype,
                   kf_stream_t stream);

/*
 * kf_rmsnorm_fwd on rows that start every ld_x (input) and ld_y (output)
 * elements, ld >= dim.  y may equal x with ld_y == ld_x (in place).  Used to
 * normalise the q and k parts of a packed qkv[B, N, 3, C] buffer in place:
 * rows = B*N, dim = C, ld = 3*C, x = y = qkv + part*C.  Replaces the q_norm /
 * k_norm RMSNorm modules of LiteLA.forward (SANA_LinearAttention/
 * original.py:91-94, 129-130), which normalise over the C channels of each
 * token; the arithmetic is kf_rmsnorm_fwd's.
 */
int kf_rmsnorm_fwd_strided(const void* x, const void* weight, void* y,
                           int64_t rows, int64_t dim, int64_t ld_x, int64_t ld_y,
                           float eps, int dtype, kf_stream_t stream);

/*
 * kf_rmsnorm_fwd with torch's type promotion between x and the weight:
 * y = y_dtype( float(x_dtype(x * inv)) * float(weight) ), where y_dtype must
 * be promote(x_dtype, w_dtype) (equal types stay, any mix of fp32, fp16 and
 * bf16 gives KF_F32).  Replaces RMSNorm.forward (rmsnorm/original.py:51-52)
 * when the module's weight keeps its default fp32 dtype (original.py:25) and
 * x is bf16 or fp16: `output * self.weight` then returns fp32.
 * x: [rows, dim] of x_dtype; weight: [dim] of w_dtype; y: [rows, dim] of y_dtype.
 */
int kf_rmsnorm_fwd_mixed(const void* x, const void* weight, void* y,
                         int64_t rows, int64_t dim, float eps,
                         int x_dtype, int w_dtype, int y_dtype, kf_stream_t stream);

/* Workspace bytes kf_rmsnorm_bwd needs (fp32 weight-gradient partials). */
int64_t kf_rmsnorm_bwd_workspace_bytes(int64_t rows, int64_t dim);

/*
 * Gradients of kf_rmsnorm_fwd_mixed for the output gradient dy (of the
 * promoted dtype), with the casts of RMSNorm.forward taken as identities,
 * which is how torch's autograd differentiates rmsnorm/original.py:38, 51-52:
 *   g  = float(x_dtype(dy * weight)),   n = x_dtype(x * inv),
 *   dx = x_dtype(inv * g - x * inv^3 * sum(g * x) / dim),
 *   dweight = w_dtype(sum over rows of dy * n)   (fp32 sum).
 * dx: [rows, dim] of x_dtype; dweight: [dim] of w_dtype.  The weight
 * gradient is summed over rows in a fixed order (deterministic, no atomics).
 * workspace: at least kf_rmsnorm_bwd_workspace_bytes(rows, dim) bytes.
 */
int kf_rmsnorm_bwd(const void* x, const void* weight, const void* dy, void* dx,
                   void* dweight, void* workspace, int64_t workspace_bytes,
                   int64_t rows, int64_t dim, float eps, int x_dtype, int w_dtype,
                   kf_stream_t stream);

/*
 * Weight-free fp32 RMSNorm with the two-scan baseline's semantics:
 * b[r, :] = a[r, :] / sqrt(sum_c a[r, c]^2 / n + eps).
 *
 * Replaces rms_norm(A, blk_m) (the TileLang "original" baseline,
 * rmsnorm/original.py:55-78, which hard-codes eps = 1e-12).
 * a, b: fp32 [rows, n].
 */
int kf_rmsnorm_noweight_f32(const float* a, float* b, int64_t rows, int64_t n,
                            float eps, kf_stream_t stream);

/* ------------------------------------------------------------------ */
/* SANA ReLU linear attention                                          */
/* ------------------------------------------------------------------ */

/*
 * Sequence split count the host dispatcher uses for a shape (>= 1).
 * Mirrors the role of the split heuristic in qkv_attn_matmul
 * (SANA_LinearAttention/custom.py:355-368), re-derived for 256 CUs.
 */
int64_t kf_linattn_default_splits(int64_t batch, int64_t heads, int64_t dim,
                                  int64_t seq_len);

/*
 * Workspace bytes kf_linattn_fwd needs for `splits` sequence splits: a fixed
 * region of control words (arrival counters of the fused kernel), then the
 * fp32 split partials [B, H, splits, D+1, D] and the reduced states.
 */
int64_t kf_linattn_workspace_bytes(int64_t batch, int64_t heads, int64_t dim,
                                   int64_t splits);

/*
 * Prepare a new SANA workspace: zeroes its control words on `stream`.  A
 * workspace's control words must be zero before its first kf_linattn_fwd
 * call (memory from a zeroing allocator needs no init); every call leaves
 * them zero again, so a workspace is initialised once and then reused for
 * any shape it is large enough for.  Calls sharing a workspace must be
 * ordered (one stream, or synchronised streams).
 */
int kf_linattn_workspace_init(void* workspace, int64_t workspace_bytes, kf_stream_t stream);

/*
 * out[b, n, h*D + r] = sum_c S[r][c] relu(q)[n,c] / (sum_c z[c] relu(q)[n,c] + eps)
 * with S = sum_n v[n,:]^T relu(k)[n,:] and z = sum_n relu(k)[n,:] per (b, h),
 * accumulated in fp32 over `splits` sequence splits and reduced across
 * splits in a fixed order (deterministic, no atomics on data).
 *
 * Replaces run(qkv) returned by
 *   qkv_attn_matmul(batch, heads, dim, seq_len, eps, dtype, output_dtype,
 *                   reduce_splits)          SANA_LinearAttention/custom.py:340-388
 * with the arithmetic of LiteLA.attn_matmul SANA_LinearAttention/original.py:99-117
 * (fp32_attention semantics) on the packed layout of
 * LiteLA.forward                          SANA_LinearAttention/original.py:124-134.
 *
 * qkv: [batch, seq_len, 3, heads*dim] of in_dtype (KF_BF16 or KF_F16, or KF_F32);
 * out: [batch, seq_len, heads*dim] of out_dtype (KF_F32, KF_F16 or KF_BF16).
 * dim must be 32 for the MFMA kernel in this build (one launch: the split
 * workgroups of a (batch, head pair) meet at a counter in the workspace's
 * control words); other head dims and fp32 input take a three-launch VALU
 * path.  splits <= 0 selects kf_linattn_default_splits; any positive count is
 * accepted and used as an upper bound: it is cut to the sequence length and,
 * for the fused kernel, to the number of its workgroups the device holds at
 * once (occupancy per CU x CUs: 256 on MI355X for fp32 output), because a
 * group's split workgroups wait for each other and must be resident
 * together.  Each split then takes whole 128-token tiles (32 on the VALU
 * path), so fewer splits than requested may run.
 * workspace: at least kf_linattn_workspace_bytes bytes for the requested
 * splits, 256-byte aligned, control words zero on entry
 * (kf_linattn_workspace_init); they are zero again on return.  The split
 * workgroups of a group wait for each other a bounded time (2^20 polls,
 * about a second); should other work on the device keep some of them from
 * being resident that long, the ones that stop waiting set the workspace's
 * error word (the second 32-bit control word) to 1 and write NaN for their
 * tokens instead of a result.  kf_linattn_check reports and clears it.
 */
int kf_linattn_fwd(const void* qkv, void* out, void* workspace,
                   int64_t workspace_bytes, int64_t batch, int64_t seq_len,
                   int64_t heads, int64_t dim, int64_t splits, float eps,
                   int in_dtype, int out_dtype, kf_stream_t stream);

/*
 * LiteLA.attn_matmul(q, k, v)               SANA_LinearAttention/original.py:99-117
 * for q, k, v that are the views LiteLA.forward makes of one packed buffer
 * (original.py:122-134): the arithmetic of kf_linattn_fwd, with the result
 * written as attn_matmul returns it, fp32 out[batch, heads, dim, seq_len]
 * (contiguous; element (b, h, r, n) at ((b*heads + h)*dim + r)*seq_len + n).
 * qkv, workspace and splits as for kf_linattn_fwd (in_dtype KF_BF16, KF_F16
 * or KF_F32; head dim 32 with 16-bit input runs the fused MFMA kernel).
 */
int kf_linattn_attn_matmul(const void* qkv, float* out, void* workspace,
                           int64_t workspace_bytes, int64_t batch, int64_t seq_len,
                           int64_t heads, int64_t dim, int64_t splits, float eps,
                           int in_dtype, kf_stream_t stream);

/*
 * Status of the SANA launches that used `workspace` since its last check:
 * waits for `stream` (the one exception to the no-synchronisation rule, so
 * not for use under graph capture), reads the workspace's error word and
 * returns KF_OK, or KF_E_INCOMPLETE with a message when a group wait gave
 * up (those outputs hold NaN) or the control words were not zero on entry;
 * in that case the control words are cleared for the next call.
 */
int kf_linattn_check(void* workspace, int64_t workspace_bytes, kf_stream_t stream);

/*
 * Largest scratch, in bytes, that kf_linattn_fwd_noalloc can use: the size
 * of its static device array (16 MiB), which must hold
 * kf_linattn_workspace_bytes(batch, heads, dim, splits).
 */
int64_t kf_linattn_noalloc_max_bytes(void);

/*
 * kf_linattn_fwd without a workspace argument and without any allocation:
 * the split partials and reduced states live in a static device array of
 * kf_linattn_noalloc_max_bytes() bytes that each GPU holds until the process
 * ends.  No counterpart in the reference; it exists for callers that cannot
 * allocate (code under HIP graph capture, serving loops, harnesses that
 * forbid hipMalloc).  Same arguments, kernels and results as kf_linattn_fwd
 * with the same splits (splits <= 0 selects kf_linattn_default_splits).
 * Returns KF_E_WORKSPACE, before any device work, when the request needs more
 * scratch than the array holds (pass fewer splits or use kf_linattn_fwd).
 * Every call on one GPU shares that GPU's array, so calls that overlap on
 * one GPU (concurrent streams or threads) race and must be serialised by the
 * caller.  The array keeps the last call's contents; its control words start
 * at zero (the first call on a device zeroes them with a fill kernel on the
 * caller's stream) and every call leaves them zero.
 */
int kf_linattn_fwd_noalloc(const void* qkv, void* out, int64_t batch, int64_t seq_len,
                           int64_t heads, int64_t dim, int64_t splits, float eps,
                           int in_dtype, int out_dtype, kf_stream_t stream);

/*
 * kf_linattn_check for the current device's static scratch, the status of
 * the kf_linattn_fwd_noalloc calls on it.  No counterpart in the reference;
 * for the callers of kf_linattn_fwd_noalloc.
 */
int kf_linattn_noalloc_check(kf_stream_t stream);

/*
 * Rotary position embedding, in place on the q and k parts of a packed
 * qkv[batch, seq_len, 3, heads*dim] buffer (v untouched): within each head,
 * channels (2i, 2i+1) rotate as a complex pair by the angle whose cosine and
 * sine are cos[n][2i..2i+1], sin[n][2i..2i+1] (fp32 [seq_len][dim]):
 *   out[2i] = x[2i] cos - x[2i+1] sin,  out[2i+1] = x[2i+1] cos + x[2i] sin,
 * products and sum rounded in fp32 and the result in the storage type
 * (dtype KF_F32/F16/BF16).  dim % 8 == 0, qkv 16-byte aligned.  Replaces
 * apply_rotary_emb(.., use_real_unbind_dim=-2) on q and k in LiteLA.forward
 * (SANA_LinearAttention/original.py:14-58, 136-138).
 */
int kf_rope_packed(void* qkv, const float* cos, const float* sin,
                   int64_t batch, int64_t seq_len, int64_t heads, int64_t dim,
                   int dtype, kf_stream_t stream);

/* ------------------------------------------------------------------ */
/* SANA projections                                                    */
/* ------------------------------------------------------------------ */

#define KF_WEIGHT_NK 0 /* weight[n][k]: torch.nn.Linear.weight          */
#define KF_WEIGHT_KN 1 /* weight_t[k][n]: the reference's prepacked WeightT */

/*
 * y[i, j] = dt( sum_c x[i, c] * W[j, c] (+ bias[j]) ), fp32 accumulation,
 * the bias (when not NULL) added in fp32, one round-to-nearest-even to the
 * storage dtype at the end.
 *
 * Replaces the TileLang kernels
 *   _qkv_projection(batch, seq_len, channels, dtype)   SANA_LinearAttention/custom.py:23-85
 *     (no bias, WeightT [C, 3C]), and
 *   _output_projection(batch, seq_len, channels, dtype) SANA_LinearAttention/custom.py:457-523
 *     (bias, WeightT [C, C]),
 * with m = batch * seq_len rows.
 *
 * x: [m, ldx] (first k columns used); y: [m, ldy] (first n columns written);
 * weight: dense [n, k] (KF_WEIGHT_NK) or [k, n] (KF_WEIGHT_KN); bias: [n] or
 * NULL; all of `dtype` (KF_BF16 or KF_F16).  n % 8 == 0, k % 8 == 0,
 * ldx % 8 == 0, ldy % 4 == 0; x and weight 16-byte aligned, y and bias 8-byte
 * aligned.  m == 0 is a no-op.
 */
int kf_proj_gemm(const void* x, const void* weight, const void* bias, void* y,
                 int64_t m, int64_t n, int64_t k, int64_t ldx, int64_t ldy,
                 int weight_layout, int dtype, kf_stream_t stream);

/*
 * LiteLA attention with the QKV projection fused in, up to (not including)
 * the output projection, head dim 32:
 *   q, k, v = dt(x W^T + bias)       (W = qkv_weight [3C, C], rows q | k | v)
 *   out[b, t, 32h + r] = dt( sum_c S[r][c] relu(q[t][32h+c])
 *                            / (sum_c z[c] relu(q[t][32h+c]) + eps) ),
 *   S[r][c] = sum_t v[t][32h+r] relu(k[t][32h+c]),  z[c] = sum_t relu(k[t][32h+c])
 * with q, k, v never written to memory.  C = 32 * heads.
 *
 * Replaces the fused projection kernels of GroupedFull64QOutLiteLA
 *   grouped_full64_kv_vk_producer / partial_reduce_joint_qout
 *     SANA_LinearAttention/custom.py:606-809
 * (there for B=1, N=1024, C=1152 only) for any batch, length and head count.
 *
 * x, out: [batch, seq_len, C]; qkv_weight: [3C, C]; qkv_bias: [3C] or NULL;
 * all of `dtype` (KF_BF16 or KF_F16); x, qkv_weight and out 16-byte aligned.
 * dim must be 32 (KF_E_UNSUPPORTED otherwise).  Three launches: k/v
 * projection with the per-(batch, head, 256-token tile) state partials, their
 * fixed-order sum (deterministic), q projection with the output.  The
 * workspace holds the partials and states: at least
 * kf_litela_fused_workspace_bytes(batch, seq_len, heads) bytes, 256-byte
 * aligned, no initialisation needed.  Calls that share a workspace must not
 * overlap.
 */
int64_t kf_litela_fused_workspace_bytes(int64_t batch, int64_t seq_len, int64_t heads);
int kf_litela_fused_attn(const void* x, const void* qkv_weight, const void* qkv_bias, void* out,
                         void* workspace, int64_t workspace_bytes,
                         int64_t batch, int64_t seq_len, int64_t heads, int64_t dim,
                         float eps, int dtype, kf_stream_t stream);

/* ------------------------------------------------------------------ */
/* FlashAttention forward and JVP                                      */
/* ------------------------------------------------------------------ */

/*
 * Layouts: q, tq, o, to: [B, Nq, Hq, D]; k, v, tk, tv: [B, Nk, Hkv, D];
 * lse: fp32 [B, Hq, Nq], natural log.  dtype is KF_F16 or KF_BF16.
 * Hq % Hkv == 0 (GQA/MQA), D % 8 == 0 and D <= 256.  causal selects the
 * bottom-right aligned mask col <= row + Nk - Nq.  Rows with no valid key
 * produce o = 0, to = 0 and lse = +inf.
 */

/*
 * O and LSE.  Replaces the forward FlashAttentionFunction.forward calls
 * (flash_attention_jvp/custom.py:229-238, flash-attn _flash_attn_forward).
 */
int kf_fa_fwd(const void* q, const void* k, const void* v, void* o, float* lse,
              int64_t B, int64_t Nq, int64_t Nk, int64_t Hq, int64_t Hkv,
              int64_t D, float scale, int causal, int dtype, kf_stream_t stream);

/*
 * tO from the cached LSE (standalone JVP, no forward launch):
 *   P = exp(scale*q k^T - lse),  tS = scale*(tq k^T + q tk^T),  H = P*tS,
 *   tO = P tv + H v - rowsum(H) * O.
 * O is the cached `o`, as in the reference, while |rowsum(H)/l| * max(max|O|,
 * 1) <= 1 on every row of a 128-row tile (l = rowsum of the 16-bit P); a tile
 * past that bound, where rowsum(H) could amplify o's rounding beyond about a
 * fifth of the bf16 tolerance, is redone by a second launch that recomputes
 * O in fp32 from the same P (U = P v) and does not read `o`.  Two launches,
 * the second exits at once for tiles under the bound.
 * Any of tq, tk, tv may be NULL, meaning a zero tangent.
 * Replaces kernelforge::flash_attention_jvp / _attention_jvp_kernel
 * (flash_attention_jvp/custom.py:12-120, 137-152).
 */
int kf_fa_jvp(const void* q, const void* k, const void* v,
              const void* tq, const void* tk, const void* tv,
              const void* o, const float* lse, void* to,
              int64_t B, int64_t Nq, int64_t Nk, int64_t Hq, int64_t Hkv,
              int64_t D, float scale, int causal, int dtype, kf_stream_t stream);

/*
 * Fused single pass: O, LSE and tO in one scan over the K/V tiles with the
 * online recurrences of flash-attention-jvp-derivation.md:388-558
 * (states m, l, U, r, G).  The reference implements this path as two
 * launches (flash-attn forward + _attention_jvp_kernel,
 * flash_attention_jvp/custom.py:229-276); this entry point replaces both.
 * Any of tq, tk, tv may be NULL (zero tangent).
 */
int kf_fa_fwd_jvp(const void* q, const void* k, const void* v,
                  const void* tq, const void* tk, const void* tv,
                  void* o, float* lse, void* to,
                  int64_t B, int64_t Nq, int64_t Nk, int64_t Hq, int64_t Hkv,
                  int64_t D, float scale, int causal, int dtype,
                  kf_stream_t stream);

/*
 * Workspace bytes kf_fa_bwd needs (fp32 per-row statistics, rows padded to
 * the kernel's query tile); -1 for an invalid shape.
 */
int64_t kf_fa_bwd_workspace_bytes(int64_t B, int64_t Nq, int64_t Hq, int64_t D);

/*
 * Gradients dq, dk, dv (layouts of q, k, v) of the attention output for the
 * output cotangent dout [B, Nq, Hq, D], from the forward's o and natural-log
 * lse (P = exp(scale*q k^T - lse), recomputed; +inf rows contribute 0):
 *   Delta = rowsum(dout * o),  dS = P * (dout v^T - Delta),
 *   dq = scale*dS k,  dk = scale*dS^T q,  dv = P^T dout,
 * dk/dv summed over the query heads of each KV head.  Deterministic (no
 * atomics).  workspace: at least kf_fa_bwd_workspace_bytes, device memory.
 * Replaces flash-attn's _flash_attn_backward as called by
 * FlashAttentionFunction.backward (flash_attention_jvp/custom.py:252-267).
 */
int kf_fa_bwd(const void* q, const void* k, const void* v, const void* o,
              const float* lse, const void* dout, void* dq, void* dk, void* dv,
              void* workspace, int64_t workspace_bytes,
              int64_t B, int64_t Nq, int64_t Nk, int64_t Hq, int64_t Hkv,
              int64_t D, float scale, int causal, int dtype, kf_stream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* KERNELFORGE_AMD_H */
