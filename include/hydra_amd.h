/*
 * hydra_amd.h -- C ABI of the MI355X (gfx950) hot path of HYDRA.
 *
 * Every entry point takes plain device pointers, sizes and strides (in
 * elements), and a HIP stream passed as `void*` (a hipStream_t; NULL is the
 * null stream).  Nothing here allocates device memory except where a comment
 * says so, nothing synchronises the host, and every launch goes on `stream`.
 *
 * Return value: 0 on success, otherwise one of HYDRA_ERR_*; the message for
 * the last failure on the calling thread is returned by hydra_last_error().
 *
 * Each declaration names the reference interface it replaces
 * (paths relative to the mcpirate17/HYDRA tree).
 */
#ifndef HYDRA_AMD_H
#define HYDRA_AMD_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- status codes and element types ------------------------------------ */
#define HYDRA_OK            0
#define HYDRA_ERR_ARG       1  /* bad shape / stride / dtype / flag          */
#define HYDRA_ERR_LAUNCH    2  /* a HIP launch or runtime call failed        */
#define HYDRA_ERR_UNSUPPORTED 3 /* valid request this build does not cover   */

#define HYDRA_F32  0
#define HYDRA_BF16 1
#define HYDRA_F16  2

/* Message of the last failure on this thread ("" if none). */
const char* hydra_last_error(void);
/* ABI version (major*10000 + minor*100 + patch). */
int hydra_abi_version(void);

/* ---- fused element ops (hydra/kernels/fused_ops.py) -------------------- */

/* RMSNorm forward: y[r,:] = x[r,:] * rsqrt(mean(x[r,:]^2) + eps) * w, with the
 * sum of squares and the products in fp32, one rounding into `dtype`.
 * Replaces fused_rms_norm (hydra/kernels/fused_ops.py:1114-1132) and its
 * kernel _fused_rms_norm_kernel (fused_ops.py:969-1007).
 * x: [rows, dim] with row stride x_rs; w: [dim] (same dtype);
 * y: [rows, dim] with row stride y_rs. */
int hydra_rms_norm_fwd(const void* x, const void* w, void* y,
                       int64_t rows, int64_t dim, int64_t x_rs, int64_t y_rs,
                       float eps, int dtype, void* stream);

/* RoPE forward on interleaved pairs:
 *   o[..,2i]   = x[..,2i]*cos[s,i] - x[..,2i+1]*sin[s,i]
 *   o[..,2i+1] = x[..,2i]*sin[s,i] + x[..,2i+1]*cos[s,i]
 * Replaces fused_rope (hydra/kernels/fused_ops.py:240-258) and
 * _fused_rope_triton / _fused_rope_kernel (fused_ops.py:185-297).
 * x: [B,H,S,D] with element strides xs[4] (xs[3] must be 1);
 * cos/sin: [S, D/2] with row stride cs_rs (element stride 1), type cs_dtype;
 * out: contiguous [B,H,S,D] in `dtype`. */
int hydra_rope_fwd(const void* x, const void* cos, const void* sin, void* out,
                   int64_t B, int64_t H, int64_t S, int64_t D,
                   const int64_t* xs, int64_t cs_rs, int dtype, int cs_dtype,
                   void* stream);

/* SwiGLU activation: out = silu(gate) * up, fp32 math, one rounding.
 * Replaces fused_swiglu (hydra/kernels/fused_ops.py:808-820) and
 * _fused_swiglu_kernel (fused_ops.py:703-725).  gate/up may be the two
 * halves of one [rows, 2*hidden] tensor (row strides g_rs/u_rs);
 * out: [rows, hidden] with row stride o_rs. */
int hydra_swiglu_fwd(const void* gate, const void* up, void* out,
                     int64_t rows, int64_t hidden,
                     int64_t g_rs, int64_t u_rs, int64_t o_rs,
                     int dtype, void* stream);

/* QK L2-normalisation + scale:
 *   q_out = q * rsqrt(sum(q^2) + 1e-8) * scale
 *   k_out = k * rsqrt(sum(k^2) + 1e-8) * scale * temperature
 * Replaces fused_qk_norm (hydra/kernels/fused_ops.py:474-493) and
 * _fused_qk_norm_kernel (fused_ops.py:323-369).  q: [q_rows, hd],
 * k: [k_rows, hd], all contiguous, same dtype. */
int hydra_qk_norm_fwd(const void* q, const void* k, void* q_out, void* k_out,
                      int64_t q_rows, int64_t k_rows, int64_t hd,
                      float scale, float temperature, int dtype, void* stream);

/* ---- backward of the fused ops ---------------------------------------- */
/* Each follows the reference's PyTorch backward (fp32 math, every gradient
 * clamped to [-100, 100], one rounding into `dtype`), which its Triton
 * backward kernel reproduces. */

/* RMSNorm backward.  Per row r = rsqrt(mean(x^2) + eps), xn = x * r:
 *   grad_x = clamp(g * w * r - xn * mean(g * w * xn))
 *   grad_w = clamp(sum over rows of xn * g)          (fp32 sum, then rounded)
 * The grad_x correction term is the reference's as written (the exact
 * derivative carries one more factor r).  Replaces FusedRMSNormFunction.
 * backward (hydra/kernels/fused_ops.py:1161-1172) with
 * _rms_norm_backward_pytorch (:1251-1281) / _fused_rms_norm_backward_kernel
 * (:1027-1111) + the grad_w reduction (:1244-1246).  x, grad_y, grad_x:
 * [rows, dim] with row strides x_rs, gy_rs, gx_rs; w, grad_w: [dim] of
 * w_dtype (`dtype`, or HYDRA_F32 for an fp32 master weight, read and
 * written in fp32 as the reference's kernel loads it,
 * fused_ops.py:1072, and casts its fp32 sum, :1244-1246).  The weight
 * gradient is summed in a fixed order (deterministic) through per-block
 * partial rows in caller-provided device scratch `workspace` of
 * workspace_bytes >= hydra_rms_norm_bwd_workspace(rows, dim) bytes (an
 * error when smaller); the library keeps no memory between calls. */
int hydra_rms_norm_bwd(const void* x, const void* w, const void* grad_y, void* grad_x,
                       void* grad_w, int64_t rows, int64_t dim, int64_t x_rs, int64_t gy_rs,
                       int64_t gx_rs, float eps, int dtype, int w_dtype, void* workspace,
                       int64_t workspace_bytes, void* stream);

/* Device scratch bytes hydra_rms_norm_bwd needs for rows x dim (768 fp32
 * partial rows of dim; 0 when rows or dim is 0).  Host-only, no device
 * call.  No counterpart in the reference (its scratch is torch's). */
int64_t hydra_rms_norm_bwd_workspace(int64_t rows, int64_t dim);

/* hydra_rms_norm_bwd without any allocation: the same kernels and results
 * (bit for bit), with the weight-gradient partials in a fixed 12 MiB device
 * array of the library (one per device, held until the process ends) instead
 * of caller-provided scratch.  No counterpart in the reference: it is for
 * callers that cannot allocate device memory (code under HIP graph capture,
 * serving loops, harnesses that forbid hipMalloc).  Limit: dim <= 4096
 * (HYDRA_ERR_ARG beyond).  Calls that overlap on one device share the array
 * and race; calls on one stream are ordered. */
int hydra_rms_norm_bwd_noalloc(const void* x, const void* w, const void* grad_y, void* grad_x,
                               void* grad_w, int64_t rows, int64_t dim, int64_t x_rs, int64_t gy_rs,
                               int64_t gx_rs, float eps, int dtype, int w_dtype, void* stream);

/* RoPE backward: grad_x = the rotation of hydra_rope_fwd transposed,
 *   gx[..,2i] = g[..,2i]*cos + g[..,2i+1]*sin, gx[..,2i+1] = -g[..,2i]*sin + g[..,2i+1]*cos.
 * The reference's Triton RoPE records no gradient (fused_ops.py:256-297);
 * this is what autograd gives through its CPU path _rope_pytorch (:300-306).
 * grad_y: [B,H,S,D] with element strides gys[4] (gys[3] must be 1);
 * grad_x: contiguous [B,H,S,D]. */
int hydra_rope_bwd(const void* grad_y, const void* cos, const void* sin, void* grad_x,
                   int64_t B, int64_t H, int64_t S, int64_t D, const int64_t* gys, int64_t cs_rs,
                   int dtype, int cs_dtype, void* stream);

/* SwiGLU backward, s = sigmoid(gate):
 *   grad_gate = clamp(g * up * s * (1 + gate * (1 - s))), grad_up = clamp(g * gate * s).
 * Replaces FusedSwiGLUFunction.backward (hydra/kernels/fused_ops.py:845-862)
 * with _swiglu_backward_pytorch (:926-948) / _fused_swiglu_backward_kernel
 * (:748-805).  All [rows, hidden] with their own row strides (gate/up may be
 * the halves of one gate_up tensor, grad_gate/grad_up of one grad tensor). */
int hydra_swiglu_bwd(const void* gate, const void* up, const void* grad_y, void* grad_gate,
                     void* grad_up, int64_t rows, int64_t hidden, int64_t g_rs, int64_t u_rs,
                     int64_t gy_rs, int64_t gg_rs, int64_t gu_rs, int dtype, void* stream);

/* QK-norm backward.  Per row n = max(||x||, 1e-6), xn = x / n:
 *   grad = clamp(s / n * (g - xn * <xn, g>)),  s = scale for q, scale * temperature for k.
 * Replaces FusedQKNormFunction.backward (hydra/kernels/fused_ops.py:533-545)
 * with _qk_norm_backward_pytorch (:638-672) / _fused_qk_norm_backward_kernel
 * (:389-471).  q, grad_qo, grad_q: [q_rows, hd]; k, grad_ko, grad_k:
 * [k_rows, hd]; all contiguous, same dtype. */
int hydra_qk_norm_bwd(const void* q, const void* k, const void* grad_qo, const void* grad_ko,
                      void* grad_q, void* grad_k, int64_t q_rows, int64_t k_rows, int64_t hd,
                      float scale, float temperature, int dtype, void* stream);

/* ---- CCGQA attention (hydra/attention/backends/ccgqa) ------------------ */

/* Feature bits of hydra_ccgqa_prep_fwd, mirroring the CCGQAAttention ctor
 * switches (attention.py:74-88). */
#define HYDRA_CCGQA_CONVS       1
#define HYDRA_CCGQA_QK_MEAN     2
#define HYDRA_CCGQA_VALUE_SHIFT 4
#define HYDRA_CCGQA_QK_NORM     8
#define HYDRA_CCGQA_ROPE        16
#define HYDRA_CCGQA_V_TRANSPOSED 32 /* write v as [B, Hkv, hd, S] */
#define HYDRA_CCGQA_W_TILED     64  /* conv weights in MFMA-fragment order (below) */

/* Everything of CCGQAAttention.forward between the qkv GEMM and the attention
 * core, in one pass over token tiles: split of the fused projection, value
 * shift, causal grouped conv1 + dense conv2 (conv_ks taps, each left-padded
 * by conv_ks - 1; the reference's default is 3) on q and k, QK-mean
 * coupling from the pre-conv q/k, L2-norm of q and of k times the key
 * temperature, and RoPE.  Replaces attention.py:205-266 with
 * OptimizedConvSequence.forward (kernels/fused_conv.py:39-62; the conv
 * sequences are built with conv_kernel_size at attention.py:132-145).
 *
 * qkv:  [B, S, L + 2K] (row stride qkv_rs), L = Hq*hd, K = Hkv*hd; column
 *       order q | k | v_curr | v_prev (v: | v when no value shift).
 * wq1/wq2/wk1/wk2: the four Conv1d weights (q_conv.conv1/conv2,
 *       k_conv.conv1/conv2) in tap-major layout [ks][out][in/groups], i.e.
 *       PyTorch's [out, in/groups, ks] permuted (2, 0, 1), ks = conv_ks:
 *       wq1 [ks][L][hd], wq2 [ks][L][L], wk1 [ks][K][hd], wk2 [ks][K][K]
 *       (unused and may be NULL without HYDRA_CCGQA_CONVS).
 *       With HYDRA_CCGQA_W_TILED each tap-major weight [3][O][I] is instead
 *       given as [3][O/32][I/16][2][32][8]: element (t, o/32, i/16, (i/8)%2,
 *       o%32, i%8), so one 32x16 MFMA operand block is 1 KB contiguous; only
 *       the MFMA path reads it (HYDRA_ERR_UNSUPPORTED otherwise).
 * temp: key temperature, 1 element of `dtype` (NULL without QK_NORM).
 * cos/sin: fp32 [S, hd/2] row stride cs_rs (NULL without ROPE).
 * q_out: [B, Hq, S, hd]; k_out: [B, Hkv, S, hd]; v_out: [B, Hkv, S, hd], or
 * [B, Hkv, hd, S] with HYDRA_CCGQA_V_TRANSPOSED (the layout hydra_attn_fwd
 * stages without a transpose); all contiguous.
 * bf16 with hd in {16, 32, 64, 128} and conv_ks = 3 runs both convs on MFMA
 * (up to ~140 KB of LDS per workgroup at L+K = 320); other cases (any
 * conv_ks in [1, 16]) run on the VALU. */
int hydra_ccgqa_prep_fwd(const void* qkv, int64_t qkv_rs,
                         const void* wq1, const void* wq2,
                         const void* wk1, const void* wk2,
                         const void* temp, const float* cos, const float* sin,
                         int64_t cs_rs,
                         void* q_out, void* k_out, void* v_out,
                         int64_t B, int64_t S, int64_t Hq, int64_t Hkv,
                         int64_t hd, int64_t conv_ks, int flags, int dtype, void* stream);

/* 1 when hydra_ccgqa_prep_fwd takes its MFMA path for these heads and
 * dtype on the current device (given 16-byte aligned pointers and, with
 * V_TRANSPOSED, S % 8 == 0), i.e. when HYDRA_CCGQA_W_TILED weights are
 * accepted; 0 otherwise.  No counterpart in the reference: it tells the
 * host which conv-weight layout to pack. */
int hydra_ccgqa_prep_tiled_ok(int64_t Hq, int64_t Hkv, int64_t hd, int dtype);

/* Number of hydra_ccgqa_prep_fwd tiles on the current device, since the
 * library was loaded, whose epilogue timed out waiting for the QK-mean
 * terms of its own workgroup (their outputs are written as NaN).  Always 0
 * on a working device; a health check for tests.  Synchronous (reads a
 * device counter).  No counterpart in the reference. */
int hydra_ccgqa_prep_faults(unsigned int* count);

/* Backward of hydra_ccgqa_prep_fwd's pointwise chain: what torch autograd
 * computes through attention.py:211-266 (value shift, QK-mean, F.normalize
 * with the key temperature, RoPE) given the gradients dq [B,Hq,S,hd] and
 * dk, dv [B,Hkv,S,hd] (contiguous) of its outputs.  y2q/y2k: the conv
 * outputs ([B,Hq,S,hd] / [B,Hkv,S,hd], i.e. hydra_ccgqa_prep_fwd with
 * HYDRA_CCGQA_CONVS alone), required with HYDRA_CCGQA_CONVS.  Writes
 *   dy [B,S,L+K]: gradient of the conv outputs (with CONVS),
 *   dqkv [B,S,L+2K] (row stride dqkv_rs): [:L+K] the QK-mean part of the
 *     q0/k0 gradient (plus the direct part without CONVS), [L+K:] the v
 *     part (value shift undone),
 *   dtemp_tok [B*S] (may be NULL): per-token partial of the temperature
 *     gradient (their sum is the gradient).
 * The flags are the forward's; V_TRANSPOSED is rejected.  L+K <= 4096. */
int hydra_ccgqa_prep_bwd(const void* qkv, int64_t qkv_rs, const void* y2q,
                         const void* y2k, const void* temp, const float* cos,
                         const float* sin, int64_t cs_rs, const void* dq,
                         const void* dk, const void* dv, void* dy, void* dqkv,
                         int64_t dqkv_rs, float* dtemp_tok, int64_t B, int64_t S,
                         int64_t Hq, int64_t Hkv, int64_t hd, int flags, int dtype,
                         void* stream);

/* The `taps`-tap causal conv of OptimizedConvSequence (kernels/fused_conv.py:
 * 52-57, left padding taps-1 per batch row) as a GEMM operand: x [B,S,G*cg]
 * (row stride x_rs) -> out [G][B*S][taps*cg] contiguous,
 * out[g][b*S+s][t*cg+c] = x[b, s+t-(taps-1), g*cg+c] (0 before the row
 * start).  A conv with weight W[o, c, t] (groups G) is then out[g] @
 * Wr[g]^T with Wr[g][o][t*cg+c].  taps in [1, 16]. */
int hydra_causal_im2col(const void* x, int64_t x_rs, void* out, int64_t B, int64_t S,
                        int64_t G, int64_t cg, int64_t taps, int dtype, void* stream);

/* The transpose of hydra_causal_im2col: out[b,s,g*cg+c] (row stride out_rs)
 * = sum over taps t of in[g][b*S+s+(taps-1)-t][t*cg+c] for
 * s+(taps-1)-t < S, added to out's contents when accumulate != 0 (the
 * conv's input gradient from the GEMM dY @ Wr). */
int hydra_causal_col2im(const void* in, void* out, int64_t out_rs, int64_t B, int64_t S,
                        int64_t G, int64_t cg, int64_t taps, int accumulate, int dtype,
                        void* stream);

/* Key-mask modes of hydra_attn_fwd (key_mask: uint8 [B,S], nonzero = keep).
 * KEY_PADDING: key t is visible to query s iff key_mask[b,t] != 0 (and t <= s
 *   when causal).
 * REFERENCE_SDPA: the literal behaviour of CCGQAAttention.forward when it is
 *   given a padding mask (attention.py:268-299): it builds
 *   triu(1) | (mask == 0) as "True = masked" and hands it to SDPA, whose
 *   boolean masks mean "True = attend", so key t is visible to query s iff
 *   t > s or key_mask[b,t] == 0.  Kept for result parity; requires causal=1. */
#define HYDRA_MASK_NONE           0
#define HYDRA_MASK_KEY_PADDING    1
#define HYDRA_MASK_REFERENCE_SDPA 2

/* Causal / full GQA softmax attention forward:
 *   o[b,h,s] = sum_{t visible} softmax_t(scale * q[b,h,s].k[b,j,t]) v[b,j,t]
 * with j = h / (Hq/Hkv) (repeat_interleave order), "visible" = t <= s when
 * causal, refined by mask_mode.
 * Replaces ccgqa_attention_fused (kernels/fused_attention.py:826-840, kernels
 * _fwd_gqa_kernel :14-110 and _fwd_kernel :341-429) and the SDPA call of
 * CCGQAAttention.forward (attention.py:268-327).
 * q: [B,Hq,S,hd], k/v: [B,Hkv,S,hd], element strides qs/ks/vs[4]; q and k
 *    need unit stride along hd; v needs it along hd or along S (the strides
 *    of a [B,Hkv,hd,S] buffer, which the bf16 path stages without a
 *    transpose; then S must be a multiple of 8);
 * o: element strides os[4] (last = 1) -- pass the strides of a [B,S,Hq,hd]
 *    buffer to write the merged-heads layout directly;
 * lse: optional fp32 [B,Hq,S] natural-log sum-exp of the scaled scores.
 * score_bound: beta >= max |q_i . k_j| (before the scale), or <= 0 when no
 *   bound is known.  When 0 < scale * beta * log2(e) <= 48 and no key mask
 *   is given, the bf16 kernel uses the fixed reference max scale * beta for
 *   every row instead of a running row max: no per-tile max and no
 *   rescaling (the softmax is the same; its exponentials are taken relative
 *   to another reference).  A beta below the true maximum overflows.  With
 *   the QK L2-norm of CCGQAAttention (unit-norm q, k of norm |temperature|,
 *   RoPE a rotation) beta = 1.03 * |temperature| holds: the 3% covers the
 *   bf16 roundings of the norm, the normalised vector, the temperature
 *   product and RoPE.
 * bound_temperature (device pointer to one bf16 or fp32 value, dtype code
 *   bound_temperature_dtype; may be NULL): the same bound taken on the
 *   device, beta = 1.03 * |*bound_temperature|, read by the kernel at each
 *   launch -- no host read of the temperature, and a captured graph follows
 *   its later values.  Takes precedence over score_bound; ignored with a
 *   key mask.  (No counterpart in the reference: its Triton kernel always
 *   keeps a running max.)
 * A query row with no visible key gets o = 0 (as CPU SDPA) and lse = -inf.
 * bf16 with hd in {16,32,64,128} runs on MFMA; other cases on the VALU.
 * workspace / workspace_bytes: caller-provided device scratch, at least
 * hydra_attn_fwd_workspace(...) bytes for the same shapes and strides (the
 * stream-K schedule's partials; 0 bytes, and NULL allowed, for every other
 * schedule); the library keeps no memory between calls. */
int hydra_attn_fwd(const void* q, const void* k, const void* v, void* o,
                   float* lse, const uint8_t* key_mask, int mask_mode,
                   int64_t B, int64_t Hq, int64_t Hkv, int64_t S, int64_t hd,
                   const int64_t* qs, const int64_t* ks, const int64_t* vs,
                   const int64_t* os, int causal, float scale,
                   float score_bound, const void* bound_temperature,
                   int bound_temperature_dtype, int dtype, void* workspace,
                   int64_t workspace_bytes, void* stream);

/* *bytes = device scratch hydra_attn_fwd needs for these shapes, strides,
 * mask mode and dtype on the current device (pointers 16-byte aligned
 * assumed; an upper bound otherwise).  Host-only, no device call.  No
 * counterpart in the reference. */
int hydra_attn_fwd_workspace(int64_t B, int64_t Hq, int64_t Hkv, int64_t S, int64_t hd,
                             const int64_t* qs, const int64_t* ks, const int64_t* vs,
                             const int64_t* os, int causal, int mask_mode, int dtype,
                             int64_t* bytes);

/* Causal / full GQA attention backward: given the forward's q, k, v, its
 * output o and lse (hydra_attn_fwd's fp32 [B,Hq,S] natural-log sum-exp of
 * the scaled scores, contiguous), and the upstream gradient grad_o, writes
 *   grad_v[b,j] = sum_g P^T grad_o,  grad_k[b,j] = sum_g dS^T q * scale,
 *   grad_q = dS k * scale,  dS = P (grad_o v^T - rowsum(grad_o * o)),
 * with P recomputed from lse, summing the G = Hq/Hkv query heads of K/V
 * head j.  key_mask / mask_mode: the forward's ([B,S] uint8, nonzero =
 * keep; HYDRA_MASK_KEY_PADDING or HYDRA_MASK_REFERENCE_SDPA, the latter
 * with causal = 1), so P is zero exactly where the forward's was -- the
 * backward of the padding-mask SDPA call (attention.py:268-299), which
 * the reference trains through autograd.  fp32 accumulation, outputs
 * rounded once; no atomics (repeat calls are bit-identical).
 * Replaces CCGQAAttentionFused.backward (kernels/fused_attention.py:706-823)
 * and its kernels _bwd_gqa_kv_kernel / _bwd_gqa_dq_kernel (:113-338) and
 * _bwd_kernel / _bwd_dq_kernel (:432-635).
 * q, o, grad_o, grad_q: [B,Hq,S,hd]; k, v, grad_k, grad_v: [B,Hkv,S,hd];
 * element strides *s[4], unit stride along hd for all.  bf16 with hd in
 * {32, 64, 128}, 16-byte aligned pointers and strides that are multiples of
 * 8 and no key mask run on MFMA; every other case on the VALU path
 * (hd <= 256).  Scratch
 * (8 * B * Hq * S bytes of row statistics, plus the dK/dV chunk partials
 * of long causal walks) comes from the caller: workspace_bytes >=
 * hydra_attn_bwd_workspace(...) for the same shapes; the library keeps no
 * memory between calls.  On the MFMA path the dQ launch runs on a side
 * stream of the library's (one per device, default priority), forked from
 * `stream` after the row statistics and joined back before the call
 * returns, so everything queued on `stream` afterwards (and a graph
 * captured from it) sees all three gradients. */
int hydra_attn_bwd(const void* q, const void* k, const void* v, const void* o,
                   const void* grad_o, const float* lse, void* grad_q, void* grad_k,
                   void* grad_v, int64_t B, int64_t Hq, int64_t Hkv, int64_t S, int64_t hd,
                   const int64_t* qs, const int64_t* ks, const int64_t* vs, const int64_t* os,
                   const int64_t* gos, const int64_t* gqs, const int64_t* gks,
                   const int64_t* gvs, const uint8_t* key_mask, int mask_mode, int causal,
                   float scale, int dtype, void* workspace, int64_t workspace_bytes,
                   void* stream);

/* *bytes = device scratch hydra_attn_bwd needs for these shapes and strides
 * (pointers 16-byte aligned assumed; an upper bound otherwise).  Host-only,
 * no device call.  No counterpart in the reference. */
int hydra_attn_bwd_workspace(int64_t B, int64_t Hq, int64_t Hkv, int64_t S, int64_t hd,
                             const int64_t* qs, const int64_t* ks, const int64_t* vs,
                             const int64_t* os, const int64_t* gos, const int64_t* gqs,
                             const int64_t* gks, const int64_t* gvs, int mask_mode, int causal,
                             int dtype, int64_t* bytes);

#define HYDRA_LINEAR_W_TILED 1 /* W in MFMA-fragment order (below)             */

/* Output projection y = x W^T (F.linear without bias), the CCGQA o_proj
 * (attention.py:329-331: out.reshape(B, S, L) @ o_proj.weight^T).  x: [M, K]
 * (row stride x_rs), y: [M, N] (row stride y_rs), W: [N, K] (row stride
 * w_rs), or with HYDRA_LINEAR_W_TILED packed as [N/32][K/16][2][32][8]
 * (element [j][s][h][n][e] = W[32 j + n][16 s + 8 h + e]; w_rs unused), the
 * layout the kernel loads with one coalesced 16-byte read per lane and
 * fragment.  Takes bf16 with K in {64, 128, 256}, N % 64 == 0 and 16-byte
 * aligned rows; returns HYDRA_ERR_UNSUPPORTED for anything else (the caller
 * then uses a library GEMM).  fp32 accumulation, one rounding. */
int hydra_linear_fwd(const void* x, int64_t x_rs, const void* w, int64_t w_rs, void* y,
                     int64_t y_rs, int64_t M, int64_t N, int64_t K, int flags, int dtype,
                     void* stream);

/* ---- LM-head loss (hydra/kernels/fused_ops.py) ------------------------- */

/* Token-row softmax cross-entropy of a logits block x [rows, vocab] (unit
 * column stride, row stride logits_rs): loss[r] = logsumexp(x[r]) - x[r, t]
 * in fp32 (0 when targets[r] == ignore_index; other targets are clamped
 * into [0, vocab)); lse[r] (optional) = logsumexp(x[r]).  With grad
 * non-null, also writes grad[r] = (softmax(x[r]) - onehot(t)) * grad_scale[0]
 * (zero rows for ignored tokens; grad may alias logits; grad_scale is a
 * device pointer, so the caller's loss scale needs no host round trip).
 * targets: int64.  Replaces the per-chunk F.cross_entropy and the gradient
 * of ChunkedCrossEntropyFunction (fused_ops.py:1303-1379, 1382-1531); the
 * projections around it stay plain GEMMs. */
int hydra_ce_rows(const void* logits, int64_t rows, int64_t vocab, int64_t logits_rs,
                  const int64_t* targets, int64_t ignore_index, float* loss, float* lse,
                  void* grad, int64_t grad_rs, const float* grad_scale, int dtype,
                  void* stream);

/* ---- block compositions (hydra/model/framework, hydra/layers) --------- */

/* Token embedding: out[r, :] = table[clamp(ids[r], 0, vocab-1), :] * scale,
 * one rounding into `dtype`.  Replaces _safe_embedding_lookup
 * (hydra/model/framework/model.py:51-73: ids always clamped, embedding(x) *
 * sqrt(dim)).  ids: int64 [n]; table: [vocab, dim] (row stride table_rs);
 * out: [n, dim] (row stride out_rs). */
int hydra_embedding_fwd(const int64_t* ids, int64_t n, const void* table, int64_t vocab,
                        int64_t dim, int64_t table_rs, float scale, void* out, int64_t out_rs,
                        int dtype, void* stream);

#define HYDRA_NORM_NONE 0 /* residual only                                   */
#define HYDRA_NORM_RMS  1 /* RMSNorm: fp32 math, one rounding                */
#define HYDRA_NORM_ADA  2 /* AdaRMSNorm: the reference's input-dtype steps   */

/* Residual add fused with the pre-norm of the next sublayer.  Per row, each
 * step rounded into `dtype` as the reference's tensor ops are:
 *   v = x + (alpha == 1 ? r : round(alpha * r))   (r optional)
 *   v = v + b1;  v = v + b2                         ([dim] vectors, optional)
 *   h_out = v                                       (optional)
 *   y_out = norm(v):
 *     RMS: v * rsqrt(mean(v^2) + eps) * w in fp32, one rounding
 *          (RMSNorm, hydra/layers/common.py:74-118);
 *     ADA: AdaRMSNorm._rmsnorm (common.py:153-157) in the input dtype:
 *          m = round(mean(round(v^2))), s = round(rsqrt(round(m + eps))),
 *          y = round(round(v * s) * w).
 * Replaces, in HydraBlock.forward (hydra/model/framework/blocks.py:68-70),
 * `h = x + attention(...)` with norm2(h); in HydraMoRBlock._forward_mor
 * (blocks.py:614-633) `x + residual_scale * attention(...)`; and in
 * MoRExecutor.forward (hydra/routing/mixture_of_recursions.py:459-465)
 * `norm(current + recursion_bias[i] + recursion_embed[i])`.
 * x, r, h_out, y_out: [rows, dim] with row strides; b1, b2: [dim] of dtype;
 * w: [dim] of w_dtype (dtype, or HYDRA_F32 for an fp32 weight).
 * y_out is required exactly when norm != NONE. */
int hydra_residual_norm_fwd(const void* x, int64_t x_rs, const void* r, int64_t r_rs,
                            float alpha, const void* b1, const void* b2, const void* w,
                            float eps, int norm, void* h_out, int64_t h_rs, void* y_out,
                            int64_t y_rs, int64_t rows, int64_t dim, int dtype, int w_dtype,
                            void* stream);

/* One recursion's update of MoRExecutor.forward
 * (hydra/routing/mixture_of_recursions.py:466-476), in place, per token row
 * with depth d = depth[row]:
 *   current = current + round(delta * (d >= recursion))
 *   output  = output + round(current * (d == recursion))
 * (the straight-through factor (1 + ste_grad) is exactly 1 in the forward).
 * current, delta, output: [rows, dim] with row strides; depth: int64 [rows]. */
int hydra_mor_update(void* current, int64_t c_rs, const void* delta, int64_t d_rs,
                     void* output, int64_t o_rs, const int64_t* depth, int64_t rows,
                     int64_t dim, int64_t recursion, int dtype, void* stream);

/* MoR depth routing from the router's logits (MoRRouter.forward,
 * hydra/routing/mixture_of_recursions.py:259-288), per token, each step
 * rounded into `dtype`:
 *   l = round(round(tanh(round(logit / 2))) * 3);  p = round(sigmoid(l));
 *   dc = round(p * (R - 1)), or round(min_d + round(p * (R - 1 - min_d)))
 *   depth = clamp(round_half_even(dc), min_d, R - 1).
 * logits: [n]; probs, logits_out: [n] of dtype (optional); depth: int64 [n]. */
int hydra_mor_route(const void* logits, int64_t n, void* probs, void* logits_out,
                    int64_t* depth, int64_t n_recursions, int64_t min_depth, int dtype,
                    void* stream);

/* ---- Mixture-of-Depths hard routing (hydra/routing, model/framework) --- */

/* Per-row top-k of router scores, ties broken by the lower index, in the
 * total order of torch.topk(largest=True) (NaN above +inf, -0.0 == +0.0).
 * Replaces torch.topk + mask.scatter_ in MoDRouter.forward
 * (hydra/routing/mixture_of_depths.py:179-191) and the torch.sort of the
 * indices in MoDMLPWrapper._forward_hard (model/framework/blocks.py:261).
 * scores: [B, L] (row stride s_rs) of score_dtype (HYDRA_F32/BF16/F16);
 * idx_desc: int64 [B, k] in value-descending order (may be NULL);
 * idx_sorted: int64 [B, k] ascending (may be NULL);
 * mask: [B, L] of mask_dtype, 1 for selected tokens else 0 (may be NULL).
 * Limits: 1 <= k <= L < 2^31, B <= 65535; rows longer than 8192 also need
 * B * L < 2^31 and take a global-memory radix sort whose workspace is
 * allocated and freed stream-ordered (hipMallocAsync / hipFreeAsync) on
 * `stream`. */
int hydra_mod_topk(const void* scores, int64_t B, int64_t L, int64_t s_rs,
                   int64_t k, int64_t* idx_desc, int64_t* idx_sorted,
                   void* mask, int score_dtype, int mask_dtype, void* stream);

/* Row gather: xs[b,j,:] = x[b, idx[b,j], :].
 * Replaces gather_by_indices (hydra/routing/ops.py:257-272) and the gather
 * of MoDMLPWrapper._forward_hard (blocks.py:263-264).
 * x: [B, L, D] (strides x_bs, x_ls; unit stride on D); idx: int64 [B, k];
 * xs: contiguous [B, k, D].  Indices must lie in [0, L). */
int hydra_mod_gather(const void* x, const int64_t* idx, void* xs,
                     int64_t B, int64_t L, int64_t k, int64_t D,
                     int64_t x_bs, int64_t x_ls, int dtype, void* stream);

#define HYDRA_SCATTER_ADD     0 /* out[b,idx] += w * y  (residual add)    */
#define HYDRA_SCATTER_REPLACE 1 /* out[b,idx]  = y      (clone + scatter) */
#define HYDRA_SCATTER_ADD_SEQ 2 /* out[b,idx] += y, repeated idx allowed  */

/* In-place weighted residual scatter into out: [B, L, D] (strides o_bs,
 * o_ls), from y: contiguous [B, k, D], at idx: int64 [B, k].
 * w: optional fp32 [B, k] per-row weights (NULL = 1; ADD only).
 * ADD (idx distinct per row) replaces the zeros_like + scatter_ + residual
 * add of MoDMLPWrapper._forward_hard and its caller (blocks.py:266-268,
 * :603); sums are fp32, one rounding.  REPLACE (idx distinct per row)
 * replaces the clone + scatter_ of MixtureOfDepthsBlock.forward
 * (mixture_of_depths.py:291-295); with y == NULL it clears the rows.
 * ADD_SEQ replaces scatter_add_by_indices (hydra/routing/ops.py:275-293,
 * torch.scatter_add_): repeated indices accumulate in index order, rounded
 * after every add, one thread per (row, column) (not a hot path).
 * Indices outside [0, L) are skipped. */
int hydra_mod_scatter(void* out, const void* y, const int64_t* idx,
                      const float* w, int64_t B, int64_t L, int64_t k,
                      int64_t D, int64_t o_bs, int64_t o_ls, int mode,
                      int dtype, void* stream);

/* ---- measurement aid ----------------------------------------------------- */

/* dst[0, bytes) = src[0, bytes): a plain device-to-device copy with
 * non-temporal 16-byte loads and stores, one chunk per thread.  No
 * counterpart in the reference: it gives callers (bench.py) the copy rate
 * of the same bytes on the same device, the practical ceiling of a
 * one-pass HBM-bound kernel.  bytes % 16 == 0, both pointers 16-byte
 * aligned, the ranges must not overlap. */
int hydra_stream_copy(const void* src, void* dst, int64_t bytes, void* stream);

/* The shader clock under matrix-core load: nwg workgroups of 8 waves each
 * run `iters` iterations of four bf16 32x32x16 MFMAs and 16 v_exp_f32 (the
 * attention tile's instruction kinds) and write, per workgroup, 5 uint64
 * to stamps (device memory): shader-clock counter (s_memtime) before and
 * after, wall-clock counter (s_memrealtime) before and after, and a sink
 * value.  *wall_khz receives the wall clock's constant rate.  The clock is
 * sum(shader ticks) / sum(wall ticks) * wall_khz.  No counterpart in the
 * reference: bench.py reports the clock the matrix-core fraction was
 * reached at. */
int hydra_clock_probe(void* stamps, int nwg, int iters, int64_t* wall_khz, void* stream);

/* Installs (stamps != NULL) or removes (NULL) a device buffer of
 * 4 * max_workgroups uint64 into which every later launch of
 * hydra_attn_fwd's key-split kernel with at most max_workgroups
 * workgroups writes, per workgroup: the shader-clock counter (s_memtime)
 * at its start and after its last store, and the wall-clock counter
 * (s_memrealtime) at the same two points.  Process-wide; the caller keeps
 * the buffer alive while installed.  No counterpart in the reference:
 * bench.py reads the clock the attention kernel itself ran at. */
int hydra_attn_clock_stamps(void* stamps, int64_t max_workgroups);

#ifdef __cplusplus
}
#endif
#endif /* HYDRA_AMD_H */
