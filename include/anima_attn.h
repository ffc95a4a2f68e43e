/*
 * anima_attn.h — C ABI of the MI355X (gfx950) DiT attention path.
 *
 * One shared library, libanima_attn.so, holds every kernel of the path:
 * the QK-RMSNorm + 3D-RoPE prologue, per-head RMSNorm of cross-attention
 * queries, the non-causal flash-attention forward (self, and key-length
 * masked cross-attention with an optional fused padding correction), the
 * flash-attention backward, and the padding-correction kernels on their own.
 *
 * Conventions shared by every entry point:
 *   - Tensors are device pointers. Attention tensors are [B, S, H, hd]
 *     ("BSHD") with the head-dim stride fixed to 1 and the other three
 *     strides passed in elements (int64). Prologue tensors are contiguous.
 *   - `stream` is a hipStream_t passed as void* (NULL = the null stream).
 *     Every call is asynchronous on that stream; no call synchronises the
 *     host and none allocates or frees device memory: outputs and
 *     workspaces are allocated by the caller.
 *   - Return codes: AA_OK (0); AA_EINVAL (-1) for a bad argument (null
 *     pointer, inconsistent shape, misaligned pointer or stride);
 *     AA_EUNSUPPORTED (-2) for a shape or dtype the kernels do not
 *     implement; AA_EHIP (-3) when a HIP launch reports an error.
 *     aa_last_error() returns the calling thread's last message.
 *   - Only dtype AA_DTYPE_BF16 is implemented for activations; weights,
 *     rotary tables, LSE and padding logs are float32; key lengths int32.
 *   - hd (head_dim) must be 128; aa_attn_fwd (and its workspace and no-alloc
 *     forms) also takes 384, the VAE decoder's single-head attention.
 *
 * The reference (anima-flat) has no C FFI of its own: its path is Python
 * calling FlashAttention-4 (CuTe DSL) and Triton kernels. Each entry point
 * below names the reference function (file:line under src/) whose work it
 * replaces; the Python host layer in anima-flat_amd/ keeps those functions'
 * signatures and calls these entry points through ctypes.
 */
#ifndef ANIMA_ATTN_H
#define ANIMA_ATTN_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define AA_ABI_VERSION 3

enum {
  AA_OK = 0,
  AA_EINVAL = -1,
  AA_EUNSUPPORTED = -2,
  AA_EHIP = -3,
};

enum {
  AA_DTYPE_BF16 = 0,
  AA_DTYPE_FP16 = 1, /* reserved: rejected with AA_EUNSUPPORTED */
};

/* ABI version of the loaded library (AA_ABI_VERSION when built from this header). */
int aa_abi_version(void);

/* Last error message of the calling thread ("" if none). Valid until the next call. */
const char* aa_last_error(void);

/* ------------------------------------------------------------------------ */
/* Prologue                                                                  */
/* ------------------------------------------------------------------------ */

/*
 * Per-head RMSNorm of the q and k sections of a fused QKV projection output,
 * rounded to the activation dtype, then rotate-half RoPE; optional V copy.
 *   qkv [B, S, 3*H*hd] contiguous; q, k [B, S, H, hd] contiguous outputs;
 *   v   [B, S, H, hd] output or NULL (NULL: V is not copied);
 *   q_weight, k_weight [hd] float32; cos, sin [S, hd/2] float32;
 *   position of token (b, s) is s.
 * Replaces: src/kernels/rope.py:175-193 (_qkv_norm_rope, v == NULL) and
 *           src/kernels/rope.py:504-523 (_qkv_norm_rope_v, v != NULL),
 *           kernel src/kernels/rope.py:61-143.
 */
int aa_qkv_norm_rope_fwd(const void* qkv, void* q, void* k, void* v,
                         const float* q_weight, const float* k_weight,
                         const float* cos, const float* sin,
                         int64_t B, int64_t S, int64_t H, int64_t hd,
                         float eps, int dtype, void* stream);

/*
 * QKV projection fused with the prologue: q, k, v = aa_qkv_norm_rope_fwd of
 * qkv = hid @ weight^T (bf16), without qkv ever reaching memory.
 *   hid [B*S rows, H*hd], row r at hid + r * hid_row_stride elements
 *   (hid_row_stride >= H*hd, a multiple of 8, at most 2^27); weight [3*H*hd, H*hd]
 *   contiguous (nn.Linear layout, no bias); q, k, v [B, S, H, hd] contiguous
 *   outputs (v is the projection's V section as it is); q_weight, k_weight,
 *   cos, sin as for aa_qkv_norm_rope_fwd. H <= 64.
 * Replaces: src/model.py:308-316 (b.qkv(hid), model.py:134, followed by
 *           qkv_norm_rope, src/kernels/rope.py:616-645) on the inference path.
 */
int aa_qkv_proj_norm_rope(const void* hid, int64_t hid_row_stride, const void* weight,
                          void* q, void* k, void* v,
                          const float* q_weight, const float* k_weight,
                          const float* cos, const float* sin,
                          int64_t B, int64_t S, int64_t H, int64_t hd,
                          float eps, int dtype, void* stream);

/*
 * A projection fused with per-head RMSNorm: y = aa_head_norm_fwd of
 * x @ weight^T (bf16), the projection never reaching memory.
 *   x [B*S rows, K], row r at x + r * x_row_stride elements (x_row_stride >= K,
 *   a multiple of 8, at most 2^27; K a multiple of 32); weight [H*hd, K] contiguous (nn.Linear
 *   layout, no bias); y [B, S, H, hd] contiguous; norm_weight [hd] float32.
 * Replaces: src/model.py:324 (b.xq(hid), model.py:138, followed by head_norm,
 *           src/kernels/rope.py:648-652) on the inference path.
 */
int aa_proj_head_norm(const void* x, int64_t x_row_stride, const void* weight, int64_t K,
                      void* y, const float* norm_weight,
                      int64_t B, int64_t S, int64_t H, int64_t hd,
                      float eps, int dtype, void* stream);

/*
 * The context's keys and values with the key-side RMSNorm fused:
 * kv = ctx @ weight^T (bf16, [B, S, 2, H, hd]), k = RMSNorm(kv[:, :, 0]) with
 * k_weight, v = kv[:, :, 1], kv never reaching memory.
 *   ctx [B*S rows, K] as x above; weight [2*H*hd, K] contiguous; k, v
 *   [B, S, H, hd] contiguous; k_weight [hd] float32 (pass the bf16 weight
 *   widened, as F.rms_norm applies it in the activation dtype).
 * Replaces: src/model.py:256-258 (b.xkv(ctx), model.py:139, .view().unbind(),
 *           F.rms_norm of k) in encode_context, inference path.
 */
int aa_kv_proj_norm(const void* ctx, int64_t ctx_row_stride, const void* weight, int64_t K,
                    void* k, void* v, const float* k_weight,
                    int64_t B, int64_t S, int64_t H, int64_t hd,
                    float eps, int dtype, void* stream);

/*
 * Per-head RMSNorm: x [B, S, H*hd] contiguous -> y [B, S, H, hd] contiguous.
 * Replaces: src/kernels/rope.py:203-212 (_head_norm), kernel rope.py:146-172.
 */
int aa_head_norm_fwd(const void* x, void* y, const float* weight,
                     int64_t B, int64_t S, int64_t H, int64_t hd,
                     float eps, int dtype, void* stream);

/* Bytes of workspace aa_qkv_norm_rope_bwd needs (weight-grad partials: one
 * 2*hd float record per 8 tokens). */
size_t aa_qkv_norm_rope_bwd_workspace(int64_t B, int64_t S, int64_t H, int64_t hd);

/*
 * Backward of aa_qkv_norm_rope_fwd (with V copied):
 *   dq, dk, dv [B, S, H, hd] contiguous -> dqkv [B, S, 3*H*hd],
 *   dq_weight, dk_weight [hd] float32 (sums over every token and head).
 * The weight-gradient reduction runs in a fixed order (deterministic).
 * Replaces: src/kernels/rope.py:540-577 (_qkv_norm_rope_bwd),
 *           kernel rope.py:277-383, helper rope.py:223-274.
 */
int aa_qkv_norm_rope_bwd(const void* qkv, const void* dq, const void* dk,
                         const void* dv, void* dqkv,
                         const float* q_weight, const float* k_weight,
                         const float* cos, const float* sin,
                         float* dq_weight, float* dk_weight,
                         void* workspace, size_t workspace_bytes,
                         int64_t B, int64_t S, int64_t H, int64_t hd,
                         float eps, int dtype, void* stream);

/* Bytes of workspace aa_head_norm_bwd needs (as above with hd floats). */
size_t aa_head_norm_bwd_workspace(int64_t B, int64_t S, int64_t H, int64_t hd);

/*
 * Backward of aa_head_norm_fwd: x, dy [B, S, H*hd] -> dx [B, S, H*hd],
 * dweight [hd] float32.
 * Replaces: src/kernels/rope.py:443-471 (_head_norm_bwd), kernel rope.py:386-436.
 */
int aa_head_norm_bwd(const void* x, const void* dy, void* dx,
                     const float* weight, float* dweight,
                     void* workspace, size_t workspace_bytes,
                     int64_t B, int64_t S, int64_t H, int64_t hd,
                     float eps, int dtype, void* stream);

/* ------------------------------------------------------------------------ */
/* Flash attention                                                           */
/* ------------------------------------------------------------------------ */

typedef struct aa_attn_fwd_args {
  const void* q;        /* [B, Sq, H, hd] */
  const void* k;        /* [B, Sk, H, hd]; may be NULL when Sk == 0 */
  const void* v;        /* [B, Sk, H, hd]; may be NULL when Sk == 0 */
  void* out;            /* [B, Sq, H, hd]; Sk == 0 gives out = 0 and lse = -inf */
  float* lse;           /* [B, H, Sq] contiguous natural-log LSE, or NULL */
  const int32_t* seqused_k; /* [B] keys attended per batch item, or NULL (all Sk) */
  const float* ln_pad;  /* [B] log(#padding keys) for the fused padding
                           correction out *= 1/(1+exp(ln_pad-lse)), or NULL */
  int64_t q_stride[3];  /* batch, seq, head strides in elements */
  int64_t k_stride[3];
  int64_t v_stride[3];
  int64_t out_stride[3];
  int64_t B, Sq, Sk, H, hd;
  float softmax_scale;  /* usually 1/sqrt(hd) */
  int dtype;
  void* workspace;      /* device scratch of aa_attn_fwd_workspace() bytes (may be 0) */
  size_t workspace_bytes;
} aa_attn_fwd_args;

/* Bytes of device workspace aa_attn_fwd needs on the current device: partial
 * results (bf16 normalised O and fp32 LSE, at both head dims) when the work items (256
 * queries of one (batch, head); 128 at hd 384) of a partial last round of
 * workgroups (at hd 384: of too few work items to fill the device) are split
 * over key ranges, else 0. */
size_t aa_attn_fwd_workspace(int64_t B, int64_t Sq, int64_t Sk, int64_t H, int64_t hd);

/*
 * out = softmax(q k^T * softmax_scale) v, non-causal, per (batch, head);
 * keys j >= seqused_k[b] are excluded when seqused_k != NULL; lse is the
 * natural-log row log-sum-exp of the scaled scores over the attended keys.
 * One kernel launch, plus a combine pass when aa_attn_fwd_workspace() > 0.
 * From about two rounds of 64-tile work items on (e.g. B=2 at 4096 keys),
 * the hd-128 forward keeps each row's first key tile max and follows its
 * launch with a fix-up launch that re-runs, with a running max, the work
 * items whose scores left that exponent range (AA_FWD_FIRST_TILE_MAX=0|1
 * forces the form). Every launch goes to `stream`; none allocates.
 * Replaces: src/attention.py:43-53 (anima_flat::fa_fwd),
 *           src/attention.py:63-66 (anima_flat::fa_fwd_nolse),
 *           src/attention.py:74-81 (anima_flat::fa_fwd_k), and with
 *           ln_pad != NULL also the ctx_scale pass of
 *           src/attention.py:156-180 (cross_attention_trimmed).
 * With hd == 384 (one kernel for that width, plus a combine pass when its keys
 * are split): replaces the VAE's mid-block attention, src/vae.py:239
 * (ffpa_attn_func / SDPA on [B, 1, S, 384], vae.py:10-13, 230-241).
 */
int aa_attn_fwd(const aa_attn_fwd_args* args, void* stream);

/*
 * aa_attn_fwd without a caller workspace and without any allocation: the
 * split partials go to a fixed device array of 25,296,896 bytes that the
 * library holds on each device it runs on until the process ends (every
 * forward, head_dim 128 or 384, on a 256-CU device fits; a plan that needs
 * more returns AA_EUNSUPPORTED). args->workspace / workspace_bytes are ignored. Calls on
 * one device share that array: calls that overlap on one device (two streams
 * at once) race and must be serialised by the caller. Same results as
 * aa_attn_fwd (same kernels). No counterpart in the reference: for callers
 * that cannot allocate device memory (code under HIP graph capture, serving
 * loops, harnesses that forbid hipMalloc).
 */
int aa_attn_fwd_noalloc(const aa_attn_fwd_args* args, void* stream);

typedef struct aa_attn_bwd_args {
  const void* dout;     /* [B, Sq, H, hd] */
  const void* q;
  const void* k;
  const void* v;
  const void* out;
  const float* lse;     /* [B, H, Sq] contiguous, from aa_attn_fwd */
  void* dq;             /* [B, Sq, H, hd] */
  void* dk;             /* [B, Sk, H, hd] */
  void* dv;             /* [B, Sk, H, hd] */
  int64_t dout_stride[3];
  int64_t q_stride[3];
  int64_t k_stride[3];
  int64_t v_stride[3];
  int64_t out_stride[3];
  int64_t dq_stride[3];
  int64_t dk_stride[3];
  int64_t dv_stride[3];
  int64_t B, Sq, Sk, H, hd;
  float softmax_scale;
  int dtype;
} aa_attn_bwd_args;

/* Bytes of workspace aa_attn_bwd needs, 16-byte aligned: 1 KB of softmax
 * statistics per 64 queries, for every (batch, head); 0 if Sq == 0. */
size_t aa_attn_bwd_workspace(int64_t B, int64_t Sq, int64_t Sk, int64_t H, int64_t hd);

/*
 * dq, dk, dv of aa_attn_fwd (no key mask), softmax recomputed from lse.
 * Deterministic: no atomics, every sum runs in a fixed order.
 * Replaces: src/attention.py:91-103 (anima_flat::fa_bwd), reached through
 *           the autograd registration at src/attention.py:111-123.
 */
int aa_attn_bwd(const aa_attn_bwd_args* args, void* workspace,
                size_t workspace_bytes, void* stream);

/* ------------------------------------------------------------------------ */
/* Padding correction of trimmed cross-attention                             */
/* ------------------------------------------------------------------------ */

/*
 * y = out * 1/(1 + exp(ln_pad[b] - lse[b, h, s])); out, y [B, S, H, hd]
 * contiguous, lse [B, H, S], ln_pad [B].
 * Replaces: src/kernels/ctx_scale.py:39-55 (kernel ctx_scale.py:8-36).
 */
int aa_ctx_scale_fwd(const void* out, const float* lse, const float* ln_pad,
                     void* y, int64_t B, int64_t S, int64_t H, int64_t hd,
                     int dtype, void* stream);

/*
 * dout = dy * g, dlse[b,h,s] = sum_d(dy * out) * g * (1 - g) with
 * g = 1/(1 + exp(ln_pad[b] - lse[b,h,s])).
 * Replaces: src/kernels/ctx_scale.py:98-117 (kernel ctx_scale.py:63-95).
 */
int aa_ctx_scale_bwd(const void* out, const float* lse, const float* ln_pad,
                     const void* dy, void* dout, float* dlse,
                     int64_t B, int64_t S, int64_t H, int64_t hd,
                     int dtype, void* stream);

/* ------------------------------------------------------------------------ */
/* Text-context length bookkeeping                                           */
/* ------------------------------------------------------------------------ */

/* Bytes of workspace aa_context_lengths needs (one int32 per 32 rows per item). */
size_t aa_context_lengths_workspace(int64_t B, int64_t S);

/*
 * Lengths of a zero-padded text context ctx [B, S, C] (element strides
 * stride_b, stride_s; last dim contiguous; elem_bytes 2 for bf16/fp16 or 4
 * for fp32): seqused[b] = 1-based index of the last row with a non-zero
 * element, at least 1 (int32 [B]); ln_pad[b] = log(S - seqused[b]) (float
 * [B], -inf when nothing is padded). Computed on the device with no host
 * read: K/V projected from the untrimmed context can go straight to
 * aa_attn_fwd with seqused_k / ln_pad, which reads only the first seqused[b]
 * keys, so the reference's trim to roundup8(max length) rows (and its
 * device-to-host read) is not needed. Rows must be 16-byte aligned and
 * C * elem_bytes a multiple of 16.
 * Replaces: src/model.py:248-253 (the length, seqused and ln_pad lines of
 *           encode_context's trim; the ctx[:, :keep] slice is dropped).
 */
int aa_context_lengths(const void* ctx, int64_t B, int64_t S, int64_t C,
                       int64_t stride_b, int64_t stride_s, int elem_bytes,
                       int32_t* seqused, float* ln_pad,
                       void* workspace, size_t workspace_bytes, void* stream);

/* ------------------------------------------------------------------------ */
/* FP8 row quantisation (consumer of the attention output)                   */
/* ------------------------------------------------------------------------ */

/*
 * Per-row FP8 quantisation: for each of `rows` rows of x [rows, K] bf16
 * (contiguous), y = x or GELU(x) (gelu != 0; Abramowitz-Stegun 7.1.26 erf),
 * s[row] = max(max|y|, 1e-12) / 448 (float), q = e4m3fn(clamp(y / s, +-448))
 * rounded to nearest even (uint8 [rows, K], OCP E4M3 "fn" bytes).
 * K a multiple of 8 and at most 8192; x 16-byte and q 8-byte aligned.
 * Replaces: src/kernels/fp8.py:295-328 (rowquant, op anima_flat::rowquant),
 *           kernel fp8.py:275-292.
 */
int aa_rowquant(const void* x, int64_t rows, int64_t K, int gelu,
                void* q, float* s, int dtype, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* ANIMA_ATTN_H */
