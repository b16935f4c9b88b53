/*
 * fa_gfx950.h - C ABI of the MI355X (gfx950) sliding-window + sink FlashAttention-2 library.
 *
 * The library computes causal attention with grouped-query heads (Hq query heads share Hkv
 * key/value heads, head h reads KV head h / (Hq/Hkv)), a sliding window W and S positional
 * "sink" keys:
 *
 *     allowed(q, k) = k <= q  &&  (q - k < W  ||  k < S)
 *
 * (reference predicate: benchmark_backward_speed.py:40-46 create_mask_bool and :110-115
 * _compute_mask; flash_attention_gpt_oss.py:82-86, 116-120, 150-155 for the repo kernels).
 *
 * Layouts follow the reference autograd function (flash_attention_gpt_oss.py:340-438):
 * q/o/dout/dq are [B, Hq, L, D], k/v/dk/dv are [B, Hkv, L, D], lse is float32 [B, Hq, L].
 * Every tensor is described by a base pointer and its batch/head/sequence strides in elements;
 * the head-dim stride must be 1.  lse holds the natural-log log-sum-exp of the scaled, masked
 * scores of each query row (the reference repo keeps a log2-domain row max instead,
 * flash_attention_gpt_oss.py:178-180; the statistic never leaves the autograd context).
 *
 * Rules shared by every entry point:
 *   - the library never allocates or frees device memory; the caller passes every buffer,
 *     including the backward workspace sized by fa_bwd_workspace_bytes() (fa_bwd_scratch uses
 *     the library's own static per-GPU buffer instead);
 *   - launches are asynchronous on `stream` (a hipStream_t; NULL means the legacy default
 *     stream); nothing synchronises the host;
 *   - arguments are validated on the host before any HIP call; on failure a negative FA_ERR_*
 *     code is returned and nothing is launched.  fa_strerror() names each code;
 *   - apart from fa_bwd_scratch's buffer, the library holds no mutable global state, so
 *     concurrent calls on different streams are safe.
 */
#ifndef FA_GFX950_H
#define FA_GFX950_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define FA_GFX950_VERSION 10400 /* 1.4.0 */

/* Element types of q/k/v/o/dout/dq/dk/dv.  All of them share one type per call, except in
 * fa_fwd_fp8 and fa_fwd_fp8_pv: FA_DTYPE_FP8_E4M3 means OCP float8 e4m3 q, k, v and a bf16 o.
 * FA_DTYPE_F32: float32 tensors, computed in float32 throughout (every product on the fp32
 * matrix instruction, P and dS kept in float32), as the reference accepts float32 q/k/v
 * (flash_attention_gpt_oss.py:356-357; benchmark_backward_speed.py:35-36). */
enum fa_dtype { FA_DTYPE_BF16 = 1, FA_DTYPE_F16 = 2, FA_DTYPE_FP8_E4M3 = 3, FA_DTYPE_F32 = 4 };

enum fa_status {
  FA_OK = 0,
  FA_ERR_NULL = -1,        /* a required pointer is NULL */
  FA_ERR_SHAPE = -2,       /* B, Hq, Hkv or L < 1, or Hq % Hkv != 0 */
  FA_ERR_HEAD_DIM = -3,    /* D not in {16, 32, 64, 128} */
  FA_ERR_DTYPE = -4,       /* dtype not an fa_dtype */
  FA_ERR_ALIGN = -5,       /* a tensor's base not 16-byte aligned, or a stride negative or not a
                              multiple of 16 bytes (8 16-bit, 4 float32 or 16 e4m3 elements); lse
                              not 4-byte aligned */
  FA_ERR_MASK = -6,        /* window < 1 and sink < 1: every query row would be fully masked */
  FA_ERR_WORKSPACE = -7,   /* workspace NULL or smaller than fa_bwd_workspace_bytes() */
  FA_ERR_LAUNCH = -8,      /* a HIP launch failed */
  FA_ERR_OVERFLOW = -9,    /* a size or element offset does not fit the kernels' index math */
  FA_ERR_SCALE = -10,      /* softmax_scale is NaN or infinite */
  FA_ERR_SCRATCH = -11     /* fa_bwd_scratch: the problem needs more workspace than FA_SCRATCH_BYTES */
};

/* Size of the library's own device scratch buffer used by fa_bwd_scratch (per GPU). */
#define FA_SCRATCH_BYTES (72u << 20) /* 72 MiB: the largest benchmark configuration (c5) needs 66.6 */

/* Forward pass.  Replaces the launch in FlashSWDAWithSink.forward
 * (flash_attention_gpt_oss.py:341-385) and the Triton _forward_kernel of the benchmark
 * (benchmark_backward_speed.py:146-217). */
typedef struct fa_fwd_params {
  const void* q;          /* [B, Hq, L, D]  */
  const void* k;          /* [B, Hkv, L, D] */
  const void* v;          /* [B, Hkv, L, D] */
  void* o;                /* [B, Hq, L, D]  output */
  float* lse;             /* [B, Hq, L]     output, natural-log log-sum-exp */
  int64_t q_stride[3];    /* batch, head, sequence strides in elements */
  int64_t k_stride[3];
  int64_t v_stride[3];
  int64_t o_stride[3];
  int64_t lse_stride[3];  /* any non-negative strides; lse needs 4-byte alignment only */
  int32_t batch, heads_q, heads_kv, seqlen, head_dim;
  int32_t window;         /* W: key k is in the window of query q when q - k < W */
  int32_t sink;           /* S: keys k < S are visible to every query q >= k */
  float softmax_scale;    /* the reference default is 1/sqrt(D), flash_attention_gpt_oss.py:345-346 */
  int32_t dtype;          /* enum fa_dtype */
} fa_fwd_params;

/* Backward pass.  Replaces FlashSWDAWithSink.backward's delta computation and kernel launch
 * (flash_attention_gpt_oss.py:387-435) and the split dQ / dK-dV kernels of the benchmark
 * (benchmark_backward_speed.py:312-466, 574-612).  dq, dk and dv are written in the input
 * dtype; dk and dv are complete sums over the Hq/Hkv query heads of each group, computed
 * without atomics, so reruns are bitwise identical. */
typedef struct fa_bwd_params {
  const void* q;
  const void* k;
  const void* v;
  const void* o;          /* forward output */
  const void* dout;       /* gradient of the loss with respect to o */
  const float* lse;       /* forward statistic from fa_fwd */
  void* dq;               /* [B, Hq, L, D]  output */
  void* dk;               /* [B, Hkv, L, D] output */
  void* dv;               /* [B, Hkv, L, D] output */
  int64_t q_stride[3];
  int64_t k_stride[3];
  int64_t v_stride[3];
  int64_t o_stride[3];
  int64_t do_stride[3];
  int64_t lse_stride[3];
  int64_t dq_stride[3];
  int64_t dk_stride[3];
  int64_t dv_stride[3];
  int32_t batch, heads_q, heads_kv, seqlen, head_dim;
  int32_t window;
  int32_t sink;
  float softmax_scale;
  int32_t dtype;
} fa_bwd_params;

/* Launches the forward kernel.  Returns FA_OK or a negative fa_status. */
int fa_fwd(const fa_fwd_params* p, void* stream);

/* Bytes of device workspace fa_bwd / fa_bwd_sinks need for this problem (row statistics of the
 * backward, per-chunk partial sums for the sink keys and per-row-block partial sums of the
 * learned sinks' gradient).  Returns 0 for an invalid problem.  The
 * reference instead allocates fp32 dK/dV staging buffers inside backward
 * (flash_attention_gpt_oss.py:397-400). */
size_t fa_bwd_workspace_bytes(int32_t batch, int32_t heads_q, int32_t heads_kv, int32_t seqlen,
                              int32_t head_dim, int32_t window, int32_t sink);

/* Launches the backward kernels (fa_bwd_dq then fa_bwd_dkdv).  `workspace` must hold
 * fa_bwd_workspace_bytes() bytes of device memory, 256-byte aligned; its contents on entry do
 * not matter. */
int fa_bwd(const fa_bwd_params* p, void* workspace, size_t workspace_bytes, void* stream);

/* The two stages of fa_bwd, for callers that schedule or time them separately.
 * fa_bwd_dq computes dq and stores the row statistic delta = rowsum(dout * o) in the workspace
 * (replaces the _backward_dq_kernel launch, benchmark_backward_speed.py:586-596, and the delta
 * computation of flash_attention_gpt_oss.py:403).  fa_bwd_dkdv computes dk and dv from that
 * workspace (replaces the _backward_dkdv_kernel launch, benchmark_backward_speed.py:600-611); it
 * must run after fa_bwd_dq on the same workspace, in stream order. */
int fa_bwd_dq(const fa_bwd_params* p, void* workspace, size_t workspace_bytes, void* stream);
int fa_bwd_dkdv(const fa_bwd_params* p, void* workspace, size_t workspace_bytes, void* stream);

/* fa_bwd without a workspace argument, for callers that cannot allocate device memory (code under
 * HIP graph capture, tight serving or training loops, harnesses that forbid hipMalloc).  No
 * counterpart in the reference (its backward allocates fp32 staging tensors,
 * flash_attention_gpt_oss.py:397-400).  The workspace is the library's own static device buffer
 * of FA_SCRATCH_BYTES bytes, one per GPU.  The buffer is part of the library's code object, so it is
 * reserved on a GPU when that object loads there (at the first launch of any of the library's
 * kernels on it, forward-only use included, whether or not fa_bwd_scratch is ever called) and held
 * until the process ends; the call itself allocates and frees nothing.  Its first call on a GPU looks
 * up the buffer's address there (hipGetSymbolAddress): make that call outside any graph capture,
 * after which calls may be captured.  Same arguments, checks, kernels and
 * results as fa_bwd (bitwise).  Returns FA_ERR_SCRATCH when fa_bwd_workspace_bytes() of the
 * problem exceeds FA_SCRATCH_BYTES.  Every call on one GPU shares that GPU's buffer: calls that
 * overlap in time on one GPU (concurrent streams, or host threads launching without ordering)
 * race on it and must be serialised by the caller; calls in one stream are ordered and safe. */
int fa_bwd_scratch(const fa_bwd_params* p, void* stream);

/* Learned attention sinks (GPT-OSS).  The reference has no such entry point: its sinks are the
 * first S key positions (benchmark_backward_speed.py:45, README.md:15).  GPT-OSS models instead
 * give every query head h a learned logit sinks[h] that joins each row's softmax denominator
 * without a value row:
 *     P[q, k] = exp(s[q, k] - lse[q]),
 *     lse[q]  = log( sum over allowed k of exp(s[q, k])  +  exp(sinks[h]) ),
 * which is the eager GptOssAttention path of HF transformers (the logits get one more column
 * holding the sink, are softmaxed, and the column is dropped).  The window and the positional
 * sinks of p still apply; GPT-OSS itself uses p->sink = 0 with window 128 (sliding layers) or
 * window >= L (full layers).  sinks is float32 [Hq], 4-byte aligned.
 * fa_fwd_sinks writes o and an lse that includes the sink term; fa_bwd_sinks must get that lse.
 * fa_bwd_sinks computes dq, dk and dv as fa_bwd does, and writes
 *     dsinks[h] = - sum over b, q of P_sink[b, h, q] * delta[b, h, q],
 *     P_sink = exp(sinks[h] - lse),  delta = rowsum(dout * o),
 * to dsinks (float32 [Hq], overwritten; summed in a fixed order, so reruns are identical). */
int fa_fwd_sinks(const fa_fwd_params* p, const float* sinks, void* stream);
int fa_bwd_sinks(const fa_bwd_params* p, const float* sinks, float* dsinks, void* workspace,
                 size_t workspace_bytes, void* stream);

/* Variable-length batches: `batch` sequences of different lengths whose rows are packed back to
 * back, as in a finetuning batch of concatenated samples.  The reference has fixed [B, H, L, D]
 * inputs only (flash_attention_gpt_oss.py:348); these entry points are the varlen form of
 * fa_fwd / fa_fwd_sinks and fa_bwd / fa_bwd_sinks.
 *   - q, o, dout, dq: [total_rows, Hq, D]; k, v, dk, dv: [total_rows, Hkv, D]; lse: float32 with
 *     one value per (head, row), e.g. [Hq, total_rows].  The head and row strides of each tensor
 *     are given as usual; batch strides are ignored.
 *   - cu_seqlens: int32 [batch + 1] in DEVICE memory, cu_seqlens[0] = 0, non-decreasing,
 *     cu_seqlens[batch] <= total_rows: sequence b is rows [cu_seqlens[b], cu_seqlens[b + 1]).
 *   - p->seqlen: the longest sequence (lengths are clamped to it, offsets to total_rows, so bad
 *     offsets cannot address memory outside the tensors; the results are then meaningless).
 *   - Causality, the window and the S positional sinks apply within each sequence: a row never
 *     sees another sequence's keys, and the sinks are each sequence's first S keys.
 *   - Rows that belong to no sequence, [0, cu_seqlens[0]) and [cu_seqlens[batch], total_rows),
 *     get o = 0 and lse = -inf from fa_fwd_varlen and zero dq, dk, dv from fa_bwd_varlen (one
 *     small extra launch, which exits at once when every row is covered).
 *   - sinks (float32 [Hq]) may be NULL; fa_bwd_varlen takes sinks and dsinks together or
 *     neither.  The workspace is fa_bwd_workspace_bytes(batch, Hq, Hkv, p->seqlen, D, W, S). */
int fa_fwd_varlen(const fa_fwd_params* p, const int32_t* cu_seqlens, int32_t total_rows, const float* sinks,
                  void* stream);
int fa_bwd_varlen(const fa_bwd_params* p, const int32_t* cu_seqlens, int32_t total_rows, const float* sinks,
                  float* dsinks, void* workspace, size_t workspace_bytes, void* stream);

/* FP8 forward: q, k and v hold OCP float8 e4m3 values (p->dtype = FA_DTYPE_FP8_E4M3, strides in
 * elements, i.e. bytes, multiples of 16, bases 16-byte aligned); the values they stand for are
 * q_descale * q, k_descale * k and v_descale * v.  o is written in bf16 (strides in bf16
 * elements, multiples of 8) and lse as by fa_fwd.  head_dim is 64 or 128.  Q K^T runs on the fp8
 * matrix cores; V is widened to bf16 exactly and P V runs as in fa_fwd, so the result is fa_fwd's
 * bf16 result for the dequantised inputs.  sinks (float32 [Hq] learned logits) may be NULL.  The
 * reference has no fp8 path (its kernels take fp16 / bf16 / fp32 tensors,
 * flash_attention_gpt_oss.py:356-383); this is the forward for the compute-bound shapes (long
 * full-causal layers, D = 128), forward only. */
int fa_fwd_fp8(const fa_fwd_params* p, float q_descale, float k_descale, float v_descale, const float* sinks,
               void* stream);

/* fa_fwd_fp8 with P V on the fp8 matrix cores as well (same arguments, checks and outputs).  The
 * softmax weights are rounded to e4m3 before the product.  A row's weights still sum to one (the
 * row sum adds the rounded values); a weight of at least 2^-10 of the row's largest carries a
 * relative rounding error of at most 2^-4, a smaller one an absolute error of at most 2^-14 of the
 * largest.  So o moves by at most 2^-4 of the weighted spread of v around o plus that absolute
 * term (the bound the tests check), and lse by at most -ln(1 - 2^-4) from fa_fwd_fp8's.  Same reference counterpart as
 * fa_fwd_fp8 (none: flash_attention_gpt_oss.py:356-383 takes 16/32-bit tensors only). */
int fa_fwd_fp8_pv(const fa_fwd_params* p, float q_descale, float k_descale, float v_descale, const float* sinks,
                  void* stream);

/* Host-only argument checks used by fa_fwd / fa_bwd (no HIP call is made). */
int fa_check_fwd(const fa_fwd_params* p);
int fa_check_bwd(const fa_bwd_params* p);

/* Static text for a status code. */
const char* fa_strerror(int status);

/* FA_GFX950_VERSION of the built library. */
int fa_version(void);

#ifdef __cplusplus
}
#endif

#endif /* FA_GFX950_H */
