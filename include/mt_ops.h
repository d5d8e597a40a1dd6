/*
 * C ABI of the decoder operators around the attention (also in
 * libmt_attn.so): RMSNorm, residual-add + RMSNorm, the SwiGLU gate and the
 * stand-alone RoPE, forward and backward, and the cross-entropy rows of the
 * fused linear cross-entropy loss head, for MI355X (gfx950).  Plain pointers
 * and sizes only.
 *
 * They replace these reference operators (src/mega_trading/kernels/triton_ops.py):
 *
 *   mt_rms_norm_fwd      <- _TritonRMSNorm.forward :135-156 (kernel :528-539),
 *                           reached from triton_rms_norm :11-15 and
 *                           RMSNorm.forward, src/mega_trading/model.py:267-268
 *   mt_rms_norm_bwd      <- _TritonRMSNorm.backward :158-184 (kernel :633-666,
 *                           dW = partial_weight.sum(dim=0) :183)
 *   mt_add_rms_norm_fwd  <- _TritonAddRMSNorm.forward :219-249 (kernel :541-566),
 *                           reached from triton_add_rms_norm :18-42
 *   mt_add_rms_norm_bwd  <- _TritonAddRMSNorm.backward :251-291 (kernel :569-608)
 *   mt_swiglu_fwd        <- _TritonSwiGLUGate.forward :433-453 (kernel :774-782),
 *                           reached from triton_swiglu_gate :57-61 and
 *                           SwiGLU.forward, src/mega_trading/model.py:252-253
 *   mt_swiglu_bwd        <- _TritonSwiGLUGate.backward :455-474 (kernel :799-819)
 *   mt_rms_norm_fwd_mixed, mt_add_rms_norm_fwd_mixed, mt_rms_norm_bwd_mixed
 *                           no counterpart: the norms with an fp32 residual
 *                           stream and 16-bit activations (autocast decoder)
 *   mt_swiglu_packed_fwd / _bwd  no counterpart: the same gate on the packed
 *                           output of one GEMM against the stacked (w1; w3)
 *                           weights (this build's "hip" decoder route)
 *   mt_apply_rope        <- _TritonRoPE.forward / .backward :187-214 (kernel
 *                           _rope_kernel :690-761, launcher :477-525), reached
 *                           from triton_apply_rope :45-54 and
 *                           RotaryEmbedding.forward, src/mega_trading/model.py:292-293
 *   mt_linear_rows       <- the bias-free nn.Linear products of the decoder
 *                           (src/mega_trading/model.py:209-212, 243-245; applied at
 *                           :220-222, :237, :250-256) for the few rows of a decode
 *                           step (one token per rollout), several weights per launch
 *   mt_topk_sample       <- the top-k draw of TradingModel.generate
 *                           (src/mega_trading/model.py:141-145: topk, masked_fill,
 *                           softmax, multinomial for one sample) in one launch
 *   mt_cross_entropy_rows <- _fused_ce_row_kernel :822-887, the per-chunk loss and
 *                           in-place logits-gradient step of
 *                           _TritonFusedLinearCrossEntropy.forward :312-400,
 *                           reached from triton_fused_linear_cross_entropy :64-92
 *                           and TradingModel.forward_with_loss,
 *                           src/mega_trading/model.py:113-123
 *
 * Conventions (as in mt_attention.h): device pointers on the current device,
 * asynchronous on `stream`, no allocation, no synchronisation; 0 = success,
 * negative = argument error (MT_E_*), positive = hipError_t; the message is in
 * mt_last_error().
 *
 *   - dtype / weight_dtype: MT_DTYPE_BF16, MT_DTYPE_FP16 or MT_DTYPE_FP32;
 *     weight_dtype is either dtype or MT_DTYPE_FP32.  Arithmetic is fp32.
 *   - RMSNorm rows: x is [rows, dim] with row stride x_row_stride (elements,
 *     last stride 1); every other [rows, dim] tensor is contiguous.
 *     dim % 8 == 0 and 8 <= dim <= 4096; base pointers and row starts
 *     16-byte aligned.  rstd is fp32 [rows]: 1 / sqrt(mean(x^2) + eps).
 *   - SwiGLU: n values, contiguous, 16-byte aligned, any n >= 0.
 */
#ifndef MT_OPS_H_
#define MT_OPS_H_

#include <stddef.h>
#include <stdint.h>

#include "mt_attention.h"

#ifdef __cplusplus
extern "C" {
#endif

#define MT_DTYPE_FP32 2

/* y = x * rstd * weight; rstd written per row. */
int mt_rms_norm_fwd(const void* x, int64_t x_row_stride, const void* weight, void* y, float* rstd, int64_t rows,
                    int dim, float eps, int dtype, int weight_dtype, void* stream);

/* new_residual = x + residual (stored in dtype), y = RMSNorm(new_residual) computed
 * from the unrounded fp32 sum; rstd written per row. */
int mt_add_rms_norm_fwd(const void* x, int64_t x_row_stride, const void* residual, int64_t residual_row_stride,
                        const void* weight, void* new_residual, void* y, float* rstd, int64_t rows, int dim,
                        float eps, int dtype, int weight_dtype, void* stream);

/* Bytes of fp32 workspace the RMSNorm backward needs (per-workgroup dW partial rows). */
size_t mt_rms_norm_bwd_workspace_size(int64_t rows, int dim);

/* dx = rstd (dy w - x rstd^2 / dim * sum(dy w x)); dweight = sum over rows of dy x rstd
 * (written in weight_dtype).  x, dy, dx contiguous [rows, dim] in dtype. */
int mt_rms_norm_bwd(const void* x, const void* weight, const float* rstd, const void* dy, void* dx, void* dweight,
                    void* workspace, size_t workspace_bytes, int64_t rows, int dim, int dtype, int weight_dtype,
                    void* stream);

/* As mt_rms_norm_bwd on the stored new_residual, plus d_new_residual added to dx
 * (dx is the gradient of both x and residual). */
int mt_add_rms_norm_bwd(const void* new_residual, const void* weight, const float* rstd, const void* d_new_residual,
                        const void* dy, void* dx, void* dweight, void* workspace, size_t workspace_bytes,
                        int64_t rows, int dim, int dtype, int weight_dtype, void* stream);

/* Mixed-dtype forms for an autocast decoder: the residual stream (x of the
 * plain norm, residual / new_residual of the add) and the weight are fp32,
 * the activations (the branch output x of the add, y, dy) 16-bit
 * (act_dtype bf16 or fp16).  y is the fp32 result rounded once to act_dtype:
 * what the reference's fp32 norm followed by the next projection's autocast
 * cast produces (model.py:184-187 with F.rms_norm, model.py:267-268), with
 * the residual add of the block in front (new_residual = x + residual in
 * fp32, as torch promotes it).  No counterpart in the reference's Triton
 * operators (triton_ops.py:18-42 takes one dtype).
 *
 * mt_rms_norm_fwd_mixed: y = round(x * rstd * w), x fp32 (row stride), y act_dtype. */
int mt_rms_norm_fwd_mixed(const void* x, int64_t x_row_stride, const void* weight, void* y, float* rstd, int64_t rows,
                          int dim, float eps, int y_dtype, int weight_dtype, void* stream);

/* new_residual = x + residual (fp32), y = round(RMSNorm(new_residual)); x act_dtype. */
int mt_add_rms_norm_fwd_mixed(const void* x, int64_t x_row_stride, const void* residual, int64_t residual_row_stride,
                              const void* weight, void* new_residual, void* y, float* rstd, int64_t rows, int dim,
                              float eps, int act_dtype, int weight_dtype, void* stream);

/* Backward of both: s = the fp32 normalised input (x, or new_residual), dy
 * act_dtype; ds (fp32) = the norm backward plus d_new_residual when that is
 * not NULL; ds16, when not NULL, receives ds rounded to act_dtype (the
 * gradient of the add's 16-bit branch input).  dweight fp32; workspace as
 * for mt_rms_norm_bwd. */
int mt_rms_norm_bwd_mixed(const void* s, const void* weight, const float* rstd, const void* d_new_residual,
                          const void* dy, void* ds, void* ds16, void* dweight, void* workspace, size_t workspace_bytes,
                          int64_t rows, int dim, int act_dtype, int weight_dtype, void* stream);

/* out = round(silu(gate)) * up, silu(g) = g / (1 + exp(-g)). */
int mt_swiglu_fwd(const void* gate, const void* up, void* out, int64_t n, int dtype, void* stream);

/* dgate = round(dout * up) * sig * (1 + gate (1 - sig)), dup = dout * round(silu(gate)). */
int mt_swiglu_bwd(const void* gate, const void* up, const void* dout, void* dgate, void* dup, int64_t n, int dtype,
                  void* stream);

/* The same gate on the packed [rows, 2*cols] output of one GEMM against the
 * stacked (w1; w3) weights: gate = columns [0, cols) and up = [cols, 2*cols) of
 * each row; out [rows, cols] contiguous.  No counterpart in the reference (its
 * gate takes the two products separately, triton_ops.py:57-61): the packed form
 * lets the two FFN input projections share one GEMM without copies.
 * cols % 8 == 0, rows * cols / 8 < 2^31, pointers 16-byte aligned. */
int mt_swiglu_packed_fwd(const void* gu, void* out, int64_t rows, int64_t cols, int dtype, void* stream);

/* Backward of mt_swiglu_packed_fwd: dgu (gu's packed layout) = (dgate | dup) as in mt_swiglu_bwd. */
int mt_swiglu_packed_bwd(const void* gu, const void* dout, void* dgu, int64_t rows, int64_t cols, int dtype,
                         void* stream);

/* Cross-entropy rows: for each of `rows` rows of `vocab` logits (row stride
 * row_stride elements, dtype), loss_rows[r] = (logsumexp(row) - row[labels[r]]) / n_valid,
 * with *n_valid (device int64) the number of labels != ignore_index; rows labelled
 * ignore_index give 0.  With write_grad != 0 the logits are overwritten in place by
 * (softmax(row) - onehot(label)) / n_valid (zero rows for ignored labels).  A label
 * outside [0, vocab) gives a NaN loss.  Any vocab >= 1; row_stride is a multiple
 * of 8 and at least vocab rounded up to 8: when vocab % 8 != 0 the columns
 * [vocab, row_stride) of each row are read as padding (ignored) and, with
 * write_grad, overwritten with 0.  Rows 16-byte aligned. */
int mt_cross_entropy_rows(void* logits, int64_t row_stride, const int64_t* labels, int64_t rows, int vocab,
                          const int64_t* n_valid, int64_t ignore_index, float* loss_rows, int write_grad, int dtype,
                          void* stream);

/* Stand-alone RoPE of q [B, Hq, T, D] and k [B, Hkv, T, D]: each
 * interleaved pair (x[2i], x[2i+1]) = (e, o) of row t becomes
 *   (e c - o s, e s + o c),  c = rope_cos[t * table_stride + i], s = rope_sin[...]
 * with s negated when inverse != 0 (the backward: gradients rotated by -theta,
 * the reference's NEGATE_SIN).  strides: 16 element strides, (b, h, t, d) of
 * q, q_out, k, k_out in that order; any values (rows with d stride 1, D % 8 == 0
 * and 16-byte alignment take 8-value vector accesses).  An output may be its
 * input (same pointer and strides).  Tables fp32, d stride 1, at least T rows.
 * D even; arithmetic fp32, one rounding to dtype per value. */
int mt_apply_rope(const void* q, const void* k, void* q_out, void* k_out, int B, int Hq, int Hkv, int T, int D,
                  const int64_t* strides, const float* rope_cos, const float* rope_sin, int64_t table_stride,
                  int table_rows, int inverse, int dtype, void* stream);

/* Products of a few rows against grouped weights, fp32:
 *   y[m, off_g + n] = sum_k x[m, k] w_g[n, k],  off_g = out_features[0] + ... + out_features[g-1],
 * for m < rows, n < out_features[g], g < groups: the bias-free nn.Linear of each
 * weight w_g [out_features[g], in_features] (row stride w_row_strides[g]), the
 * results side by side in y's rows (y row stride y_row_stride >= the sum of
 * out_features).  `weights` and `out_features`, `w_row_strides` are host arrays
 * (device pointers in `weights`).  x is [rows, in_features] with row stride
 * x_row_stride, of type `dtype`: MT_DTYPE_FP32, or MT_DTYPE_BF16 / MT_DTYPE_FP16
 * (widened to fp32 exactly, as x.float() would); weights and y are fp32.  One
 * launch reads every weight in place (no concatenation): the decode step's
 * q|k|v and w1|w3 projections, and o_proj on the 16-bit attention output.
 * 1 <= groups <= 4; 1 <= rows <= 64; in_features a positive multiple of 128;
 * weights 16-byte aligned, x 16-byte (fp32) or 8-byte (16-bit) aligned, row
 * strides multiples of 4 elements.  Sums in fp32 (MFMA), in an order of this
 * kernel's own. */
int mt_linear_rows(const void* x, int64_t x_row_stride, const void* const* weights, const int* out_features,
                   const int64_t* w_row_strides, int groups, void* y, int64_t y_row_stride, int rows, int in_features,
                   int dtype, void* stream);

/* One sampled token per row: the logits >= the k-th largest of the row are
 * kept (ties at the k-th value included), p = softmax over the kept values,
 * and tokens[r] = the first index of the largest p / E[r, i] over the kept i,
 * with E the caller's Exponential(1) noise (one value per logit, e.g. drawn by
 * torch's exponential_ from its generator): the draw torch.multinomial makes for
 * one sample, without its host-side validity check.  logits and noise are fp32
 * [rows, vocab] with row strides >= vocab; tokens int64 [rows].  dtype
 * MT_DTYPE_FP32; 1 <= vocab <= 32768; 1 <= k <= vocab; rows >= 0. */
int mt_topk_sample(const void* logits, int64_t row_stride, const void* noise, int64_t noise_row_stride, int rows,
                   int vocab, int k, int64_t* tokens, int dtype, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* MT_OPS_H_ */
