/*
 * C ABI of the MI355X (gfx950) causal grouped-query attention library
 * (libmt_attn.so).  Plain pointers and sizes only; no torch types.
 *
 * These entry points replace the reference's operator boundary for its
 * attention hot path (paths relative to the duoan/mega-trading tree):
 *
 *   mt_gqa_attn_fwd  <- _TritonCausalAttention.forward,
 *                       src/mega_trading/kernels/triton_attention.py:28-78
 *                       (the kernel launches at :40-74).  With rope_cos /
 *                       rope_sin set it also replaces the RoPE launch that
 *                       precedes it, triton_apply_rope / _TritonRoPE.forward,
 *                       src/mega_trading/kernels/triton_ops.py:45-54,187-202,
 *                       as called from src/mega_trading/model.py:223.
 *   mt_gqa_attn_bwd  <- _TritonCausalAttention.backward,
 *                       src/mega_trading/kernels/triton_attention.py:80-111,
 *                       and _triton_attention_server_backward :134-245
 *                       (dQ kernel :154, dK/dV kernel :197).  With RoPE tables
 *                       it also replaces _TritonRoPE.backward,
 *                       src/mega_trading/kernels/triton_ops.py:204-214.
 *
 * Conventions shared by every entry point:
 *   - All tensor pointers are device pointers on the current HIP device.
 *   - Tensors are [B, H, T, D]; strides are in elements and ordered
 *     (b, h, t, d); the d stride must be 1 (the others are free, so the
 *     [B, T, H, D]-physical views the model produces are accepted as is).
 *   - K and V have Hkv heads, Q / O / dO / dQ have Hq = Hkv * repeats heads;
 *     query head h reads KV head h / repeats (triton_attention.py:299).
 *   - Causal, top-left aligned, Tq == Tk == T, any T >= 1.
 *   - D in {32, 64, 128}; dtype MT_DTYPE_BF16 or MT_DTYPE_FP16, or MT_DTYPE_FP32
 *     for the forward and backward (computed in full fp32 on fp32 MFMA: at
 *     least the precision of the reference's fp32 path, whose forward dots
 *     run in TF32 and whose backward is dense fp32, triton_attention.py:88-111).
 *     Decode takes 16-bit caches only.
 *   - lse is fp32 [B, Hq, T] contiguous, the natural-log logsumexp of the
 *     scaled scores (triton_attention.py:346-349).
 *   - rope_cos / rope_sin: either both NULL (no RoPE) or both fp32
 *     [>= T, D/2] contiguous tables, row t = position t
 *     (src/mega_trading/model.py:279-284).  The rotation acts on interleaved
 *     pairs (x[2i], x[2i+1]) (model.py:312-316).
 *   - stream is a hipStream_t (NULL = the legacy default stream).  Calls are
 *     asynchronous, never synchronise, never allocate device memory, and are
 *     safe to record into a HIP graph.
 *   - Return 0 on success.  Negative values are argument errors
 *     (MT_E_*), positive values are hipError_t codes from the launch.
 *     mt_last_error() describes the most recent failure of the calling thread.
 */
#ifndef MT_ATTENTION_H_
#define MT_ATTENTION_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define MT_DTYPE_BF16 0
#define MT_DTYPE_FP16 1
#define MT_DTYPE_FP32 2 /* attention forward / backward only; full-fp32 MFMA kernels */

#define MT_OK 0
#define MT_E_NULL (-1)      /* a required pointer is NULL */
#define MT_E_SHAPE (-2)     /* B/H/T/D/repeats inconsistent or unsupported */
#define MT_E_STRIDE (-3)    /* d stride != 1, or misaligned rows / buffers */
#define MT_E_DTYPE (-4)     /* dtype code not supported */
#define MT_E_ROPE (-5)      /* exactly one of rope_cos / rope_sin given */
#define MT_E_WORKSPACE (-6) /* backward workspace smaller than required */
#define MT_E_DEVICE (-7)    /* the stream belongs to a device other than the current one */

/* Library version, (major << 16) | minor. */
int mt_version(void);

/* Message of the calling thread's last failure ("" if none). */
const char* mt_last_error(void);

/*
 * Forward.  O = softmax(scale * rot(Q) rot(K)^T + causal) V and its LSE.
 *   q [B,Hq,T,D], k/v [B,Hkv,T,D], o [B,Hq,T,D] (written), lse [B,Hq,T] (written).
 *   strides: 16 int64 = q, k, v, o, 4 each in (b, h, t, d) order.
 *   With RoPE tables: q_rot [B,Hq,T,D] and k_rot [B,Hkv,T,D] (contiguous,
 *   written) receive the rotated Q and K; the backward consumes them in place
 *   of q and k.  Without tables both may be NULL.
 */
int mt_gqa_attn_fwd(const void* q, const void* k, const void* v, void* o, float* lse,
                    void* q_rot, void* k_rot,
                    int B, int Hq, int Hkv, int T, int D,
                    const int64_t* strides, float scale, int dtype,
                    const float* rope_cos, const float* rope_sin, void* stream);

/* Bytes of device workspace mt_gqa_attn_bwd needs for this shape on the
 * current device (0 for an invalid shape), for 16-bit inputs: an upper bound
 * for every dtype (fp32 inputs need only the delta / LSE vectors). */
size_t mt_gqa_attn_bwd_workspace_size(int B, int Hq, int Hkv, int T, int D);

/* As mt_gqa_attn_bwd_workspace_size for one dtype (MT_DTYPE_*): the exact
 * size mt_gqa_attn_bwd checks against for that dtype.  No separate reference
 * counterpart: the reference's backward allocates its own buffers
 * (triton_attention.py:88-111, 148-150). */
size_t mt_gqa_attn_bwd_workspace_size_dtype(int B, int Hq, int Hkv, int T, int D, int dtype);

/*
 * Backward.  Given dO, writes dQ, dK, dV.
 *   q, k: the tensors the forward's scores were computed from -- q_rot and
 *   k_rot when RoPE tables are given, in which case dQ and dK are rotated back
 *   by -theta and returned in the un-rotated basis (triton_ops.py:205-214).
 *   workspace: 256-byte aligned device buffer of at least
 *   mt_gqa_attn_bwd_workspace_size_dtype() bytes (delta = rowsum(O * dO),
 *   triton_attention.py:561, and fp32 dK/dV partial sums).
 *   strides: 32 int64 = q, k, v, o, dO, dQ, dK, dV, 4 each in (b, h, t, d) order.
 *   dQ/dK/dV are fully overwritten (no zero-fill needed).
 */
int mt_gqa_attn_bwd(const void* q, const void* k, const void* v, const void* o, const float* lse,
                    const void* dout, void* dq, void* dk, void* dv, void* workspace, size_t workspace_size,
                    int B, int Hq, int Hkv, int T, int D,
                    const int64_t* strides, float scale, int dtype,
                    const float* rope_cos, const float* rope_sin, void* stream);

/*
 * Allocation-free backward.  No counterpart in the reference: it is for
 * callers that cannot allocate device memory -- code under HIP graph capture,
 * tight serving loops, harnesses that forbid hipMalloc.  Same arguments and
 * results as mt_gqa_attn_bwd without the workspace: the delta / LSE vectors
 * and the dK/dV partial sums live in a fixed device array of
 * MT_NOALLOC_SCRATCH_BYTES that each GPU the library runs on holds until the
 * process ends.  The dK/dV head split is mt_gqa_attn_bwd's when its partials
 * fit (then the results are bit-identical), else the largest smaller one that
 * fits; a shape whose delta and LSE vectors alone (8 * B * Hq * T bytes,
 * rounded up) exceed the array returns MT_E_WORKSPACE, and an invalid shape
 * its MT_E_* code, before any device call.
 * Nothing in the array needs to start at zero: every value read was written
 * earlier in the same call.  All calls on one GPU share that GPU's array, so
 * calls that overlap in time on one GPU (other streams, other threads) race;
 * serialise them.  Calls no hipMalloc / hipFree.  The stream, when given,
 * must belong to the current device (else MT_E_DEVICE).
 */
#define MT_NOALLOC_SCRATCH_BYTES ((size_t)64 << 20)
int mt_gqa_attn_bwd_noalloc(const void* q, const void* k, const void* v, const void* o, const float* lse,
                            const void* dout, void* dq, void* dk, void* dv, int B, int Hq, int Hkv, int T, int D,
                            const int64_t* strides, float scale, int dtype, const float* rope_cos,
                            const float* rope_sin, void* stream);

/*
 * The two halves of mt_gqa_attn_bwd, for callers that schedule or time the
 * backward kernels separately (same arguments and conventions).
 *   mt_gqa_attn_bwd_dq  <- _triton_attention_backward_dq_server_kernel launch,
 *                          triton_attention.py:154-195; writes dQ and delta.
 *   mt_gqa_attn_bwd_dkv <- _triton_attention_backward_dkv_server_kernel launch,
 *                          triton_attention.py:197-244; reads delta, so it
 *                          must follow mt_gqa_attn_bwd_dq on the same stream.
 */
int mt_gqa_attn_bwd_dq(const void* q, const void* k, const void* v, const void* o, const float* lse,
                       const void* dout, void* dq, void* dk, void* dv, void* workspace, size_t workspace_size,
                       int B, int Hq, int Hkv, int T, int D,
                       const int64_t* strides, float scale, int dtype,
                       const float* rope_cos, const float* rope_sin, void* stream);
int mt_gqa_attn_bwd_dkv(const void* q, const void* k, const void* v, const void* o, const float* lse,
                        const void* dout, void* dq, void* dk, void* dv, void* workspace, size_t workspace_size,
                        int B, int Hq, int Hkv, int T, int D,
                        const int64_t* strides, float scale, int dtype,
                        const float* rope_cos, const float* rope_sin, void* stream);

/*
 * Kernel timing (no counterpart in the reference, whose benchmark times the
 * whole op, scripts/benchmark_triton_attention.py:164-176).  Arms two created
 * HIP events (hipEvent_t, passed as void*) that the next mt_gqa_attn_* call
 * made by this thread attaches to its main kernel (attn_fwd, attn_bwd_dq or
 * attn_bwd_dkv -- the first of these it launches) through hipExtLaunchKernel,
 * so their elapsed time is that dispatch's own duration, without helper passes
 * such as the K RoPE pass and the dK/dV partial-sum combine.  The events are
 * disarmed after that launch.  Both NULL disarms.  For benchmarks and
 * profilers.
 */
int mt_time_next_kernel(void* start_event, void* stop_event);

/*
 * As mt_time_next_kernel for the next n main kernels launched by any thread
 * of the process, in launch order: launch i takes start_events[i] and
 * stop_events[i].  A thread's own mt_time_next_kernel arming is used first.
 * For timing kernels that a framework launches from its own threads (the
 * backward runs on the autograd engine's device thread).  The arrays are
 * copied; n = 0 disarms.  No reference counterpart (benchmark support).
 */
int mt_time_kernel_queue(void* const* start_events, void* const* stop_events, int n);

/*
 * Decode attention for KV-cached generation: one new query token per sequence
 * (at position L-1) against cached keys/values 0..L-1.  It replaces the
 * attention inside the per-token full recompute of TradingModel.generate,
 * src/mega_trading/model.py:134-147 (model.py:139-140 runs the whole context
 * through every layer for each new token): the result equals the last row of
 * the causal forward over the L cached positions (triton_attention.py:28-78).
 *   q [B,Hq,1,D] (rotated if RoPE is used), k_cache / v_cache [B,Hkv,>=L,D]
 *   (rotated keys), o [B,Hq,1,D] written; strides: 16 int64 = q, k_cache,
 *   v_cache, o in (b, h, t, d) order (the t stride of q and o is unused).
 *   Hq / Hkv <= 8; L >= 1.  The fp32 workspace (16-byte aligned) holds one
 *   partial per 64-key split (mt_gqa_attn_decode_workspace_size).
 */
size_t mt_gqa_attn_decode_workspace_size(int B, int Hq, int L, int D);
int mt_gqa_attn_decode(const void* q, const void* k_cache, const void* v_cache, void* o, int B, int Hq, int Hkv,
                       int L, int D, const int64_t* strides, float scale, int dtype, void* workspace,
                       size_t workspace_bytes, void* stream);
/* As mt_gqa_attn_decode with the length read from device memory (*length_dev,
 * clamped to [1, capacity]) when the kernels run, so one recorded launch
 * (e.g. in a HIP graph) serves every decode step; the grid and the workspace
 * (mt_gqa_attn_decode_workspace_size(B, Hq, capacity, D)) cover the capacity. */
int mt_gqa_attn_decode_dev(const void* q, const void* k_cache, const void* v_cache, void* o, int B, int Hq, int Hkv,
                           int capacity, const int* length_dev, int D, const int64_t* strides, float scale, int dtype,
                           void* workspace, size_t workspace_bytes, void* stream);

/*
 * The decode step's RoPE and cache append (no reference counterpart as one
 * call: it is the per-token share of model.py:223's rotation plus the cache
 * write that KV-cached generation adds).  q [B,Hq,D], k/v [B,Hkv,D] (views of
 * the new token's projections, in_strides: 6 int64 = (b, h) of q, k, v; d
 * stride 1; in_dtype bf16, fp16 or 2 = fp32) are rounded to the cache dtype,
 * rotated by position `pos` (fp32 tables [>= pos+1, D/2]) and written: q_rot
 * [B,Hq,1,D] contiguous, k_cache[:, :, pos] and v_cache[:, :, pos]
 * (cache_strides: 6 int64 = (b, h, t) of k_cache, v_cache).  With pos_dev set
 * the position is read from device memory when the kernel runs, clamped to
 * [0, pos] (pass the last valid position as pos).  table_rows (rows of the
 * RoPE tables) and capacity (positions of the caches) bound pos: a pos at or
 * past either is rejected before the launch.
 */
int mt_decode_rope_append(const void* q, const void* k, const void* v, const int64_t* in_strides,
                          const float* rope_cos, const float* rope_sin, int table_rows, int pos, const int* pos_dev,
                          void* q_rot, void* k_cache, void* v_cache, const int64_t* cache_strides, int capacity,
                          int B, int Hq, int Hkv, int D, int in_dtype, int dtype, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* MT_ATTENTION_H_ */
