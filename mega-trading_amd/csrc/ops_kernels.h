// gfx950 kernels for the decoder's memory-bound operators around the
// attention: RMSNorm (optionally fused with the residual add), the SwiGLU
// gate and the stand-alone RoPE, forward and backward.
//
// Reference operators (src/mega_trading/kernels/triton_ops.py):
//   RMSNorm          :11-15, :133-184, kernels :528-539 (forward), :633-666 (backward)
//   add + RMSNorm    :18-42, :217-291, kernels :541-566, :569-608
//   SwiGLU gate      :57-61, :431-474, kernels :774-782, :799-819
//   cross-entropy rows of the fused linear cross-entropy :294-412, kernel :822-887
//   RoPE             :45-54, :187-214, kernel :690-761
//
// All of them move each byte once: one wave owns one row (RMSNorm, rows of D
// <= 4096 values held in registers as 8-value chunks), the SwiGLU gate streams
// 8 values per lane per step.  Arithmetic is fp32; storage is bf16, fp16 or
// fp32 (tensor dtype codes as in include/mt_ops.h).  The roundings the
// reference performs between steps are reproduced (e.g. silu(g) is rounded to
// the storage type before it multiplies `up`), so 16-bit results match the
// reference's to the last bit up to the last-ulp differences of exp.
#pragma once

#include <type_traits>

#include "mt_common.h"

namespace mt {
namespace ops {

constexpr int kDtBF16 = 0;
constexpr int kDtFP16 = 1;
constexpr int kDtFP32 = 2;

// ---------------------------------------------------------------------------
// storage <-> fp32, 8 consecutive values at a time (16 bytes for 16-bit types,
// 32 bytes for fp32); element offsets must be multiples of 8
// ---------------------------------------------------------------------------
template <int DT>
struct IO {
  static __device__ __forceinline__ void load8(const void* base, int64_t i, float* v) {
    if constexpr (DT == kDtFP32) {
      const f32x4* p = reinterpret_cast<const f32x4*>(static_cast<const float*>(base) + i);
      const f32x4 a = p[0], b = p[1];
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        v[k] = a[k];
        v[4 + k] = b[k];
      }
    } else {
      using E = typename std::conditional<DT == kDtBF16, BF16, FP16>::type;
      const u32x4 w = *reinterpret_cast<const u32x4*>(static_cast<const uint16_t*>(base) + i);
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        v[2 * k] = lo_f<E>(w[k]);
        v[2 * k + 1] = hi_f<E>(w[k]);
      }
    }
  }
  static __device__ __forceinline__ void store8(void* base, int64_t i, const float* v) {
    if constexpr (DT == kDtFP32) {
      f32x4* p = reinterpret_cast<f32x4*>(static_cast<float*>(base) + i);
      p[0] = f32x4{v[0], v[1], v[2], v[3]};
      p[1] = f32x4{v[4], v[5], v[6], v[7]};
    } else {
      using E = typename std::conditional<DT == kDtBF16, BF16, FP16>::type;
      u32x4 w;
#pragma unroll
      for (int k = 0; k < 4; ++k) w[k] = pack2<E>(v[2 * k], v[2 * k + 1]);
      *reinterpret_cast<u32x4*>(static_cast<uint16_t*>(base) + i) = w;
    }
  }
  static __device__ __forceinline__ float load1(const void* base, int64_t i) {
    if constexpr (DT == kDtFP32) return static_cast<const float*>(base)[i];
    else if constexpr (DT == kDtBF16) return BF16::to_f(static_cast<const uint16_t*>(base)[i]);
    else return FP16::to_f(static_cast<const uint16_t*>(base)[i]);
  }
  static __device__ __forceinline__ void store1(void* base, int64_t i, float x) {
    if constexpr (DT == kDtFP32) static_cast<float*>(base)[i] = x;
    else if constexpr (DT == kDtBF16) static_cast<uint16_t*>(base)[i] = uint16_t(pack2<BF16>(x, 0.f) & 0xffffu);
    else static_cast<uint16_t*>(base)[i] = uint16_t(pack2<FP16>(x, 0.f) & 0xffffu);
  }
  // the value x takes after a store to and a load from this storage type
  static __device__ __forceinline__ float round(float x) {
    if constexpr (DT == kDtFP32) return x;
    else if constexpr (DT == kDtBF16) return lo_f<BF16>(pack2<BF16>(x, 0.f));
    else return lo_f<FP16>(pack2<FP16>(x, 0.f));
  }
};

// Sum over the 64 lanes of a wave; every lane gets the same, bit-identical
// value (each butterfly level adds the same two operands on both partners).
__device__ __forceinline__ float wave_sum(float x) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) x += __shfl_xor(x, o, 64);
  return x;
}

// sigmoid(g) = 1 / (1 + e^-g) from the hardware exp2 and reciprocal
// (v_exp_f32, v_rcp_f32, about 1 ulp each) rather than the correctly rounded
// library sequences, which made the SwiGLU kernels issue-bound; e^-g = inf
// gives 0 and e^-g = 0 gives 1, as the exact formula does.
__device__ __forceinline__ float sigmoid_fast(float g) {
  return __builtin_amdgcn_rcpf(1.f + __builtin_amdgcn_exp2f(-g * kLog2e));
}

// ===========================================================================
// RMSNorm forward (ADD: the residual add fused in front)
//   ADD:  s = x + r (fp32), new_res = s (stored in ST), y = s * rstd * w
//   else: y = x * rstd * w
//   rstd = 1 / sqrt(mean(s^2) + eps) (fp32, one per row)
// Storage types: x in XT, residual and new_res in ST, y in YT.  One dtype for
// all of them is the reference operator; the mixed form (x and y 16-bit, the
// residual stream fp32) is the autocast decoder's residual add followed by
// the next norm, whose output the next projection reads in 16 bits anyway.
// One wave per row; lane L holds chunks L, L + 64, ... (8 values each).
// ===========================================================================
template <int XT, int ST, int YT, int WT, int NCH, bool ADD>
__global__ __launch_bounds__(256) void rmsnorm_fwd_kernel(const void* x, int64_t sx, const void* res, int64_t sr,
                                                          const void* w, void* new_res, void* y, float* rstd,
                                                          int64_t rows, int D, float eps) {
  const int wave = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * 4 + wave;
  if (row >= rows) return;
  const int nch = D >> 3;
  float v[NCH][8];
  float ss = 0.f;
#pragma unroll
  for (int k = 0; k < NCH; ++k) {
    const int c = lane + 64 * k;
    if (c < nch) {
      IO<XT>::load8(x, row * sx + 8 * c, v[k]);
      if constexpr (ADD) {
        float r[8];
        IO<ST>::load8(res, row * sr + 8 * c, r);
#pragma unroll
        for (int j = 0; j < 8; ++j) v[k][j] += r[j];
        IO<ST>::store8(new_res, row * D + 8 * c, v[k]);
      }
#pragma unroll
      for (int j = 0; j < 8; ++j) ss += v[k][j] * v[k][j];
    }
  }
  ss = wave_sum(ss);
  const float inv = __builtin_amdgcn_rsqf(ss / float(D) + eps);
#pragma unroll
  for (int k = 0; k < NCH; ++k) {
    const int c = lane + 64 * k;
    if (c < nch) {
      float wv[8], o[8];
      IO<WT>::load8(w, 8 * c, wv);
#pragma unroll
      for (int j = 0; j < 8; ++j) o[j] = v[k][j] * inv * wv[j];
      IO<YT>::store8(y, row * D + 8 * c, o);
    }
  }
  if (lane == 0) rstd[row] = inv;
}

// ===========================================================================
// RMSNorm backward.  With g = dy * w (fp32) and c = sum(g * s) over the row:
//   ds = rstd * (g - s * rstd^2 / D * c)        (+ d_new_res when ADD)
//   dw = sum over rows of dy * s * rstd         (per-workgroup partial sums)
// s is x (or the stored new residual when ADD).  s, d_new_res and ds in ST,
// dy in GT; when ds16 is not null ds is also written there in GT (the
// gradient of a 16-bit branch input of the mixed add).  Waves stride over
// rows; each lane accumulates its dw chunks in registers, the 4 waves of a
// workgroup combine them in LDS and write one fp32 partial row per workgroup.
// ===========================================================================
template <int ST, int GT, int WT, int NCH, bool ADD>
__global__ __launch_bounds__(256) void rmsnorm_bwd_kernel(const void* s, const void* w, const float* rstd,
                                                          const void* dy, const void* dres, void* ds, void* ds16,
                                                          float* partial, int64_t rows, int D) {
  __shared__ float red[3][NCH * 512];
  const int wave = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63;
  const int nch = D >> 3;
  const float inv_d = 1.f / float(D);
  float wv[NCH][8], acc[NCH][8];
#pragma unroll
  for (int k = 0; k < NCH; ++k) {
    const int c = lane + 64 * k;
#pragma unroll
    for (int j = 0; j < 8; ++j) acc[k][j] = 0.f;
    if (c < nch) IO<WT>::load8(w, 8 * c, wv[k]);
  }
  // U rows per iteration, all loads issued before any arithmetic, so each wave
  // keeps U rows of traffic in flight
  constexpr int U = NCH <= 2 ? 2 : 1;
  const int64_t waves = (int64_t)gridDim.x * 4;
  for (int64_t row0 = (int64_t)blockIdx.x * 4 + wave; row0 < rows; row0 += U * waves) {
    float sv[U][NCH][8], g[U][NCH][8], r[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int64_t row = row0 + u * waves;
      if (row < rows) {
        r[u] = rstd[row];
#pragma unroll
        for (int k = 0; k < NCH; ++k) {
          const int c = lane + 64 * k;
          if (c < nch) {
            IO<ST>::load8(s, row * D + 8 * c, sv[u][k]);
            IO<GT>::load8(dy, row * D + 8 * c, g[u][k]);
          }
        }
      }
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int64_t row = row0 + u * waves;
      if (row >= rows) break;
      float cs = 0.f;
#pragma unroll
      for (int k = 0; k < NCH; ++k) {
        const int c = lane + 64 * k;
        if (c < nch) {
#pragma unroll
          for (int j = 0; j < 8; ++j) {
            acc[k][j] += g[u][k][j] * sv[u][k][j] * r[u];
            g[u][k][j] *= wv[k][j];
            cs += g[u][k][j] * sv[u][k][j];
          }
        }
      }
      cs = wave_sum(cs);
      const float f = r[u] * r[u] * inv_d * cs;
#pragma unroll
      for (int k = 0; k < NCH; ++k) {
        const int c = lane + 64 * k;
        if (c < nch) {
          float o[8];
#pragma unroll
          for (int j = 0; j < 8; ++j) o[j] = r[u] * (g[u][k][j] - sv[u][k][j] * f);
          if constexpr (ADD) {
            float dr[8];
            IO<ST>::load8(dres, row * D + 8 * c, dr);
#pragma unroll
            for (int j = 0; j < 8; ++j) o[j] += dr[j];
          }
          IO<ST>::store8(ds, row * D + 8 * c, o);
          if (ds16) IO<GT>::store8(ds16, row * D + 8 * c, o);
        }
      }
    }
  }
  // workgroup reduction of dw: waves 1..3 park their sums, wave 0 adds them
  if (wave > 0) {
#pragma unroll
    for (int k = 0; k < NCH; ++k)
#pragma unroll
      for (int j = 0; j < 8; ++j) red[wave - 1][(lane + 64 * k) * 8 + j] = acc[k][j];
  }
  __syncthreads();
  if (wave == 0) {
#pragma unroll
    for (int k = 0; k < NCH; ++k) {
      const int c = lane + 64 * k;
      if (c < nch) {
        float o[8];
#pragma unroll
        for (int j = 0; j < 8; ++j)
          o[j] = acc[k][j] + red[0][c * 8 + j] + red[1][c * 8 + j] + red[2][c * 8 + j];
        IO<kDtFP32>::store8(partial, (int64_t)blockIdx.x * D + 8 * c, o);
      }
    }
  }
}

// dw[d] = sum over nb partial rows, stored as WT.  A block of 16 waves owns 64
// columns; wave q sums rows q, q + 16, ... into 8 independent accumulators (8
// loads in flight per lane), then wave 0 adds the 16 wave sums.  The order of
// every addition is fixed, so the result is deterministic.
constexpr int kColWaves = 16;

template <int WT>
__global__ __launch_bounds__(64 * kColWaves) void column_sum_kernel(const float* partial, int nb, int D, void* out) {
  __shared__ float part[kColWaves][64];
  const int wave = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63;
  const int d = blockIdx.x * 64 + lane;
  float acc = 0.f;
  if (d < D) {
    float a[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    int b = wave;
    for (; b + 7 * kColWaves < nb; b += 8 * kColWaves) {
#pragma unroll
      for (int k = 0; k < 8; ++k) a[k] += partial[(int64_t)(b + kColWaves * k) * D + d];
    }
    for (; b < nb; b += kColWaves) a[0] += partial[(int64_t)b * D + d];
    acc = ((a[0] + a[1]) + (a[2] + a[3])) + ((a[4] + a[5]) + (a[6] + a[7]));
  }
  part[wave][lane] = acc;
  __syncthreads();
  if (wave == 0 && d < D) {
    float t = 0.f;
#pragma unroll
    for (int q = 0; q < kColWaves; ++q) t += part[q][lane];
    IO<WT>::store1(out, d, t);
  }
}

// ===========================================================================
// SwiGLU gate: out = silu(g) * u, silu(g) = g / (1 + exp(-g)) in fp32.
// Forward rounds silu(g) to the storage type before the product
// (triton_ops.py:781: silu.to(up.dtype) * up).  Backward
// (triton_ops.py:814-819):
//   t  = dy * u                 rounded to the storage type
//   dg = (t * sig) * (1 + g (1 - sig)),  sig = 1 / (1 + exp(-g))
//   du = dy * round(silu(g))
// with silu(g) evaluated as in the forward, so du uses exactly the rounded
// forward activation.
// Flat over n values; lanes take 8 consecutive values, the last n % 8 values
// are handled one per lane.
// ===========================================================================
template <int DT>
__global__ __launch_bounds__(256) void swiglu_fwd_kernel(const void* gate, const void* up, void* out, int64_t n) {
  // two 8-value chunks per thread per iteration, both loaded before any arithmetic
  const int64_t nvec = n >> 3;
  const int64_t stride = (int64_t)gridDim.x * 256;
  for (int64_t i0 = (int64_t)blockIdx.x * 256 + threadIdx.x; i0 < nvec; i0 += 2 * stride) {
    float g[2][8], u[2][8];
#pragma unroll
    for (int q = 0; q < 2; ++q) {
      const int64_t i = i0 + q * stride;
      if (i < nvec) {
        IO<DT>::load8(gate, 8 * i, g[q]);
        IO<DT>::load8(up, 8 * i, u[q]);
      }
    }
#pragma unroll
    for (int q = 0; q < 2; ++q) {
      const int64_t i = i0 + q * stride;
      if (i < nvec) {
        float o[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) o[j] = IO<DT>::round(g[q][j] * sigmoid_fast(g[q][j])) * u[q][j];
        IO<DT>::store8(out, 8 * i, o);
      }
    }
  }
  const int64_t t = 8 * nvec + (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (t < n && (int64_t)blockIdx.x * 256 + threadIdx.x < 8) {
    const float g = IO<DT>::load1(gate, t);
    IO<DT>::store1(out, t, IO<DT>::round(g * sigmoid_fast(g)) * IO<DT>::load1(up, t));
  }
}

template <int DT>
__global__ __launch_bounds__(256) void swiglu_bwd_kernel(const void* gate, const void* up, const void* dout,
                                                         void* dgate, void* dup, int64_t n) {
  const int64_t nvec = n >> 3;
  const int64_t stride = (int64_t)gridDim.x * 256;
  for (int64_t i0 = (int64_t)blockIdx.x * 256 + threadIdx.x; i0 < nvec; i0 += 2 * stride) {
    float g[2][8], u[2][8], dy[2][8];
#pragma unroll
    for (int q = 0; q < 2; ++q) {
      const int64_t i = i0 + q * stride;
      if (i < nvec) {
        IO<DT>::load8(gate, 8 * i, g[q]);
        IO<DT>::load8(up, 8 * i, u[q]);
        IO<DT>::load8(dout, 8 * i, dy[q]);
      }
    }
#pragma unroll
    for (int q = 0; q < 2; ++q) {
      const int64_t i = i0 + q * stride;
      if (i < nvec) {
        float dg[8], du[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          const float sg = sigmoid_fast(g[q][j]);
          const float t = IO<DT>::round(dy[q][j] * u[q][j]);
          dg[j] = (t * sg) * (1.f + g[q][j] * (1.f - sg));
          du[j] = dy[q][j] * IO<DT>::round(g[q][j] * sg);
        }
        IO<DT>::store8(dgate, 8 * i, dg);
        IO<DT>::store8(dup, 8 * i, du);
      }
    }
  }
  const int64_t t = 8 * nvec + (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (t < n && (int64_t)blockIdx.x * 256 + threadIdx.x < 8) {
    const float g = IO<DT>::load1(gate, t), u = IO<DT>::load1(up, t), dy = IO<DT>::load1(dout, t);
    const float sg = sigmoid_fast(g);
    IO<DT>::store1(dgate, t, (IO<DT>::round(dy * u) * sg) * (1.f + g * (1.f - sg)));
    IO<DT>::store1(dup, t, dy * IO<DT>::round(g * sg));
  }
}

// The same gate over the packed output of one GEMM against the stacked
// (w1; w3) weights: row r of `gu` holds gate in columns [0, cols) and up in
// [cols, 2 cols); `out` is [rows, cols] and the backward's `dgu` has gu's
// layout.  cols % 8 == 0; thread i takes the 8-value chunk (r, c) =
// (i / cpr, i % cpr), cpr = cols / 8, with rows * cpr < 2^31.
template <int DT>
__global__ __launch_bounds__(256) void swiglu_packed_fwd_kernel(const void* gu, void* out, int rows, int cpr) {
  const int n = rows * cpr;
  for (int i = blockIdx.x * 256 + threadIdx.x; i < n; i += gridDim.x * 256) {
    const int r = i / cpr, c = i - r * cpr;
    const int64_t g0 = (int64_t)r * (16 * cpr) + 8 * c;
    float g[8], u[8], o[8];
    IO<DT>::load8(gu, g0, g);
    IO<DT>::load8(gu, g0 + 8 * cpr, u);
#pragma unroll
    for (int j = 0; j < 8; ++j) o[j] = IO<DT>::round(g[j] * sigmoid_fast(g[j])) * u[j];
    IO<DT>::store8(out, 8 * (int64_t)i, o);
  }
}

template <int DT>
__global__ __launch_bounds__(256) void swiglu_packed_bwd_kernel(const void* gu, const void* dout, void* dgu, int rows,
                                                                int cpr) {
  const int n = rows * cpr;
  for (int i = blockIdx.x * 256 + threadIdx.x; i < n; i += gridDim.x * 256) {
    const int r = i / cpr, c = i - r * cpr;
    const int64_t g0 = (int64_t)r * (16 * cpr) + 8 * c;
    float g[8], u[8], dy[8], dg[8], du[8];
    IO<DT>::load8(gu, g0, g);
    IO<DT>::load8(gu, g0 + 8 * cpr, u);
    IO<DT>::load8(dout, 8 * (int64_t)i, dy);
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const float sg = sigmoid_fast(g[j]);
      const float t = IO<DT>::round(dy[j] * u[j]);
      dg[j] = (t * sg) * (1.f + g[j] * (1.f - sg));
      du[j] = dy[j] * IO<DT>::round(g[j] * sg);
    }
    IO<DT>::store8(dgu, g0, dg);
    IO<DT>::store8(dgu, g0 + 8 * cpr, du);
  }
}

// ===========================================================================
// Cross-entropy over rows of logits (the loss head of the fused linear
// cross-entropy).  One workgroup (256 threads) per row of V logits:
//   pass 1: running (max, sum of exp) over the row, combined across the
//           threads;  lse = max + log(sum);  loss[row] = (lse - logit[label]) / n_valid
//   pass 2 (GRAD): logits[row] <- (exp(logit - lse) - [j == label]) / n_valid,
//           written over the logits in place
// With NCH > 0 each thread keeps its NCH chunks of 8 logits in registers
// between the passes (V <= 2048 * NCH: the row is read once); NCH == 0 streams
// the row twice.  exp is the hardware exp2 (v_exp_f32 on x * log2 e), accurate
// to a few fp32 ulps, far below the bf16 rounding of the logits.
// Rows whose label is ignore_index get loss 0 and (GRAD) a zero row.  n_valid is
// read from device memory (no host synchronisation); n_valid = 0 gives zeros.  A
// label outside [0, V) gives a NaN loss (the row is still read in bounds).
// When V is not a multiple of 8 the row's last chunk reaches into the row's
// padding (the row stride is at least V rounded up to 8): those columns count
// as -inf in pass 1 and are written 0 in pass 2.
// ===========================================================================
struct MaxSum {
  float m, s;
};

__device__ __forceinline__ MaxSum ms_combine(MaxSum a, MaxSum b) {
  if (a.m == -INFINITY) return b;
  if (b.m == -INFINITY) return a;
  const float m = fmaxf(a.m, b.m);
  return MaxSum{m, a.s * __expf(a.m - m) + b.s * __expf(b.m - m)};
}

// columns j >= n of a chunk of 8 are padding: -inf (no contribution)
__device__ __forceinline__ void mask_tail(float* v, int n) {
#pragma unroll
  for (int j = 0; j < 8; ++j)
    if (j >= n) v[j] = -INFINITY;
}

__device__ __forceinline__ MaxSum chunk_max_sum(const float* v) {
  float m = v[0];
#pragma unroll
  for (int j = 1; j < 8; ++j) m = fmaxf(m, v[j]);
  float sum = 0.f;
#pragma unroll
  for (int j = 0; j < 8; ++j) sum += __expf(v[j] - m);
  return MaxSum{m, sum};
}

template <int DT, bool GRAD, int NCH>
__global__ __launch_bounds__(256) void ce_rows_kernel(void* logits, int64_t ld, const int64_t* labels, int V,
                                                      const int64_t* n_valid, int64_t ignore_index, float* loss) {
  __shared__ MaxSum part[4];
  const int64_t row = blockIdx.x;
  const int tid = threadIdx.x;
  const int64_t base = row * ld;
  const int nvec = (V + 7) >> 3;
  const int tail = V - 8 * (nvec - 1);  // real columns of the last chunk (1..8)
  const int64_t label = labels[row];
  const int64_t nv = *n_valid;
  const float inv_n = nv > 0 ? 1.f / float(nv) : 0.f;
  if (label == ignore_index) {
    if constexpr (GRAD) {
      const float z[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
      for (int c = tid; c < nvec; c += 256) IO<DT>::store8(logits, base + 8 * c, z);
    }
    if (tid == 0) loss[row] = 0.f;
    return;
  }
  MaxSum acc{-INFINITY, 0.f};
  float v[NCH > 0 ? NCH : 1][8];
  if constexpr (NCH > 0) {
#pragma unroll
    for (int k = 0; k < NCH; ++k) {
      const int c = tid + 256 * k;
      if (c < nvec) {
        IO<DT>::load8(logits, base + 8 * c, v[k]);
        if (c == nvec - 1) mask_tail(v[k], tail);
      }
    }
#pragma unroll
    for (int k = 0; k < NCH; ++k)
      if (tid + 256 * k < nvec) acc = ms_combine(acc, chunk_max_sum(v[k]));
  } else {
    for (int c = tid; c < nvec; c += 256) {
      IO<DT>::load8(logits, base + 8 * c, v[0]);
      if (c == nvec - 1) mask_tail(v[0], tail);
      acc = ms_combine(acc, chunk_max_sum(v[0]));
    }
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    MaxSum other{__shfl_xor(acc.m, o, 64), __shfl_xor(acc.s, o, 64)};
    acc = ms_combine(acc, other);
  }
  if ((tid & 63) == 0) part[tid >> 6] = acc;
  __syncthreads();
  const MaxSum tot = ms_combine(ms_combine(part[0], part[1]), ms_combine(part[2], part[3]));
  const float lse = tot.m + __logf(tot.s);
  const bool ok = label >= 0 && label < V;
  if (tid == 0) {
    const float ly = IO<DT>::load1(logits, base + (ok ? label : 0));
    loss[row] = ok ? (lse - ly) * inv_n : __builtin_nanf("");
  }
  if constexpr (GRAD) {
    __syncthreads();  // the label's logit is read above before it is overwritten below
    auto grad8 = [&](int c, float* x) {
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const float p = __expf(x[j] - lse);  // 0 for the -inf padding
        x[j] = (p - (8 * c + j == label ? 1.f : 0.f)) * inv_n;
      }
      IO<DT>::store8(logits, base + 8 * c, x);
    };
    if constexpr (NCH > 0) {
#pragma unroll
      for (int k = 0; k < NCH; ++k) {
        const int c = tid + 256 * k;
        if (c < nvec) grad8(c, v[k]);
      }
    } else {
      for (int c = tid; c < nvec; c += 256) {
        IO<DT>::load8(logits, base + 8 * c, v[0]);
        if (c == nvec - 1) mask_tail(v[0], tail);
        grad8(c, v[0]);
      }
    }
  }
}

// ===========================================================================
// Stand-alone RoPE (triton_ops.py:187-214, kernel :690-761): every
// interleaved pair (e, o) of q and k becomes (e c - o s, e s + o c), with s
// negated for the backward (a rotation by -theta).  One launch covers the
// B*Hq*T query rows, then the B*Hkv*T key rows.  VEC (every d stride 1,
// D % 8 == 0, 16-byte aligned rows and table rows): a lane takes 8 values (4
// pairs); otherwise a lane takes one pair, any strides.  A lane reads its
// values before writing the same positions, so the output may be the input.
// ===========================================================================
struct RopeArgs {
  const void* src[2];  // q, k
  void* dst[2];        // q_out, k_out
  int64_t ss[2][4];    // (b, h, t, d) element strides of src
  int64_t sd[2][4];    // ... of dst
  int heads[2];        // Hq, Hkv
  int T;
  int half;            // D / 2
  const float* cos;    // [rows >= T, D / 2], row stride tstride, d stride 1
  const float* sin;
  int64_t tstride;
  float sign;          // +1 forward, -1 inverse
  int64_t n0;          // lane units of q
  int64_t n;           // lane units of q and k
};

// I: the index type of the (unit -> b, h, t, pair) decomposition; uint32_t
// whenever the unit count allows (64-bit divisions are long instruction
// sequences).  Rows are visited in memory order: (b, h, t) for [B, H, T, D]
// storage, (b, t, h) when the heads are interleaved per token (the model's
// projection views, [B, T, H, D] storage).
template <int DT, bool VEC, class I>
__global__ __launch_bounds__(256) void rope_kernel(RopeArgs a) {
  const I u = (I)blockIdx.x * 256 + threadIdx.x;
  if ((int64_t)u >= a.n) return;
  const int w = (int64_t)u >= a.n0 ? 1 : 0;
  const I local = u - (w ? (I)a.n0 : (I)0);
  constexpr int P = VEC ? 4 : 1;  // pairs per lane
  const I per_row = (I)(a.half / P);
  const int i = int(local % per_row) * P;  // first pair
  const I row = local / per_row;
  int t, h;
  I bq;
  if (a.ss[w][1] <= a.ss[w][2]) {  // heads inside tokens: row = (b T + t) H + h
    h = int(row % (I)a.heads[w]);
    const I bt = row / (I)a.heads[w];
    t = int(bt % (I)a.T);
    bq = bt / (I)a.T;
  } else {  // row = (b H + h) T + t
    t = int(row % (I)a.T);
    const I bh = row / (I)a.T;
    h = int(bh % (I)a.heads[w]);
    bq = bh / (I)a.heads[w];
  }
  const int64_t b = (int64_t)bq;
  const int64_t so = b * a.ss[w][0] + h * a.ss[w][1] + t * a.ss[w][2];
  const int64_t dO = b * a.sd[w][0] + h * a.sd[w][1] + t * a.sd[w][2];
  const float* cp = a.cos + t * a.tstride + i;
  const float* sp = a.sin + t * a.tstride + i;
  if constexpr (VEC) {
    float v[8];
    IO<DT>::load8(a.src[w], so + 2 * i, v);
    const f32x4 c = *reinterpret_cast<const f32x4*>(cp);
    const f32x4 s = *reinterpret_cast<const f32x4*>(sp);
#pragma unroll
    for (int p = 0; p < 4; ++p) {
      const float e = v[2 * p], o = v[2 * p + 1], sn = s[p] * a.sign;
      v[2 * p] = e * c[p] - o * sn;
      v[2 * p + 1] = e * sn + o * c[p];
    }
    IO<DT>::store8(a.dst[w], dO + 2 * i, v);
  } else {
    const int64_t sdd = a.ss[w][3], ddd = a.sd[w][3];
    const float e = IO<DT>::load1(a.src[w], so + 2 * i * sdd);
    const float o = IO<DT>::load1(a.src[w], so + (2 * i + 1) * sdd);
    const float c = *cp, sn = *sp * a.sign;
    IO<DT>::store1(a.dst[w], dO + 2 * i * ddd, e * c - o * sn);
    IO<DT>::store1(a.dst[w], dO + (2 * i + 1) * ddd, e * sn + o * c);
  }
}

}  // namespace ops
}  // namespace mt
