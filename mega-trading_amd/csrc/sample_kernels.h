// Top-k sampling of one token per row, for generation: the draw that
// TradingModel.generate makes after each decode step (the reference's
// model.py:141-145: keep the logits >= the k-th largest, softmax,
// torch.multinomial for one sample), in the form torch.multinomial uses for
// one sample -- argmax over the row of p / E with E ~ Exponential(1), the
// noise E coming from the caller (drawn by torch from its generator, so the
// same seed gives the same stream).  One launch instead of a dozen library
// kernels (a multi-pass radix top-k, the mask, the softmax, the division, the
// argmax).
//
// One workgroup of 1024 threads per row, the row held in registers
// (EPT values per thread, vocab <= 1024 EPT).  The k-th largest value is
// found bit by bit on order-preserving 32-bit keys: from the most significant
// bit down, a bit is kept when at least k keys are >= the prefix with it set
// (32 block-wide counts); ties at the k-th value are all kept, as the
// reference's `logits < values[:, [-1]]` mask keeps them.  Then the maximum,
// the sum of exp(x - max) over the kept values, p = exp(x - max) / sum, and
// the first index of the largest p / E.
#pragma once

#include "mt_common.h"

namespace mt {

constexpr int kSampleThreads = 1024;

// order-preserving key of a float (larger float, larger key; NaN excluded)
__device__ __forceinline__ uint32_t sample_key(float x) {
  const uint32_t u = __float_as_uint(x);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

// block-wide max or sum of one float per thread (every thread gets it);
// `buf` holds kSampleThreads / 64 floats, reused: a barrier guards both ends
template <bool MAX>
__device__ __forceinline__ float block_reduce(float v, float* buf) {
  v = wave_reduce<0, MAX>(v);
  const int wave = threadIdx.x >> 6;
  __syncthreads();  // the previous reduction's reads of buf are done
  if ((threadIdx.x & 63) == 0) buf[wave] = v;
  __syncthreads();
  float r = buf[0];
#pragma unroll
  for (int w = 1; w < kSampleThreads / 64; ++w) r = red_op<MAX>(r, buf[w]);
  return r;
}

template <int EPT>
__global__ __launch_bounds__(kSampleThreads) void topk_sample_kernel(const float* logits, int64_t ld,
                                                                     const float* noise, int64_t ldn, int V, int k,
                                                                     int64_t* out) {
  __shared__ float buf[kSampleThreads / 64];
  const int tid = threadIdx.x;
  const float* x = logits + (int64_t)blockIdx.x * ld;
  const float* e = noise + (int64_t)blockIdx.x * ldn;
  float v[EPT];
  uint32_t key[EPT];
#pragma unroll
  for (int j = 0; j < EPT; ++j) {
    const int i = tid + j * kSampleThreads;
    v[j] = i < V ? x[i] : -INFINITY;
    key[j] = i < V ? sample_key(v[j]) : 0u;  // padding: below every real key (k <= V)
  }
  // the k-th largest key: the largest t with count(key >= t) >= k
  uint32_t t = 0;
  for (int bit = 31; bit >= 0; --bit) {
    const uint32_t cand = t | (1u << bit);
    float c = 0.f;
#pragma unroll
    for (int j = 0; j < EPT; ++j) c += key[j] >= cand ? 1.f : 0.f;
    if (block_reduce<false>(c, buf) >= (float)k) t = cand;
  }
  float m = -INFINITY;
#pragma unroll
  for (int j = 0; j < EPT; ++j)
    if (key[j] >= t) m = fmaxf(m, v[j]);
  m = block_reduce<true>(m, buf);
  float s = 0.f;
#pragma unroll
  for (int j = 0; j < EPT; ++j)
    if (key[j] >= t) s += expf(v[j] - m);
  s = block_reduce<false>(s, buf);
  const float inv = 1.f / s;
  // the largest p / E, first index among equals
  float best = -1.f, bi = (float)V;
#pragma unroll
  for (int j = 0; j < EPT; ++j) {
    const int i = tid + j * kSampleThreads;
    if (i < V && key[j] >= t) {
      const float q = expf(v[j] - m) * inv / e[i];
      if (q > best) {  // j ascending: the first index wins among this thread's equals
        best = q;
        bi = (float)i;
      }
    }
  }
  const float top = block_reduce<true>(best, buf);
  const float first = -block_reduce<true>(best == top ? -bi : -(float)V, buf);
  if (tid == 0) out[blockIdx.x] = (int64_t)first;
}

}  // namespace mt
