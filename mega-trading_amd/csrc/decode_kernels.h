// gfx950 decode attention: one new query token per sequence against a KV cache,
// for KV-cached generation (the reference's TradingModel.generate,
// src/mega_trading/model.py:134-147, recomputes the whole context per token
// instead; the maths is the causal GQA attention of triton_attention.py for the
// last query row, whose keys are all cached positions).
//
// Split-K ("flash decoding"): the cached keys 0..L-1 are cut into 256-key
// splits; workgroup (batch, KV head, split) scores its split for all R query
// heads of the KV group (each K/V row is read once for the R heads), forms the
// split's softmax numerator and running offset, and writes an fp32 partial
// (o, m, l).  A second kernel merges the splits with the log-sum-exp rule.
// The work is HBM-bound (the cache is read once), so it uses plain fp32 FMAs:
// with one query row per head there is no matrix product to feed the MFMAs.
#pragma once

#include "mt_common.h"

namespace mt {

constexpr int kDecSplit = 256;  // keys per split (one per thread in the score pass)
constexpr int kDecMaxR = 8;     // query heads per KV head supported

struct DecodeParams {
  const uint16_t* q;  // [B, Hq, 1, D] (rotated when RoPE is used)
  const uint16_t* k;  // [B, Hkv, >= L, D] cache (rotated keys)
  const uint16_t* v;  // [B, Hkv, >= L, D] cache
  uint16_t* out;      // [B, Hq, 1, D]
  float* part;        // [B, Hq, nsplit, D + 2] fp32: o (unnormalised), m (log2), l
  int64_t sq[2], sk[3], sv[3], so[2];  // strides (b, h) for q / o, (b, h, t) for the caches
  const int* length_dev;  // when set, L is read from device memory (graph-replayable decode)
  int B, Hq, Hkv, R, L, nsplit;  // nsplit: splits in the grid (of the capacity when length_dev is set)
  float scale_log2;  // softmax scale * log2(e)
};

// With length_dev, L holds the capacity and the device value is clamped to [1, capacity].
__device__ __forceinline__ int decode_length(const DecodeParams& p) {
  return p.length_dev ? min(max(*p.length_dev, 1), p.L) : p.L;
}

template <class E, int D>
__global__ __launch_bounds__(256) void attn_decode_split_kernel(DecodeParams p) {
  __shared__ float qs[kDecMaxR][D];
  __shared__ float ps[kDecMaxR][kDecSplit];
  __shared__ float red[kDecMaxR][4];
  __shared__ float red_buf[(256 / (D / 8)) * kDecMaxR * D];  // V-pass key-group sums (64 KB)
  const int tid = threadIdx.x;
  const int wave = tid >> 6;
  const int lane = tid & 63;
  const int s = blockIdx.x % p.nsplit;
  const int g = blockIdx.x / p.nsplit;
  const int kvh = g % p.Hkv;
  const int b = g / p.Hkv;
  const int R = p.R;
  const int k0 = s * kDecSplit;
  const int L = decode_length(p);
  if (k0 >= L) return;  // a split past the current length (device-length launches cover the capacity)
  const int n = min(kDecSplit, L - k0);

  // Every K and V load of this thread is issued first, so the score, softmax
  // and V passes wait on one memory round trip: the K row of key k0 + tid,
  // and the 16-byte V chunks of the V pass (chunk c = tid % NC of keys
  // tid / NC, tid / NC + G, ...).
  constexpr int NC = D / 8;      // 16-byte chunks per V row
  constexpr int G = 256 / NC;    // key groups of the V pass
  constexpr int NV = kDecSplit / G;  // V chunks per thread
  u32x4 kw[D / 8], vw[NV];
  if (tid < n) {
    const uint16_t* krow = p.k + b * p.sk[0] + (int64_t)kvh * p.sk[1] + (int64_t)(k0 + tid) * p.sk[2];
#pragma unroll
    for (int c = 0; c < D / 8; ++c) kw[c] = *reinterpret_cast<const u32x4*>(krow + 8 * c);
  }
  const uint16_t* vbase = p.v + b * p.sv[0] + (int64_t)kvh * p.sv[1] + (int64_t)k0 * p.sv[2];
  const int c = tid % NC;
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const int j = tid / NC + i * G;
    if (j < n) vw[i] = *reinterpret_cast<const u32x4*>(vbase + (int64_t)j * p.sv[2] + 8 * c);
  }

  for (int i = tid; i < R * D; i += 256) {
    const int h = i / D, d = i % D;
    qs[h][d] = E::to_f(p.q[b * p.sq[0] + (int64_t)(kvh * R + h) * p.sq[1] + d]);
  }
  __syncthreads();

  // scores of key k0 + tid for every head (log2 units)
  float sc[kDecMaxR];
#pragma unroll
  for (int h = 0; h < kDecMaxR; ++h) sc[h] = 0.f;
  if (tid < n) {
#pragma unroll
    for (int c8 = 0; c8 < D / 8; ++c8) {
      const u32x4 w = kw[c8];
      float kv[8];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        kv[2 * e] = lo_f<E>(w[e]);
        kv[2 * e + 1] = hi_f<E>(w[e]);
      }
#pragma unroll
      for (int h = 0; h < kDecMaxR; ++h)
        if (h < R)
#pragma unroll
          for (int e = 0; e < 8; ++e) sc[h] = __builtin_fmaf(qs[h][8 * c8 + e], kv[e], sc[h]);
    }
  }
  // per-head max over the split
#pragma unroll
  for (int h = 0; h < kDecMaxR; ++h) {
    if (h >= R) break;
    float v = tid < n ? sc[h] * p.scale_log2 : -INFINITY;
    sc[h] = v;
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
    if (lane == 0) red[h][wave] = v;
  }
  __syncthreads();
  float m[kDecMaxR];
#pragma unroll
  for (int h = 0; h < kDecMaxR; ++h)
    m[h] = h < R ? fmaxf(fmaxf(red[h][0], red[h][1]), fmaxf(red[h][2], red[h][3])) : 0.f;
  __syncthreads();  // red is reused for the sums
  // probabilities (0 past the split's last key) and their per-head sums
#pragma unroll
  for (int h = 0; h < kDecMaxR; ++h) {
    if (h >= R) break;
    const float e = tid < n ? exp2_fast(sc[h] - m[h]) : 0.f;
    ps[h][tid] = e;
    float v = e;
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
    if (lane == 0) red[h][wave] = v;
  }
  __syncthreads();

  // o[h][d] = sum_j p[h][j] V[k0 + j][d].  Thread t takes the 8-value d chunk
  // c = t % NC of keys j = t / NC, t / NC + G, ... (one 16-byte load per key,
  // issued at the start, feeds 8 d values of every head), then the G key
  // groups are summed through LDS.
  float acc[kDecMaxR][8];
#pragma unroll
  for (int h = 0; h < kDecMaxR; ++h)
#pragma unroll
    for (int e = 0; e < 8; ++e) acc[h][e] = 0.f;
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const int j = tid / NC + i * G;
    if (j >= n) break;
    const u32x4 w = vw[i];
    float vv[8];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      vv[2 * e] = lo_f<E>(w[e]);
      vv[2 * e + 1] = hi_f<E>(w[e]);
    }
#pragma unroll
    for (int h = 0; h < kDecMaxR; ++h) {
      if (h < R) {
        const float pj = ps[h][j];
#pragma unroll
        for (int e = 0; e < 8; ++e) acc[h][e] = __builtin_fmaf(pj, vv[e], acc[h][e]);
      }
    }
  }
  // key-group partial sums: red_o[g][h][d]
  float* red_o = red_buf;
  const int kg = tid / NC;
#pragma unroll
  for (int h = 0; h < kDecMaxR; ++h)
    if (h < R)
#pragma unroll
      for (int e = 0; e < 8; ++e) red_o[(kg * kDecMaxR + h) * D + 8 * c + e] = acc[h][e];
  __syncthreads();
  for (int i = tid; i < R * D; i += 256) {
    const int h = i / D, d = i % D;
    float o = 0.f;
#pragma unroll 8
    for (int gg = 0; gg < G; ++gg) o += red_o[(gg * kDecMaxR + h) * D + d];
    float* dst = p.part + (((int64_t)b * p.Hq + kvh * R + h) * p.nsplit + s) * (D + 2);
    dst[d] = o;
    if (d == 0) {
      dst[D] = m[h];
      dst[D + 1] = (red[h][0] + red[h][1]) + (red[h][2] + red[h][3]);
    }
  }
}

// Merge the splits of each (batch, query head): M = max m_s,
// O = sum_s 2^(m_s - M) o_s / sum_s 2^(m_s - M) l_s.  One thread per d value.
template <class E, int D>
__global__ __launch_bounds__(256) void attn_decode_combine_kernel(DecodeParams p) {
  constexpr int PER = 256 / D;  // (batch, head) pairs per workgroup
  const int pair = blockIdx.x * PER + threadIdx.x / D;
  const int d = threadIdx.x % D;
  if (pair >= p.B * p.Hq) return;
  const int b = pair / p.Hq, h = pair % p.Hq;
  const float* src = p.part + (int64_t)pair * p.nsplit * (D + 2);
  const int ns = (decode_length(p) + kDecSplit - 1) / kDecSplit;  // splits holding keys
  float M = -INFINITY;
  for (int s = 0; s < ns; ++s) M = fmaxf(M, src[s * (D + 2) + D]);
  float o = 0.f, l = 0.f;
  for (int s = 0; s < ns; ++s) {
    const float w = exp2_fast(src[s * (D + 2) + D] - M);
    o = __builtin_fmaf(w, src[s * (D + 2) + d], o);
    l = __builtin_fmaf(w, src[s * (D + 2) + D + 1], l);
  }
  const float r = o / l;
  p.out[b * p.so[0] + (int64_t)h * p.so[1] + d] = uint16_t(pack2<E>(r, 0.f) & 0xffffu);
}

// ---------------------------------------------------------------------------
// The new token's RoPE and cache append, in one launch: q_rot = rot(q) (written
// [B, Hq, 1, D]), k_cache[:, :, pos] = rot(k), v_cache[:, :, pos] = v.  The
// inputs (views of the projections, [B, H, D] with strides (b, h), d stride 1)
// are first rounded to the cache's 16-bit type, then rotated in fp32 with the
// fp32 tables row `pos` and rounded again -- the sequence the fused forward
// kernels apply to the prompt, so cached and recomputed keys are identical.
// One thread per interleaved pair (x[2i], x[2i+1]).
// ---------------------------------------------------------------------------
struct RopeAppendParams {
  const void* q;
  const void* k;
  const void* v;
  int64_t sq[2], sk[2], sv[2];
  const float* cos;  // [>= pos + 1, D/2]
  const float* sin;
  uint16_t* q_out;   // [B, Hq, 1, D] contiguous
  uint16_t* kc;      // [B, Hkv, cap, D] with strides (b, h, t)
  uint16_t* vc;
  int64_t skc[3], svc[3];
  const int* pos_dev;  // when set, the position is read from device memory, clamped to [0, pos]
  int B, Hq, Hkv, D, pos;
};

template <class E, int XT>
__device__ __forceinline__ float load_in(const void* base, int64_t i) {
  if constexpr (XT == 2) return E::to_f(uint16_t(pack2<E>(static_cast<const float*>(base)[i], 0.f) & 0xffffu));
  else return E::to_f(static_cast<const uint16_t*>(base)[i]);
}

template <class E, int XT>
__global__ __launch_bounds__(256) void decode_rope_append_kernel(RopeAppendParams p) {
  const int half = p.D / 2;
  const int pos = p.pos_dev ? min(max(*p.pos_dev, 0), p.pos) : p.pos;
  const int64_t nq = (int64_t)p.B * p.Hq * half, nk = (int64_t)p.B * p.Hkv * half;
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= nq + 2 * nk) return;
  if (i < nq + nk) {
    const bool isq = i < nq;
    const int64_t j = isq ? i : i - nq;
    const int H = isq ? p.Hq : p.Hkv;
    const int pr = int(j % half);
    const int h = int((j / half) % H);
    const int b = int(j / half / H);
    const void* src = isq ? p.q : p.k;
    const int64_t off = b * (isq ? p.sq[0] : p.sk[0]) + (int64_t)h * (isq ? p.sq[1] : p.sk[1]) + 2 * pr;
    const float x0 = load_in<E, XT>(src, off), x1 = load_in<E, XT>(src, off + 1);
    const float c = p.cos[(int64_t)pos * half + pr], sn = p.sin[(int64_t)pos * half + pr];
    const uint32_t w = pack2<E>(x0 * c - x1 * sn, x0 * sn + x1 * c);
    uint16_t* dst = isq ? p.q_out + ((int64_t)b * p.Hq + h) * p.D + 2 * pr
                        : p.kc + b * p.skc[0] + (int64_t)h * p.skc[1] + (int64_t)pos * p.skc[2] + 2 * pr;
    dst[0] = uint16_t(w & 0xffffu);
    dst[1] = uint16_t(w >> 16);
  } else {
    const int64_t j = i - nq - nk;
    const int pr = int(j % half);
    const int h = int((j / half) % p.Hkv);
    const int b = int(j / half / p.Hkv);
    const int64_t off = b * p.sv[0] + (int64_t)h * p.sv[1] + 2 * pr;
    const uint32_t w = pack2<E>(load_in<E, XT>(p.v, off), load_in<E, XT>(p.v, off + 1));
    uint16_t* dst = p.vc + b * p.svc[0] + (int64_t)h * p.svc[1] + (int64_t)pos * p.svc[2] + 2 * pr;
    dst[0] = uint16_t(w & 0xffffu);
    dst[1] = uint16_t(w >> 16);
  }
}

}  // namespace mt
