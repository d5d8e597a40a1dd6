// gfx950 decode attention: one new query token per sequence against a KV cache,
// for KV-cached generation (the reference's TradingModel.generate,
// src/mega_trading/model.py:134-147, recomputes the whole context per token
// instead; the maths is the causal GQA attention of triton_attention.py for the
// last query row, whose keys are all cached positions).
//
// Split-K ("flash decoding"): the cached keys 0..L-1 are cut into 64-key
// splits and each split is one wave (workgroup (batch, KV head, split)).  The
// wave scores its split for all R query heads of the KV group (each K/V row is
// read once for the R heads), forms the split's softmax numerator and offset,
// and writes an fp32 partial (o, m, l).  A second kernel merges the splits
// with the log-sum-exp rule; a cache of at most 8 splits is decoded in one
// launch instead (one workgroup per (batch, KV head), its waves merged in
// LDS).  The work is HBM- and latency-bound (the cache is read once; at the
// decoder's shapes a split's data is a few KB), so it runs on the vector ALUs
// -- with one query row per head there is no matrix product to feed the
// MFMAs: q . k as v_dot2 on the stored 16-bit pairs, p V as fp32 FMAs -- and
// is laid out for few dependent steps: every K and V load of a lane is issued
// at entry, the reductions stay inside the wave (DPP within 16-lane rows,
// permlane swaps across rows), and one LDS exchange hands the probabilities
// from the score layout (lane = key) to the V layout.
#pragma once

#include "mt_common.h"

namespace mt {

constexpr int kDecSplit = 64;   // keys per split: one wave, one key per lane in the score pass
constexpr int kDecMaxR = 8;     // query heads per KV head supported

// fp32 floats per partial: o[0..D), m (log2), l, two pad floats (16-byte rows)
template <int D>
constexpr int dec_row() { return D + 4; }

struct DecodeParams {
  const uint16_t* q;  // [B, Hq, 1, D] (rotated when RoPE is used)
  const uint16_t* k;  // [B, Hkv, >= L, D] cache (rotated keys)
  const uint16_t* v;  // [B, Hkv, >= L, D] cache
  uint16_t* out;      // [B, Hq, 1, D]
  float* part;        // [B, Hq, nsplit, D + 4] fp32: o (unnormalised), m (log2), l
  int64_t sq[2], sk[3], sv[3], so[2];  // strides (b, h) for q / o, (b, h, t) for the caches
  const int* length_dev;  // when set, L is read from device memory (graph-replayable decode)
  int B, Hq, Hkv, R, L, nsplit;  // nsplit: splits in the grid (of the capacity when length_dev is set)
  float scale_log2;  // softmax scale * log2(e)
};

// With length_dev, L holds the capacity and the device value is clamped to [1, capacity].
__device__ __forceinline__ int decode_length(const DecodeParams& p) {
  return p.length_dev ? min(max(*p.length_dev, 1), p.L) : p.L;
}

// q . k of one cached row for each of the R heads: two products per
// v_dot2c_f32 (exact 16-bit products, fp32 sums) straight from the stored
// pairs, with no conversion of k.
template <class E, int NC, int R>
__device__ __forceinline__ void dec_scores(const u32x4 (&qs)[R][NC], const u32x4 (&kw)[NC], float (&sc)[R]) {
#pragma unroll
  for (int h = 0; h < R; ++h) sc[h] = 0.f;
#pragma unroll
  for (int cc = 0; cc < NC; ++cc)
#pragma unroll
    for (int h = 0; h < R; ++h) {
      const u32x4 qv = qs[h][cc];
#pragma unroll
      for (int e = 0; e < 4; ++e) sc[h] = E::dot2(qv[e], kw[cc][e], sc[h]);
    }
}

// One 64-key split [k0, k0 + n) of one (batch, KV head), computed by one wave
// for the R query heads of the group; shared by the split kernel (which writes
// the result to HBM) and the fused kernel (which merges its waves in LDS).
//
// Layouts.  Score pass: lane = key k0 + lane.  V pass: lane = (d chunk
// c = lane % NC, key group lane / NC), keys j = lane / NC + i G.  Keys past the
// split's end load its last key instead (in bounds; their probabilities are
// zero), so the loads need no branches.
template <int D>
struct DecLayout {
  static constexpr int NC = D / 8;          // 16-byte chunks per row
  static constexpr int G = 64 / NC;         // key groups of the V pass
  static constexpr int NV = kDecSplit / G;  // V chunks per lane
  static constexpr int LO = NC == 4 ? 2 : NC == 8 ? 3 : 4;  // log2(NC): lane bits of the d chunk
};

// Every K and V load of the split, issued together (one memory round trip).
template <int D>
__device__ __forceinline__ void dec_load(const DecodeParams& p, int b, int kvh, int k0, int n, int lane,
                                         u32x4 (&kw)[DecLayout<D>::NC], u32x4 (&vw)[DecLayout<D>::NV]) {
  using Ly = DecLayout<D>;
  const int c = lane % Ly::NC, kg = lane / Ly::NC;
  const uint16_t* krow = p.k + b * p.sk[0] + (int64_t)kvh * p.sk[1] + (int64_t)(k0 + min(lane, n - 1)) * p.sk[2];
#pragma unroll
  for (int cc = 0; cc < Ly::NC; ++cc) kw[cc] = *reinterpret_cast<const u32x4*>(krow + 8 * cc);
  const uint16_t* vbase = p.v + b * p.sv[0] + (int64_t)kvh * p.sv[1] + (int64_t)k0 * p.sv[2] + 8 * c;
#pragma unroll
  for (int i = 0; i < Ly::NV; ++i)
    vw[i] = *reinterpret_cast<const u32x4*>(vbase + (int64_t)min(kg + i * Ly::G, n - 1) * p.sv[2]);
}

// The group's q rows, [R][NC] 16-byte chunks as stored, staged in LDS by the
// workgroup's threads (read back as broadcasts).
template <int D, int R>
__device__ __forceinline__ void dec_stage_q(const DecodeParams& p, int b, int kvh, int tid, int nthreads,
                                            u32x4 (&qs)[R][DecLayout<D>::NC]) {
  constexpr int NC = DecLayout<D>::NC;
  const uint16_t* qb = p.q + b * p.sq[0] + (int64_t)(kvh * R) * p.sq[1];
  for (int i = tid; i < R * NC; i += nthreads) {
    const int h = i / NC, cc = i % NC;
    qs[h][cc] = *reinterpret_cast<const u32x4*>(qb + (int64_t)h * p.sq[1] + 8 * cc);
  }
}

// The split's softmax offset m and sum l per head (log2 units) and its
// unnormalised o[h][8 c .. 8 c + 7] = sum_j p[h][j] V[k0 + j][...], summed
// over the key groups (lanes with kg = 0 hold the result).  ps is the wave's
// own [R][64] LDS block; one exchange through it moves the probabilities from
// the score layout to the V layout.
template <class E, int D, int R>
__device__ __forceinline__ void dec_split(const DecodeParams& p, int n, int lane, const u32x4 (&qs)[R][DecLayout<D>::NC],
                                          const u32x4 (&kw)[DecLayout<D>::NC], const u32x4 (&vw)[DecLayout<D>::NV],
                                          float (&ps)[R][kDecSplit], float (&m)[R], float (&l)[R],
                                          float (&acc)[R][8]) {
  using Ly = DecLayout<D>;
  float sc[R];
  dec_scores<E, Ly::NC, R>(qs, kw, sc);
  const bool live = lane < n;
#pragma unroll
  for (int h = 0; h < R; ++h) {
    const float x = live ? sc[h] * p.scale_log2 : -INFINITY;
    m[h] = wave_reduce<0, true>(x);  // lane 0 is always live: finite
    const float e = live ? exp2_fast(x - m[h]) : 0.f;
    ps[h][lane] = e;
    l[h] = wave_reduce<0, false>(e);
  }
  // LDS operations of one wave complete in order: a wave-scope fence (a
  // compiler barrier) suffices between the writes and the reads
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  const int kg = lane / Ly::NC;
#pragma unroll
  for (int h = 0; h < R; ++h)
#pragma unroll
    for (int e = 0; e < 8; ++e) acc[h][e] = 0.f;
#pragma unroll
  for (int i = 0; i < Ly::NV; ++i) {
    const int j = kg + i * Ly::G;
    float vv[8];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      vv[2 * e] = lo_f<E>(vw[i][e]);
      vv[2 * e + 1] = hi_f<E>(vw[i][e]);
    }
#pragma unroll
    for (int h = 0; h < R; ++h) {
      const float pj = ps[h][j];
#pragma unroll
      for (int e = 0; e < 8; ++e) acc[h][e] = __builtin_fmaf(pj, vv[e], acc[h][e]);
    }
  }
#pragma unroll
  for (int h = 0; h < R; ++h)
#pragma unroll
    for (int e = 0; e < 8; ++e) acc[h][e] = wave_reduce<Ly::LO, false>(acc[h][e]);
}

// R (query heads of the KV group) is a template parameter: the per-head loops
// then unroll into straight-line code whose LDS reads issue back to back (with
// a run-time R every head is a branch with its own wait on its reads).
template <class E, int D, int R>
__global__ __launch_bounds__(64) void attn_decode_split_kernel(DecodeParams p) {
  static_assert(D == 32 || D == 64 || D == 128, "head size");
  static_assert(R >= 1 && R <= kDecMaxR, "group size");
  using Ly = DecLayout<D>;
  __shared__ u32x4 qs[R][Ly::NC];
  __shared__ float ps[R][kDecSplit];
  const int lane = threadIdx.x;
  const int s = blockIdx.x % p.nsplit;
  const int g = blockIdx.x / p.nsplit;
  const int kvh = g % p.Hkv;
  const int b = g / p.Hkv;
  const int k0 = s * kDecSplit;
  const int L = decode_length(p);
  if (k0 >= L) return;  // a split past the current length (device-length launches cover the capacity)
  const int n = min(kDecSplit, L - k0);
  u32x4 kw[Ly::NC], vw[Ly::NV];
  dec_load<D>(p, b, kvh, k0, n, lane, kw, vw);
  dec_stage_q<D, R>(p, b, kvh, lane, 64, qs);
  __syncthreads();
  float m[R], l[R], acc[R][8];
  dec_split<E, D, R>(p, n, lane, qs, kw, vw, ps, m, l, acc);
  if (lane / Ly::NC == 0) {
    const int c = lane;
#pragma unroll
    for (int h = 0; h < R; ++h) {
      float* dst = p.part + (((int64_t)b * p.Hq + kvh * R + h) * p.nsplit + s) * dec_row<D>();
      *reinterpret_cast<f32x4*>(dst + 8 * c) = f32x4{acc[h][0], acc[h][1], acc[h][2], acc[h][3]};
      *reinterpret_cast<f32x4*>(dst + 8 * c + 4) = f32x4{acc[h][4], acc[h][5], acc[h][6], acc[h][7]};
      if (c == 0) *reinterpret_cast<f32x2*>(dst + D) = f32x2{m[h], l[h]};
    }
  }
}

// ---------------------------------------------------------------------------
// Short caches: split and combine in one launch.
// ---------------------------------------------------------------------------
// One workgroup of kDecWaves waves per (batch, KV head); wave w computes split
// w exactly as the split kernel does, writes its (m, l, o) to LDS, and the
// workgroup merges the waves with the log-sum-exp rule and writes O: no
// partials in HBM and no second launch.  The launcher uses it when the cache
// (its capacity, for device-length launches) holds at most kDecWaves splits,
// where the split + combine pair is latency-bound.  With more splits per
// workgroup the B * Hkv workgroups, one per CU, become bound by their CU's
// VALU and load bandwidth, and the split kernel's grid spread over every CU
// is faster.
constexpr int kDecWaves = 8;

template <class E, int D, int R>
__global__ __launch_bounds__(64 * kDecWaves) void attn_decode_fused_kernel(DecodeParams p) {
  static_assert(D == 32 || D == 64 || D == 128, "head size");
  static_assert(R >= 1 && R <= kDecMaxR, "group size");
  using Ly = DecLayout<D>;
  __shared__ u32x4 qs[R][Ly::NC];
  __shared__ float ps[kDecWaves][R][kDecSplit];
  __shared__ float wo[kDecWaves][R][D];   // the waves' unnormalised o
  __shared__ float wml[kDecWaves][R][2];  // and (m, l)
  const int tid = threadIdx.x;
  const int wave = tid >> 6;
  const int lane = tid & 63;
  const int kvh = blockIdx.x % p.Hkv;
  const int b = blockIdx.x / p.Hkv;
  const int L = decode_length(p);
  const int k0 = wave * kDecSplit;
  const bool active = k0 < L;  // wave-uniform
  const int n = min(kDecSplit, L - k0);
  u32x4 kw[Ly::NC], vw[Ly::NV];
  if (active) dec_load<D>(p, b, kvh, k0, n, lane, kw, vw);
  dec_stage_q<D, R>(p, b, kvh, tid, 64 * kDecWaves, qs);
  __syncthreads();
  if (active) {
    float m[R], l[R], acc[R][8];
    dec_split<E, D, R>(p, n, lane, qs, kw, vw, ps[wave], m, l, acc);
    if (lane / Ly::NC == 0) {
      const int c = lane;
#pragma unroll
      for (int h = 0; h < R; ++h) {
        *reinterpret_cast<f32x4*>(&wo[wave][h][8 * c]) = f32x4{acc[h][0], acc[h][1], acc[h][2], acc[h][3]};
        *reinterpret_cast<f32x4*>(&wo[wave][h][8 * c + 4]) = f32x4{acc[h][4], acc[h][5], acc[h][6], acc[h][7]};
        if (c == 0) {
          wml[wave][h][0] = m[h];
          wml[wave][h][1] = l[h];
        }
      }
    }
  }
  __syncthreads();
  // merge the active waves (0 .. na - 1; wave 0 holds key 0, so na >= 1):
  // M = max m_w, O = sum_w 2^(m_w - M) o_w / sum_w 2^(m_w - M) l_w
  const int na = min(kDecWaves, (L + kDecSplit - 1) / kDecSplit);
  for (int i = tid; i < R * D; i += 64 * kDecWaves) {
    const int h = i / D, d = i % D;
    float M = wml[0][h][0];
    for (int w = 1; w < na; ++w) M = fmaxf(M, wml[w][h][0]);
    float o = 0.f, lt = 0.f;
    for (int w = 0; w < na; ++w) {
      const float a = exp2_fast(wml[w][h][0] - M);
      o = __builtin_fmaf(a, wo[w][h][d], o);
      lt = __builtin_fmaf(a, wml[w][h][1], lt);
    }
    p.out[b * p.so[0] + (int64_t)(kvh * R + h) * p.so[1] + d] = uint16_t(pack2<E>(o / lt, 0.f) & 0xffffu);
  }
}

// Merge the splits of each (batch, query head): M = max m_s,
// O = sum_s 2^(m_s - M) o_s / sum_s 2^(m_s - M) l_s.  One thread per d value;
// the splits are read 16 at a time with every load of a batch issued before
// its first use (one memory round trip per 16 splits).
template <class E, int D>
__global__ __launch_bounds__(256) void attn_decode_combine_kernel(DecodeParams p) {
  constexpr int PER = 256 / D;  // (batch, head) pairs per workgroup
  constexpr int ROW = dec_row<D>();
  constexpr int BATCH = 16;
  const int pair = blockIdx.x * PER + threadIdx.x / D;
  const int d = threadIdx.x % D;
  if (pair >= p.B * p.Hq) return;
  const int b = pair / p.Hq, h = pair % p.Hq;
  const float* src = p.part + (int64_t)pair * p.nsplit * ROW;
  const int ns = (decode_length(p) + kDecSplit - 1) / kDecSplit;  // splits holding keys
  float M = -INFINITY, o = 0.f, l = 0.f;
  for (int s0 = 0; s0 < ns; s0 += BATCH) {
    float ms[BATCH], os[BATCH], ls[BATCH];
#pragma unroll
    for (int i = 0; i < BATCH; ++i) {
      const bool in = s0 + i < ns;
      const float* r = src + (int64_t)(in ? s0 + i : 0) * ROW;
      const f32x2 ml = *reinterpret_cast<const f32x2*>(r + D);
      ms[i] = in ? ml[0] : -INFINITY;
      ls[i] = in ? ml[1] : 0.f;
      os[i] = in ? r[d] : 0.f;
    }
    float mn = M;
#pragma unroll
    for (int i = 0; i < BATCH; ++i) mn = fmaxf(mn, ms[i]);
    const float a = exp2_fast(M - mn);  // 0 on the first batch (M = -inf)
    o *= a;
    l *= a;
#pragma unroll
    for (int i = 0; i < BATCH; ++i) {
      const float w = exp2_fast(ms[i] - mn);
      o = __builtin_fmaf(w, os[i], o);
      l = __builtin_fmaf(w, ls[i], l);
    }
    M = mn;
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
