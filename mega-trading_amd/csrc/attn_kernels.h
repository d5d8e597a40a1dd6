// gfx950 causal grouped-query attention: forward, backward-dQ, backward-dK/dV.
//
// Reference algorithm: src/mega_trading/kernels/triton_attention.py
//   forward  :260-358  (online softmax, LSE = m + ln l, P rounded to the input
//                       dtype before the PV product)
//   dQ       :481-615  (delta = rowsum(O*dO), P = exp(S - LSE), dS = P (dP - delta),
//                       dQ = scale dS K)
//   dK/dV    :618-747  (per KV block, loop over the group's query heads and the
//                       causal row blocks; dV = P^T dO, dK = scale dS^T Q)
// and the interleaved RoPE of src/mega_trading/model.py:312-316, fused into the
// Q/K tile loads (the backward emits dQ/dK in the un-rotated basis, i.e. rotated
// by -theta as src/mega_trading/kernels/triton_ops.py:205-214 does).
//
// Tiling.  A "row block" is 64 query rows of one head, a "KV tile" 64 keys.
//   * forward / dQ: a workgroup is 4 waves; each wave owns one (query head,
//     row block).  The 4 waves are the R_SUB = min(R, 4) heads of one KV group
//     times 4/R_SUB consecutive row blocks, so every K/V tile staged in LDS
//     feeds all of them.  S^T = K Q^T puts one query per lane (lane % 32),
//     keys along the accumulator slots; the row max needs one lane^32 swap.
//   * dK/dV: a workgroup is 2 waves over 64 keys (32 keys each) of one KV head;
//     it walks every (query head of the group, row block on or below the
//     diagonal) and stages Q/dO in LDS once per step for both waves.
// Fully masked causal tiles are never visited; only the diagonal tile masks.
#pragma once

#include "mt_common.h"

namespace mt {

constexpr int kBlk = 64;   // rows per row block == keys per KV tile
constexpr int kPad = 8;    // LDS row padding in 16-bit elements

struct AttnParams {
  // [B, H, T, D] tensors, element strides (b, h, t); the d stride is 1.
  const uint16_t* q;
  const uint16_t* k;
  const uint16_t* v;
  const uint16_t* o;
  const uint16_t* dout;
  uint16_t* out;   // forward: O.  backward: dQ
  uint16_t* dk;
  uint16_t* dv;
  float* lse;      // [B, Hq, T] natural-log LSE (written by fwd, read by bwd)
  float* delta;    // [B, Hq, T] rowsum(O * dO) workspace (bwd)
  const float* cos;  // [T, D/2] fp32 or null
  const float* sin;
  int64_t sq[3], sk[3], sv[3], so[3], sdo[3], sout[3], sdk[3], sdv[3];
  int B, Hq, Hkv, T, R;
  int r_sub;      // heads of a group per workgroup (fwd / dQ)
  int n_hsub;     // R / r_sub
  int rb;         // row blocks per workgroup (4 / r_sub)
  int nqb;        // ceil(T / 64)
  int nsb;        // ceil(nqb / rb)
  float scale;       // softmax scale (1/sqrt(D) by default)
  float scale_log2;  // scale * log2(e)
};

// ---------------------------------------------------------------------------
// Global -> register tile loads.  A "chunk" is 8 consecutive d values of one
// row (16 bytes).  Rows at or beyond T read as zero.
// ---------------------------------------------------------------------------
__device__ __forceinline__ u32x4 load_chunk(const uint16_t* base, int64_t st, int row, int T, int d0) {
  if (row < T) return *reinterpret_cast<const u32x4*>(base + (int64_t)row * st + d0);
  return zero4();
}

template <int D>
__device__ __forceinline__ void load_rope_cs(const float* cos, const float* sin, int row, int T, int d0, f32x4& c, f32x4& s) {
  if (row < T) {
    c = *reinterpret_cast<const f32x4*>(cos + (int64_t)row * (D / 2) + d0 / 2);
    s = *reinterpret_cast<const f32x4*>(sin + (int64_t)row * (D / 2) + d0 / 2);
  } else {
    c = f32x4{1.f, 1.f, 1.f, 1.f};
    s = f32x4{0.f, 0.f, 0.f, 0.f};
  }
}

// Write a chunk row-major: dst[row][d0..d0+7].
template <int LD>
__device__ __forceinline__ void st_row(uint16_t* dst, int row, int d0, u32x4 x) {
  *reinterpret_cast<u32x4*>(dst + row * LD + d0) = x;
}
// Write a chunk transposed: dst[d0 + e][row] for e = 0..7.
template <int LD>
__device__ __forceinline__ void st_col(uint16_t* dst, int row, int d0, u32x4 x) {
#pragma unroll
  for (int p = 0; p < 4; ++p) {
    dst[(d0 + 2 * p) * LD + row] = uint16_t(x[p] & 0xffffu);
    dst[(d0 + 2 * p + 1) * LD + row] = uint16_t(x[p] >> 16);
  }
}

// A operand read along a transposed tile: 8 slots = columns c0 + 4h + {0..3}
// and c0 + 8 + 4h + {0..3} of row `row` (the permuted contraction order that
// matches a C tile fed back as a B operand).
template <class E, int LD>
__device__ __forceinline__ typename E::v8 ld_perm(const uint16_t* src, int row, int c0, int h) {
  const uint16_t* p = src + row * LD + c0 + 4 * h;
  u32x2 lo = *reinterpret_cast<const u32x2*>(p);
  u32x2 hi = *reinterpret_cast<const u32x2*>(p + 8);
  u32x4 w = {lo[0], lo[1], hi[0], hi[1]};
  return __builtin_bit_cast(typename E::v8, w);
}

template <class E, int LD>
__device__ __forceinline__ typename E::v8 ld_row8(const uint16_t* src, int row, int c0) {
  return __builtin_bit_cast(typename E::v8, *reinterpret_cast<const u32x4*>(src + row * LD + c0));
}

// Pack C-tile slots [i0, i0+8) to an 8-wide 16-bit operand.
template <class E>
__device__ __forceinline__ typename E::v8 pack8(const f32x16& x, int i0) {
  u32x4 w;
#pragma unroll
  for (int p = 0; p < 4; ++p) w[p] = pack2<E>(x[i0 + 2 * p], x[i0 + 2 * p + 1]);
  return __builtin_bit_cast(typename E::v8, w);
}

// Workgroup -> (batch, kv head, head subset, super block) for fwd / dQ; the
// longest causal rows are issued first.  Consecutive workgroups share a
// (batch, kv head, subset) slot modulo the group count, so with a group count
// that is a multiple of 8 every KV stream stays on one XCD.
struct RowTask {
  int b, kvh, hs, sb;
};
__device__ __forceinline__ RowTask row_task(const AttnParams& p) {
  int groups = p.B * p.Hkv * p.n_hsub;
  int L = blockIdx.x;
  RowTask t;
  t.sb = p.nsb - 1 - L / groups;
  int g = L % groups;
  t.hs = g % p.n_hsub;
  int bk = g / p.n_hsub;
  t.kvh = bk % p.Hkv;
  t.b = bk / p.Hkv;
  return t;
}

// ===========================================================================
// Forward
// ===========================================================================
template <class E, int D, bool ROPE>
__global__ __launch_bounds__(256, 2) void attn_fwd_kernel(AttnParams p) {
  using V8 = typename E::v8;
  constexpr int KT = D / 16;            // k-steps over d
  constexpr int DT = D / 32;            // 32-wide d tiles
  constexpr int LDK = D + kPad;         // Ks row stride
  constexpr int LDV = kBlk + kPad;      // VsT row stride
  constexpr int CH = kBlk * D / 8;      // chunks per tile
  constexpr int CPT = CH / 256;         // chunks per thread
  __shared__ __attribute__((aligned(16))) uint16_t Ks[2][kBlk * LDK];
  __shared__ __attribute__((aligned(16))) uint16_t VsT[2][D * LDV];

  const RowTask task = row_task(p);
  const int tid = threadIdx.x;
  const int wave = tid >> 6;
  const int lane = tid & 63;
  const int l32 = lane & 31;
  const int hh = lane >> 5;
  const int head = task.kvh * p.R + task.hs * p.r_sub + (wave % p.r_sub);
  const int qb = task.sb * p.rb + wave / p.r_sub;   // this wave's row block
  const int q0 = qb * kBlk;
  const bool active = qb < p.nqb;
  // last KV tile any wave of the workgroup needs
  const int jlast = min(p.nqb - 1, task.sb * p.rb + p.rb - 1);

  const uint16_t* kbase = p.k + task.b * p.sk[0] + (int64_t)task.kvh * p.sk[1];
  const uint16_t* vbase = p.v + task.b * p.sv[0] + (int64_t)task.kvh * p.sv[1];

  // Q^T as B operands (N = query, k = d), rotated if RoPE.
  V8 qop[2][KT];
  {
    const uint16_t* qbase = p.q + task.b * p.sq[0] + (int64_t)head * p.sq[1];
#pragma unroll
    for (int nt = 0; nt < 2; ++nt) {
      const int row = q0 + nt * 32 + l32;
#pragma unroll
      for (int kk = 0; kk < KT; ++kk) {
        const int d0 = 16 * kk + 8 * hh;
        u32x4 x = active ? load_chunk(qbase, p.sq[2], row, p.T, d0) : zero4();
        if constexpr (ROPE) {
          f32x4 c, s;
          load_rope_cs<D>(p.cos, p.sin, active ? row : p.T, p.T, d0, c, s);
          x = rope_chunk<E>(x, c, s);
        }
        qop[nt][kk] = __builtin_bit_cast(V8, x);
      }
    }
  }

  f32x16 oacc[DT][2];
#pragma unroll
  for (int dt = 0; dt < DT; ++dt)
#pragma unroll
    for (int nt = 0; nt < 2; ++nt)
#pragma unroll
      for (int i = 0; i < 16; ++i) oacc[dt][nt][i] = 0.f;
  float mrun[2] = {-INFINITY, -INFINITY};
  float lrun[2] = {0.f, 0.f};

  // staging registers (prefetch of the next KV tile)
  u32x4 kreg[CPT], vreg[CPT];
  f32x4 kc[CPT], ks[CPT];
  auto fetch = [&](int j) {
#pragma unroll
    for (int i = 0; i < CPT; ++i) {
      const int c = tid + i * 256;
      const int row = c / (D / 8);
      const int d0 = (c % (D / 8)) * 8;
      const int key = j * kBlk + row;
      kreg[i] = load_chunk(kbase, p.sk[2], key, p.T, d0);
      vreg[i] = load_chunk(vbase, p.sv[2], key, p.T, d0);
      if constexpr (ROPE) load_rope_cs<D>(p.cos, p.sin, key, p.T, d0, kc[i], ks[i]);
    }
  };
  auto commit = [&](int buf) {
#pragma unroll
    for (int i = 0; i < CPT; ++i) {
      const int c = tid + i * 256;
      const int row = c / (D / 8);
      const int d0 = (c % (D / 8)) * 8;
      u32x4 x = kreg[i];
      if constexpr (ROPE) x = rope_chunk<E>(x, kc[i], ks[i]);
      st_row<LDK>(Ks[buf], row, d0, x);
      st_col<LDV>(VsT[buf], row, d0, vreg[i]);
    }
  };

  fetch(0);
  commit(0);
  __syncthreads();

  const float c2 = p.scale_log2;
  for (int j = 0; j <= jlast; ++j) {
    const int buf = j & 1;
    if (j < jlast) fetch(j + 1);
    if (active && j <= qb) {
      const uint16_t* K = Ks[buf];
      const uint16_t* Vt = VsT[buf];
      f32x16 st[2][2];
#pragma unroll
      for (int mt = 0; mt < 2; ++mt)
#pragma unroll
        for (int nt = 0; nt < 2; ++nt)
#pragma unroll
          for (int i = 0; i < 16; ++i) st[mt][nt][i] = 0.f;
#pragma unroll
      for (int kk = 0; kk < KT; ++kk) {
#pragma unroll
        for (int mt = 0; mt < 2; ++mt) {
          V8 a = ld_row8<E, LDK>(K, mt * 32 + l32, 16 * kk + 8 * hh);
#pragma unroll
          for (int nt = 0; nt < 2; ++nt) st[mt][nt] = E::mfma(a, qop[nt][kk], st[mt][nt]);
        }
      }
      if (j == qb) {
        // diagonal tile: key (row m of S^T) > query (col n) is masked
#pragma unroll
        for (int mt = 0; mt < 2; ++mt)
#pragma unroll
          for (int nt = 0; nt < 2; ++nt)
#pragma unroll
            for (int i = 0; i < 16; ++i) {
              const int kr = mt * 32 + 8 * (i >> 2) + 4 * hh + (i & 3);
              const int qr = nt * 32 + l32;
              if (kr > qr) st[mt][nt][i] = -INFINITY;
            }
      }
      V8 pop[2][4];
#pragma unroll
      for (int nt = 0; nt < 2; ++nt) {
        float mx = -INFINITY;
#pragma unroll
        for (int mt = 0; mt < 2; ++mt)
#pragma unroll
          for (int i = 0; i < 16; ++i) mx = fmaxf(mx, st[mt][nt][i]);
        mx = max_with_partner(mx) * c2;
        const float mnew = fmaxf(mrun[nt], mx);
        const float alpha = exp2_fast(mrun[nt] - mnew);
        mrun[nt] = mnew;
        float ls = 0.f;
#pragma unroll
        for (int mt = 0; mt < 2; ++mt)
#pragma unroll
          for (int i = 0; i < 16; ++i) {
            const float pv = exp2_fast(__builtin_fmaf(st[mt][nt][i], c2, -mnew));
            st[mt][nt][i] = pv;
            ls += pv;
          }
        lrun[nt] = lrun[nt] * alpha + ls;
#pragma unroll
        for (int dt = 0; dt < DT; ++dt)
#pragma unroll
          for (int i = 0; i < 16; ++i) oacc[dt][nt][i] *= alpha;
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) pop[nt][ks] = pack8<E>(st[ks >> 1][nt], (ks & 1) * 8);
      }
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) {
#pragma unroll
        for (int dt = 0; dt < DT; ++dt) {
          V8 a = ld_perm<E, LDV>(Vt, dt * 32 + l32, 16 * ks, hh);
#pragma unroll
          for (int nt = 0; nt < 2; ++nt) oacc[dt][nt] = E::mfma(a, pop[nt][ks], oacc[dt][nt]);
        }
      }
    }
    if (j < jlast) commit(buf ^ 1);
    __syncthreads();
  }

  if (!active) return;
  uint16_t* obase = p.out + task.b * p.so[0] + (int64_t)head * p.so[1];
  float* lbase = p.lse + ((int64_t)task.b * p.Hq + head) * p.T;
#pragma unroll
  for (int nt = 0; nt < 2; ++nt) {
    const float lt = sum_with_partner(lrun[nt]);
    const float inv = 1.f / lt;
    const int row = q0 + nt * 32 + l32;
    if (row < p.T) {
#pragma unroll
      for (int dt = 0; dt < DT; ++dt)
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const int d = dt * 32 + 8 * g + 4 * hh;
          u32x2 w = {pack2<E>(oacc[dt][nt][4 * g] * inv, oacc[dt][nt][4 * g + 1] * inv),
                     pack2<E>(oacc[dt][nt][4 * g + 2] * inv, oacc[dt][nt][4 * g + 3] * inv)};
          *reinterpret_cast<u32x2*>(obase + (int64_t)row * p.so[2] + d) = w;
        }
      if (hh == 0) lbase[row] = (mrun[nt] + __builtin_amdgcn_logf(lt)) * kLn2;
    }
  }
}

// ===========================================================================
// Backward, dQ (also writes delta = rowsum(O * dO))
// ===========================================================================
template <class E, int D, bool ROPE>
__global__ __launch_bounds__(256, 2) void attn_bwd_dq_kernel(AttnParams p) {
  using V8 = typename E::v8;
  constexpr int KT = D / 16;
  constexpr int DT = D / 32;
  constexpr int LDK = D + kPad;      // Ks / Vs row stride
  constexpr int LDT = kBlk + kPad;   // KsT row stride
  constexpr int CH = kBlk * D / 8;
  constexpr int CPT = CH / 256;
  __shared__ __attribute__((aligned(16))) uint16_t Ks[2][kBlk * LDK];
  __shared__ __attribute__((aligned(16))) uint16_t Vs[2][kBlk * LDK];
  __shared__ __attribute__((aligned(16))) uint16_t KsT[2][D * LDT];

  const RowTask task = row_task(p);
  const int tid = threadIdx.x;
  const int wave = tid >> 6;
  const int lane = tid & 63;
  const int l32 = lane & 31;
  const int hh = lane >> 5;
  const int head = task.kvh * p.R + task.hs * p.r_sub + (wave % p.r_sub);
  const int qb = task.sb * p.rb + wave / p.r_sub;
  const int q0 = qb * kBlk;
  const bool active = qb < p.nqb;
  const int jlast = min(p.nqb - 1, task.sb * p.rb + p.rb - 1);

  const uint16_t* kbase = p.k + task.b * p.sk[0] + (int64_t)task.kvh * p.sk[1];
  const uint16_t* vbase = p.v + task.b * p.sv[0] + (int64_t)task.kvh * p.sv[1];
  const int64_t rowbase = ((int64_t)task.b * p.Hq + head) * p.T;

  V8 qop[2][KT], gop[2][KT];
  float lse2[2], dlt[2];
  {
    const uint16_t* qbase = p.q + task.b * p.sq[0] + (int64_t)head * p.sq[1];
    const uint16_t* gbase = p.dout + task.b * p.sdo[0] + (int64_t)head * p.sdo[1];
    const uint16_t* obase = p.o + task.b * p.so[0] + (int64_t)head * p.so[1];
#pragma unroll
    for (int nt = 0; nt < 2; ++nt) {
      const int row = q0 + nt * 32 + l32;
      const bool ok = active && row < p.T;
      float dsum = 0.f;
#pragma unroll
      for (int kk = 0; kk < KT; ++kk) {
        const int d0 = 16 * kk + 8 * hh;
        u32x4 x = ok ? load_chunk(qbase, p.sq[2], row, p.T, d0) : zero4();
        if constexpr (ROPE) {
          f32x4 c, s;
          load_rope_cs<D>(p.cos, p.sin, ok ? row : p.T, p.T, d0, c, s);
          x = rope_chunk<E>(x, c, s);
        }
        qop[nt][kk] = __builtin_bit_cast(V8, x);
        u32x4 g = ok ? load_chunk(gbase, p.sdo[2], row, p.T, d0) : zero4();
        u32x4 o = ok ? load_chunk(obase, p.so[2], row, p.T, d0) : zero4();
        gop[nt][kk] = __builtin_bit_cast(V8, g);
#pragma unroll
        for (int w = 0; w < 4; ++w)
          dsum += lo_f<E>(g[w]) * lo_f<E>(o[w]) + hi_f<E>(g[w]) * hi_f<E>(o[w]);
      }
      dsum = sum_with_partner(dsum);
      dlt[nt] = dsum;
      lse2[nt] = ok ? p.lse[rowbase + row] * kLog2e : 0.f;
      if (ok && hh == 0) p.delta[rowbase + row] = dsum;
    }
  }

  f32x16 dqacc[DT][2];
#pragma unroll
  for (int dt = 0; dt < DT; ++dt)
#pragma unroll
    for (int nt = 0; nt < 2; ++nt)
#pragma unroll
      for (int i = 0; i < 16; ++i) dqacc[dt][nt][i] = 0.f;

  u32x4 kreg[CPT], vreg[CPT];
  f32x4 kc[CPT], ksn[CPT];
  auto fetch = [&](int j) {
#pragma unroll
    for (int i = 0; i < CPT; ++i) {
      const int c = tid + i * 256;
      const int row = c / (D / 8);
      const int d0 = (c % (D / 8)) * 8;
      const int key = j * kBlk + row;
      kreg[i] = load_chunk(kbase, p.sk[2], key, p.T, d0);
      vreg[i] = load_chunk(vbase, p.sv[2], key, p.T, d0);
      if constexpr (ROPE) load_rope_cs<D>(p.cos, p.sin, key, p.T, d0, kc[i], ksn[i]);
    }
  };
  auto commit = [&](int buf) {
#pragma unroll
    for (int i = 0; i < CPT; ++i) {
      const int c = tid + i * 256;
      const int row = c / (D / 8);
      const int d0 = (c % (D / 8)) * 8;
      u32x4 x = kreg[i];
      if constexpr (ROPE) x = rope_chunk<E>(x, kc[i], ksn[i]);
      st_row<LDK>(Ks[buf], row, d0, x);
      st_col<LDT>(KsT[buf], row, d0, x);
      st_row<LDK>(Vs[buf], row, d0, vreg[i]);
    }
  };

  fetch(0);
  commit(0);
  __syncthreads();

  const float c2 = p.scale_log2;
  for (int j = 0; j <= jlast; ++j) {
    const int buf = j & 1;
    if (j < jlast) fetch(j + 1);
    if (active && j <= qb) {
      const uint16_t* K = Ks[buf];
      const uint16_t* Vr = Vs[buf];
      const uint16_t* Kt = KsT[buf];
#pragma unroll
      for (int nt = 0; nt < 2; ++nt) {
        f32x16 st[2], dpt[2];
#pragma unroll
        for (int mt = 0; mt < 2; ++mt)
#pragma unroll
          for (int i = 0; i < 16; ++i) { st[mt][i] = 0.f; dpt[mt][i] = 0.f; }
#pragma unroll
        for (int kk = 0; kk < KT; ++kk) {
#pragma unroll
          for (int mt = 0; mt < 2; ++mt) {
            V8 a = ld_row8<E, LDK>(K, mt * 32 + l32, 16 * kk + 8 * hh);
            st[mt] = E::mfma(a, qop[nt][kk], st[mt]);
            V8 b = ld_row8<E, LDK>(Vr, mt * 32 + l32, 16 * kk + 8 * hh);
            dpt[mt] = E::mfma(b, gop[nt][kk], dpt[mt]);
          }
        }
        const int qr = nt * 32 + l32;
#pragma unroll
        for (int mt = 0; mt < 2; ++mt)
#pragma unroll
          for (int i = 0; i < 16; ++i) {
            float pv = exp2_fast(__builtin_fmaf(st[mt][i], c2, -lse2[nt]));
            if (j == qb) {
              const int kr = mt * 32 + 8 * (i >> 2) + 4 * hh + (i & 3);
              if (kr > qr) pv = 0.f;
            }
            st[mt][i] = pv * (dpt[mt][i] - dlt[nt]);
          }
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) {
          V8 b = pack8<E>(st[ks >> 1], (ks & 1) * 8);
#pragma unroll
          for (int dt = 0; dt < DT; ++dt) {
            V8 a = ld_perm<E, LDT>(Kt, dt * 32 + l32, 16 * ks, hh);
            dqacc[dt][nt] = E::mfma(a, b, dqacc[dt][nt]);
          }
        }
      }
    }
    if (j < jlast) commit(buf ^ 1);
    __syncthreads();
  }

  if (!active) return;
  uint16_t* dqbase = p.out + task.b * p.sout[0] + (int64_t)head * p.sout[1];
#pragma unroll
  for (int nt = 0; nt < 2; ++nt) {
    const int row = q0 + nt * 32 + l32;
    if (row >= p.T) continue;
#pragma unroll
    for (int dt = 0; dt < DT; ++dt)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int d = dt * 32 + 8 * g + 4 * hh;
        float x0 = dqacc[dt][nt][4 * g] * p.scale, x1 = dqacc[dt][nt][4 * g + 1] * p.scale;
        float x2 = dqacc[dt][nt][4 * g + 2] * p.scale, x3 = dqacc[dt][nt][4 * g + 3] * p.scale;
        if constexpr (ROPE) {
          // rotate back by -theta: (e, o) -> (e c + o s, -e s + o c)
          const float* cp = p.cos + (int64_t)row * (D / 2) + d / 2;
          const float* sp = p.sin + (int64_t)row * (D / 2) + d / 2;
          f32x2 c = *reinterpret_cast<const f32x2*>(cp);
          f32x2 s = *reinterpret_cast<const f32x2*>(sp);
          float y0 = x0 * c[0] + x1 * s[0], y1 = x1 * c[0] - x0 * s[0];
          float y2 = x2 * c[1] + x3 * s[1], y3 = x3 * c[1] - x2 * s[1];
          x0 = y0; x1 = y1; x2 = y2; x3 = y3;
        }
        u32x2 w = {pack2<E>(x0, x1), pack2<E>(x2, x3)};
        *reinterpret_cast<u32x2*>(dqbase + (int64_t)row * p.sout[2] + d) = w;
      }
  }
}

// ===========================================================================
// Backward, dK / dV
// ===========================================================================
constexpr int kKvWaves = 2;                 // waves per dK/dV workgroup
constexpr int kKvKeys = 32 * kKvWaves;      // keys per dK/dV workgroup (== kBlk)
static_assert(kKvKeys == kBlk, "dK/dV key block must equal the row block");

template <class E, int D, bool ROPE>
__global__ __launch_bounds__(64 * kKvWaves, 2) void attn_bwd_dkv_kernel(AttnParams p) {
  using V8 = typename E::v8;
  constexpr int NT = 64 * kKvWaves;
  constexpr int KT = D / 16;
  constexpr int DT = D / 32;
  constexpr int LDR = D + kPad;      // row-major Q / dO stride
  constexpr int LDT = kBlk + kPad;   // transposed Q^T / dO^T stride
  constexpr int CH = kBlk * D / 8;
  constexpr int CPT = CH / NT;
  __shared__ __attribute__((aligned(16))) uint16_t Qs[2][kBlk * LDR];
  __shared__ __attribute__((aligned(16))) uint16_t Gs[2][kBlk * LDR];
  __shared__ __attribute__((aligned(16))) uint16_t QsT[2][D * LDT];
  __shared__ __attribute__((aligned(16))) uint16_t GsT[2][D * LDT];
  __shared__ __attribute__((aligned(16))) float Ls[2][kBlk];
  __shared__ __attribute__((aligned(16))) float Ds[2][kBlk];

  // heaviest key blocks (smallest index: most causal rows) first
  const int groups = p.B * p.Hkv;
  const int L = blockIdx.x;
  const int kb = L / groups;
  const int g = L % groups;
  const int kvh = g % p.Hkv;
  const int b = g / p.Hkv;

  const int tid = threadIdx.x;
  const int wave = tid >> 6;
  const int lane = tid & 63;
  const int l32 = lane & 31;
  const int hh = lane >> 5;
  const int k0 = kb * kBlk + wave * 32;     // this wave's first key
  const int key = k0 + l32;                 // this lane's key (C column)

  // K and V rows as B operands (N = key, k = d)
  V8 kop[KT], vop[KT];
  {
    const uint16_t* kbase = p.k + b * p.sk[0] + (int64_t)kvh * p.sk[1];
    const uint16_t* vbase = p.v + b * p.sv[0] + (int64_t)kvh * p.sv[1];
#pragma unroll
    for (int kk = 0; kk < KT; ++kk) {
      const int d0 = 16 * kk + 8 * hh;
      u32x4 x = load_chunk(kbase, p.sk[2], key, p.T, d0);
      if constexpr (ROPE) {
        f32x4 c, s;
        load_rope_cs<D>(p.cos, p.sin, key, p.T, d0, c, s);
        x = rope_chunk<E>(x, c, s);
      }
      kop[kk] = __builtin_bit_cast(V8, x);
      vop[kk] = __builtin_bit_cast(V8, load_chunk(vbase, p.sv[2], key, p.T, d0));
    }
  }

  f32x16 dkacc[DT], dvacc[DT];
#pragma unroll
  for (int dt = 0; dt < DT; ++dt)
#pragma unroll
    for (int i = 0; i < 16; ++i) { dkacc[dt][i] = 0.f; dvacc[dt][i] = 0.f; }

  const int nblk_q = p.nqb - kb;          // row blocks on or below the diagonal
  const int n_it = p.R * nblk_q;

  u32x4 qreg[CPT], greg[CPT];
  f32x4 qc[CPT], qs[CPT];
  float lreg = 0.f, dreg = 0.f;
  auto fetch = [&](int it) {
    const int r = it / nblk_q;
    const int qb = kb + it % nblk_q;
    const int head = kvh * p.R + r;
    const uint16_t* qbase = p.q + b * p.sq[0] + (int64_t)head * p.sq[1];
    const uint16_t* gbase = p.dout + b * p.sdo[0] + (int64_t)head * p.sdo[1];
#pragma unroll
    for (int i = 0; i < CPT; ++i) {
      const int c = tid + i * NT;
      const int row = c / (D / 8);
      const int d0 = (c % (D / 8)) * 8;
      const int t = qb * kBlk + row;
      qreg[i] = load_chunk(qbase, p.sq[2], t, p.T, d0);
      greg[i] = load_chunk(gbase, p.sdo[2], t, p.T, d0);
      if constexpr (ROPE) load_rope_cs<D>(p.cos, p.sin, t, p.T, d0, qc[i], qs[i]);
    }
    if (tid < kBlk) {
      const int t = qb * kBlk + tid;
      const int64_t rb = ((int64_t)b * p.Hq + head) * p.T;
      lreg = t < p.T ? p.lse[rb + t] * kLog2e : 0.f;
      dreg = t < p.T ? p.delta[rb + t] : 0.f;
    }
  };
  auto commit = [&](int buf) {
#pragma unroll
    for (int i = 0; i < CPT; ++i) {
      const int c = tid + i * NT;
      const int row = c / (D / 8);
      const int d0 = (c % (D / 8)) * 8;
      u32x4 x = qreg[i];
      if constexpr (ROPE) x = rope_chunk<E>(x, qc[i], qs[i]);
      st_row<LDR>(Qs[buf], row, d0, x);
      st_col<LDT>(QsT[buf], row, d0, x);
      st_row<LDR>(Gs[buf], row, d0, greg[i]);
      st_col<LDT>(GsT[buf], row, d0, greg[i]);
    }
    if (tid < kBlk) {
      Ls[buf][tid] = lreg;
      Ds[buf][tid] = dreg;
    }
  };

  fetch(0);
  commit(0);
  __syncthreads();

  const float c2 = p.scale_log2;
  for (int it = 0; it < n_it; ++it) {
    const int buf = it & 1;
    if (it + 1 < n_it) fetch(it + 1);
    const int qb = kb + it % nblk_q;
    const int qbase_row = qb * kBlk;
    {
      const uint16_t* Q = Qs[buf];
      const uint16_t* G = Gs[buf];
      const uint16_t* Qt = QsT[buf];
      const uint16_t* Gt = GsT[buf];
      V8 pop[4], dsop[4];
#pragma unroll
      for (int mt = 0; mt < 2; ++mt) {
        f32x16 s, dp;
#pragma unroll
        for (int i = 0; i < 16; ++i) { s[i] = 0.f; dp[i] = 0.f; }
#pragma unroll
        for (int kk = 0; kk < KT; ++kk) {
          V8 a = ld_row8<E, LDR>(Q, mt * 32 + l32, 16 * kk + 8 * hh);
          s = E::mfma(a, kop[kk], s);
          V8 a2 = ld_row8<E, LDR>(G, mt * 32 + l32, 16 * kk + 8 * hh);
          dp = E::mfma(a2, vop[kk], dp);
        }
#pragma unroll
        for (int g4 = 0; g4 < 4; ++g4) {
          const int qr = mt * 32 + 8 * g4 + 4 * hh;   // first of 4 query rows in these slots
          f32x4 l4 = *reinterpret_cast<const f32x4*>(&Ls[buf][qr]);
          f32x4 d4 = *reinterpret_cast<const f32x4*>(&Ds[buf][qr]);
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const int i = 4 * g4 + e;
            const int qg = qbase_row + qr + e;
            float pv = exp2_fast(__builtin_fmaf(s[i], c2, -l4[e]));
            if (key > qg || qg >= p.T) pv = 0.f;
            s[i] = pv;
            dp[i] = pv * (dp[i] - d4[e]);
          }
        }
        pop[2 * mt] = pack8<E>(s, 0);
        pop[2 * mt + 1] = pack8<E>(s, 8);
        dsop[2 * mt] = pack8<E>(dp, 0);
        dsop[2 * mt + 1] = pack8<E>(dp, 8);
      }
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) {
#pragma unroll
        for (int dt = 0; dt < DT; ++dt) {
          V8 a = ld_perm<E, LDT>(Gt, dt * 32 + l32, 16 * ks, hh);
          dvacc[dt] = E::mfma(a, pop[ks], dvacc[dt]);
          V8 a2 = ld_perm<E, LDT>(Qt, dt * 32 + l32, 16 * ks, hh);
          dkacc[dt] = E::mfma(a2, dsop[ks], dkacc[dt]);
        }
      }
    }
    if (it + 1 < n_it) commit(buf ^ 1);
    __syncthreads();
  }

  if (key >= p.T) return;
  uint16_t* dkbase = p.dk + b * p.sdk[0] + (int64_t)kvh * p.sdk[1] + (int64_t)key * p.sdk[2];
  uint16_t* dvbase = p.dv + b * p.sdv[0] + (int64_t)kvh * p.sdv[1] + (int64_t)key * p.sdv[2];
#pragma unroll
  for (int dt = 0; dt < DT; ++dt)
#pragma unroll
    for (int g4 = 0; g4 < 4; ++g4) {
      const int d = dt * 32 + 8 * g4 + 4 * hh;
      float x0 = dkacc[dt][4 * g4] * p.scale, x1 = dkacc[dt][4 * g4 + 1] * p.scale;
      float x2 = dkacc[dt][4 * g4 + 2] * p.scale, x3 = dkacc[dt][4 * g4 + 3] * p.scale;
      if constexpr (ROPE) {
        const float* cp = p.cos + (int64_t)key * (D / 2) + d / 2;
        const float* sp = p.sin + (int64_t)key * (D / 2) + d / 2;
        f32x2 c = *reinterpret_cast<const f32x2*>(cp);
        f32x2 s = *reinterpret_cast<const f32x2*>(sp);
        float y0 = x0 * c[0] + x1 * s[0], y1 = x1 * c[0] - x0 * s[0];
        float y2 = x2 * c[1] + x3 * s[1], y3 = x3 * c[1] - x2 * s[1];
        x0 = y0; x1 = y1; x2 = y2; x3 = y3;
      }
      u32x2 wk = {pack2<E>(x0, x1), pack2<E>(x2, x3)};
      *reinterpret_cast<u32x2*>(dkbase + d) = wk;
      u32x2 wv = {pack2<E>(dvacc[dt][4 * g4], dvacc[dt][4 * g4 + 1]), pack2<E>(dvacc[dt][4 * g4 + 2], dvacc[dt][4 * g4 + 3])};
      *reinterpret_cast<u32x2*>(dvbase + d) = wv;
    }
}

}  // namespace mt
