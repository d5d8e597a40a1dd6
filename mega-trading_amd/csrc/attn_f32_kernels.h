// fp32 causal grouped-query attention on fp32 MFMA (v_mfma_f32_32x32x2_f32).
//
// The reference takes fp32 tensors on its Triton path
// (src/mega_trading/kernels/triton_attention.py:16): its forward dots run on
// fp32 inputs (TF32 by Triton's default) and its backward is the dense fp32
// fallback (:88-111).  These kernels compute both in full fp32: the MFMA
// multiplies fp32 operands exactly and accumulates in fp32, P and dS stay fp32
// (the reference casts P to V's dtype, fp32 here, :340), and the softmax runs
// in fp32.  They favour simplicity over speed: one wave owns 32 query rows (or
// 32 keys), reads its K / V (or Q / dO) rows straight from global memory (no
// LDS staging, no sharing across the group's heads beyond the L2) and runs the
// diagonal tile masked.
//
// MFMA layout (32x32x2, fp32): A[m][k] comes from lane m + 32 k, B[k][n] from
// lane n + 32 k, and lane l holds C[m][n = l % 32] for m = 8 (i / 4) + 4 (l / 32)
// + i % 4, i = 0..15.  A lane's half h = l / 32 feeds contraction slot k = h.
//  * Scores: the contraction runs over d, lane half h supplying the d values
//    [h D/2, (h + 1) D/2) of its row (the pairing is the same on both operands,
//    so the product is the full dot product).
//  * Products that contract over the 32 keys (or rows) of a score tile use the
//    score accumulator itself as the B operand: step j pairs slot k = h with
//    key 8 (j / 4) + 4 h + j % 4, exactly the key that lane holds in its slot
//    j, and the A operand reads the matching row.
#pragma once

#include "attn_kernels.h"

namespace mt {

__device__ __forceinline__ f32x16 mfma_f32(float a, float b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, c, 0, 0, 0);
}

// the row (key) a lane's accumulator slot i refers to, within a 32-row tile
__device__ __forceinline__ int f32_slot_row(int i, int hh) { return 8 * (i >> 2) + 4 * hh + (i & 3); }

// wave task t -> (batch, head, 32-row block), longest causal rows first; the
// four waves of a workgroup share a row block when B * H is a multiple of 4
struct F32Task {
  int b, h, blk;
};
__device__ __forceinline__ F32Task f32_task(int t, int B, int H, int nblk, bool reverse) {
  F32Task r;
  const int bh = t % (B * H);
  r.blk = reverse ? nblk - 1 - t / (B * H) : t / (B * H);
  r.h = bh % H;
  r.b = bh / H;
  return r;
}

__device__ __forceinline__ const float* fptr(const uint16_t* p) { return reinterpret_cast<const float*>(p); }
__device__ __forceinline__ float* fptr(uint16_t* p) { return reinterpret_cast<float*>(p); }

// Y = rot(X) for an fp32 [B, H, T, D] tensor, Y contiguous; one thread per 4
// consecutive d values (two interleaved pairs).
template <int D>
__global__ __launch_bounds__(256) void rope_f32_kernel(const float* x, int64_t s0, int64_t s1, int64_t s2, float* y,
                                                       const float* cos, const float* sin, int H, int T,
                                                       int64_t n4) {
  const int64_t c = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (c >= n4) return;
  const int d0 = int(c % (D / 4)) * 4;
  const int64_t row = c / (D / 4);
  const int t = int(row % T);
  const int64_t bh = row / T;
  const int h = int(bh % H);
  const int64_t b = bh / H;
  const f32x4 v = *reinterpret_cast<const f32x4*>(x + b * s0 + h * s1 + (int64_t)t * s2 + d0);
  const f32x2 cs = *reinterpret_cast<const f32x2*>(cos + (int64_t)t * (D / 2) + d0 / 2);
  const f32x2 sn = *reinterpret_cast<const f32x2*>(sin + (int64_t)t * (D / 2) + d0 / 2);
  const f32x4 r = {v[0] * cs[0] - v[1] * sn[0], v[0] * sn[0] + v[1] * cs[0], v[2] * cs[1] - v[3] * sn[1],
                   v[2] * sn[1] + v[3] * cs[1]};
  *reinterpret_cast<f32x4*>(y + row * D + d0) = r;
}

// ---------------------------------------------------------------------------
// Forward: online softmax over 32-key tiles, O and LSE.
// ---------------------------------------------------------------------------
template <int D, bool ROPE>
__global__ __launch_bounds__(256) void attn_fwd_f32_kernel(AttnParams p) {
  constexpr int HD = D / 2;  // d values per lane
  constexpr int DT = D / 32;
  __shared__ f32x4 red_o[3][DT * 4][64];  // waves 1-3: [wave - 1][dt, g][lane] unnormalised O
  __shared__ f32x2 red_ml[3][64];         // and (m, l)
  const int lane = threadIdx.x & 63, l32 = lane & 31, hh = lane >> 5;
  const int wave = threadIdx.x >> 6;
  const int nblk = (p.T + 31) / 32;
  const int t = blockIdx.x;
  if (t >= p.B * p.Hq * nblk) return;  // (workgroup-uniform)
  const F32Task task = f32_task(t, p.B, p.Hq, nblk, true);
  const int kvh = task.h / p.R;
  const int row = task.blk * 32 + l32;
  const int rc = min(row, p.T - 1);

  // the lane's half of its query row, rotated if RoPE (and written to q_rot,
  // by wave 0)
  float qv[HD];
  {
    const float* qr = fptr(p.q) + task.b * p.sq[0] + (int64_t)task.h * p.sq[1] + (int64_t)rc * p.sq[2] + hh * HD;
#pragma unroll
    for (int j = 0; j < HD / 4; ++j) {
      f32x4 x = *reinterpret_cast<const f32x4*>(qr + 4 * j);
      if constexpr (ROPE) {
        const int d0 = hh * HD + 4 * j;
        const f32x2 cs = *reinterpret_cast<const f32x2*>(p.cos + (int64_t)rc * (D / 2) + d0 / 2);
        const f32x2 sn = *reinterpret_cast<const f32x2*>(p.sin + (int64_t)rc * (D / 2) + d0 / 2);
        x = f32x4{x[0] * cs[0] - x[1] * sn[0], x[0] * sn[0] + x[1] * cs[0], x[2] * cs[1] - x[3] * sn[1],
                  x[2] * sn[1] + x[3] * cs[1]};
        if (wave == 0 && row < p.T)
          *reinterpret_cast<f32x4*>(fptr(p.qrot) + (((int64_t)task.b * p.Hq + task.h) * p.T + row) * D + d0) = x;
      }
#pragma unroll
      for (int c = 0; c < 4; ++c) qv[4 * j + c] = x[c];
    }
  }
  const float* kbase = fptr(p.k) + task.b * p.sk[0] + (int64_t)kvh * p.sk[1];
  const float* vbase = fptr(p.v) + task.b * p.sv[0] + (int64_t)kvh * p.sv[1];
  const float c2 = p.scale_log2;

  f32x16 oacc[DT];
#pragma unroll
  for (int dt = 0; dt < DT; ++dt) zero16(oacc[dt]);
  float m = -INFINITY, l = 0.f;
  // the key tiles on or left of the diagonal are dealt to the 4 waves in turn;
  // each keeps its own running offset and sums, merged below
  for (int kt = wave; kt <= task.blk; kt += 4) {
    // S^T (lane = query, slots = keys)
    const float* kr = kbase + (int64_t)min(kt * 32 + l32, p.T - 1) * p.sk[2] + hh * HD;
    f32x16 s = {};
#pragma unroll
    for (int j = 0; j < HD / 4; ++j) {
      const f32x4 k4 = *reinterpret_cast<const f32x4*>(kr + 4 * j);
#pragma unroll
      for (int c = 0; c < 4; ++c) s = mfma_f32(k4[c], qv[4 * j + c], s);
    }
    float mx = -INFINITY;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int key = kt * 32 + f32_slot_row(i, hh);
      s[i] = (key <= row && key < p.T) ? s[i] * c2 : -INFINITY;
      mx = fmaxf(mx, s[i]);
    }
    // every tile left of the diagonal is unmasked and the diagonal tile holds
    // key 32 kt <= row, so m is finite after a wave's first tile
    const float mnew = fmaxf(m, max_with_partner(mx));
    const float alpha = exp2_fast(m - mnew);
    float ps = 0.f;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      s[i] = exp2_fast(s[i] - mnew);
      ps += s[i];
    }
    l = l * alpha + ps;
    m = mnew;
#pragma unroll
    for (int dt = 0; dt < DT; ++dt)
#pragma unroll
      for (int i = 0; i < 16; ++i) oacc[dt][i] *= alpha;
    // O^T += V^T P^T over the tile's 32 keys
#pragma unroll
    for (int j = 0; j < 16; ++j) {
      const float* vr = vbase + (int64_t)min(kt * 32 + f32_slot_row(j, hh), p.T - 1) * p.sv[2] + l32;
#pragma unroll
      for (int dt = 0; dt < DT; ++dt) oacc[dt] = mfma_f32(vr[32 * dt], s[j], oacc[dt]);
    }
  }
  // merge the four waves' (O, m, l) with the log-sum-exp rule (a wave that
  // had no tile has m = -inf and contributes nothing); m is the same on a
  // lane and its lane^32 partner
  if (wave > 0) {
#pragma unroll
    for (int dt = 0; dt < DT; ++dt)
#pragma unroll
      for (int g = 0; g < 4; ++g)
        red_o[wave - 1][dt * 4 + g][lane] =
            f32x4{oacc[dt][4 * g], oacc[dt][4 * g + 1], oacc[dt][4 * g + 2], oacc[dt][4 * g + 3]};
    red_ml[wave - 1][lane] = f32x2{m, l};
  }
  __syncthreads();
  if (wave > 0) return;
  {
    f32x2 ml[3];
    float mm = m;
#pragma unroll
    for (int w = 0; w < 3; ++w) {
      ml[w] = red_ml[w][lane];
      mm = fmaxf(mm, ml[w][0]);
    }
    const float a0 = exp2_fast(m - mm);
    l *= a0;
#pragma unroll
    for (int dt = 0; dt < DT; ++dt)
#pragma unroll
      for (int i = 0; i < 16; ++i) oacc[dt][i] *= a0;
#pragma unroll
    for (int w = 0; w < 3; ++w) {
      const float aw = exp2_fast(ml[w][0] - mm);
      l = __builtin_fmaf(aw, ml[w][1], l);
#pragma unroll
      for (int dt = 0; dt < DT; ++dt)
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const f32x4 o = red_o[w][dt * 4 + g][lane];
#pragma unroll
          for (int e = 0; e < 4; ++e) oacc[dt][4 * g + e] = __builtin_fmaf(aw, o[e], oacc[dt][4 * g + e]);
        }
    }
    m = mm;
  }
  if (row >= p.T) return;
  const float lt = sum_with_partner(l);
  const float inv = 1.f / lt;
  float* ob = fptr(p.out) + task.b * p.so[0] + (int64_t)task.h * p.so[1] + (int64_t)row * p.so[2];
#pragma unroll
  for (int dt = 0; dt < DT; ++dt)
#pragma unroll
    for (int g = 0; g < 4; ++g)
      *reinterpret_cast<f32x4*>(ob + 32 * dt + 8 * g + 4 * hh) =
          f32x4{oacc[dt][4 * g] * inv, oacc[dt][4 * g + 1] * inv, oacc[dt][4 * g + 2] * inv, oacc[dt][4 * g + 3] * inv};
  if (hh == 0) p.lse[((int64_t)task.b * p.Hq + task.h) * p.T + row] = (m + __builtin_amdgcn_logf(lt)) * kLn2;
}

// ---------------------------------------------------------------------------
// Backward prep: -delta = -rowsum(O * dO) and -LSE log2(e) (fp32 O and dO).
// ---------------------------------------------------------------------------
template <int D>
__global__ __launch_bounds__(256) void attn_bwd_prep_f32_kernel(AttnParams p) {
  constexpr int LPR = D / 4;  // lanes per row, one 16-byte chunk each
  const int64_t rows = (int64_t)p.B * p.Hq * p.T;
  const int64_t row = (int64_t)blockIdx.x * (256 / LPR) + threadIdx.x / LPR;
  const int c = threadIdx.x % LPR;
  float sum = 0.f;
  if (row < rows) {
    const int t = int(row % p.T);
    const int64_t bh = row / p.T;
    const int h = int(bh % p.Hq);
    const int64_t b = bh / p.Hq;
    const f32x4 o = *reinterpret_cast<const f32x4*>(fptr(p.o) + b * p.so[0] + h * p.so[1] + (int64_t)t * p.so[2] + 4 * c);
    const f32x4 g =
        *reinterpret_cast<const f32x4*>(fptr(p.dout) + b * p.sdo[0] + h * p.sdo[1] + (int64_t)t * p.sdo[2] + 4 * c);
    sum = o[0] * g[0] + o[1] * g[1] + o[2] * g[2] + o[3] * g[3];
  }
#pragma unroll
  for (int msk = 1; msk < LPR; msk <<= 1) sum += __shfl_xor(sum, msk, LPR);
  if (c == 0 && row < rows) {
    p.ndelta[row] = -sum;
    p.nlse2[row] = -p.lse[row] * kLog2e;
  }
}

// ---------------------------------------------------------------------------
// Backward dQ: per workgroup 32 query rows of one head; the 32-key tiles on
// or left of the diagonal are dealt to the 4 waves in turn (each recomputes
// S^T and dP^T for its tiles, lane = query: P = 2^(S c - LSE2), dS = P (dP -
// delta), dQ^T += K^T dS^T), and the four partial sums are added through LDS.
// ---------------------------------------------------------------------------
template <int D, bool ROPE>
__global__ __launch_bounds__(256) void attn_bwd_dq_f32_kernel(AttnParams p) {
  constexpr int HD = D / 2;
  constexpr int DT = D / 32;
  __shared__ f32x4 red[3][DT * 4][64];  // waves 1-3: [wave - 1][dt, g][lane]
  const int lane = threadIdx.x & 63, l32 = lane & 31, hh = lane >> 5;
  const int wave = threadIdx.x >> 6;
  const int nblk = (p.T + 31) / 32;
  const int t = blockIdx.x;
  if (t >= p.B * p.Hq * nblk) return;  // (workgroup-uniform)
  const F32Task task = f32_task(t, p.B, p.Hq, nblk, true);
  const int kvh = task.h / p.R;
  const int row = task.blk * 32 + l32;
  const int rc = min(row, p.T - 1);
  const int64_t rowbase = ((int64_t)task.b * p.Hq + task.h) * p.T;

  float qv[HD], gv[HD];
  {
    const float* qr = fptr(p.q) + task.b * p.sq[0] + (int64_t)task.h * p.sq[1] + (int64_t)rc * p.sq[2] + hh * HD;
    const float* gr = fptr(p.dout) + task.b * p.sdo[0] + (int64_t)task.h * p.sdo[1] + (int64_t)rc * p.sdo[2] + hh * HD;
#pragma unroll
    for (int j = 0; j < HD / 4; ++j) {
      const f32x4 a = *reinterpret_cast<const f32x4*>(qr + 4 * j);
      const f32x4 b = *reinterpret_cast<const f32x4*>(gr + 4 * j);
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        qv[4 * j + c] = a[c];
        gv[4 * j + c] = b[c];
      }
    }
  }
  const float nl2 = p.nlse2[rowbase + rc];
  const float nd = p.ndelta[rowbase + rc];
  const float* kbase = fptr(p.k) + task.b * p.sk[0] + (int64_t)kvh * p.sk[1];
  const float* vbase = fptr(p.v) + task.b * p.sv[0] + (int64_t)kvh * p.sv[1];
  const float c2 = p.scale_log2;

  f32x16 dq[DT];
#pragma unroll
  for (int dt = 0; dt < DT; ++dt) zero16(dq[dt]);
  for (int kt = wave; kt <= task.blk; kt += 4) {
    const int kc = min(kt * 32 + l32, p.T - 1);
    const float* kr = kbase + (int64_t)kc * p.sk[2] + hh * HD;
    const float* vr = vbase + (int64_t)kc * p.sv[2] + hh * HD;
    f32x16 s = {}, dp = {};
#pragma unroll
    for (int j = 0; j < HD / 4; ++j) {
      const f32x4 k4 = *reinterpret_cast<const f32x4*>(kr + 4 * j);
      const f32x4 v4 = *reinterpret_cast<const f32x4*>(vr + 4 * j);
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        s = mfma_f32(k4[c], qv[4 * j + c], s);
        dp = mfma_f32(v4[c], gv[4 * j + c], dp);
      }
    }
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int key = kt * 32 + f32_slot_row(i, hh);
      const float pv = (key <= row && key < p.T && row < p.T) ? exp2_fast(__builtin_fmaf(s[i], c2, nl2)) : 0.f;
      s[i] = pv * (dp[i] + nd);  // dS
    }
#pragma unroll
    for (int j = 0; j < 16; ++j) {
      const float* kj = kbase + (int64_t)min(kt * 32 + f32_slot_row(j, hh), p.T - 1) * p.sk[2] + l32;
#pragma unroll
      for (int dt = 0; dt < DT; ++dt) dq[dt] = mfma_f32(kj[32 * dt], s[j], dq[dt]);
    }
  }
  // the four waves' partial sums: waves 1-3 hand theirs to wave 0
  if (wave > 0) {
#pragma unroll
    for (int dt = 0; dt < DT; ++dt)
#pragma unroll
      for (int g = 0; g < 4; ++g)
        red[wave - 1][dt * 4 + g][lane] = f32x4{dq[dt][4 * g], dq[dt][4 * g + 1], dq[dt][4 * g + 2], dq[dt][4 * g + 3]};
  }
  __syncthreads();
  if (wave > 0) return;
#pragma unroll
  for (int w = 0; w < 3; ++w)
#pragma unroll
    for (int dt = 0; dt < DT; ++dt)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const f32x4 a = red[w][dt * 4 + g][lane];
#pragma unroll
        for (int e = 0; e < 4; ++e) dq[dt][4 * g + e] += a[e];
      }
  if (row >= p.T) return;
  float* out = fptr(p.out) + task.b * p.sout[0] + (int64_t)task.h * p.sout[1] + (int64_t)row * p.sout[2];
#pragma unroll
  for (int dt = 0; dt < DT; ++dt)
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const int d = 32 * dt + 8 * g + 4 * hh;
      float x0 = dq[dt][4 * g] * p.scale, x1 = dq[dt][4 * g + 1] * p.scale;
      float x2 = dq[dt][4 * g + 2] * p.scale, x3 = dq[dt][4 * g + 3] * p.scale;
      if constexpr (ROPE)
        rope_back4(x0, x1, x2, x3, p.cos + (int64_t)row * (D / 2) + d / 2, p.sin + (int64_t)row * (D / 2) + d / 2);
      *reinterpret_cast<f32x4*>(out + d) = f32x4{x0, x1, x2, x3};
    }
}

// ---------------------------------------------------------------------------
// Backward dK / dV: per workgroup 32 keys of one KV head, K and V in
// registers; the (query head, 32-row tile on or below the diagonal) pairs of
// the block are dealt to the 4 waves in turn (each recomputes S and dP for its
// pairs: lane = key, slots = rows; dV^T += dO^T P, dK^T += Q^T dS), and the
// four partial sums are added through LDS.  A wave per key block would leave
// most of the GPU idle at small shapes (32 waves on 1024
// SIMDs, the longest walking every row of its heads).
// ---------------------------------------------------------------------------
template <int D, bool ROPE>
__global__ __launch_bounds__(256) void attn_bwd_dkv_f32_kernel(AttnParams p) {
  constexpr int HD = D / 2;
  constexpr int DT = D / 32;
  __shared__ f32x4 red[3][2 * DT * 4][64];  // waves 1-3: [wave - 1][dK / dV, dt, g][lane]
  const int lane = threadIdx.x & 63, l32 = lane & 31, hh = lane >> 5;
  const int wave = threadIdx.x >> 6;
  const int nblk = (p.T + 31) / 32;
  const int t = blockIdx.x;
  if (t >= p.B * p.Hkv * nblk) return;  // (workgroup-uniform)
  const F32Task task = f32_task(t, p.B, p.Hkv, nblk, false);  // smallest key block (most rows) first
  const int key = task.blk * 32 + l32;
  const int kc = min(key, p.T - 1);

  float kv[HD], vv[HD];
  {
    const float* kr = fptr(p.k) + task.b * p.sk[0] + (int64_t)task.h * p.sk[1] + (int64_t)kc * p.sk[2] + hh * HD;
    const float* vr = fptr(p.v) + task.b * p.sv[0] + (int64_t)task.h * p.sv[1] + (int64_t)kc * p.sv[2] + hh * HD;
#pragma unroll
    for (int j = 0; j < HD / 4; ++j) {
      const f32x4 a = *reinterpret_cast<const f32x4*>(kr + 4 * j);
      const f32x4 b = *reinterpret_cast<const f32x4*>(vr + 4 * j);
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        kv[4 * j + c] = a[c];
        vv[4 * j + c] = b[c];
      }
    }
  }
  const float c2 = p.scale_log2;
  f32x16 dk[DT], dv[DT];
#pragma unroll
  for (int dt = 0; dt < DT; ++dt) {
    zero16(dk[dt]);
    zero16(dv[dt]);
  }
  const int ntile = nblk - task.blk;  // row tiles per head on or below the diagonal
  for (int u = wave; u < p.R * ntile; u += 4) {
    const int r = u % p.R;
    const int qt = task.blk + u / p.R;
    const int head = task.h * p.R + r;
    const float* qbase = fptr(p.q) + task.b * p.sq[0] + (int64_t)head * p.sq[1];
    const float* gbase = fptr(p.dout) + task.b * p.sdo[0] + (int64_t)head * p.sdo[1];
    const int64_t rowbase = ((int64_t)task.b * p.Hq + head) * p.T;
    {
      // S and dP: rows m = the tile's queries, lane = key
      const int qa = min(qt * 32 + l32, p.T - 1);
      const float* qr = qbase + (int64_t)qa * p.sq[2] + hh * HD;
      const float* gr = gbase + (int64_t)qa * p.sdo[2] + hh * HD;
      f32x16 s = {}, dp = {};
#pragma unroll
      for (int j = 0; j < HD / 4; ++j) {
        const f32x4 q4 = *reinterpret_cast<const f32x4*>(qr + 4 * j);
        const f32x4 g4 = *reinterpret_cast<const f32x4*>(gr + 4 * j);
#pragma unroll
        for (int c = 0; c < 4; ++c) {
          s = mfma_f32(q4[c], kv[4 * j + c], s);
          dp = mfma_f32(g4[c], vv[4 * j + c], dp);
        }
      }
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int qrow = qt * 32 + f32_slot_row(i, hh);
        const int qcl = min(qrow, p.T - 1);
        const bool ok = key <= qrow && qrow < p.T && key < p.T;
        const float pv = ok ? exp2_fast(__builtin_fmaf(s[i], c2, p.nlse2[rowbase + qcl])) : 0.f;
        s[i] = pv;
        dp[i] = pv * (dp[i] + p.ndelta[rowbase + qcl]);  // dS
      }
#pragma unroll
      for (int j = 0; j < 16; ++j) {
        const int qj = min(qt * 32 + f32_slot_row(j, hh), p.T - 1);
        const float* qrj = qbase + (int64_t)qj * p.sq[2] + l32;
        const float* grj = gbase + (int64_t)qj * p.sdo[2] + l32;
#pragma unroll
        for (int dt = 0; dt < DT; ++dt) {
          dv[dt] = mfma_f32(grj[32 * dt], s[j], dv[dt]);
          dk[dt] = mfma_f32(qrj[32 * dt], dp[j], dk[dt]);
        }
      }
    }
  }
  // the four waves' partial sums: waves 1-3 hand theirs to wave 0
  if (wave > 0) {
#pragma unroll
    for (int dt = 0; dt < DT; ++dt)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        red[wave - 1][dt * 4 + g][lane] = f32x4{dk[dt][4 * g], dk[dt][4 * g + 1], dk[dt][4 * g + 2], dk[dt][4 * g + 3]};
        red[wave - 1][(DT + dt) * 4 + g][lane] =
            f32x4{dv[dt][4 * g], dv[dt][4 * g + 1], dv[dt][4 * g + 2], dv[dt][4 * g + 3]};
      }
  }
  __syncthreads();
  if (wave > 0) return;
#pragma unroll
  for (int w = 0; w < 3; ++w)
#pragma unroll
    for (int dt = 0; dt < DT; ++dt)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const f32x4 a = red[w][dt * 4 + g][lane], b = red[w][(DT + dt) * 4 + g][lane];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          dk[dt][4 * g + e] += a[e];
          dv[dt][4 * g + e] += b[e];
        }
      }
  if (key >= p.T) return;
  float* dkr = fptr(p.dk) + task.b * p.sdk[0] + (int64_t)task.h * p.sdk[1] + (int64_t)key * p.sdk[2];
  float* dvr = fptr(p.dv) + task.b * p.sdv[0] + (int64_t)task.h * p.sdv[1] + (int64_t)key * p.sdv[2];
#pragma unroll
  for (int dt = 0; dt < DT; ++dt)
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const int d = 32 * dt + 8 * g + 4 * hh;
      float x0 = dk[dt][4 * g] * p.scale, x1 = dk[dt][4 * g + 1] * p.scale;
      float x2 = dk[dt][4 * g + 2] * p.scale, x3 = dk[dt][4 * g + 3] * p.scale;
      if constexpr (ROPE)
        rope_back4(x0, x1, x2, x3, p.cos + (int64_t)key * (D / 2) + d / 2, p.sin + (int64_t)key * (D / 2) + d / 2);
      *reinterpret_cast<f32x4*>(dkr + d) = f32x4{x0, x1, x2, x3};
      *reinterpret_cast<f32x4*>(dvr + d) = f32x4{dv[dt][4 * g], dv[dt][4 * g + 1], dv[dt][4 * g + 2], dv[dt][4 * g + 3]};
    }
}

}  // namespace mt
