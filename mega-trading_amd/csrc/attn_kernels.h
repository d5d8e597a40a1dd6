// gfx950 causal grouped-query attention: forward, backward-dQ, backward-dK/dV.
//
// Reference algorithm: src/mega_trading/kernels/triton_attention.py
//   forward  :260-358  (online softmax, LSE = m + ln l, P rounded to the input
//                       dtype before the PV product)
//   dQ       :481-615  (delta = rowsum(O*dO), P = exp(S - LSE), dS = P (dP - delta),
//                       dQ = scale dS K)
//   dK/dV    :618-747  (per KV block, loop over the group's query heads and the
//                       causal row blocks; dV = P^T dO, dK = scale dS^T Q)
// and the interleaved RoPE of src/mega_trading/model.py:312-316.
//
// RoPE.  The forward rotates each Q tile as it loads it into registers and
// writes the rotated rows out (Q_rot); K is rotated once per call by a
// streaming pass (K_rot) whose output feeds the forward's K tiles.  The
// backward consumes Q_rot / K_rot directly and rotates dQ / dK back by -theta
// in its epilogues (src/mega_trading/kernels/triton_ops.py:205-214).
//
// Tiling.  A "row block" is 64 query rows of one head.
//   * forward / dQ (D <= 64): a workgroup is 4 waves; each wave owns one
//     (query head, row block).  The 4 waves are the R_SUB = min(R, 4) heads of
//     one KV group times 4/R_SUB consecutive row blocks, so every K/V tile
//     staged in LDS feeds all of them (forward: 128-key tiles, dQ: 64-key
//     tiles, both double-buffered).  S^T = K Q^T puts one query per lane
//     (lane % 32), keys along the accumulator slots; the row max needs one
//     lane^32 swap.  At D = 128 the same (head, row block) pairs are split
//     into two 32-row waves (8 waves per workgroup, two per SIMD), which keeps
//     the wider rows within 256 registers.
//   * dK/dV: a workgroup is 4 waves of 32 keys each (a 128-key block of one
//     KV head, K and V held in registers); it walks (query head, 128-row step
//     on or below the diagonal) with the Q / dO rows of each step staged in
//     LDS once for all 4 waves.  The group's heads may be split over several
//     workgroups (fp32 partial sums, combined by attn_bwd_combine_kernel) so
//     the causal triangle spreads over enough workgroups to balance.
//   * Backward launches: a prep pass writes -delta and -LSE log2(e) per query
//     row; at D <= 64 the dQ and dK/dV workgroups then share one grid
//     (attn_bwd_kernel), at D = 128 they are two launches.
// Fully masked causal tiles are never visited; only diagonal tiles mask.
#pragma once

#include "lds_tile.h"
#include "mt_common.h"

namespace mt {

constexpr int kBlk = 64;   // rows per row block (and keys per dQ K/V tile)

struct AttnParams {
  // [B, H, T, D] tensors, element strides (b, h, t); the d stride is 1.
  const uint16_t* q;     // forward: un-rotated Q.  backward: the Q scores used (rotated if RoPE)
  const uint16_t* k;     // forward: K (rotated if RoPE: the K_rot buffer).  backward: as for q
  const uint16_t* v;
  const uint16_t* o;
  const uint16_t* dout;
  uint16_t* out;   // forward: O.  backward: dQ
  uint16_t* qrot;  // forward with RoPE: rotated Q out (contiguous [B,Hq,T,D])
  uint16_t* dk;
  uint16_t* dv;
  float* lse;      // [B, Hq, T] natural-log LSE (written by fwd, read by bwd)
  float* ndelta;   // [B, Hq, T] -rowsum(O * dO) workspace (written by the prep pass, read by dQ and dK/dV)
  float* nlse2;    // [B, Hq, T] -LSE * log2(e) workspace (written by the prep pass, read by dQ and dK/dV)
  float* part;     // [n_split, 2, B, Hkv, T, D] fp32 dK/dV partial sums (bwd, n_split > 1)
  const float* cos;  // [T, D/2] fp32 or null
  const float* sin;
  int64_t sq[3], sk[3], sv[3], so[3], sdo[3], sout[3], sdk[3], sdv[3];
  int B, Hq, Hkv, T, R;
  int r_sub;      // heads of a group per workgroup (fwd / dQ)
  int n_hsub;     // R / r_sub
  int rb;         // row blocks per workgroup (4 / r_sub)
  int nqb;        // ceil(T / 64)
  int nsb;        // ceil(nqb / rb)
  int n_split;    // dK/dV: workgroups sharing one key block (each sums a range of the R heads)
  int nkb;        // dK/dV: key blocks
  int n_kv_tasks; // attn_bwd_kernel: dK/dV workgroups in the grid
  int n_dq_tasks; // attn_bwd_kernel: dQ workgroups in the grid
  int fwd_fold;   // forward grids of one resident round: workgroups past this index run in reverse order (0: off)
  // attn_bwd_kernel task order, in chunks (of 8 workgroups, or of 1): mg_head
  // chunks of one kind (dK/dV if mg_head_kv), then mg_mid_kv dK/dV and
  // mg_mid_dq dQ chunks interleaved in proportion, then the rest of one kind
  int mg_head, mg_head_kv, mg_mid_kv, mg_mid_dq;
  float scale;       // softmax scale (1/sqrt(D) by default)
  float scale_log2;  // scale * log2(e)
};

// ---------------------------------------------------------------------------
// small helpers
// ---------------------------------------------------------------------------
__device__ __forceinline__ u32x4 load_chunk(const uint16_t* base, int64_t st, int row, int T, int d0) {
  if (row < T) return *reinterpret_cast<const u32x4*>(base + (int64_t)row * st + d0);
  return zero4();
}

template <int D>
__device__ __forceinline__ void load_rope_cs(const float* cos, const float* sin, int row, int d0, f32x4& c, f32x4& s) {
  c = *reinterpret_cast<const f32x4*>(cos + (int64_t)row * (D / 2) + d0 / 2);
  s = *reinterpret_cast<const f32x4*>(sin + (int64_t)row * (D / 2) + d0 / 2);
}

// Pack C-tile slots [i0, i0+8) to an 8-wide 16-bit operand.
template <class E>
__device__ __forceinline__ typename E::v8 pack8(const f32x16& x, int i0) {
  u32x4 w;
#pragma unroll
  for (int p = 0; p < 4; ++p) w[p] = pack2<E>(x[i0 + 2 * p], x[i0 + 2 * p + 1]);
  return __builtin_bit_cast(typename E::v8, w);
}

__device__ __forceinline__ void zero16(f32x16& x) {
#pragma unroll
  for (int i = 0; i < 16; ++i) x[i] = 0.f;
}

// Rotate 4 consecutive d values (2 interleaved pairs) by -theta in place.
__device__ __forceinline__ void rope_back4(float& x0, float& x1, float& x2, float& x3, const float* cs, const float* sn) {
  const f32x2 c = *reinterpret_cast<const f32x2*>(cs);
  const f32x2 s = *reinterpret_cast<const f32x2*>(sn);
  const float y0 = x0 * c[0] + x1 * s[0], y1 = x1 * c[0] - x0 * s[0];
  const float y2 = x2 * c[1] + x3 * s[1], y3 = x3 * c[1] - x2 * s[1];
  x0 = y0; x1 = y1; x2 = y2; x3 = y3;
}

// Workgroup -> (batch, kv head, head subset, super block) for fwd / dQ; the
// longest causal rows are issued first.  Consecutive workgroups share a
// (batch, kv head, subset) slot modulo the group count, so with a group count
// that is a multiple of 8 every KV stream stays on one XCD.
struct RowTask {
  int b, kvh, hs, sb;
};
__device__ __forceinline__ RowTask row_task(const AttnParams& p, int L) {
  const int groups = p.B * p.Hkv * p.n_hsub;
  RowTask t;
  t.sb = p.nsb - 1 - L / groups;
  const int g = L % groups;
  t.hs = g % p.n_hsub;
  const int bk = g / p.n_hsub;
  t.kvh = bk % p.Hkv;
  t.b = bk / p.Hkv;
  return t;
}

// A forward grid that fits one resident round (at most two workgroups per CU)
// gets no dynamic balancing: every workgroup starts at once, and a CU's time
// is the sum of its two workgroups' causal lengths.  The first `fold`
// workgroups (one per CU) keep the heaviest-first order; the rest run in
// reverse, lightest first, so the workgroup that shares a CU with the k-th
// heaviest is the k-th lightest and every CU gets about the same work.  The
// reversal moves whole chunks of 8 workgroups, so a workgroup keeps its XCD
// (index mod 8).
__device__ __forceinline__ int fold_order(int L, int n, int fold) {
  if (fold == 0 || L < fold) return L;
  const int m = n - fold, j = L - fold;
  if (((m | fold) & 7) == 0) return fold + (m - 8 - (j & ~7)) + (j & 7);
  return fold + (m - 1 - j);
}

// ===========================================================================
// RoPE streaming pass: Y = rot(X) for a [B, H, T, D] tensor, Y contiguous.
// One thread per 16-byte chunk (4 interleaved pairs).
// ===========================================================================
template <class E, int D>
__global__ __launch_bounds__(256) void rope_rows_kernel(const uint16_t* x, int64_t s0, int64_t s1, int64_t s2,
                                                        uint16_t* y, const float* cos, const float* sin,
                                                        int H, int T, int64_t n_chunks) {
  const int64_t c = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (c >= n_chunks) return;
  constexpr int NC = D / 8;
  const int d0 = int(c % NC) * 8;
  const int64_t row = c / NC;  // (b*H + h)*T + t
  const int t = int(row % T);
  const int64_t bh = row / T;
  const int h = int(bh % H);
  const int64_t b = bh / H;
  u32x4 v = *reinterpret_cast<const u32x4*>(x + b * s0 + h * s1 + (int64_t)t * s2 + d0);
  f32x4 cs, sn;
  load_rope_cs<D>(cos, sin, t, d0, cs, sn);
  *reinterpret_cast<u32x4*>(y + row * D + d0) = rope_chunk<E>(v, cs, sn);
}

// ===========================================================================
// Forward
// ===========================================================================
// Lazy rescaling: the running row offset m (log2 units) is only raised when a
// quarter's probabilities P = 2^(s*c - m) may exceed 2^kRescaleSlack, which is
// detected from the quarter's row sums (any P above the bound makes the sum
// exceed it; a NaN sum -- the first quarter, with m = -inf -- also fails the
// test).  The row max is computed only then, O and l are rescaled and the
// quarter's P recomputed.  P stays below 2^kRescaleSlack (fits fp16 too), and
// O = acc / l and LSE = (m + log2 l) ln 2 are exact for any m, so the result
// does not depend on when rescales happen.  Row sums add the packed 16-bit P
// (v_dot2c with 1.0, 1.0), i.e. exactly the weights the PV product uses.
constexpr float kRescaleSlack = 8.0f;
constexpr float kSumLimit = 256.0f;  // 2^kRescaleSlack
constexpr int kFwdKeys = 128;  // keys per staged K/V tile (two 64-row halves)

// One 128-key tile for one wave (64 query rows, two 32-row column tiles nt).
// Quarter h = keys kt0 + 32h .. +31.  Pipeline (issue order):
//   S0 | S1 + E0 | C0 | PV0 + S2 + E1 | C1 | PV1 + S3 + E2 | C2 | PV2 + E3 | C3 | PV3
// Sh = scores of quarter h, Eh = its exponentials, packing and row sums,
// Ch = the overflow test and (rare, wave-uniform) rescale, PVh = O += P V.
// With MASK (the tile holding this wave's diagonal) keys above the query are
// masked and quarters wholly above the wave's rows are skipped.
template <class E, int D, bool MASK>
__device__ __forceinline__ void fwd_tile(const char* K, const char* Vt, const typename E::v8 (*qop)[D / 16],
                                         f32x16 (*oacc)[2], float* mrun, float* lrun, int rbase, TrBase tbase,
                                         int lane, int kt0, int q0, float c2) {
  using V8 = typename E::v8;
  using TL = Tile<D>;
  constexpr int KT = D / 16;
  constexpr int DT = D / 32;
  const int hh = lane >> 5;
  const int l32 = lane & 31;
  bool live[4];
#pragma unroll
  for (int h = 0; h < 4; ++h) live[h] = !MASK || (kt0 + 32 * h <= q0 + 63);

  auto sq = [&](int h, f32x16* st) {
    const char* Kh = K + (h >> 1) * TL::BYTES;
    const int r0 = 32 * (h & 1);
    V8 a = TL::template row_op<E>(Kh, rbase, r0, 0);
#pragma unroll
    for (int nt = 0; nt < 2; ++nt) st[nt] = E::mfma(a, qop[nt][0], f32x16{});
#pragma unroll
    for (int kk = 1; kk < KT; ++kk) {
      a = TL::template row_op<E>(Kh, rbase, r0, kk);
#pragma unroll
      for (int nt = 0; nt < 2; ++nt) st[nt] = E::mfma(a, qop[nt][kk], st[nt]);
    }
  };
  // P = 2^(S c2 - m) packed to 16 bits (S kept for a possible rescale);
  // qs = this lane's share of the quarter's row sums
  auto ex = [&](int h, f32x16* st, V8 (*pk)[2], float* qs) {
#pragma unroll
    for (int nt = 0; nt < 2; ++nt) {
      if constexpr (MASK) {
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          const int kr = kt0 + 32 * h + 8 * (i >> 2) + 4 * hh + (i & 3);
          if (kr > q0 + 32 * nt + l32) st[nt][i] = -INFINITY;
        }
      }
      const float moff = mrun[nt];
      u32x4 w[2];
#pragma unroll
      for (int p2 = 0; p2 < 8; ++p2) {
        const float a = exp2_fast(__builtin_fmaf(st[nt][2 * p2], c2, -moff));
        const float b = exp2_fast(__builtin_fmaf(st[nt][2 * p2 + 1], c2, -moff));
        w[p2 >> 2][p2 & 3] = pack2<E>(a, b);
      }
      float s0 = E::sum2(w[0][0], 0.f), s1 = E::sum2(w[1][0], 0.f);
#pragma unroll
      for (int p = 1; p < 4; ++p) {
        s0 = E::sum2(w[0][p], s0);
        s1 = E::sum2(w[1][p], s1);
      }
      qs[nt] = s0 + s1;
      pk[nt][0] = __builtin_bit_cast(V8, w[0]);
      pk[nt][1] = __builtin_bit_cast(V8, w[1]);
    }
  };
  // overflow test; on failure raise m to the row max, rescale O and l, redo E
  auto chk = [&](int h, f32x16* st, V8 (*pk)[2], float* qs) {
    const bool bad = !(qs[0] <= kSumLimit) || !(qs[1] <= kSumLimit);
    if (__builtin_amdgcn_ballot_w64(bad)) {
#pragma unroll
      for (int nt = 0; nt < 2; ++nt) {
        float v = -INFINITY;
#pragma unroll
        for (int i = 0; i < 16; ++i) v = fmaxf(v, st[nt][i]);
        const float mnew = fmaxf(mrun[nt], max_with_partner(v) * c2);
        const float alpha = exp2_fast(mrun[nt] - mnew);
        mrun[nt] = mnew;
        lrun[nt] *= alpha;
#pragma unroll
        for (int dt = 0; dt < DT; ++dt)
#pragma unroll
          for (int i = 0; i < 16; ++i) oacc[dt][nt][i] *= alpha;
      }
      ex(h, st, pk, qs);
    }
    lrun[0] += qs[0];
    lrun[1] += qs[1];
  };
  auto pv = [&](int h, V8 (*pk)[2]) {
    const char* Vh = Vt + (h >> 1) * TL::BYTES;
#pragma unroll
    for (int k2 = 0; k2 < 2; ++k2)
#pragma unroll
      for (int dt = 0; dt < DT; ++dt) {
        const V8 a = TL::template tr_op<E>(Vh, tbase, 2 * (h & 1) + k2, dt);
#pragma unroll
        for (int nt = 0; nt < 2; ++nt) oacc[dt][nt] = E::mfma(a, pk[nt][k2], oacc[dt][nt]);
      }
  };

  f32x16 st[2][2];                 // ring: two quarters' scores [slot][nt]
  V8 pk[2][2][2];                  // ring: two quarters' packed P [slot][nt][k2]
  float qs[2];
  // LDS operand reads run one step ahead of the MFMAs that consume them
  if (live[0]) sq(0, st[0]);
  __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
#pragma unroll
  for (int i = 0; i < KT; ++i) {
    __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
    __builtin_amdgcn_sched_group_barrier(0x008, 2, 0);
  }
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int h = 0; h < 4; ++h) {
    // region: PV(h-1) + S(h+1) MFMAs interleaved with E(h)
    if (h > 0 && live[h - 1]) pv(h - 1, pk[(h + 1) & 1]);
    if (h < 3 && live[h + 1]) sq(h + 1, st[(h + 1) & 1]);
    if (live[h]) ex(h, st[h & 1], pk[h & 1], qs);
    // the interleaving inside the stage is left to the scheduler (explicit
    // sched_group_barrier patterns of k VALU per MFMA measured slower)
    __builtin_amdgcn_sched_barrier(0);
    // C(h): after PV(h-1), so a rescale of O covers everything accumulated
    if (live[h]) chk(h, st[h & 1], pk[h & 1], qs);
    __builtin_amdgcn_sched_barrier(0);
  }
  if (live[3]) pv(3, pk[1]);
}

// PEEL: as for the dQ kernel, the 4 waves share one row block, so the
// diagonal (masked) tile is the last one and runs after the loop.
template <class E, int D, bool ROPE, bool PEEL>
__global__ __launch_bounds__(256, 2) void attn_fwd_kernel(AttnParams p) {
  static_assert(D <= 64, "D = 128 uses attn_fwd_w8_kernel");
  using V8 = typename E::v8;
  using TL = Tile<D>;
  constexpr int KT = D / 16;            // k-steps over d
  constexpr int DT = D / 32;            // 32-wide d tiles
  // [buf][K, V] x 128 rows (two 64-row tiles back to back)
  __shared__ __attribute__((aligned(1024))) char smem[2][2][2 * TL::BYTES];

  const RowTask task = row_task(p, fold_order(blockIdx.x, gridDim.x, p.fwd_fold));
  const int tid = threadIdx.x;
  const int wave = tid >> 6;
  const int lane = tid & 63;
  const int l32 = lane & 31;
  const int hh = lane >> 5;
  const int head = task.kvh * p.R + task.hs * p.r_sub + (wave % p.r_sub);
  const int qb = task.sb * p.rb + wave / p.r_sub;   // this wave's row block
  const int q0 = qb * kBlk;
  const bool active = qb < p.nqb;
  const int jw = (q0 + kBlk - 1) / kFwdKeys;        // this wave's diagonal tile
  // last KV tile any wave of the workgroup needs
  const int last_row = min(p.T, (task.sb * p.rb + p.rb) * kBlk) - 1;
  const int jlast = last_row / kFwdKeys;

  const uint16_t* kbase = p.k + task.b * p.sk[0] + (int64_t)task.kvh * p.sk[1];
  const uint16_t* vbase = p.v + task.b * p.sv[0] + (int64_t)task.kvh * p.sv[1];

  // Q^T as B operands (N = query, k = d), rotated if RoPE (and written out).
  // Every load is issued before the first use and the first Q_rot store, so
  // the prologue costs one memory round trip (rows past T load row T-1 and
  // are zeroed).
  V8 qop[2][KT];
  {
    const uint16_t* qbase = p.q + task.b * p.sq[0] + (int64_t)head * p.sq[1];
    uint16_t* rbase = ROPE ? p.qrot + ((int64_t)task.b * p.Hq + head) * p.T * D : nullptr;
    u32x4 x[2][KT];
    f32x4 cs[2][ROPE ? KT : 1], sn[2][ROPE ? KT : 1];
#pragma unroll
    for (int nt = 0; nt < 2; ++nt) {
      const int rc = min(q0 + nt * 32 + l32, p.T - 1);
#pragma unroll
      for (int kk = 0; kk < KT; ++kk) {
        const int d0 = 16 * kk + 8 * hh;
        x[nt][kk] = *reinterpret_cast<const u32x4*>(qbase + (int64_t)rc * p.sq[2] + d0);
        if constexpr (ROPE) load_rope_cs<D>(p.cos, p.sin, rc, d0, cs[nt][kk], sn[nt][kk]);
      }
    }
#pragma unroll
    for (int nt = 0; nt < 2; ++nt) {
      const int row = q0 + nt * 32 + l32;
      const bool ok = active && row < p.T;
#pragma unroll
      for (int kk = 0; kk < KT; ++kk) {
        const int d0 = 16 * kk + 8 * hh;
        u32x4 y = ok ? x[nt][kk] : zero4();
        if constexpr (ROPE) {
          y = rope_chunk<E>(y, cs[nt][kk], sn[nt][kk]);
          if (ok) *reinterpret_cast<u32x4*>(rbase + (int64_t)row * D + d0) = y;
        }
        qop[nt][kk] = __builtin_bit_cast(V8, y);
      }
    }
  }

  f32x16 oacc[DT][2];
#pragma unroll
  for (int dt = 0; dt < DT; ++dt)
#pragma unroll
    for (int nt = 0; nt < 2; ++nt) zero16(oacc[dt][nt]);
  float mrun[2] = {-INFINITY, -INFINITY};
  float lrun[2] = {0.f, 0.f};

  Stager<D, 4> ks_stage, vs_stage;
  ks_stage.init(p.sk[2], wave, lane);
  vs_stage.init(p.sv[2], wave, lane);
  const int rbase_op = TL::row_base(lane);
  const TrBase tbase_op = TL::tr_base(lane);
  auto stage = [&](int j, int buf) {
    const int r0 = j * kFwdKeys;
    ks_stage.stage(smem[buf][0], kbase, p.sk[2], r0, p.T);
    vs_stage.stage(smem[buf][1], vbase, p.sv[2], r0, p.T);
    ks_stage.stage(smem[buf][0] + TL::BYTES, kbase, p.sk[2], r0 + kBlk, p.T);
    vs_stage.stage(smem[buf][1] + TL::BYTES, vbase, p.sv[2], r0 + kBlk, p.T);
  };

  stage(0, 0);
  wait_vmem();
  __syncthreads();

  const float c2 = p.scale_log2;
  for (int j = 0; j < (PEEL ? jlast : jlast + 1); ++j) {
    const int buf = j & 1;
    if (j < jlast) stage(j + 1, buf ^ 1);
    if (active && j <= jw) {
      if (PEEL || j < jw)
        fwd_tile<E, D, false>(smem[buf][0], smem[buf][1], qop, oacc, mrun, lrun, rbase_op, tbase_op, lane,
                              j * kFwdKeys, q0, c2);
      else
        fwd_tile<E, D, true>(smem[buf][0], smem[buf][1], qop, oacc, mrun, lrun, rbase_op, tbase_op, lane,
                             j * kFwdKeys, q0, c2);
    }
    wait_vmem();
    __syncthreads();
  }
  if (PEEL && active)  // jw == jlast
    fwd_tile<E, D, true>(smem[jlast & 1][0], smem[jlast & 1][1], qop, oacc, mrun, lrun, rbase_op, tbase_op, lane,
                         jlast * kFwdKeys, q0, c2);

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
// Forward for D = 128: 8 waves of 32 query rows per workgroup
// ===========================================================================
// At D = 128 the 64-row waves of attn_fwd_kernel need one SIMD each and spill.
// Here a workgroup is 8 waves: the 4 (head, 64-row block) pairs of a RowTask
// split into two 32-row waves, two waves per SIMD, so each staged 128-key K/V
// tile still feeds 256 query rows and no wave spills.  The softmax is that of
// attn_fwd_kernel (fp32 scale and offset per score, lazy rescaling).
constexpr int kFwdW8Waves = 8;

// NQ 32-key quarters per staged tile (4: 128 keys, 2: 64 keys).  AHEAD:
// quarter h+1's scores are issued before quarter h's softmax (two score
// tiles live); without it one is, for 4 waves per SIMD at D = 64.
template <class E, int D, bool MASK, int NQ = 4, bool AHEAD = true>
__device__ __forceinline__ void fwd32_tile(const char* K, const char* Vt, const typename E::v8* qop, f32x16* oacc,
                                           float& mrun, float& lrun, int rbase, TrBase tbase, int lane, int kt0,
                                           int q0, float c2) {
  using V8 = typename E::v8;
  using TL = Tile<D>;
  constexpr int KT = D / 16;
  constexpr int DT = D / 32;
  const int hh = lane >> 5;
  const int l32 = lane & 31;
  bool live[NQ];
#pragma unroll
  for (int h = 0; h < NQ; ++h) live[h] = !MASK || (kt0 + 32 * h <= q0 + 31);

  auto sq = [&](int h, f32x16& st) {
    const char* Kh = K + (h >> 1) * TL::BYTES;
    const int r0 = 32 * (h & 1);
    st = E::mfma(TL::template row_op<E>(Kh, rbase, r0, 0), qop[0], f32x16{});
#pragma unroll
    for (int kk = 1; kk < KT; ++kk) st = E::mfma(TL::template row_op<E>(Kh, rbase, r0, kk), qop[kk], st);
  };
  // P = 2^(s*c - m) packed to 16 bits (the scores kept for a possible
  // rescale); returns this lane's share of the quarter's row sum
  auto ex = [&](int h, f32x16& st, V8* pk) {
    if constexpr (MASK) {
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int kr = kt0 + 32 * h + 8 * (i >> 2) + 4 * hh + (i & 3);
        if (kr > q0 + l32) st[i] = -INFINITY;
      }
    }
    const float moff = mrun;
    u32x4 w[2];
#pragma unroll
    for (int p2 = 0; p2 < 8; ++p2)
      w[p2 >> 2][p2 & 3] = pack2<E>(exp2_fast(__builtin_fmaf(st[2 * p2], c2, -moff)),
                                    exp2_fast(__builtin_fmaf(st[2 * p2 + 1], c2, -moff)));
    float s0 = E::sum2(w[0][0], 0.f), s1 = E::sum2(w[1][0], 0.f);
#pragma unroll
    for (int q = 1; q < 4; ++q) {
      s0 = E::sum2(w[0][q], s0);
      s1 = E::sum2(w[1][q], s1);
    }
    pk[0] = __builtin_bit_cast(V8, w[0]);
    pk[1] = __builtin_bit_cast(V8, w[1]);
    return s0 + s1;
  };
  // overflow test (the first quarter, m = -inf, fails it by construction); on
  // failure raise m to the row max, rescale O and l and redo E
  auto chk = [&](int h, f32x16& st, V8* pk, float qs) {
    if (__builtin_amdgcn_ballot_w64(!(qs <= kSumLimit))) {
      float v = -INFINITY;
#pragma unroll
      for (int i = 0; i < 16; ++i) v = fmaxf(v, st[i]);
      const float mnew = fmaxf(mrun, max_with_partner(v) * c2);
      const float alpha = exp2_fast(mrun - mnew);
      mrun = mnew;
      lrun *= alpha;
#pragma unroll
      for (int dt = 0; dt < DT; ++dt)
#pragma unroll
        for (int i = 0; i < 16; ++i) oacc[dt][i] *= alpha;
      qs = ex(h, st, pk);
    }
    lrun += qs;
  };
  auto pv = [&](int h, const V8* pk) {
    const char* Vh = Vt + (h >> 1) * TL::BYTES;
#pragma unroll
    for (int k2 = 0; k2 < 2; ++k2)
#pragma unroll
      for (int dt = 0; dt < DT; ++dt)
        oacc[dt] = E::mfma(TL::template tr_op<E>(Vh, tbase, 2 * (h & 1) + k2, dt), pk[k2], oacc[dt]);
  };

  // S(h+1) is issued before E(h) so the score MFMAs overlap the softmax
  f32x16 st[AHEAD ? 2 : 1];
  V8 pk[2];
  if (AHEAD && live[0]) sq(0, st[0]);
#pragma unroll
  for (int h = 0; h < NQ; ++h) {
    if constexpr (AHEAD) {
      if (h < NQ - 1 && live[h + 1]) sq(h + 1, st[(h + 1) & 1]);
    } else {
      if (live[h]) sq(h, st[0]);
    }
    float qs = 0.f;
    if (live[h]) qs = ex(h, st[AHEAD ? (h & 1) : 0], pk);
    __builtin_amdgcn_sched_barrier(0);
    if (live[h]) {
      chk(h, st[AHEAD ? (h & 1) : 0], pk, qs);
      pv(h, pk);
    }
    __builtin_amdgcn_sched_barrier(0);
  }
}

// NW waves per workgroup (the RowTask's NW / 2 (head, row block) pairs; the
// launch sets r_sub and rb for that many), KEYS keys per staged K / V tile.
// Occupancy: two workgroups per CU at D <= 64 (NW / 2 waves per SIMD, so at
// most 128 VGPRs with NW = 8), two waves per SIMD at D = 128.
template <class E, int D, bool ROPE, bool PEEL, int NW = kFwdW8Waves, int KEYS = kFwdKeys>
__global__ __launch_bounds__(64 * NW, D <= 64 ? NW / 2 : 2) void attn_fwd_w8_kernel(AttnParams p) {
  using V8 = typename E::v8;
  using TL = Tile<D>;
  constexpr int KT = D / 16;
  constexpr int DT = D / 32;
  constexpr int NQ = KEYS / 32;
  constexpr bool kAhead = !(D == 64 && NW == 8);     // register budget of 4 waves per SIMD
  constexpr int SW = TL::INSTR < NW ? TL::INSTR : NW;  // waves that stage tiles
  __shared__ __attribute__((aligned(1024))) char smem[2][2][(KEYS / 64) * TL::BYTES];  // [buf][K, V] x KEYS rows

  const RowTask task = row_task(p, fold_order(blockIdx.x, gridDim.x, p.fwd_fold));
  const int tid = threadIdx.x;
  const int wave = tid >> 6;
  const int lane = tid & 63;
  const int l32 = lane & 31;
  const int hh = lane >> 5;
  const int pw = wave >> 1;                         // (head, row block) pair of this wave
  const int head = task.kvh * p.R + task.hs * p.r_sub + (pw % p.r_sub);
  const int qb = task.sb * p.rb + pw / p.r_sub;     // this wave's row block
  const int q0 = qb * kBlk + 32 * (wave & 1);       // this wave's first row
  const bool active = qb < p.nqb && q0 < p.T;
  const int jw = (q0 + 31) / KEYS;                  // this wave's diagonal tile
  const int last_row = min(p.T, (task.sb * p.rb + p.rb) * kBlk) - 1;
  const int jlast = last_row / KEYS;

  const uint16_t* kbase = p.k + task.b * p.sk[0] + (int64_t)task.kvh * p.sk[1];
  const uint16_t* vbase = p.v + task.b * p.sv[0] + (int64_t)task.kvh * p.sv[1];

  // Q^T as B operands, rotated if RoPE (and written out); rows past T load
  // row T-1 and are zeroed
  V8 qop[KT];
  {
    const uint16_t* qbase = p.q + task.b * p.sq[0] + (int64_t)head * p.sq[1];
    uint16_t* rbase = ROPE ? p.qrot + ((int64_t)task.b * p.Hq + head) * p.T * D : nullptr;
    const int row = q0 + l32;
    const int rc = min(row, p.T - 1);
    const bool ok = active && row < p.T;
    u32x4 x[KT];
    f32x4 cs[ROPE ? KT : 1], sn[ROPE ? KT : 1];
#pragma unroll
    for (int kk = 0; kk < KT; ++kk) {
      const int d0 = 16 * kk + 8 * hh;
      x[kk] = *reinterpret_cast<const u32x4*>(qbase + (int64_t)rc * p.sq[2] + d0);
      if constexpr (ROPE) load_rope_cs<D>(p.cos, p.sin, rc, d0, cs[kk], sn[kk]);
    }
#pragma unroll
    for (int kk = 0; kk < KT; ++kk) {
      const int d0 = 16 * kk + 8 * hh;
      u32x4 y = ok ? x[kk] : zero4();
      if constexpr (ROPE) {
        y = rope_chunk<E>(y, cs[kk], sn[kk]);
        if (ok) *reinterpret_cast<u32x4*>(rbase + (int64_t)row * D + d0) = y;
      }
      qop[kk] = __builtin_bit_cast(V8, y);
    }
  }

  f32x16 oacc[DT];
#pragma unroll
  for (int dt = 0; dt < DT; ++dt) zero16(oacc[dt]);
  float mrun = -INFINITY;
  float lrun = 0.f;
  const float c2 = p.scale_log2;

  Stager<D, SW> ks_stage, vs_stage;
  const bool stager = wave < SW;
  ks_stage.init(p.sk[2], wave, lane);
  vs_stage.init(p.sv[2], wave, lane);
  const int rbase_op = TL::row_base(lane);
  const TrBase tbase_op = TL::tr_base(lane);
  auto stage = [&](int j, int buf) {
    if (!stager) return;
    const int r0 = j * KEYS;
    ks_stage.stage(smem[buf][0], kbase, p.sk[2], r0, p.T);
    vs_stage.stage(smem[buf][1], vbase, p.sv[2], r0, p.T);
    if constexpr (KEYS == 128) {
      ks_stage.stage(smem[buf][0] + TL::BYTES, kbase, p.sk[2], r0 + kBlk, p.T);
      vs_stage.stage(smem[buf][1] + TL::BYTES, vbase, p.sv[2], r0 + kBlk, p.T);
    }
  };

  stage(0, 0);
  wait_vmem();
  __syncthreads();
  for (int j = 0; j < (PEEL ? jlast : jlast + 1); ++j) {
    const int buf = j & 1;
    if (j < jlast) stage(j + 1, buf ^ 1);
    if (active && j <= jw) {
      if (PEEL || j < jw)
        fwd32_tile<E, D, false, NQ, kAhead>(smem[buf][0], smem[buf][1], qop, oacc, mrun, lrun, rbase_op, tbase_op, lane,
                                j * KEYS, q0, c2);
      else
        fwd32_tile<E, D, true, NQ, kAhead>(smem[buf][0], smem[buf][1], qop, oacc, mrun, lrun, rbase_op, tbase_op, lane,
                               j * KEYS, q0, c2);
    }
    wait_vmem();
    __syncthreads();
  }
  if (PEEL && active)  // jw == jlast
    fwd32_tile<E, D, true, NQ, kAhead>(smem[jlast & 1][0], smem[jlast & 1][1], qop, oacc, mrun, lrun, rbase_op, tbase_op,
                           lane, jlast * KEYS, q0, c2);

  if (!active) return;
  const int row = q0 + l32;
  if (row >= p.T) return;
  uint16_t* obase = p.out + task.b * p.so[0] + (int64_t)head * p.so[1];
  float* lbase = p.lse + ((int64_t)task.b * p.Hq + head) * p.T;
  const float lt = sum_with_partner(lrun);
  const float inv = 1.f / lt;
#pragma unroll
  for (int dt = 0; dt < DT; ++dt)
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const int d = dt * 32 + 8 * g + 4 * hh;
      u32x2 w = {pack2<E>(oacc[dt][4 * g] * inv, oacc[dt][4 * g + 1] * inv),
                 pack2<E>(oacc[dt][4 * g + 2] * inv, oacc[dt][4 * g + 3] * inv)};
      *reinterpret_cast<u32x2*>(obase + (int64_t)row * p.so[2] + d) = w;
    }
  if (hh == 0) lbase[row] = (mrun + __builtin_amdgcn_logf(lt)) * kLn2;
}

// ===========================================================================
// Backward, dQ
// ===========================================================================
// One 64-key K/V tile against the wave's 64 query rows: S^T and dP^T
// recomputed (lane = query), P = 2^(S c2 - lse2), dS = P (dP - delta),
// dQ += dS K.  With MASK (the diagonal tile) keys above the query get P = 0.
// The two 32-key halves mt run one after the other and each K / V operand
// read from LDS (row reads for S^T / dP^T, transposed reads for dQ) feeds
// both 32-query halves nt of the wave.
// Per-wave LDS block of the dQ softmax offsets, each query's value stored 16
// times: [kind: 0 = -LSE log2(e), 1 = -delta][32-query half nt][group g][query
// l32][4 copies].  A lane's 16 accumulator slots all belong to its query, so
// four ds_read_b128 (one per group, 16 consecutive lanes reading 256
// consecutive bytes) give the MFMA accumulator its starting value without VALU
// work; the score MFMA then yields S c2 - LSE2 (Q pre-scaled by c2) and the dP
// MFMA yields dP - delta.
constexpr int kDqOffsFloats = 2 * 2 * 4 * 32 * 4;  // per wave (8 KB)

__device__ __forceinline__ f32x16 dq_offset_tile(const float* offs, int kind, int nt, int l32) {
  const float* b = offs + (kind * 2 + nt) * 512 + l32 * 4;
  f32x16 r;
#pragma unroll
  for (int g = 0; g < 4; ++g) {
    const f32x4 v = *reinterpret_cast<const f32x4*>(b + g * 128);
#pragma unroll
    for (int c = 0; c < 4; ++c) r[4 * g + c] = v[c];
  }
  return r;
}

// With MASK, qoff = (the wave's row block - the tile) * 64 >= 0: keys above
// the query are masked (only on the wave's diagonal tile, qoff = 0, does
// anything get masked; a masked tile left of it computes as an unmasked one).
template <class E, int D, bool MASK>
__device__ __forceinline__ void dq_tile(const char* K, const char* Vr, const typename E::v8 (*qop)[D / 16],
                                        const typename E::v8 (*gop)[D / 16], f32x16 (*dqacc)[2], const float* offs,
                                        int rbase, TrBase tbase, int l32, int hh, int qoff = 0) {
  using V8 = typename E::v8;
  using TL = Tile<D>;
  constexpr int KT = D / 16;
  constexpr int DT = D / 32;
#pragma unroll
  for (int mt = 0; mt < 2; ++mt) {
    f32x16 st[2], dpt[2];  // [nt]
    {
      const V8 a = TL::template row_op<E>(K, rbase, mt * 32, 0);
      const V8 b = TL::template row_op<E>(Vr, rbase, mt * 32, 0);
#pragma unroll
      for (int nt = 0; nt < 2; ++nt) {
        // accumulators start at -LSE log2(e) and -delta of the lane's query
        st[nt] = E::mfma(a, qop[nt][0], dq_offset_tile(offs, 0, nt, l32));
        dpt[nt] = E::mfma(b, gop[nt][0], dq_offset_tile(offs, 1, nt, l32));
      }
    }
#pragma unroll
    for (int kk = 1; kk < KT; ++kk) {
      const V8 a = TL::template row_op<E>(K, rbase, mt * 32, kk);
      const V8 b = TL::template row_op<E>(Vr, rbase, mt * 32, kk);
#pragma unroll
      for (int nt = 0; nt < 2; ++nt) {
        st[nt] = E::mfma(a, qop[nt][kk], st[nt]);
        dpt[nt] = E::mfma(b, gop[nt][kk], dpt[nt]);
      }
    }
    V8 dsb[2][2];  // [nt][k2]
#pragma unroll
    for (int nt = 0; nt < 2; ++nt) {
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        float pv = exp2_fast(st[nt][i]);
        if constexpr (MASK) {
          const int kr = mt * 32 + 8 * (i >> 2) + 4 * hh + (i & 3);
          if (kr > qoff + nt * 32 + l32) pv = 0.f;
        }
        st[nt][i] = pv * dpt[nt][i];
      }
      dsb[nt][0] = pack8<E>(st[nt], 0);
      dsb[nt][1] = pack8<E>(st[nt], 8);
    }
#pragma unroll
    for (int k2 = 0; k2 < 2; ++k2) {
#pragma unroll
      for (int dt = 0; dt < DT; ++dt) {
        const V8 a = TL::template tr_op<E>(K, tbase, 2 * mt + k2, dt);
#pragma unroll
        for (int nt = 0; nt < 2; ++nt) dqacc[dt][nt] = E::mfma(a, dsb[nt][k2], dqacc[dt][nt]);
      }
    }
    // keep the two halves' live ranges apart
    __builtin_amdgcn_sched_barrier(0);
  }
}

// LDS of one dQ workgroup (D <= 64): double-buffered K / V tiles, then the
// 4 waves' offset blocks.
template <int D>
struct DqLds {
  static constexpr int TILES = 2 * 2 * Tile<D>::BYTES;          // [buf][K, V]
  static constexpr int BYTES = TILES + 4 * kDqOffsFloats * 4;
};

// One dQ workgroup (task L of the dQ grid).  PEEL: the workgroup's 4 waves
// are 4 heads of one row block, so every active wave's diagonal tile is the
// workgroup's last tile and is handled after the loop; keeping the masked
// tile out of the loop keeps the loop within the register budget.  The rows'
// -delta and -LSE log2(e) come from attn_bwd_prep_kernel.
template <class E, int D, bool ROPE, bool PEEL>
__device__ __forceinline__ void dq_body(const AttnParams& p, int L, char* lds) {
  static_assert(D <= 64, "D = 128 uses attn_bwd_dq_w8_kernel");
  using V8 = typename E::v8;
  using TL = Tile<D>;
  constexpr int KT = D / 16;
  constexpr int DT = D / 32;
  char (*smem)[2][TL::BYTES] = reinterpret_cast<char (*)[2][TL::BYTES]>(lds);  // [buf][K, V]
  float (*offs_all)[kDqOffsFloats] = reinterpret_cast<float (*)[kDqOffsFloats]>(lds + DqLds<D>::TILES);

  const RowTask task = row_task(p, L);
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
  float* offs = offs_all[wave];

  const uint16_t* kbase = p.k + task.b * p.sk[0] + (int64_t)task.kvh * p.sk[1];
  const uint16_t* vbase = p.v + task.b * p.sv[0] + (int64_t)task.kvh * p.sv[1];
  const int64_t rowbase = ((int64_t)task.b * p.Hq + head) * p.T;

  V8 qop[2][KT], gop[2][KT];
  {
    const uint16_t* qbase = p.q + task.b * p.sq[0] + (int64_t)head * p.sq[1];
    const uint16_t* gbase = p.dout + task.b * p.sdo[0] + (int64_t)head * p.sdo[1];
    // all loads first (one memory round trip; rows past T load row T-1 and
    // are zeroed), then the operands and the offset block
    u32x4 qx[2][KT], gx[2][KT];
    float nlx[2], ndx[2];
#pragma unroll
    for (int nt = 0; nt < 2; ++nt) {
      const int rc = min(q0 + nt * 32 + l32, p.T - 1);
#pragma unroll
      for (int kk = 0; kk < KT; ++kk) {
        const int d0 = 16 * kk + 8 * hh;
        qx[nt][kk] = *reinterpret_cast<const u32x4*>(qbase + (int64_t)rc * p.sq[2] + d0);
        gx[nt][kk] = *reinterpret_cast<const u32x4*>(gbase + (int64_t)rc * p.sdo[2] + d0);
      }
      nlx[nt] = p.nlse2[rowbase + rc];
      ndx[nt] = p.ndelta[rowbase + rc];
    }
    const float c2 = p.scale_log2;
#pragma unroll
    for (int nt = 0; nt < 2; ++nt) {
      const int row = q0 + nt * 32 + l32;
      const bool ok = active && row < p.T;
#pragma unroll
      for (int kk = 0; kk < KT; ++kk) {
        // Q pre-multiplied by scale * log2(e) (rounded to the storage type once,
        // as the dK/dV pass does with K), so the score MFMA yields S c2 directly
        u32x4 qs = ok ? qx[nt][kk] : zero4();
#pragma unroll
        for (int w = 0; w < 4; ++w) qs[w] = pack2<E>(lo_f<E>(qs[w]) * c2, hi_f<E>(qs[w]) * c2);
        qop[nt][kk] = __builtin_bit_cast(V8, qs);
        gop[nt][kk] = __builtin_bit_cast(V8, ok ? gx[nt][kk] : zero4());
      }
      const float nlse2 = ok ? nlx[nt] : 0.f;
      const float ndelta = ok ? ndx[nt] : 0.f;
      // this wave's offset block: lanes hh = 0 / 1 fill groups 0-1 / 2-3
      const f32x4 nl = {nlse2, nlse2, nlse2, nlse2}, nd = {ndelta, ndelta, ndelta, ndelta};
#pragma unroll
      for (int g = 2 * hh; g < 2 * hh + 2; ++g) {
        *reinterpret_cast<f32x4*>(offs + (0 * 2 + nt) * 512 + g * 128 + l32 * 4) = nl;
        *reinterpret_cast<f32x4*>(offs + (1 * 2 + nt) * 512 + g * 128 + l32 * 4) = nd;
      }
    }
  }

  f32x16 dqacc[DT][2];
#pragma unroll
  for (int dt = 0; dt < DT; ++dt)
#pragma unroll
    for (int nt = 0; nt < 2; ++nt) zero16(dqacc[dt][nt]);

  Stager<D, 4> ks_stage, vs_stage;
  ks_stage.init(p.sk[2], wave, lane);
  vs_stage.init(p.sv[2], wave, lane);
  const int rbase_op = TL::row_base(lane);
  const TrBase tbase_op = TL::tr_base(lane);

  ks_stage.stage(smem[0][0], kbase, p.sk[2], 0, p.T);
  vs_stage.stage(smem[0][1], vbase, p.sv[2], 0, p.T);
  wait_vmem();
  __syncthreads();

  // Tiles before the workgroup's first row block are below every wave's
  // diagonal (unmasked loop); the rb tiles from there on hold the waves'
  // diagonals and run the masked variant (with PEEL that is the last tile).
  const int jdiag = task.sb * p.rb;
  for (int j = 0; j < jdiag; ++j) {
    const int buf = j & 1;
    ks_stage.stage(smem[buf ^ 1][0], kbase, p.sk[2], (j + 1) * kBlk, p.T);
    vs_stage.stage(smem[buf ^ 1][1], vbase, p.sv[2], (j + 1) * kBlk, p.T);
    if (active)
      dq_tile<E, D, false>(smem[buf][0], smem[buf][1], qop, gop, dqacc, offs, rbase_op, tbase_op, l32, hh);
    wait_vmem();
    __syncthreads();
  }
  if constexpr (PEEL) {
    if (active)  // qb == jdiag == jlast
      dq_tile<E, D, true>(smem[jlast & 1][0], smem[jlast & 1][1], qop, gop, dqacc, offs, rbase_op, tbase_op, l32,
                          hh);
  } else {
    for (int j = jdiag; j <= jlast; ++j) {
      const int buf = j & 1;
      if (j < jlast) {
        ks_stage.stage(smem[buf ^ 1][0], kbase, p.sk[2], (j + 1) * kBlk, p.T);
        vs_stage.stage(smem[buf ^ 1][1], vbase, p.sv[2], (j + 1) * kBlk, p.T);
      }
      if (active && j <= qb)
        dq_tile<E, D, true>(smem[buf][0], smem[buf][1], qop, gop, dqacc, offs, rbase_op, tbase_op, l32, hh,
                            (qb - j) * kBlk);
      wait_vmem();
      __syncthreads();
    }
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
        if constexpr (ROPE)
          rope_back4(x0, x1, x2, x3, p.cos + (int64_t)row * (D / 2) + d / 2, p.sin + (int64_t)row * (D / 2) + d / 2);
        u32x2 w = {pack2<E>(x0, x1), pack2<E>(x2, x3)};
        *reinterpret_cast<u32x2*>(dqbase + (int64_t)row * p.sout[2] + d) = w;
      }
  }
}


// ===========================================================================
// Backward, dQ for D = 128: 8 waves of 32 query rows per workgroup
// ===========================================================================
// As for the D = 128 forward: the 4 (head, 64-row block) pairs of a RowTask
// split into two 32-row waves, two waves per SIMD and no spills.  At D = 128
// attn_bwd_dq_kernel re-reads the K / V operands for each 32-query half
// anyway, so the narrower wave costs no extra LDS reads per MFMA.  It runs
// before the dK/dV pass (separate launches) and writes the -delta and
// -LSE log2(e) vectors that pass reads.
template <class E, int D, bool MASK>
__device__ __forceinline__ void dq32_tile(const char* K, const char* Vr, const typename E::v8* qop,
                                          const typename E::v8* gop, f32x16* dqacc, float lse2, float dlt, int rbase,
                                          TrBase tbase, int l32, int hh, int qoff, float c2) {
  using V8 = typename E::v8;
  using TL = Tile<D>;
  constexpr int KT = D / 16;
  constexpr int DT = D / 32;
#pragma unroll
  for (int mt = 0; mt < 2; ++mt) {
    // on the diagonal tile, key halves wholly above the wave's rows add nothing
    if (MASK && mt * 32 > qoff + 31) continue;
    f32x16 st, dpt;
    {
      const V8 a = TL::template row_op<E>(K, rbase, mt * 32, 0);
      const V8 b = TL::template row_op<E>(Vr, rbase, mt * 32, 0);
      st = E::mfma(a, qop[0], f32x16{});
      dpt = E::mfma(b, gop[0], f32x16{});
    }
#pragma unroll
    for (int kk = 1; kk < KT; ++kk) {
      const V8 a = TL::template row_op<E>(K, rbase, mt * 32, kk);
      const V8 b = TL::template row_op<E>(Vr, rbase, mt * 32, kk);
      st = E::mfma(a, qop[kk], st);
      dpt = E::mfma(b, gop[kk], dpt);
    }
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      float pv = exp2_fast(__builtin_fmaf(st[i], c2, -lse2));
      if constexpr (MASK) {
        const int kr = mt * 32 + 8 * (i >> 2) + 4 * hh + (i & 3);
        if (kr > qoff + l32) pv = 0.f;
      }
      st[i] = pv * (dpt[i] - dlt);
    }
    V8 dsb[2];
    dsb[0] = pack8<E>(st, 0);
    dsb[1] = pack8<E>(st, 8);
#pragma unroll
    for (int k2 = 0; k2 < 2; ++k2)
#pragma unroll
      for (int dt = 0; dt < DT; ++dt)
        dqacc[dt] = E::mfma(TL::template tr_op<E>(K, tbase, 2 * mt + k2, dt), dsb[k2], dqacc[dt]);
    __builtin_amdgcn_sched_barrier(0);
  }
}

// NW waves per workgroup: the RowTask's NW / 2 (head, row block) pairs
// (the launch sets r_sub and rb for that many pairs).
template <class E, int D, bool ROPE, bool PEEL, int NW>
__global__ __launch_bounds__(64 * NW, 2) void attn_bwd_dq_w8_kernel(AttnParams p) {
  using V8 = typename E::v8;
  using TL = Tile<D>;
  constexpr int KT = D / 16;
  constexpr int DT = D / 32;
  constexpr int SW = TL::INSTR < NW ? TL::INSTR : NW;  // waves that stage tiles
  __shared__ __attribute__((aligned(1024))) char smem[2][2][TL::BYTES];  // [buf][K, V]

  const RowTask task = row_task(p, blockIdx.x);
  const int tid = threadIdx.x;
  const int wave = tid >> 6;
  const int lane = tid & 63;
  const int l32 = lane & 31;
  const int hh = lane >> 5;
  const int pw = wave >> 1;
  const int head = task.kvh * p.R + task.hs * p.r_sub + (pw % p.r_sub);
  const int qb = task.sb * p.rb + pw / p.r_sub;
  const int qoff = 32 * (wave & 1);                 // the wave's rows within its 64-row block
  const int q0 = qb * kBlk + qoff;
  const bool active = qb < p.nqb && q0 < p.T;
  const int jlast = min(p.nqb - 1, task.sb * p.rb + p.rb - 1);

  const uint16_t* kbase = p.k + task.b * p.sk[0] + (int64_t)task.kvh * p.sk[1];
  const uint16_t* vbase = p.v + task.b * p.sv[0] + (int64_t)task.kvh * p.sv[1];
  const int64_t rowbase = ((int64_t)task.b * p.Hq + head) * p.T;

  V8 qop[KT], gop[KT];
  float lse2, dlt;  // LSE log2(e) and delta of the lane's row
  {
    // This kernel is the D = 128 backward's first pass, so it computes the
    // row's delta = rowsum(O * dO) in fp32 itself (the lane and its lane^32
    // partner hold the two halves of the row) and stores -delta and
    // -LSE log2(e) for the dK/dV pass; no separate prep pass.
    const uint16_t* qbase = p.q + task.b * p.sq[0] + (int64_t)head * p.sq[1];
    const uint16_t* gbase = p.dout + task.b * p.sdo[0] + (int64_t)head * p.sdo[1];
    const uint16_t* obase = p.o + task.b * p.so[0] + (int64_t)head * p.so[1];
    const int row = q0 + l32;
    const int rc = min(row, p.T - 1);
    const bool ok = active && row < p.T;
    u32x4 qx[KT], gx[KT], ox[KT];
#pragma unroll
    for (int kk = 0; kk < KT; ++kk) {
      const int d0 = 16 * kk + 8 * hh;
      qx[kk] = *reinterpret_cast<const u32x4*>(qbase + (int64_t)rc * p.sq[2] + d0);
      gx[kk] = *reinterpret_cast<const u32x4*>(gbase + (int64_t)rc * p.sdo[2] + d0);
      ox[kk] = *reinterpret_cast<const u32x4*>(obase + (int64_t)rc * p.so[2] + d0);
    }
    const float lse = p.lse[rowbase + rc];
    float part = 0.f;
#pragma unroll
    for (int kk = 0; kk < KT; ++kk)
#pragma unroll
      for (int w = 0; w < 4; ++w)
        part += lo_f<E>(gx[kk][w]) * lo_f<E>(ox[kk][w]) + hi_f<E>(gx[kk][w]) * hi_f<E>(ox[kk][w]);
    const float delta = sum_with_partner(part);
#pragma unroll
    for (int kk = 0; kk < KT; ++kk) {
      qop[kk] = __builtin_bit_cast(V8, ok ? qx[kk] : zero4());
      gop[kk] = __builtin_bit_cast(V8, ok ? gx[kk] : zero4());
    }
    dlt = ok ? delta : 0.f;
    lse2 = ok ? lse * kLog2e : 0.f;
    if (ok && hh == 0) {
      p.ndelta[rowbase + row] = -delta;
      p.nlse2[rowbase + row] = -lse * kLog2e;
    }
  }

  f32x16 dqacc[DT];
#pragma unroll
  for (int dt = 0; dt < DT; ++dt) zero16(dqacc[dt]);

  Stager<D, SW> ks_stage, vs_stage;
  const bool stager = wave < SW;
  ks_stage.init(p.sk[2], wave, lane);
  vs_stage.init(p.sv[2], wave, lane);
  const int rbase_op = TL::row_base(lane);
  const TrBase tbase_op = TL::tr_base(lane);

  if (stager) {
    ks_stage.stage(smem[0][0], kbase, p.sk[2], 0, p.T);
    vs_stage.stage(smem[0][1], vbase, p.sv[2], 0, p.T);
  }
  wait_vmem();
  __syncthreads();

  const float c2 = p.scale_log2;
  // unmasked tiles below every wave's diagonal, then the rb diagonal-zone
  // tiles with the masked variant (row offset from the tile: a tile left of
  // the wave's diagonal masks nothing)
  const int jdiag = task.sb * p.rb;
  for (int j = 0; j < jdiag; ++j) {
    const int buf = j & 1;
    if (stager) {
      ks_stage.stage(smem[buf ^ 1][0], kbase, p.sk[2], (j + 1) * kBlk, p.T);
      vs_stage.stage(smem[buf ^ 1][1], vbase, p.sv[2], (j + 1) * kBlk, p.T);
    }
    if (active)
      dq32_tile<E, D, false>(smem[buf][0], smem[buf][1], qop, gop, dqacc, lse2, dlt, rbase_op, tbase_op, l32, hh,
                             qoff, c2);
    wait_vmem();
    __syncthreads();
  }
  for (int j = jdiag; j <= jlast; ++j) {
    const int buf = j & 1;
    if (j < jlast && stager) {
      ks_stage.stage(smem[buf ^ 1][0], kbase, p.sk[2], (j + 1) * kBlk, p.T);
      vs_stage.stage(smem[buf ^ 1][1], vbase, p.sv[2], (j + 1) * kBlk, p.T);
    }
    if (active && j <= qb)
      dq32_tile<E, D, true>(smem[buf][0], smem[buf][1], qop, gop, dqacc, lse2, dlt, rbase_op, tbase_op, l32, hh,
                            qoff + (qb - j) * kBlk, c2);
    wait_vmem();
    __syncthreads();
  }

  if (!active) return;
  const int row = q0 + l32;
  if (row >= p.T) return;
  uint16_t* dqbase = p.out + task.b * p.sout[0] + (int64_t)head * p.sout[1];
#pragma unroll
  for (int dt = 0; dt < DT; ++dt)
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const int d = dt * 32 + 8 * g + 4 * hh;
      float x0 = dqacc[dt][4 * g] * p.scale, x1 = dqacc[dt][4 * g + 1] * p.scale;
      float x2 = dqacc[dt][4 * g + 2] * p.scale, x3 = dqacc[dt][4 * g + 3] * p.scale;
      if constexpr (ROPE)
        rope_back4(x0, x1, x2, x3, p.cos + (int64_t)row * (D / 2) + d / 2, p.sin + (int64_t)row * (D / 2) + d / 2);
      u32x2 w = {pack2<E>(x0, x1), pack2<E>(x2, x3)};
      *reinterpret_cast<u32x2*>(dqbase + (int64_t)row * p.sout[2] + d) = w;
    }
}

// dK/dV softmax step for one 32-row quarter (C layout: lane = key, slots =
// rows).  The score MFMAs start from the accumulator tiles -lse2[row] and
// -delta[row] (see dkv_step) with K pre-scaled by scale*log2(e), so on entry
// s = S*c - lse2 and dp = dP - delta; this computes P = 2^s, dS = P * dp and
// packs both into the two 16-row B operands.  With MASK, entries whose key
// exceeds the row or whose row is at or past T are zeroed (qrow = the
// quarter's first global row).
template <class E, bool MASK>
__device__ __forceinline__ void softmax_dS32(f32x16& s, f32x16& dp, int key, int qrow, int T, int hh,
                                             typename E::v8 pk[2], typename E::v8 dk[2]) {
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    float pv = exp2_fast(s[i]);
    if constexpr (MASK) {
      const int qg = qrow + 8 * (i >> 2) + 4 * hh + (i & 3);
      if (key > qg || qg >= T) pv = 0.f;
    }
    s[i] = pv;
    dp[i] = pv * dp[i];
  }
  pk[0] = pack8<E>(s, 0);
  pk[1] = pack8<E>(s, 8);
  dk[0] = pack8<E>(dp, 0);
  dk[1] = pack8<E>(dp, 8);
}

// The 16 accumulator slots of a 32-row quarter (slot i = row 8(i/4) + 4(lane/32)
// + i%4) filled from a row-indexed fp32 vector in LDS; `rows` already points at
// the quarter's first row plus 4 * (lane / 32).
__device__ __forceinline__ f32x16 row_tile(const float* rows) {
  f32x16 t;
#pragma unroll
  for (int g4 = 0; g4 < 4; ++g4) {
    const f32x4 v = *reinterpret_cast<const f32x4*>(rows + 8 * g4);
#pragma unroll
    for (int e = 0; e < 4; ++e) t[4 * g4 + e] = v[e];
  }
  return t;
}

// ===========================================================================
// Backward, dK / dV
// ===========================================================================
#ifndef MT_DKV_GROUPS
#define MT_DKV_GROUPS 0
#endif
// explicit MFMA / VALU / LDS-read interleaving of the dK/dV step (0: scheduler's choice)
#define MT_DKV_GROUP(mask, n) \
  do {                       \
    if constexpr (MT_DKV_GROUPS) __builtin_amdgcn_sched_group_barrier(mask, n, 0); \
  } while (0)
constexpr int kKvWaves = 4;    // waves per dK/dV workgroup
constexpr int kKvKpw = 32;     // keys per wave
constexpr int kKvKeys = kKvWaves * kKvKpw;
constexpr int kKvRows = 128;   // query rows staged per step (two row blocks)

// One step of a wave: rows [qrow0, qrow0 + 32 NQ) of one head against the
// wave's 32 keys (NQ = 4: both staged 64-row tiles; NQ = 2: the one tile Q,
// G point at).  Quarter h covers rows qrow0 + 32h.  MFMA / VALU pipeline
// (issue order, phases fenced by sched_barrier, MFMAs interleaved with the
// VALU work of the same phase), for NQ = 4:
//   SdP0 | SdP1 + V0 | dVdK0 + SdP2 + V1 | dVdK1 + SdP3 + V2 | dVdK2 + V3 | dVdK3
// and for NQ = 2:  SdP0 | SdP1 + V0 | dVdK0 + V1 | dVdK1
// where SdPh = S and dP of quarter h, Vh = its softmax / dS, dVdKh = its
// dV and dK updates.  Quarters with every key above every row, or every row
// at or past T, are skipped (LIVE masks only matter where MASK is set).
template <class E, int D, bool MASK, int NQ = 4>
__device__ __forceinline__ void dkv_step(const char* Q, const char* G, const float* lrow, const float* drow,
                                         const typename E::v8* kop, const typename E::v8* vop,
                                         f32x16* dkacc, f32x16* dvacc, int rbase, TrBase tbase, int lane,
                                         int key, int k0, int qrow0, int T) {
  static_assert(NQ == 2 || NQ == 4, "one or two 64-row tiles per step");
  using V8 = typename E::v8;
  using TL = Tile<D>;
  constexpr int KT = D / 16;
  constexpr int DT = D / 32;
  const int hh = lane >> 5;
  // quarter live: some key of the wave is <= the quarter's last row, and the
  // quarter's first row is below T
  bool live[NQ];
#pragma unroll
  for (int h = 0; h < NQ; ++h) live[h] = !MASK || (k0 <= qrow0 + 32 * h + 31 && qrow0 + 32 * h < T);

  auto sdp = [&](int h, f32x16& s, f32x16& dp) {
    const char* Qh = Q + (h >> 1) * TL::BYTES;
    const char* Gh = G + (h >> 1) * TL::BYTES;
    const int r0 = 32 * (h & 1);
    V8 aq = TL::template row_op<E>(Qh, rbase, r0, 0);
    V8 ag = TL::template row_op<E>(Gh, rbase, r0, 0);
    // accumulators start at -lse2 / -delta of the quarter's rows
    s = E::mfma(aq, kop[0], row_tile(lrow + 32 * h + 4 * hh));
    dp = E::mfma(ag, vop[0], row_tile(drow + 32 * h + 4 * hh));
#pragma unroll
    for (int kk = 1; kk < KT; ++kk) {
      aq = TL::template row_op<E>(Qh, rbase, r0, kk);
      ag = TL::template row_op<E>(Gh, rbase, r0, kk);
      s = E::mfma(aq, kop[kk], s);
      dp = E::mfma(ag, vop[kk], dp);
    }
  };
  auto vh = [&](int h, f32x16& s, f32x16& dp, V8* pk, V8* dk) {
    softmax_dS32<E, MASK>(s, dp, key, qrow0 + 32 * h, T, hh, pk, dk);
  };
  auto dvdk = [&](int h, const V8* pk, const V8* dk) {
    const char* Qh = Q + (h >> 1) * TL::BYTES;
    const char* Gh = G + (h >> 1) * TL::BYTES;
    const int ks0 = 2 * (h & 1);
#pragma unroll
    for (int k2 = 0; k2 < 2; ++k2)
#pragma unroll
      for (int dt = 0; dt < DT; ++dt) {
        dvacc[dt] = E::mfma(TL::template tr_op<E>(Gh, tbase, ks0 + k2, dt), pk[k2], dvacc[dt]);
        dkacc[dt] = E::mfma(TL::template tr_op<E>(Qh, tbase, ks0 + k2, dt), dk[k2], dkacc[dt]);
      }
  };
  constexpr int NS = 2 * KT;   // S/dP MFMAs of a quarter
  constexpr int NT = 4 * DT;   // dV/dK MFMAs of a quarter

  f32x16 s[2], dp[2];          // ring of two quarters' S / dP
  V8 pk[2][2], dk[2][2];       // ring of two quarters' packed P / dS
  // phase 1: SdP0
  if (live[0]) sdp(0, s[0], dp[0]);
#pragma unroll
  for (int i = 0; i < KT; ++i) {
    MT_DKV_GROUP(0x100, 2);
    MT_DKV_GROUP(0x008, 2);
  }
  __builtin_amdgcn_sched_barrier(0);
  // phase 2: SdP1 + V0
  if (live[1]) sdp(1, s[1], dp[1]);
  if (live[0]) vh(0, s[0], dp[0], pk[0], dk[0]);
#pragma unroll
  for (int i = 0; i < KT; ++i) {
    MT_DKV_GROUP(0x100, 2);
    MT_DKV_GROUP(0x008, 2);
    MT_DKV_GROUP(0x002, 16);
  }
  __builtin_amdgcn_sched_barrier(0);
  // phases 3 .. NQ: dVdK(h-2) + SdP(h) + V(h-1), h = 2 .. NQ-1
#pragma unroll
  for (int h = 2; h < NQ; ++h) {
    if (live[h - 2]) dvdk(h - 2, pk[h & 1], dk[h & 1]);
    if (live[h]) sdp(h, s[h & 1], dp[h & 1]);
    if (live[h - 1]) vh(h - 1, s[(h - 1) & 1], dp[(h - 1) & 1], pk[(h - 1) & 1], dk[(h - 1) & 1]);
#pragma unroll
    for (int i = 0; i < NT; ++i) {
      MT_DKV_GROUP(0x100, 2);
      MT_DKV_GROUP(0x008, 1);
      MT_DKV_GROUP(0x002, 6);
    }
#pragma unroll
    for (int i = 0; i < KT; ++i) {
      MT_DKV_GROUP(0x100, 2);
      MT_DKV_GROUP(0x008, 2);
      MT_DKV_GROUP(0x002, 6);
    }
    __builtin_amdgcn_sched_barrier(0);
  }
  // dVdK(NQ-2) + V(NQ-1)
  if (live[NQ - 2]) dvdk(NQ - 2, pk[0], dk[0]);
  if (live[NQ - 1]) vh(NQ - 1, s[1], dp[1], pk[1], dk[1]);
#pragma unroll
  for (int i = 0; i < NT; ++i) {
    MT_DKV_GROUP(0x100, 2);
    MT_DKV_GROUP(0x008, 1);
    MT_DKV_GROUP(0x002, 10);
  }
  __builtin_amdgcn_sched_barrier(0);
  // dVdK(NQ-1)
  if (live[NQ - 1]) dvdk(NQ - 1, pk[1], dk[1]);
#pragma unroll
  for (int i = 0; i < NT; ++i) {
    MT_DKV_GROUP(0x100, 2);
    MT_DKV_GROUP(0x008, 1);
  }
  (void)NS;
}

// LDS of one dK/dV workgroup: [buf][Q, dO] x 128 rows (two 64-row tiles back
// to back), then [buf][-lse * log2(e), -delta] of those rows.
template <int D>
struct DkvLds {
  static constexpr int TILES = 2 * 2 * 2 * Tile<D>::BYTES;
  static constexpr int BYTES = TILES + 2 * 2 * kKvRows * 4;
};

// One dK/dV workgroup (task L of the dK/dV grid), KVK keys.
//  * KVK = 128: wave w owns keys 32w .. 32w+31 of the block and runs every
//    staged 128-row step on them.
//  * KVK = 64: waves w and w+2 own keys 32(w & 1) .. +31; of each staged
//    128-row step wave w takes the first 64 rows and wave w+2 the second,
//    and the pair adds its dK / dV through LDS at the end.  A task then
//    carries half the work, so the heaviest (first) key blocks, which bound
//    the launch when the grid is one or two resident rounds, finish twice as
//    soon.
// DESC: the steps run from the last row block down to the diagonal, the
// task's heads innermost, so the dK/dV tasks of a group that are resident
// together read the same Q / dO rows at about the same time (in the
// one-launch backward this cuts its L2 fetches by a fifth at equal time);
// otherwise each head's row blocks run upwards from the diagonal.
template <class E, int D, bool ROPE, int KVK = kKvKeys, bool DESC = false>
__device__ __forceinline__ void dkv_body(const AttnParams& p, int L, char* lds) {
  static_assert(KVK == 128 || KVK == 64, "128 or 64 keys per task");
  constexpr int NQ = KVK == 128 ? 4 : 2;      // 32-row quarters per wave and step
  using V8 = typename E::v8;
  using TL = Tile<D>;
  constexpr int KT = D / 16;
  constexpr int DT = D / 32;
  char (*smem)[2][2 * TL::BYTES] = reinterpret_cast<char (*)[2][2 * TL::BYTES]>(lds);
  float (*vec)[2][kKvRows] = reinterpret_cast<float (*)[2][kKvRows]>(lds + DkvLds<D>::TILES);

  // heaviest key blocks (smallest index: most causal rows) first
  const int groups = p.B * p.Hkv * p.n_split;
  const int kb = L / groups;
  const int g = L % groups;
  const int hs = g % p.n_split;
  const int bk = g / p.n_split;
  const int kvh = bk % p.Hkv;
  const int b = bk / p.Hkv;

  const int tid = threadIdx.x;
  const int wave = tid >> 6;
  const int lane = tid & 63;
  const int l32 = lane & 31;
  const int hh = lane >> 5;
  const int kcol = KVK == 128 ? wave : (wave & 1);  // key column of the wave
  const int rsel = KVK == 128 ? 0 : (wave >> 1);    // its 64-row half of a step (KVK = 64)
  const int k0 = kb * KVK + kcol * kKvKpw;         // this wave's first key
  const int key = k0 + l32;                        // this lane's key (C column)
  const bool wave_live = k0 < p.T;

  // K and V rows as B operands (N = key, k = d).  K is pre-multiplied by
  // scale * log2(e) (rounded to the storage type once), so the score MFMA
  // yields S * c directly and the softmax needs no per-score multiply.
  V8 kop[KT], vop[KT];
  {
    const uint16_t* kbase = p.k + b * p.sk[0] + (int64_t)kvh * p.sk[1];
    const uint16_t* vbase = p.v + b * p.sv[0] + (int64_t)kvh * p.sv[1];
    u32x4 kx[KT];
#pragma unroll
    for (int kk = 0; kk < KT; ++kk) {
      const int d0 = 16 * kk + 8 * hh;
      kx[kk] = load_chunk(kbase, p.sk[2], key, p.T, d0);
      vop[kk] = __builtin_bit_cast(V8, load_chunk(vbase, p.sv[2], key, p.T, d0));
    }
    const float c2 = p.scale_log2;
#pragma unroll
    for (int kk = 0; kk < KT; ++kk) {
#pragma unroll
      for (int w = 0; w < 4; ++w) kx[kk][w] = pack2<E>(lo_f<E>(kx[kk][w]) * c2, hi_f<E>(kx[kk][w]) * c2);
      kop[kk] = __builtin_bit_cast(V8, kx[kk]);
    }
  }

  f32x16 dkacc[DT], dvacc[DT];
#pragma unroll
  for (int dt = 0; dt < DT; ++dt) { zero16(dkacc[dt]); zero16(dvacc[dt]); }

  // this task's heads: [R hs / n_split, R (hs + 1) / n_split) of the group
  // (uneven when n_split does not divide R)
  const int h_lo = (p.R * hs) / p.n_split;
  const int hpt = (p.R * (hs + 1)) / p.n_split - h_lo;  // heads per task
  const int qr0 = kb * KVK;                        // first row touching these keys
  const int nstep_h = (p.T - qr0 + kKvRows - 1) / kKvRows;  // 128-row steps per head
  const int n_it = hpt * nstep_h;

  Stager<D, kKvWaves> qs_stage, gs_stage;
  qs_stage.init(p.sq[2], wave, lane);
  gs_stage.init(p.sdo[2], wave, lane);
  const int rbase_op = TL::row_base(lane);
  const TrBase tbase_op = TL::tr_base(lane);

  // (head, first row) of a step, advanced without divisions
  auto stage = [&](int head, int row0, int buf) {
    const uint16_t* qh = p.q + b * p.sq[0] + (int64_t)head * p.sq[1];
    const uint16_t* gh = p.dout + b * p.sdo[0] + (int64_t)head * p.sdo[1];
    // both halves always (rows past T are clamped to row T-1, so the LDS
    // never holds stale or uninitialised values that could reach a product)
    qs_stage.stage(smem[buf][0], qh, p.sq[2], row0, p.T);
    gs_stage.stage(smem[buf][1], gh, p.sdo[2], row0, p.T);
    qs_stage.stage(smem[buf][0] + TL::BYTES, qh, p.sq[2], row0 + kBlk, p.T);
    gs_stage.stage(smem[buf][1] + TL::BYTES, gh, p.sdo[2], row0 + kBlk, p.T);
    const int64_t rb = ((int64_t)b * p.Hq + head) * p.T;
    const float* src = (wave & 2) ? p.ndelta + rb : p.nlse2 + rb;
    stage_vec64(reinterpret_cast<char*>(&vec[buf][wave >> 1][(wave & 1) * kBlk]), src, row0 + (wave & 1) * kBlk, p.T, lane);
  };

  const int h0 = kvh * p.R + h_lo;
  int cur_row = qr0, nxt_head = h0, nxt_row = DESC ? qr0 + (nstep_h - 1) * kKvRows : qr0;
  stage(nxt_head, nxt_row, 0);
  wait_vmem();
  __syncthreads();
  for (int it = 0; it < n_it; ++it) {
    const int buf = it & 1;
    cur_row = nxt_row;
    if constexpr (DESC) {
      if (++nxt_head == h0 + hpt) {
        nxt_head = h0;
        nxt_row -= kKvRows;
      }
    } else {
      nxt_row += kKvRows;
      if (nxt_row >= p.T) {
        nxt_row = qr0;
        ++nxt_head;
      }
    }
    if (it + 1 < n_it) stage(nxt_head, nxt_row, buf ^ 1);
    if (wave_live) {
      // this wave's rows of the step: all 128, or its 64-row half
      const int row0 = cur_row + 64 * rsel;
      const char* Qw = smem[buf][0] + rsel * TL::BYTES;
      const char* Gw = smem[buf][1] + rsel * TL::BYTES;
      const float* lw = vec[buf][0] + 64 * rsel;
      const float* dw = vec[buf][1] + 64 * rsel;
      // no mask when every key of the wave precedes every row and all rows are below T
      const bool fast = (k0 + kKvKpw - 1 <= row0) && (row0 + 32 * NQ <= p.T);
      if (fast)
        dkv_step<E, D, false, NQ>(Qw, Gw, lw, dw, kop, vop, dkacc, dvacc, rbase_op, tbase_op, lane, key, k0, row0,
                                  p.T);
      else
        dkv_step<E, D, true, NQ>(Qw, Gw, lw, dw, kop, vop, dkacc, dvacc, rbase_op, tbase_op, lane, key, k0, row0,
                                 p.T);
    }
    wait_vmem();
    __syncthreads();
  }

  if constexpr (KVK == 64) {
    // waves 2, 3 hand their sums to waves 0, 1 (same keys) through the
    // staging LDS, free after the loop's last barrier: [kcol][slot][lane]
    // 16-byte chunks, conflict-free
    constexpr int NV = DT * 16 / 4;   // f32x4 chunks per accumulator set
    f32x4* red = reinterpret_cast<f32x4*>(lds);
    if (rsel == 1 && wave_live) {
#pragma unroll
      for (int dt = 0; dt < DT; ++dt)
#pragma unroll
        for (int g4 = 0; g4 < 4; ++g4) {
          red[((kcol * 2 * NV) + dt * 4 + g4) * 64 + lane] =
              f32x4{dkacc[dt][4 * g4], dkacc[dt][4 * g4 + 1], dkacc[dt][4 * g4 + 2], dkacc[dt][4 * g4 + 3]};
          red[((kcol * 2 * NV) + NV + dt * 4 + g4) * 64 + lane] =
              f32x4{dvacc[dt][4 * g4], dvacc[dt][4 * g4 + 1], dvacc[dt][4 * g4 + 2], dvacc[dt][4 * g4 + 3]};
        }
    }
    __syncthreads();
    if (rsel == 1) return;
    if (wave_live) {
#pragma unroll
      for (int dt = 0; dt < DT; ++dt)
#pragma unroll
        for (int g4 = 0; g4 < 4; ++g4) {
          const f32x4 a = red[((kcol * 2 * NV) + dt * 4 + g4) * 64 + lane];
          const f32x4 b = red[((kcol * 2 * NV) + NV + dt * 4 + g4) * 64 + lane];
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            dkacc[dt][4 * g4 + e] += a[e];
            dvacc[dt][4 * g4 + e] += b[e];
          }
        }
    }
  }
  if (!wave_live || key >= p.T) return;
  if (p.n_split == 1) {
    uint16_t* dkrow = p.dk + b * p.sdk[0] + (int64_t)kvh * p.sdk[1] + (int64_t)key * p.sdk[2];
    uint16_t* dvrow = p.dv + b * p.sdv[0] + (int64_t)kvh * p.sdv[1] + (int64_t)key * p.sdv[2];
#pragma unroll
    for (int dt = 0; dt < DT; ++dt)
#pragma unroll
      for (int g4 = 0; g4 < 4; ++g4) {
        const int d = dt * 32 + 8 * g4 + 4 * hh;
        float x0 = dkacc[dt][4 * g4] * p.scale, x1 = dkacc[dt][4 * g4 + 1] * p.scale;
        float x2 = dkacc[dt][4 * g4 + 2] * p.scale, x3 = dkacc[dt][4 * g4 + 3] * p.scale;
        if constexpr (ROPE)
          rope_back4(x0, x1, x2, x3, p.cos + (int64_t)key * (D / 2) + d / 2, p.sin + (int64_t)key * (D / 2) + d / 2);
        u32x2 wk = {pack2<E>(x0, x1), pack2<E>(x2, x3)};
        *reinterpret_cast<u32x2*>(dkrow + d) = wk;
        u32x2 wv = {pack2<E>(dvacc[dt][4 * g4], dvacc[dt][4 * g4 + 1]),
                    pack2<E>(dvacc[dt][4 * g4 + 2], dvacc[dt][4 * g4 + 3])};
        *reinterpret_cast<u32x2*>(dvrow + d) = wv;
      }
  } else {
    // fp32 partials: part[hs][0 = dK, 1 = dV][b][kvh][key][d]
    const int64_t plane = (int64_t)p.B * p.Hkv * p.T * D;
    float* pk = p.part + (int64_t)hs * 2 * plane + (((int64_t)b * p.Hkv + kvh) * p.T + key) * D;
    float* pv = pk + plane;
#pragma unroll
    for (int dt = 0; dt < DT; ++dt)
#pragma unroll
      for (int g4 = 0; g4 < 4; ++g4) {
        const int d = dt * 32 + 8 * g4 + 4 * hh;
        f32x4 xk = {dkacc[dt][4 * g4] * p.scale, dkacc[dt][4 * g4 + 1] * p.scale,
                    dkacc[dt][4 * g4 + 2] * p.scale, dkacc[dt][4 * g4 + 3] * p.scale};
        f32x4 xv = {dvacc[dt][4 * g4], dvacc[dt][4 * g4 + 1], dvacc[dt][4 * g4 + 2], dvacc[dt][4 * g4 + 3]};
        *reinterpret_cast<f32x4*>(pk + d) = xk;
        *reinterpret_cast<f32x4*>(pv + d) = xv;
      }
  }
}

template <class E, int D, bool ROPE>
__global__ __launch_bounds__(64 * kKvWaves, D <= 64 ? 2 : 1) void attn_bwd_dkv_kernel(AttnParams p) {
  __shared__ __attribute__((aligned(1024))) char lds[DkvLds<D>::BYTES];
  dkv_body<E, D, ROPE>(p, blockIdx.x, lds);
}

// ===========================================================================
// Backward, dQ and dK/dV work in one launch (D <= 64)
// ===========================================================================
// The n_kv dK/dV tasks and the n_dq dQ tasks are independent once the prep
// pass has written -delta and -LSE log2(e), so one grid holds both, in
// longest-first order over both kinds: both lists are sorted by work, and the
// host (bwd_merge) describes their merge as a head of the kind whose tasks are
// longer than every task of the other, a middle where the two interleave in
// proportion, and a tail of the kind whose tasks are shorter than every task
// of the other.  The last workgroups to start are then the shortest of either
// kind, which keeps the end of the launch short.
//
// Workgroups are dealt to the 8 XCDs round-robin by index, and both task
// lists give task i the (batch, KV head) group i mod (B Hkv) (times the
// head split), so with 8 | B Hkv a task's group decides its XCD.  The merge
// keeps that: it orders chunks of 8 consecutive workgroups, each chunk one
// kind, so task index and workgroup index agree mod 8 and the dQ and dK/dV
// tasks of a group share one XCD's L2 (its K/V and Q/dO rows).  When a count
// is not a multiple of 8 the merge is per workgroup.  KVK = keys per dK/dV
// task (dkv_body).
template <int D>
struct BwdLds {
  static constexpr int BYTES = DqLds<D>::BYTES > DkvLds<D>::BYTES ? DqLds<D>::BYTES : DkvLds<D>::BYTES;
};

template <class E, int D, bool ROPE, bool PEEL, int KVK>
__global__ __launch_bounds__(256, 2) void attn_bwd_kernel(AttnParams p) {
  static_assert(kKvWaves == 4, "dQ and dK/dV workgroups must have the same size");
  __shared__ __attribute__((aligned(1024))) char lds[BwdLds<D>::BYTES];
  const int L = blockIdx.x;
  const int sh = ((p.n_kv_tasks | p.n_dq_tasks) & 7) == 0 ? 3 : 0;  // chunks of 8 workgroups, or of 1
  const int n = (p.n_kv_tasks + p.n_dq_tasks) >> sh;
  // Within an XCD, consecutive workgroups go to its 4 shader engines in turn
  // and are dispatched in order, so an engine with no free slot holds back
  // the next workgroups of every engine.  Where the two kinds interleave 1:1,
  // chunk c's kind would repeat with c mod 4 and each engine would get one
  // kind only; rotating the chunks of each block of 4 (32 single workgroups)
  // by the block index gives every engine both kinds.  A permutation of
  // complete blocks: every task runs once.
  const int P = sh ? 4 : 32;
  const int u = L >> sh, m = u / P, t = u - m * P;
  const int c = (m + 1) * P <= n ? m * P + (t + m) % P : u;
  const int sub = L - (u << sh);
  const int nkv = p.n_kv_tasks >> sh;
  const int kv0 = p.mg_head_kv ? p.mg_head : 0;    // first dK/dV chunk of the middle
  const int dq0 = p.mg_head_kv ? 0 : p.mg_head;    // first dQ chunk of the middle
  const int mid = p.mg_mid_kv + p.mg_mid_dq;
  bool kv;
  int idx;
  if (c < p.mg_head) {
    kv = p.mg_head_kv;
    idx = c;
  } else if (c < p.mg_head + mid) {
    const int j = c - p.mg_head;
    const int before = (int)((int64_t)j * p.mg_mid_kv / mid);
    kv = (int)((int64_t)(j + 1) * p.mg_mid_kv / mid) > before;
    idx = kv ? kv0 + before : dq0 + (j - before);
  } else {
    const int j = c - p.mg_head - mid;
    kv = kv0 + p.mg_mid_kv < nkv;
    idx = kv ? kv0 + p.mg_mid_kv + j : dq0 + p.mg_mid_dq + j;
  }
  if (kv)
    dkv_body<E, D, ROPE, KVK, true>(p, (idx << sh) + sub, lds);
  else
    dq_body<E, D, ROPE, PEEL>(p, (idx << sh) + sub, lds);
}

// ===========================================================================
// Backward prep: -delta = -rowsum(O * dO) and -LSE log2(e) per query row
// ===========================================================================
// delta is computed in fp32 from the 16-bit O and dO (triton_attention.py:561);
// both vectors are stored negated because the dQ and dK/dV passes seed their
// score and dP accumulators with them.  D/8 lanes per row, each summing one
// 16-byte chunk, then a DPP butterfly over those lanes.  Every load (O, dO and
// the row's LSE, which all the row's lanes read) is issued up front: one
// memory round trip per row.
template <class E, int D>
__global__ __launch_bounds__(256) void attn_bwd_prep_kernel(AttnParams p) {
  constexpr int LPR = D / 8;  // lanes per row: 4, 8 or 16, aligned groups of a 16-lane DPP row
  static_assert(LPR == 4 || LPR == 8 || LPR == 16, "head size");
  const int64_t rows = (int64_t)p.B * p.Hq * p.T;
  const int64_t row = (int64_t)blockIdx.x * (256 / LPR) + threadIdx.x / LPR;
  const int c = threadIdx.x % LPR;
  float sum = 0.f, lse = 0.f;
  if (row < rows) {
    const int t = int(row % p.T);
    const int64_t bh = row / p.T;
    const int h = int(bh % p.Hq);
    const int64_t b = bh / p.Hq;
    const u32x4 o = *reinterpret_cast<const u32x4*>(p.o + b * p.so[0] + h * p.so[1] + (int64_t)t * p.so[2] + 8 * c);
    const u32x4 g =
        *reinterpret_cast<const u32x4*>(p.dout + b * p.sdo[0] + h * p.sdo[1] + (int64_t)t * p.sdo[2] + 8 * c);
    lse = p.lse[row];
#pragma unroll
    for (int w = 0; w < 4; ++w) sum += lo_f<E>(g[w]) * lo_f<E>(o[w]) + hi_f<E>(g[w]) * hi_f<E>(o[w]);
  }
  // sum over the row's lanes: lane ^ 1, lane ^ 2 (quad permutations), then the
  // mirror within 8 lanes (i <-> 7 - i joins the two quads) and within 16
  sum += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(sum), 0xB1, 0xf, 0xf, false));
  sum += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(sum), 0x4E, 0xf, 0xf, false));
  if constexpr (LPR >= 8)
    sum += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(sum), 0x141, 0xf, 0xf, false));
  if constexpr (LPR >= 16)
    sum += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(sum), 0x140, 0xf, 0xf, false));
  if (c == 0 && row < rows) {
    p.ndelta[row] = -sum;
    p.nlse2[row] = -lse * kLog2e;
  }
}

// Sum the n_split fp32 partials, rotate dK back (RoPE) and store dK / dV.
// One thread per 4 consecutive d values of one key row.
template <class E, int D, bool ROPE>
__global__ __launch_bounds__(256) void attn_bwd_combine_kernel(AttnParams p) {
  const int64_t n4 = (int64_t)p.B * p.Hkv * p.T * (D / 4);
  const int64_t c = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (c >= n4) return;
  const int d = int(c % (D / 4)) * 4;
  const int64_t row = c / (D / 4);  // (b*Hkv + kvh)*T + key
  const int key = int(row % p.T);
  const int64_t bk = row / p.T;
  const int kvh = int(bk % p.Hkv);
  const int64_t b = bk / p.Hkv;
  const int64_t plane = (int64_t)p.B * p.Hkv * p.T * D;
  f32x4 sk = {0.f, 0.f, 0.f, 0.f}, sv = {0.f, 0.f, 0.f, 0.f};
  for (int s = 0; s < p.n_split; ++s) {
    const float* pk = p.part + (int64_t)s * 2 * plane + row * D + d;
    sk += *reinterpret_cast<const f32x4*>(pk);
    sv += *reinterpret_cast<const f32x4*>(pk + plane);
  }
  float x0 = sk[0], x1 = sk[1], x2 = sk[2], x3 = sk[3];
  if constexpr (ROPE)
    rope_back4(x0, x1, x2, x3, p.cos + (int64_t)key * (D / 2) + d / 2, p.sin + (int64_t)key * (D / 2) + d / 2);
  u32x2 wk = {pack2<E>(x0, x1), pack2<E>(x2, x3)};
  u32x2 wv = {pack2<E>(sv[0], sv[1]), pack2<E>(sv[2], sv[3])};
  *reinterpret_cast<u32x2*>(p.dk + b * p.sdk[0] + (int64_t)kvh * p.sdk[1] + (int64_t)key * p.sdk[2] + d) = wk;
  *reinterpret_cast<u32x2*>(p.dv + b * p.sdv[0] + (int64_t)kvh * p.sdv[1] + (int64_t)key * p.sdv[2] + d) = wv;
}

}  // namespace mt
