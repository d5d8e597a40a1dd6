// gfx950 fp32 products of a few rows against grouped weights: the decode
// step's projections.  y[m, off_g + n] = sum_k x[m, k] w_g[n, k] for every
// group g (the q, k and v projections of a layer, or its w1 and w3), from one
// launch that reads each weight matrix where it lies (and x as it lies, fp32
// or 16-bit: the decode attention's output): the "hip" decoder's
// packed GEMM otherwise concatenates the weights first (a copy of every
// weight per call), and the library GEMMs at 32 rows are latency-bound.
//
// One workgroup per 16 x 16 tile of y (16 rows, 16 columns of one group),
// 8 waves; wave w takes K / 8 values of the contraction, and its lane quarter
// q every fourth 16-byte block of them, so that the four quarters of a row
// read 64 contiguous bytes per load instruction.  A lane loads its blocks of
// one x row and one w row, all of them before the first product (up to 12:
// one memory round trip for K <= 1536), and feeds them to
// v_mfma_f32_16x16x4_f32, whose contraction slot is the lane quarter, so the
// four quarters' partial sums add inside the MFMA; the 8 waves' tiles are
// summed through LDS.  Row tiles are separate workgroups so that narrow
// outputs (512 columns: 32 column tiles) still spread over 64 or more CUs.
// fp32 throughout (the reference's eval runs the fp32 model without
// autocast).
#pragma once

#include <type_traits>

#include "mt_common.h"

namespace mt {

constexpr int kLinGroups = 4;   // weight groups per launch
constexpr int kLinWaves = 8;
constexpr int kLinCols = 16;    // columns per workgroup
constexpr int kLinMaxRows = 64; // rows per launch (four 16-row tiles)

struct LinearGroup {
  const float* w;   // [n, K], row stride ldw
  int64_t ldw;
  int n;            // output columns of the group
  int col_off;      // first column of the group in y
  int tile0;        // first workgroup of the group
};

struct LinearParams {
  const void* x;    // [M, K], row stride ldx: fp32, or 16-bit (converted to fp32 on load)
  float* y;         // [M, >= sum n], row stride ldy
  int64_t ldx, ldy;
  int M, K, groups;
  LinearGroup g[kLinGroups];
};

// MFMA layout (16x16x4, fp32): A[i][k] from lane i + 16 k, B[k][j] from lane
// j + 16 k; lane l holds D[4 (l / 16) + v][l % 16], v = 0..3.
// 4 consecutive x values as fp32: one 16-byte load, or one 8-byte load of
// 16-bit values (E = BF16 / FP16) widened exactly
template <class E>
__device__ __forceinline__ f32x4 load_x4(const void* row, int k) {
  if constexpr (std::is_same_v<E, float>) {
    return *reinterpret_cast<const f32x4*>(static_cast<const float*>(row) + k);
  } else {
    const u32x2 w = *reinterpret_cast<const u32x2*>(static_cast<const uint16_t*>(row) + k);
    return f32x4{lo_f<E>(w[0]), hi_f<E>(w[0]), lo_f<E>(w[1]), hi_f<E>(w[1])};
  }
}

// PD: chunks of 4 values per lane held in flight (all of them when K <= 128 PD).
// XT: float, or BF16 / FP16 for a 16-bit x.
template <int PD, class XT>
__global__ __launch_bounds__(64 * kLinWaves) void linear_rows_f32_kernel(LinearParams p) {
  __shared__ float red[kLinWaves][16][17];
  const int tid = threadIdx.x;
  const int wave = tid >> 6;
  const int lane = tid & 63;
  const int q = lane >> 4;   // contraction slot
  const int c = lane & 15;   // A row / B column of this lane
  const int ntiles = p.g[p.groups - 1].tile0 + (p.g[p.groups - 1].n + kLinCols - 1) / kLinCols;
  const int ct = (int)blockIdx.x % ntiles;  // column tile
  const int m0 = ((int)blockIdx.x / ntiles) * 16;
  int gi = 0;
#pragma unroll
  for (int i = 1; i < kLinGroups; ++i)
    if (i < p.groups && ct >= p.g[i].tile0) gi = i;
  const LinearGroup grp = p.g[gi];
  const int n0 = (ct - grp.tile0) * kLinCols;

  // the contraction: wave w takes the values [w K / 8, (w + 1) K / 8), and of
  // those lane quarter q the 16-byte blocks 4 j + q (j = 0 .. K / 128 - 1), so
  // for each j the four quarters of a row read 64 contiguous bytes
  const int k0 = wave * (p.K >> 3) + 4 * q;
  const float* wrow = grp.w + (int64_t)min(n0 + c, grp.n - 1) * grp.ldw + k0;
  constexpr int XB = std::is_same_v<XT, float> ? 4 : 2;  // bytes per x value
  const void* xrow = static_cast<const char*>(p.x) + ((int64_t)min(m0 + c, p.M - 1) * p.ldx + k0) * XB;

  f32x4 acc[2] = {{0.f, 0.f, 0.f, 0.f}, {0.f, 0.f, 0.f, 0.f}};  // two chains: back-to-back issue
  const int nch = p.K >> 7;
  f32x4 wb[PD], xb[PD];
  auto load = [&](int j, int kk) {
    wb[j] = *reinterpret_cast<const f32x4*>(wrow + kk);
    xb[j] = load_x4<XT>(xrow, kk);
  };
#pragma unroll
  for (int j = 0; j < PD; ++j)
    if (j < nch) load(j, 16 * j);
  for (int i0 = 0; i0 < nch; i0 += PD) {
#pragma unroll
    for (int j = 0; j < PD; ++j) {
      const int i = i0 + j;
      if (i < nch) {
#pragma unroll
        for (int e = 0; e < 4; ++e)
          acc[e & 1] = __builtin_amdgcn_mfma_f32_16x16x4f32(xb[j][e], wb[j][e], acc[e & 1], 0, 0, 0);
        if (i + PD < nch) load(j, 16 * (i + PD));
      }
    }
  }
  // the waves' tiles through LDS, then one output per thread of the first 4 waves
#pragma unroll
  for (int v = 0; v < 4; ++v) red[wave][4 * q + v][c] = acc[0][v] + acc[1][v];
  __syncthreads();
  if (tid < 256) {
    const int r = tid >> 4, col = tid & 15;
    const int m = m0 + r, n = n0 + col;
    float s = 0.f;
#pragma unroll
    for (int w = 0; w < kLinWaves; ++w) s += red[w][r][col];
    if (m < p.M && n < grp.n) p.y[(int64_t)m * p.ldy + grp.col_off + n] = s;
  }
}

}  // namespace mt
