// LDS tiles of 64 rows x D 16-bit elements for the gfx950 attention kernels.
//
// Layout: rows are stored unpadded (2*D bytes); the 16-byte chunks of row r
// are XOR-swizzled, chunk c living at slot c ^ (r % SW), so that the 8 lanes
// reading one chunk column of 8 consecutive rows hit 8 different slots.
//
// Staging uses global_load_lds_dwordx4: each lane of a wave copies 16 bytes
// from its own global address straight into LDS at (wave base + 16 * lane),
// with no VGPR round trip.  The lane -> global-address map applies the
// swizzle, so one instruction fills 1 KB of consecutive swizzled rows.
// Rows at or past T are clamped to row T-1 (in-bounds, finite values); the
// kernels mask the scores of such rows and keys.
//
// Two operand reads:
//  * row_op:  A/B operand with rows = tile rows, k = tile columns
//             (one ds_read_b128 per lane).
//  * tr_op:   A operand with M = tile columns, k = tile rows in the permuted
//             order 16*ks + 8*(j/4) + 4*h + (j%4) that matches a C tile fed
//             back as a B operand (two ds_read_b64_tr_b16 per lane).
//             ds_read_b64_tr_b16 semantics (measured on gfx950): in each
//             16-lane group, output lane i element e is element (i % 4) of the
//             8 bytes addressed by lane 4*e + i/4 of the group.  Lane j of the
//             group therefore points at X[r0 + j/4][c0 + 4*(j%4)], and output
//             lane i receives X[r0 + e][c0 + i], e = 0..3.
#pragma once

#include "mt_common.h"

namespace mt {

typedef short i16x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) i16x4 lds_i16x4;

template <int D>
struct Tile {
  static constexpr int NC = D / 8;              // 16-byte chunks per row
  static constexpr int SW = NC < 8 ? NC : 8;    // swizzle period
  static constexpr int ROW_BYTES = 2 * D;
  static constexpr int BYTES = 64 * ROW_BYTES;  // one 64-row tile
  static constexpr int INSTR = 64 * NC / 64;    // 1 KB wave instructions per tile

  static __device__ __forceinline__ int chunk_off(int row, int chunk) {
    return row * ROW_BYTES + ((chunk ^ (row % SW)) << 4);
  }
  // byte offset of element (row, col); col must be a multiple of 4
  static __device__ __forceinline__ int elem_off(int row, int col) {
    return chunk_off(row, col >> 3) + ((col & 7) << 1);
  }

  // Stage rows [row0, row0+64) of a row-strided 16-bit matrix into `lds`
  // (byte pointer to the tile).  The workgroup's NW waves split the INSTR
  // instructions; `wave`/`lane` identify the caller.
  template <int NW>
  static __device__ __forceinline__ void stage(char* lds, const uint16_t* src, int64_t row_stride, int row0,
                                               int T, int wave, int lane) {
    static_assert(INSTR % NW == 0, "tile instructions must split evenly over the waves");
#pragma unroll
    for (int i = 0; i < INSTR / NW; ++i) {
      const int f = (i * NW + wave) * 64 + lane;  // flat LDS chunk index
      const int row = f / NC;
      const int slot = f % NC;
      const int chunk = slot ^ (row % SW);
      const int grow = min(row0 + row, T - 1);
      const uint16_t* g = src + (int64_t)grow * row_stride + chunk * 8;
      __builtin_amdgcn_global_load_lds(g, (__attribute__((address_space(3))) void*)(lds + (i * NW + wave) * 1024), 16, 0, 0);
    }
  }

  template <class E>
  static __device__ __forceinline__ typename E::v8 row_op(const char* lds, int r0, int kk, int lane) {
    const int row = r0 + (lane & 31);
    const int chunk = 2 * kk + (lane >> 5);
    return *reinterpret_cast<const typename E::v8*>(lds + chunk_off(row, chunk));
  }

  template <class E>
  static __device__ __forceinline__ typename E::v8 tr_op(const char* lds, int r0, int c0, int lane) {
    const int g = lane >> 4;
    const int i = lane & 15;
    const int col = c0 + 16 * (g & 1) + 4 * (i & 3);
    const int row = r0 + 4 * (g >> 1) + (i >> 2);
    i16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)(lds + elem_off(row, col)));
    i16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)(lds + elem_off(row + 8, col)));
    u32x4 w = {__builtin_bit_cast(u32x2, lo)[0], __builtin_bit_cast(u32x2, lo)[1],
               __builtin_bit_cast(u32x2, hi)[0], __builtin_bit_cast(u32x2, hi)[1]};
    return __builtin_bit_cast(typename E::v8, w);
  }
};

// Stage 64 fp32 values (row-indexed vector, clamped at T-1) with one wave.
__device__ __forceinline__ void stage_vec64(char* lds, const float* src, int row0, int T, int lane) {
  const float* g = src + min(row0 + lane, T - 1);
  __builtin_amdgcn_global_load_lds(g, (__attribute__((address_space(3))) void*)lds, 4, 0, 0);
}

__device__ __forceinline__ void wait_vmem() { __builtin_amdgcn_s_waitcnt(0x0F70); }  // vmcnt(0)

}  // namespace mt
