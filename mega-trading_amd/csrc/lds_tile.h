// LDS tiles of 64 rows x D 16-bit elements for the gfx950 attention kernels.
//
// Layout: rows are stored unpadded (RB = 2*D bytes); the 16-byte chunks of
// row r are XOR-swizzled, chunk c living at slot c ^ f(r), f of period 16.
// The gfx950 LDS serves 256 bytes per clock: a wave's ds_read_b128 is served
// 16 lanes at a time and a ds_read_b64_tr_b16 32 lanes at a time, so an
// access is conflict-free when each such group covers 256 distinct bytes
// modulo 256.  For D = 64 (two rows per 256 bytes) f(r) = 4*((r/2) % 2) +
// (r/4) % 4 makes the 16 consecutive rows of a ds_read_b128 group (one chunk
// column) and the 4 rows x 4 chunks of a transposed-read group land on 16
// distinct 16-byte slots; for D = 128 (one row per 256 bytes) f(r) =
// 4*(r % 4) + (r/4) % 4 does the same, and for D = 32 (four rows per 256
// bytes) f(r) = (r/4) % 4.  Because the swizzle is an XOR with
// bits the operand offsets never touch and has period 16, every operand
// address is a per-lane base computed once, XOR-ed with a per-step constant,
// plus an immediate offset of a multiple of 16 rows.
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
//             back as a B operand (two ds_read_b64_tr_b16 per lane, rows
//             16ks + 0..7 and 16ks + 8..15, from two per-lane bases).
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

// Per-lane bases of the two transposed reads of a tr_op (rows 0..7 and 8..15
// of a 16-row group).
struct TrBase {
  int lo, hi;
};

template <int D>
struct Tile {
  static constexpr int NC = D / 8;              // 16-byte chunks per row
  static constexpr int RB = 2 * D;              // row bytes
  static constexpr int BYTES = 64 * RB;         // one 64-row tile
  static constexpr int INSTR = NC;              // 1 KB wave instructions per tile (64 * NC * 16 B / 1 KB)

  // slot permutation of row r (period 16)
  static __device__ __forceinline__ int swz(int row) {
    if constexpr (NC == 8) return (((row >> 1) & 1) << 2) | ((row >> 2) & 3);
    else if constexpr (NC == 16) return ((row & 3) << 2) | ((row >> 2) & 3);
    else return (row >> 2) & 3;  // NC == 4: four rows per 256 bytes
  }

  // --- operand addressing -------------------------------------------------
  // row_op base: lane (row = lane % 32, chunk = lane / 32) at r0 = 0, kk = 0.
  static __device__ __forceinline__ int row_base(int lane) {
    const int row = lane & 31;
    const int chunk = lane >> 5;
    return row * RB + ((chunk ^ swz(row)) << 4);
  }
  // tr_op bases: lane's 8-byte source in rows 0..7 and 8..15 at c0 = 0.
  static __device__ __forceinline__ TrBase tr_base(int lane) {
    const int g = lane >> 4;
    const int i = lane & 15;
    const int row = 4 * (g >> 1) + (i >> 2);
    const int col = 16 * (g & 1) + 4 * (i & 3);
    auto at = [&](int r) { return r * RB + (((col >> 3) ^ swz(r)) << 4) + ((col & 7) << 1); };
    return TrBase{at(row), at(row + 8)};
  }

  template <class E>
  static __device__ __forceinline__ typename E::v8 row_op(const char* lds, int base, int r0, int kk) {
    return *reinterpret_cast<const typename E::v8*>(lds + (base ^ (32 * kk)) + r0 * RB);
  }

  template <class E>
  static __device__ __forceinline__ typename E::v8 tr_op(const char* lds, TrBase b, int ks, int dt) {
    const char* p = lds + 16 * ks * RB;
    i16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)(p + (b.lo ^ (64 * dt))));
    i16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)(p + (b.hi ^ (64 * dt))));
    u32x4 w = {__builtin_bit_cast(u32x2, lo)[0], __builtin_bit_cast(u32x2, lo)[1],
               __builtin_bit_cast(u32x2, hi)[0], __builtin_bit_cast(u32x2, hi)[1]};
    return __builtin_bit_cast(typename E::v8, w);
  }
};

// Global -> LDS copies (global_load_lds_dword[x4]: M0 = the wave's LDS base,
// lane L's bytes land at M0 + size * L).  Issued from inline assembly so the
// compiler does not track them: it would otherwise make the first
// ds_read_b64_tr_b16 after each copy wait for every outstanding copy (it cannot
// tell that the copy targets the other buffer), serialising the next tile's
// prefetch with the current tile's compute.  Completion is enforced explicitly:
// every copied buffer is read only after wait_vmem() and a workgroup barrier,
// and a buffer is refilled only after the barrier that ends its last reads.
//
// Because the compiler does not see what these instructions read, it cannot
// insert the wait states gfx950 requires before them, so the blocks take care
// of them: each starts with `s_nop 0` after the M0 write the compiler places
// right before it (an LDS DMA reading an M0 written by a scalar instruction
// needs one wait state), and the scalar-base forms read their base from a
// scalar copy (uniform_ptr), never from the SGPRs a v_readfirstlane wrote (a
// vector-memory instruction reading an SGPR written by a vector instruction
// needs five).
__device__ __forceinline__ uint32_t lds_addr(const void* l) {
  return (uint32_t)(uintptr_t)l;
}

__device__ __forceinline__ void lds_dma16(const uint16_t* g, char* l) {
  asm volatile("s_nop 0\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(g), "{m0}"(lds_addr(l)));
}

__device__ __forceinline__ void lds_dma4(const float* g, char* l) {
  asm volatile("s_nop 0\n\tglobal_load_lds_dword %0, off" ::"v"(g), "{m0}"(lds_addr(l)));
}

// Scalar-base forms: lane L reads base + voff_L (a 32-bit byte offset), so a
// whole tile's addresses cost one 64-bit scalar add and no vector ALU work.
// `base` must be wave-uniform; it is moved to scalar registers explicitly
// (free when the compiler already holds it there) and then copied by a scalar
// instruction, which the copy blocks read.
__device__ __forceinline__ uint64_t uniform_ptr(const void* p) {
  const uint64_t v = (uint64_t)(uintptr_t)p;
  const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)v);
  const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(v >> 32));
  uint64_t r;
  asm volatile("s_mov_b64 %0, %1" : "=s"(r) : "s"(((uint64_t)hi << 32) | lo));
  return r;
}

__device__ __forceinline__ void lds_dma16_s(const void* base, uint32_t voff, uint32_t l) {
  asm volatile("s_nop 0\n\tglobal_load_lds_dwordx4 %0, %1" ::"v"(voff), "s"(uniform_ptr(base)), "{m0}"(l));
}

__device__ __forceinline__ void lds_dma4_s(const void* base, uint32_t voff, uint32_t l) {
  asm volatile("s_nop 0\n\tglobal_load_lds_dword %0, %1" ::"v"(voff), "s"(uniform_ptr(base)), "{m0}"(l));
}

// Staging of one 64-row tile by the NW waves of a workgroup: per-lane source
// offsets (elements, relative to the tile's first row) of the INSTR/NW wave
// instructions this wave issues, computed once.

template <int D, int NW>
struct Stager {
  using TL = Tile<D>;
  static_assert(TL::INSTR % NW == 0, "tile instructions must split evenly over the waves");
  static constexpr int N = TL::INSTR / NW;
  uint32_t voff[N];  // byte offsets (row * row_stride + chunk * 8) * 2 from the tile's first row
  int lds_off;       // byte offset of this wave's first 1 KB block in the tile (wave-uniform)
  int wave_, lane_;

  static __device__ __forceinline__ void place(int i, int wave, int lane, int& row, int& chunk) {
    const int f = (i * NW + wave) * 64 + lane;  // flat LDS chunk index
    row = f / TL::NC;
    chunk = (f % TL::NC) ^ TL::swz(row);
  }

  __device__ __forceinline__ void init(int64_t row_stride, int wave, int lane) {
#pragma unroll
    for (int i = 0; i < N; ++i) {
      int row, chunk;
      place(i, wave, lane, row, chunk);
      voff[i] = (uint32_t)(row * (int)row_stride + chunk * 8) * 2u;
    }
    lds_off = __builtin_amdgcn_readfirstlane(wave) * 1024;
    wave_ = wave;
    lane_ = lane;
  }

  // Stage rows [row0, row0 + 64) of the matrix at `src` (row stride as in init).
  __device__ __forceinline__ void stage(char* lds, const uint16_t* src, int64_t row_stride, int row0, int T) const {
    if (row0 + 64 <= T) {
      const uint16_t* tile = src + (int64_t)row0 * row_stride;
      const uint32_t l0 = lds_addr(lds) + (uint32_t)lds_off;
#pragma unroll
      for (int i = 0; i < N; ++i) lds_dma16_s(tile, voff[i], l0 + i * NW * 1024);
    } else {
#pragma unroll
      for (int i = 0; i < N; ++i) {
        int row, chunk;
        place(i, wave_, lane_, row, chunk);
        const int grow = min(row0 + row, T - 1);
        lds_dma16(src + (int64_t)grow * row_stride + chunk * 8, lds + lds_off + i * NW * 1024);
      }
    }
  }
};

// Stage 64 fp32 values (row-indexed vector, clamped at T-1) with one wave.
__device__ __forceinline__ void stage_vec64(char* lds, const float* src, int row0, int T, int lane) {
  if (row0 + 64 <= T)
    lds_dma4_s(src + row0, (uint32_t)lane * 4u, lds_addr(lds));
  else
    lds_dma4(src + min(row0 + lane, T - 1), lds);
}

__device__ __forceinline__ void wait_vmem() { __builtin_amdgcn_s_waitcnt(0x0F70); }  // vmcnt(0)

}  // namespace mt
