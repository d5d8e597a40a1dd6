// Shared device helpers for the gfx950 causal GQA attention kernels.
//
// MFMA layout facts used throughout (v_mfma_f32_32x32x16_{bf16,f16}, wave64),
// checked lane by lane on an MI355X:
//   A operand (32 x 16, M x K): lane l holds row m = l % 32, k-slots 8*(l/32) + j, j = 0..7
//   B operand (16 x 32, K x N): lane l holds col n = l % 32, k-slots 8*(l/32) + j
//   C/D (32 x 32):              lane l holds col n = l % 32, rows m = 8*(i/4) + 4*(l/32) + (i%4), i = 0..15
// A k-slot (half h, slot j) of A pairs with the same (h, j) of B, so any
// permutation of the contraction index that is applied to both operands gives
// the same product.  The kernels exploit that: a C tile (lane = n, slots = m)
// is fed straight back as the B operand of a product that contracts over m,
// with the A operand read in the matching permuted order.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace mt {

typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;

// Element traits: storage is always 16-bit; the MFMA builtin differs.
struct BF16 {
  using v8 = bf16x8;
  using v4 = bf16x4;
  using v2 = bf16x2;
  static __device__ __forceinline__ f32x16 mfma(v8 a, v8 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
  }
  static __device__ __forceinline__ float to_f(uint16_t x) { return __uint_as_float(uint32_t(x) << 16); }
  // acc + lo(w) + hi(w) for two packed values (v_dot2c_f32_bf16 against 1.0, 1.0)
  static __device__ __forceinline__ float sum2(uint32_t w, float acc) {
    return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, w), __builtin_bit_cast(bf16x2, 0x3F803F80u),
                                           acc, false);
  }
  // acc + lo(a) lo(b) + hi(a) hi(b) (v_dot2c_f32_bf16: exact products, fp32 sum)
  static __device__ __forceinline__ float dot2(uint32_t a, uint32_t b, float acc) {
    return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, a), __builtin_bit_cast(bf16x2, b), acc, false);
  }
};

struct FP16 {
  using v8 = f16x8;
  using v4 = f16x4;
  using v2 = f16x2;
  static __device__ __forceinline__ f32x16 mfma(v8 a, v8 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
  }
  static __device__ __forceinline__ float to_f(uint16_t x) {
    return (float)__builtin_bit_cast(_Float16, x);
  }
  static __device__ __forceinline__ float sum2(uint32_t w, float acc) {
    return __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2, w), __builtin_bit_cast(f16x2, 0x3C003C00u), acc, false);
  }
  static __device__ __forceinline__ float dot2(uint32_t a, uint32_t b, float acc) {
    return __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2, a), __builtin_bit_cast(f16x2, b), acc, false);
  }
};

// Two fp32 values -> two 16-bit values packed in a u32 (round to nearest even).
template <class E>
__device__ __forceinline__ uint32_t pack2(float a, float b) {
  f32x2 x = {a, b};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(x, typename E::v2));
}

// Low/high 16-bit halves of a u32 as fp32.
template <class E>
__device__ __forceinline__ float lo_f(uint32_t w) { return E::to_f(uint16_t(w & 0xffffu)); }
template <class E>
__device__ __forceinline__ float hi_f(uint32_t w) { return E::to_f(uint16_t(w >> 16)); }

__device__ __forceinline__ float exp2_fast(float x) { return __builtin_amdgcn_exp2f(x); }

template <int CTRL>
__device__ __forceinline__ float dpp_mov(float x) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), CTRL, 0xf, 0xf, false));
}

template <bool MAX>
__device__ __forceinline__ float red_op(float a, float b) {
  return MAX ? fmaxf(a, b) : a + b;
}

// Max or sum over lane bits [LO, 6) of a wave64; every lane receives the
// result.  Bits 0-1: quad permutations; bits 2-3: row rotations by 4 and 8
// (after them each lane holds the sum over the lanes of its row that agree
// with it in the lower bits); bits 4-5: v_permlane16/32_swap.
template <int LO, bool MAX>
__device__ __forceinline__ float wave_reduce(float x) {
  if constexpr (LO <= 0) x = red_op<MAX>(x, dpp_mov<0xB1>(x));   // quad_perm(1,0,3,2): lane ^ 1
  if constexpr (LO <= 1) x = red_op<MAX>(x, dpp_mov<0x4E>(x));   // quad_perm(2,3,0,1): lane ^ 2
  if constexpr (LO <= 2) x = red_op<MAX>(x, dpp_mov<0x124>(x));  // row_ror:4
  if constexpr (LO <= 3) x = red_op<MAX>(x, dpp_mov<0x128>(x));  // row_ror:8
  if constexpr (LO <= 4) {
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    x = red_op<MAX>(__uint_as_float(r[0]), __uint_as_float(r[1]));
  }
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return red_op<MAX>(__uint_as_float(r[0]), __uint_as_float(r[1]));
}


// Max of a value and its lane^32 partner (both halves of the wave end up equal).
__device__ __forceinline__ float max_with_partner(float x) {
  auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float sum_with_partner(float x) {
  auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// Rotate the 4 interleaved pairs held in a 16-byte chunk (8 x 16-bit) by the
// angles whose cos/sin are c[0..3], s[0..3]:  (e, o) -> (e c - o s, e s + o c).
template <class E>
__device__ __forceinline__ u32x4 rope_chunk(u32x4 x, f32x4 c, f32x4 s) {
  u32x4 out;
#pragma unroll
  for (int p = 0; p < 4; ++p) {
    float e = lo_f<E>(x[p]);
    float o = hi_f<E>(x[p]);
    out[p] = pack2<E>(e * c[p] - o * s[p], e * s[p] + o * c[p]);
  }
  return out;
}

__device__ __forceinline__ u32x4 zero4() { return u32x4{0u, 0u, 0u, 0u}; }

}  // namespace mt
