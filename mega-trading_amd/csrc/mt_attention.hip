// C ABI of libmt_attn.so: argument checks, launch geometry and dispatch to the
// gfx950 kernels in attn_kernels.h.  Declared in include/mt_attention.h.
//
// The validation mirrors the reference's Python checks
// (src/mega_trading/kernels/triton_attention.py:14-23) so a bad call fails
// before any launch, with a message retrievable through mt_last_error().
#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdio>
#include <cstring>

#include "../../include/mt_attention.h"
#include "attn_kernels.h"

namespace {

thread_local char g_err[512] = "";

int fail(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
int fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
  return code;
}

int ok() {
  g_err[0] = '\0';
  return MT_OK;
}

// Strides for one [B,H,T,D] tensor: d stride must be 1 and rows 16-byte aligned.
int check_tensor(const char* name, const void* ptr, const int64_t* s) {
  if (!ptr) return fail(MT_E_NULL, "%s is NULL", name);
  if (s[3] != 1) return fail(MT_E_STRIDE, "%s: last-dim stride must be 1 (got %lld)", name, (long long)s[3]);
  if (reinterpret_cast<uintptr_t>(ptr) % 16) return fail(MT_E_STRIDE, "%s: base pointer must be 16-byte aligned", name);
  for (int i = 0; i < 3; ++i)
    if (s[i] % 8) return fail(MT_E_STRIDE, "%s: stride %d (%lld) must be a multiple of 8 elements", name, i, (long long)s[i]);
  return MT_OK;
}

int check_common(int B, int Hq, int Hkv, int T, int D, int dtype, const float* cs, const float* sn) {
  if (B < 1 || Hq < 1 || Hkv < 1 || T < 1) return fail(MT_E_SHAPE, "B, Hq, Hkv and T must be >= 1 (got %d, %d, %d, %d)", B, Hq, Hkv, T);
  if (Hq % Hkv) return fail(MT_E_SHAPE, "query heads (%d) must equal key/value heads (%d) multiplied by repeats", Hq, Hkv);
  if (D != 32 && D != 64 && D != 128) return fail(MT_E_SHAPE, "head_dim %d unsupported (32, 64 or 128)", D);
  if (dtype != MT_DTYPE_BF16 && dtype != MT_DTYPE_FP16) return fail(MT_E_DTYPE, "dtype code %d unsupported", dtype);
  if ((cs == nullptr) != (sn == nullptr)) return fail(MT_E_ROPE, "rope_cos and rope_sin must both be given or both be NULL");
  if (cs && (reinterpret_cast<uintptr_t>(cs) % 16 || reinterpret_cast<uintptr_t>(sn) % 16))
    return fail(MT_E_ROPE, "RoPE tables must be 16-byte aligned");
  return MT_OK;
}

void fill_geometry(mt::AttnParams& p, int B, int Hq, int Hkv, int T, float scale) {
  p.B = B;
  p.Hq = Hq;
  p.Hkv = Hkv;
  p.T = T;
  p.R = Hq / Hkv;
  p.r_sub = (p.R % 4 == 0) ? 4 : (p.R % 2 == 0) ? 2 : 1;
  p.n_hsub = p.R / p.r_sub;
  p.rb = 4 / p.r_sub;
  p.nqb = (T + mt::kBlk - 1) / mt::kBlk;
  p.nsb = (p.nqb + p.rb - 1) / p.rb;
  p.scale = scale;
  p.scale_log2 = scale * mt::kLog2e;
}

void copy3(int64_t dst[3], const int64_t* s) {
  dst[0] = s[0];
  dst[1] = s[1];
  dst[2] = s[2];
}

template <class E, int D, bool ROPE>
hipError_t launch_fwd(const mt::AttnParams& p, hipStream_t st) {
  dim3 grid(p.nsb * p.B * p.Hkv * p.n_hsub);
  hipLaunchKernelGGL((mt::attn_fwd_kernel<E, D, ROPE>), grid, dim3(256), 0, st, p);
  return hipGetLastError();
}

// stage: 1 = dQ (+ delta), 2 = dK/dV, 3 = both
template <class E, int D, bool ROPE>
hipError_t launch_bwd(const mt::AttnParams& p, hipStream_t st, int stage) {
  if (stage & 1) {
    dim3 grid_dq(p.nsb * p.B * p.Hkv * p.n_hsub);
    hipLaunchKernelGGL((mt::attn_bwd_dq_kernel<E, D, ROPE>), grid_dq, dim3(256), 0, st, p);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
  }
  if (stage & 2) {
    dim3 grid_kv(p.nqb * p.B * p.Hkv);
    hipLaunchKernelGGL((mt::attn_bwd_dkv_kernel<E, D, ROPE>), grid_kv, dim3(64 * mt::kKvWaves), 0, st, p);
    return hipGetLastError();
  }
  return hipSuccess;
}

template <class E, int D, bool ROPE>
hipError_t launch_fwd_s(const mt::AttnParams& p, hipStream_t st, int) {
  return launch_fwd<E, D, ROPE>(p, st);
}

using Launcher = hipError_t (*)(const mt::AttnParams&, hipStream_t, int);

template <bool FWD, class E, int D>
Launcher pick_rope(bool rope) {
  if (FWD) return rope ? &launch_fwd_s<E, D, true> : &launch_fwd_s<E, D, false>;
  return rope ? &launch_bwd<E, D, true> : &launch_bwd<E, D, false>;
}

template <bool FWD>
Launcher pick(int dtype, int D, bool rope) {
  if (dtype == MT_DTYPE_BF16) {
    if (D == 32) return pick_rope<FWD, mt::BF16, 32>(rope);
    if (D == 64) return pick_rope<FWD, mt::BF16, 64>(rope);
    return pick_rope<FWD, mt::BF16, 128>(rope);
  }
  if (D == 32) return pick_rope<FWD, mt::FP16, 32>(rope);
  if (D == 64) return pick_rope<FWD, mt::FP16, 64>(rope);
  return pick_rope<FWD, mt::FP16, 128>(rope);
}

}  // namespace

extern "C" {

int mt_version(void) { return (0 << 16) | 1; }

const char* mt_last_error(void) { return g_err; }

int mt_gqa_attn_fwd(const void* q, const void* k, const void* v, void* o, float* lse,
                    int B, int Hq, int Hkv, int T, int D,
                    const int64_t* strides, float scale, int dtype,
                    const float* rope_cos, const float* rope_sin, void* stream) {
  int rc = check_common(B, Hq, Hkv, T, D, dtype, rope_cos, rope_sin);
  if (rc) return rc;
  if (!strides) return fail(MT_E_NULL, "strides is NULL");
  if (!lse) return fail(MT_E_NULL, "lse is NULL");
  if ((rc = check_tensor("q", q, strides + 0))) return rc;
  if ((rc = check_tensor("k", k, strides + 4))) return rc;
  if ((rc = check_tensor("v", v, strides + 8))) return rc;
  if ((rc = check_tensor("o", o, strides + 12))) return rc;

  mt::AttnParams p{};
  p.q = static_cast<const uint16_t*>(q);
  p.k = static_cast<const uint16_t*>(k);
  p.v = static_cast<const uint16_t*>(v);
  p.out = static_cast<uint16_t*>(o);
  p.lse = lse;
  p.cos = rope_cos;
  p.sin = rope_sin;
  copy3(p.sq, strides + 0);
  copy3(p.sk, strides + 4);
  copy3(p.sv, strides + 8);
  copy3(p.so, strides + 12);
  fill_geometry(p, B, Hq, Hkv, T, scale);
  hipError_t e = pick<true>(dtype, D, rope_cos != nullptr)(p, static_cast<hipStream_t>(stream), 0);
  if (e != hipSuccess) return fail(int(e), "forward launch failed: %s", hipGetErrorString(e));
  return ok();
}

static int bwd_impl(int stage, const void* q, const void* k, const void* v, const void* o, const float* lse,
                    const void* dout, void* dq, void* dk, void* dv, float* delta_ws,
                    int B, int Hq, int Hkv, int T, int D,
                    const int64_t* strides, float scale, int dtype,
                    const float* rope_cos, const float* rope_sin, void* stream) {
  int rc = check_common(B, Hq, Hkv, T, D, dtype, rope_cos, rope_sin);
  if (rc) return rc;
  if (!strides) return fail(MT_E_NULL, "strides is NULL");
  if (!lse) return fail(MT_E_NULL, "lse is NULL");
  if (!delta_ws) return fail(MT_E_NULL, "delta_ws is NULL");
  if ((rc = check_tensor("q", q, strides + 0))) return rc;
  if ((rc = check_tensor("k", k, strides + 4))) return rc;
  if ((rc = check_tensor("v", v, strides + 8))) return rc;
  if ((rc = check_tensor("o", o, strides + 12))) return rc;
  if ((rc = check_tensor("dout", dout, strides + 16))) return rc;
  if ((rc = check_tensor("dq", dq, strides + 20))) return rc;
  if ((rc = check_tensor("dk", dk, strides + 24))) return rc;
  if ((rc = check_tensor("dv", dv, strides + 28))) return rc;

  mt::AttnParams p{};
  p.q = static_cast<const uint16_t*>(q);
  p.k = static_cast<const uint16_t*>(k);
  p.v = static_cast<const uint16_t*>(v);
  p.o = static_cast<const uint16_t*>(o);
  p.dout = static_cast<const uint16_t*>(dout);
  p.out = static_cast<uint16_t*>(dq);
  p.dk = static_cast<uint16_t*>(dk);
  p.dv = static_cast<uint16_t*>(dv);
  p.lse = const_cast<float*>(lse);
  p.delta = delta_ws;
  p.cos = rope_cos;
  p.sin = rope_sin;
  copy3(p.sq, strides + 0);
  copy3(p.sk, strides + 4);
  copy3(p.sv, strides + 8);
  copy3(p.so, strides + 12);
  copy3(p.sdo, strides + 16);
  copy3(p.sout, strides + 20);
  copy3(p.sdk, strides + 24);
  copy3(p.sdv, strides + 28);
  fill_geometry(p, B, Hq, Hkv, T, scale);
  hipError_t e = pick<false>(dtype, D, rope_cos != nullptr)(p, static_cast<hipStream_t>(stream), stage);
  if (e != hipSuccess) return fail(int(e), "backward launch failed: %s", hipGetErrorString(e));
  return ok();
}

#define MT_BWD_ARGS                                                                            \
  const void *q, const void *k, const void *v, const void *o, const float *lse, const void *dout, \
      void *dq, void *dk, void *dv, float *delta_ws, int B, int Hq, int Hkv, int T, int D,         \
      const int64_t *strides, float scale, int dtype, const float *rope_cos, const float *rope_sin, \
      void *stream
#define MT_BWD_PASS \
  q, k, v, o, lse, dout, dq, dk, dv, delta_ws, B, Hq, Hkv, T, D, strides, scale, dtype, rope_cos, rope_sin, stream

int mt_gqa_attn_bwd(MT_BWD_ARGS) { return bwd_impl(3, MT_BWD_PASS); }
int mt_gqa_attn_bwd_dq(MT_BWD_ARGS) { return bwd_impl(1, MT_BWD_PASS); }
int mt_gqa_attn_bwd_dkv(MT_BWD_ARGS) { return bwd_impl(2, MT_BWD_PASS); }

}  // extern "C"
