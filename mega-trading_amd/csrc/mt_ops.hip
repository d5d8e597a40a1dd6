// C ABI of the decoder operators (RMSNorm, residual-add + RMSNorm, SwiGLU
// gate, cross-entropy rows, stand-alone RoPE): argument checks, launch geometry and dispatch to
// ops_kernels.h.
// Declared in include/mt_ops.h.
#include <hip/hip_runtime.h>

#include <cstdint>

#include "../../include/mt_ops.h"
#include "linear_kernels.h"
#include "mt_abi.h"
#include "ops_kernels.h"
#include "sample_kernels.h"

namespace {

using mt_abi::device_cus;
using mt_abi::fail;
using mt_abi::ok;
namespace K = mt::ops;

bool aligned16(const void* p) { return reinterpret_cast<uintptr_t>(p) % 16 == 0; }

int check_dtype(int dtype, int weight_dtype) {
  if (dtype != MT_DTYPE_BF16 && dtype != MT_DTYPE_FP16 && dtype != MT_DTYPE_FP32)
    return fail(MT_E_DTYPE, "dtype code %d unsupported", dtype);
  if (weight_dtype != dtype && weight_dtype != MT_DTYPE_FP32)
    return fail(MT_E_DTYPE, "weight dtype code %d must equal the tensor dtype (%d) or be fp32", weight_dtype, dtype);
  return MT_OK;
}

int check_rows(int64_t rows, int dim) {
  if (rows < 0 || rows > (int64_t(1) << 32))
    return fail(MT_E_SHAPE, "rows must be in [0, 2^32] (got %lld)", (long long)rows);
  if (dim < 8 || dim > 4096 || dim % 8)
    return fail(MT_E_SHAPE, "dim %d unsupported (a multiple of 8 in [8, 4096])", dim);
  return MT_OK;
}

int check_ptr(const char* name, const void* p) {
  if (!p) return fail(MT_E_NULL, "%s is NULL", name);
  if (!aligned16(p)) return fail(MT_E_STRIDE, "%s must be 16-byte aligned", name);
  return MT_OK;
}

int check_stride(const char* name, int64_t stride, int dim) {
  if (stride < dim || stride % 8) return fail(MT_E_STRIDE, "%s row stride %lld must be >= dim and a multiple of 8",
                                               name, (long long)stride);
  return MT_OK;
}

// chunks of 8 values per lane that hold a row of dim values: 1, 2, 4 or 8
int chunks(int dim) {
  const int nch = (dim / 8 + 63) / 64;
  return nch <= 1 ? 1 : nch <= 2 ? 2 : nch <= 4 ? 4 : 8;
}

// workgroups of the RMSNorm backward: 4 per CU (16 waves), each striding over rows
int bwd_blocks(int64_t rows) {
  const int64_t want = (rows + 3) / 4;
  const int64_t cap = 4L * device_cus();
  return (int)(want < 1 ? 1 : want < cap ? want : cap);
}

// ---- dispatch over (dtype, weight dtype, chunks) ---------------------------
// XT / ST / YT: storage of x, of the residual stream (residual, new residual)
// and of y; one dtype for all of them in the reference operators.
template <int XT, int ST, int YT, int WT, int NCH, bool ADD>
hipError_t fwd_launch_x(const void* x, int64_t sx, const void* r, int64_t sr, const void* w, void* nr, void* y,
                        float* rstd, int64_t rows, int dim, float eps, hipStream_t st) {
  const dim3 grid((unsigned)((rows + 3) / 4));
  hipLaunchKernelGGL((K::rmsnorm_fwd_kernel<XT, ST, YT, WT, NCH, ADD>), grid, dim3(256), 0, st, x, sx, r, sr, w, nr, y,
                     rstd, rows, dim, eps);
  return hipGetLastError();
}

template <int DT, int WT, int NCH, bool ADD>
hipError_t fwd_launch(const void* x, int64_t sx, const void* r, int64_t sr, const void* w, void* nr, void* y, float* rstd,
                      int64_t rows, int dim, float eps, hipStream_t st) {
  return fwd_launch_x<DT, DT, DT, WT, NCH, ADD>(x, sx, r, sr, w, nr, y, rstd, rows, dim, eps, st);
}

// ST: storage of s, d_new_res and ds; GT: of dy (and of the optional ds16 copy)
template <int ST, int GT, int WT, int NCH, bool ADD>
hipError_t bwd_launch_x(const void* s, const void* w, const float* rstd, const void* dy, const void* dres, void* ds,
                        void* ds16, void* dw, float* partial, int64_t rows, int dim, hipStream_t st) {
  const int nb = bwd_blocks(rows);
  if (rows > 0) {
    hipLaunchKernelGGL((K::rmsnorm_bwd_kernel<ST, GT, WT, NCH, ADD>), dim3(nb), dim3(256), 0, st, s, w, rstd, dy, dres,
                       ds, ds16, partial, rows, dim);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
  }
  hipLaunchKernelGGL((K::column_sum_kernel<WT>), dim3((dim + 63) / 64), dim3(64 * K::kColWaves), 0, st, partial,
                     rows > 0 ? nb : 0, dim, dw);
  return hipGetLastError();
}

template <int DT, int WT, int NCH, bool ADD>
hipError_t bwd_launch(const void* s, const void* w, const float* rstd, const void* dy, const void* dres, void* ds,
                      void* dw, float* partial, int64_t rows, int dim, hipStream_t st) {
  return bwd_launch_x<DT, DT, WT, NCH, ADD>(s, w, rstd, dy, dres, ds, nullptr, dw, partial, rows, dim, st);
}

// ---- mixed form: fp32 residual stream and weight, 16-bit activations (AT) --
template <int AT, bool ADD>
hipError_t fwd_mixed(int nch, const void* x, int64_t sx, const void* r, int64_t sr, const void* w, void* nr, void* y,
                     float* rstd, int64_t rows, int dim, float eps, hipStream_t st) {
  // x: the 16-bit branch output when ADD, else the fp32 residual stream itself
  constexpr int XT = ADD ? AT : K::kDtFP32;
  constexpr int F = K::kDtFP32;
  switch (nch) {
    case 1: return fwd_launch_x<XT, F, AT, F, 1, ADD>(x, sx, r, sr, w, nr, y, rstd, rows, dim, eps, st);
    case 2: return fwd_launch_x<XT, F, AT, F, 2, ADD>(x, sx, r, sr, w, nr, y, rstd, rows, dim, eps, st);
    case 4: return fwd_launch_x<XT, F, AT, F, 4, ADD>(x, sx, r, sr, w, nr, y, rstd, rows, dim, eps, st);
    default: return fwd_launch_x<XT, F, AT, F, 8, ADD>(x, sx, r, sr, w, nr, y, rstd, rows, dim, eps, st);
  }
}

template <int AT, bool ADD>
hipError_t bwd_mixed(int nch, const void* s, const void* w, const float* rstd, const void* dy, const void* dres,
                     void* ds, void* ds16, void* dw, float* partial, int64_t rows, int dim, hipStream_t st) {
  constexpr int F = K::kDtFP32;
  switch (nch) {
    case 1: return bwd_launch_x<F, AT, F, 1, ADD>(s, w, rstd, dy, dres, ds, ds16, dw, partial, rows, dim, st);
    case 2: return bwd_launch_x<F, AT, F, 2, ADD>(s, w, rstd, dy, dres, ds, ds16, dw, partial, rows, dim, st);
    case 4: return bwd_launch_x<F, AT, F, 4, ADD>(s, w, rstd, dy, dres, ds, ds16, dw, partial, rows, dim, st);
    default: return bwd_launch_x<F, AT, F, 8, ADD>(s, w, rstd, dy, dres, ds, ds16, dw, partial, rows, dim, st);
  }
}

int check_mixed(int act_dtype, int weight_dtype) {
  if (act_dtype != MT_DTYPE_BF16 && act_dtype != MT_DTYPE_FP16)
    return fail(MT_E_DTYPE, "activation dtype code %d unsupported (bf16 or fp16)", act_dtype);
  if (weight_dtype != MT_DTYPE_FP32) return fail(MT_E_DTYPE, "weight dtype code %d must be fp32", weight_dtype);
  return MT_OK;
}

template <int DT, int WT, bool ADD>
hipError_t fwd_nch(int nch, const void* x, int64_t sx, const void* r, int64_t sr, const void* w, void* nr, void* y,
                   float* rstd, int64_t rows, int dim, float eps, hipStream_t st) {
  switch (nch) {
    case 1: return fwd_launch<DT, WT, 1, ADD>(x, sx, r, sr, w, nr, y, rstd, rows, dim, eps, st);
    case 2: return fwd_launch<DT, WT, 2, ADD>(x, sx, r, sr, w, nr, y, rstd, rows, dim, eps, st);
    case 4: return fwd_launch<DT, WT, 4, ADD>(x, sx, r, sr, w, nr, y, rstd, rows, dim, eps, st);
    default: return fwd_launch<DT, WT, 8, ADD>(x, sx, r, sr, w, nr, y, rstd, rows, dim, eps, st);
  }
}

template <int DT, int WT, bool ADD>
hipError_t bwd_nch(int nch, const void* s, const void* w, const float* rstd, const void* dy, const void* dres, void* ds,
                   void* dw, float* partial, int64_t rows, int dim, hipStream_t st) {
  switch (nch) {
    case 1: return bwd_launch<DT, WT, 1, ADD>(s, w, rstd, dy, dres, ds, dw, partial, rows, dim, st);
    case 2: return bwd_launch<DT, WT, 2, ADD>(s, w, rstd, dy, dres, ds, dw, partial, rows, dim, st);
    case 4: return bwd_launch<DT, WT, 4, ADD>(s, w, rstd, dy, dres, ds, dw, partial, rows, dim, st);
    default: return bwd_launch<DT, WT, 8, ADD>(s, w, rstd, dy, dres, ds, dw, partial, rows, dim, st);
  }
}

template <bool ADD>
hipError_t fwd_dispatch(int dtype, int wdt, const void* x, int64_t sx, const void* r, int64_t sr, const void* w,
                        void* nr, void* y, float* rstd, int64_t rows, int dim, float eps, hipStream_t st) {
  const int n = chunks(dim);
  if (dtype == MT_DTYPE_FP32) return fwd_nch<K::kDtFP32, K::kDtFP32, ADD>(n, x, sx, r, sr, w, nr, y, rstd, rows, dim, eps, st);
  if (dtype == MT_DTYPE_BF16) {
    if (wdt == MT_DTYPE_FP32) return fwd_nch<K::kDtBF16, K::kDtFP32, ADD>(n, x, sx, r, sr, w, nr, y, rstd, rows, dim, eps, st);
    return fwd_nch<K::kDtBF16, K::kDtBF16, ADD>(n, x, sx, r, sr, w, nr, y, rstd, rows, dim, eps, st);
  }
  if (wdt == MT_DTYPE_FP32) return fwd_nch<K::kDtFP16, K::kDtFP32, ADD>(n, x, sx, r, sr, w, nr, y, rstd, rows, dim, eps, st);
  return fwd_nch<K::kDtFP16, K::kDtFP16, ADD>(n, x, sx, r, sr, w, nr, y, rstd, rows, dim, eps, st);
}

template <bool ADD>
hipError_t bwd_dispatch(int dtype, int wdt, const void* s, const void* w, const float* rstd, const void* dy,
                        const void* dres, void* ds, void* dw, float* partial, int64_t rows, int dim, hipStream_t st) {
  const int n = chunks(dim);
  if (dtype == MT_DTYPE_FP32) return bwd_nch<K::kDtFP32, K::kDtFP32, ADD>(n, s, w, rstd, dy, dres, ds, dw, partial, rows, dim, st);
  if (dtype == MT_DTYPE_BF16) {
    if (wdt == MT_DTYPE_FP32) return bwd_nch<K::kDtBF16, K::kDtFP32, ADD>(n, s, w, rstd, dy, dres, ds, dw, partial, rows, dim, st);
    return bwd_nch<K::kDtBF16, K::kDtBF16, ADD>(n, s, w, rstd, dy, dres, ds, dw, partial, rows, dim, st);
  }
  if (wdt == MT_DTYPE_FP32) return bwd_nch<K::kDtFP16, K::kDtFP32, ADD>(n, s, w, rstd, dy, dres, ds, dw, partial, rows, dim, st);
  return bwd_nch<K::kDtFP16, K::kDtFP16, ADD>(n, s, w, rstd, dy, dres, ds, dw, partial, rows, dim, st);
}

int swiglu_blocks(int64_t n) {
  const int64_t nvec = n / 8;
  const int64_t want = (nvec + 255) / 256;
  const int64_t cap = 8L * device_cus();
  return (int)(want < 1 ? 1 : want < cap ? want : cap);
}

// register-resident rows up to 2048 * 8 = 16384 logits, streamed beyond
template <int DT, bool GRAD, int NCH>
void ce_launch(dim3 grid, hipStream_t st, void* logits, int64_t ld, const int64_t* labels, int V, const int64_t* nv,
               int64_t ignore, float* loss) {
  hipLaunchKernelGGL((K::ce_rows_kernel<DT, GRAD, NCH>), grid, dim3(256), 0, st, logits, ld, labels, V, nv, ignore, loss);
}

template <int DT>
void ce_dispatch(int nch, bool grad, dim3 grid, hipStream_t st, void* logits, int64_t ld, const int64_t* labels, int V,
                 const int64_t* nv, int64_t ignore, float* loss) {
  if (grad) {
    if (nch <= 1) ce_launch<DT, true, 1>(grid, st, logits, ld, labels, V, nv, ignore, loss);
    else if (nch <= 2) ce_launch<DT, true, 2>(grid, st, logits, ld, labels, V, nv, ignore, loss);
    else if (nch <= 4) ce_launch<DT, true, 4>(grid, st, logits, ld, labels, V, nv, ignore, loss);
    else if (nch <= 8) ce_launch<DT, true, 8>(grid, st, logits, ld, labels, V, nv, ignore, loss);
    else ce_launch<DT, true, 0>(grid, st, logits, ld, labels, V, nv, ignore, loss);
  } else {
    if (nch <= 8) ce_launch<DT, false, 8>(grid, st, logits, ld, labels, V, nv, ignore, loss);
    else ce_launch<DT, false, 0>(grid, st, logits, ld, labels, V, nv, ignore, loss);
  }
}

int rms_bwd_common(const void* s, const void* w, const float* rstd, const void* dy, void* dx, void* dw, void* ws,
                   size_t ws_bytes, int64_t rows, int dim, int dtype, int wdt) {
  int rc;
  if ((rc = check_dtype(dtype, wdt)) || (rc = check_rows(rows, dim))) return rc;
  if ((rc = check_ptr("weight", w)) || (rc = check_ptr("dweight", dw)) || (rc = check_ptr("workspace", ws))) return rc;
  if (rows > 0) {
    if ((rc = check_ptr("x", s)) || (rc = check_ptr("dy", dy)) || (rc = check_ptr("dx", dx))) return rc;
    if (!rstd) return fail(MT_E_NULL, "rstd is NULL");
  }
  if (ws_bytes < mt_rms_norm_bwd_workspace_size(rows, dim))
    return fail(MT_E_WORKSPACE, "workspace of %zu bytes is smaller than the %zu required", ws_bytes,
                mt_rms_norm_bwd_workspace_size(rows, dim));
  return MT_OK;
}

}  // namespace

namespace {
template <int DT>
void rope_launch(bool vec, dim3 grid, hipStream_t st, const K::RopeArgs& a) {
  if (a.n + 256 < (int64_t(1) << 32)) {
    if (vec) hipLaunchKernelGGL((K::rope_kernel<DT, true, uint32_t>), grid, dim3(256), 0, st, a);
    else hipLaunchKernelGGL((K::rope_kernel<DT, false, uint32_t>), grid, dim3(256), 0, st, a);
  } else {
    if (vec) hipLaunchKernelGGL((K::rope_kernel<DT, true, int64_t>), grid, dim3(256), 0, st, a);
    else hipLaunchKernelGGL((K::rope_kernel<DT, false, int64_t>), grid, dim3(256), 0, st, a);
  }
}
}  // namespace

extern "C" {

int mt_rms_norm_fwd(const void* x, int64_t x_row_stride, const void* weight, void* y, float* rstd, int64_t rows,
                    int dim, float eps, int dtype, int weight_dtype, void* stream) {
  int rc;
  if ((rc = check_dtype(dtype, weight_dtype)) || (rc = check_rows(rows, dim))) return rc;
  if ((rc = check_ptr("weight", weight))) return rc;
  if (rows == 0) return ok();
  if ((rc = check_ptr("x", x)) || (rc = check_ptr("y", y)) || (rc = check_stride("x", x_row_stride, dim))) return rc;
  if (!rstd) return fail(MT_E_NULL, "rstd is NULL");
  const hipError_t e = fwd_dispatch<false>(dtype, weight_dtype, x, x_row_stride, nullptr, 0, weight, nullptr, y, rstd,
                                           rows, dim, eps, (hipStream_t)stream);
  return e == hipSuccess ? ok() : fail((int)e, "launch failed: %s", hipGetErrorString(e));
}

int mt_add_rms_norm_fwd(const void* x, int64_t x_row_stride, const void* residual, int64_t residual_row_stride,
                        const void* weight, void* new_residual, void* y, float* rstd, int64_t rows, int dim,
                        float eps, int dtype, int weight_dtype, void* stream) {
  int rc;
  if ((rc = check_dtype(dtype, weight_dtype)) || (rc = check_rows(rows, dim))) return rc;
  if ((rc = check_ptr("weight", weight))) return rc;
  if (rows == 0) return ok();
  if ((rc = check_ptr("x", x)) || (rc = check_ptr("residual", residual)) || (rc = check_ptr("new_residual", new_residual)) ||
      (rc = check_ptr("y", y)) || (rc = check_stride("x", x_row_stride, dim)) ||
      (rc = check_stride("residual", residual_row_stride, dim)))
    return rc;
  if (!rstd) return fail(MT_E_NULL, "rstd is NULL");
  const hipError_t e = fwd_dispatch<true>(dtype, weight_dtype, x, x_row_stride, residual, residual_row_stride, weight,
                                          new_residual, y, rstd, rows, dim, eps, (hipStream_t)stream);
  return e == hipSuccess ? ok() : fail((int)e, "launch failed: %s", hipGetErrorString(e));
}

size_t mt_rms_norm_bwd_workspace_size(int64_t rows, int dim) {
  if (rows < 0 || dim < 0) return 0;
  return ((size_t)bwd_blocks(rows) * (size_t)dim * sizeof(float) + 255) / 256 * 256;
}

int mt_rms_norm_bwd(const void* x, const void* weight, const float* rstd, const void* dy, void* dx, void* dweight,
                    void* workspace, size_t workspace_bytes, int64_t rows, int dim, int dtype, int weight_dtype,
                    void* stream) {
  const int rc = rms_bwd_common(x, weight, rstd, dy, dx, dweight, workspace, workspace_bytes, rows, dim, dtype,
                                weight_dtype);
  if (rc) return rc;
  const hipError_t e = bwd_dispatch<false>(dtype, weight_dtype, x, weight, rstd, dy, nullptr, dx, dweight,
                                           static_cast<float*>(workspace), rows, dim, (hipStream_t)stream);
  return e == hipSuccess ? ok() : fail((int)e, "launch failed: %s", hipGetErrorString(e));
}

int mt_add_rms_norm_bwd(const void* new_residual, const void* weight, const float* rstd, const void* d_new_residual,
                        const void* dy, void* dx, void* dweight, void* workspace, size_t workspace_bytes,
                        int64_t rows, int dim, int dtype, int weight_dtype, void* stream) {
  int rc = rms_bwd_common(new_residual, weight, rstd, dy, dx, dweight, workspace, workspace_bytes, rows, dim, dtype,
                          weight_dtype);
  if (rc) return rc;
  if (rows > 0 && (rc = check_ptr("d_new_residual", d_new_residual))) return rc;
  const hipError_t e = bwd_dispatch<true>(dtype, weight_dtype, new_residual, weight, rstd, dy, d_new_residual, dx,
                                          dweight, static_cast<float*>(workspace), rows, dim, (hipStream_t)stream);
  return e == hipSuccess ? ok() : fail((int)e, "launch failed: %s", hipGetErrorString(e));
}

int mt_rms_norm_fwd_mixed(const void* x, int64_t x_row_stride, const void* weight, void* y, float* rstd, int64_t rows,
                          int dim, float eps, int y_dtype, int weight_dtype, void* stream) {
  int rc;
  if ((rc = check_mixed(y_dtype, weight_dtype)) || (rc = check_rows(rows, dim))) return rc;
  if ((rc = check_ptr("weight", weight))) return rc;
  if (rows == 0) return ok();
  if ((rc = check_ptr("x", x)) || (rc = check_ptr("y", y)) || (rc = check_stride("x", x_row_stride, dim))) return rc;
  if (!rstd) return fail(MT_E_NULL, "rstd is NULL");
  const int n = chunks(dim);
  hipStream_t st = (hipStream_t)stream;
  const hipError_t e =
      y_dtype == MT_DTYPE_BF16
          ? fwd_mixed<K::kDtBF16, false>(n, x, x_row_stride, nullptr, 0, weight, nullptr, y, rstd, rows, dim, eps, st)
          : fwd_mixed<K::kDtFP16, false>(n, x, x_row_stride, nullptr, 0, weight, nullptr, y, rstd, rows, dim, eps, st);
  return e == hipSuccess ? ok() : fail((int)e, "launch failed: %s", hipGetErrorString(e));
}

int mt_add_rms_norm_fwd_mixed(const void* x, int64_t x_row_stride, const void* residual, int64_t residual_row_stride,
                              const void* weight, void* new_residual, void* y, float* rstd, int64_t rows, int dim,
                              float eps, int act_dtype, int weight_dtype, void* stream) {
  int rc;
  if ((rc = check_mixed(act_dtype, weight_dtype)) || (rc = check_rows(rows, dim))) return rc;
  if ((rc = check_ptr("weight", weight))) return rc;
  if (rows == 0) return ok();
  if ((rc = check_ptr("x", x)) || (rc = check_ptr("residual", residual)) ||
      (rc = check_ptr("new_residual", new_residual)) || (rc = check_ptr("y", y)) ||
      (rc = check_stride("x", x_row_stride, dim)) || (rc = check_stride("residual", residual_row_stride, dim)))
    return rc;
  if (!rstd) return fail(MT_E_NULL, "rstd is NULL");
  const int n = chunks(dim);
  hipStream_t st = (hipStream_t)stream;
  const hipError_t e =
      act_dtype == MT_DTYPE_BF16
          ? fwd_mixed<K::kDtBF16, true>(n, x, x_row_stride, residual, residual_row_stride, weight, new_residual, y,
                                        rstd, rows, dim, eps, st)
          : fwd_mixed<K::kDtFP16, true>(n, x, x_row_stride, residual, residual_row_stride, weight, new_residual, y,
                                        rstd, rows, dim, eps, st);
  return e == hipSuccess ? ok() : fail((int)e, "launch failed: %s", hipGetErrorString(e));
}

int mt_rms_norm_bwd_mixed(const void* s, const void* weight, const float* rstd, const void* d_new_residual,
                          const void* dy, void* ds, void* ds16, void* dweight, void* workspace, size_t workspace_bytes,
                          int64_t rows, int dim, int act_dtype, int weight_dtype, void* stream) {
  int rc;
  if ((rc = check_mixed(act_dtype, weight_dtype)) || (rc = check_rows(rows, dim))) return rc;
  if ((rc = check_ptr("weight", weight)) || (rc = check_ptr("dweight", dweight)) ||
      (rc = check_ptr("workspace", workspace)))
    return rc;
  if (rows > 0) {
    if ((rc = check_ptr("s", s)) || (rc = check_ptr("dy", dy)) || (rc = check_ptr("ds", ds))) return rc;
    if (d_new_residual && (rc = check_ptr("d_new_residual", d_new_residual))) return rc;
    if (ds16 && (rc = check_ptr("ds16", ds16))) return rc;
    if (!rstd) return fail(MT_E_NULL, "rstd is NULL");
  }
  if (workspace_bytes < mt_rms_norm_bwd_workspace_size(rows, dim))
    return fail(MT_E_WORKSPACE, "workspace of %zu bytes is smaller than the %zu required", workspace_bytes,
                mt_rms_norm_bwd_workspace_size(rows, dim));
  const int n = chunks(dim);
  hipStream_t st = (hipStream_t)stream;
  float* part = static_cast<float*>(workspace);
  hipError_t e;
  if (act_dtype == MT_DTYPE_BF16)
    e = d_new_residual
            ? bwd_mixed<K::kDtBF16, true>(n, s, weight, rstd, dy, d_new_residual, ds, ds16, dweight, part, rows, dim, st)
            : bwd_mixed<K::kDtBF16, false>(n, s, weight, rstd, dy, nullptr, ds, ds16, dweight, part, rows, dim, st);
  else
    e = d_new_residual
            ? bwd_mixed<K::kDtFP16, true>(n, s, weight, rstd, dy, d_new_residual, ds, ds16, dweight, part, rows, dim, st)
            : bwd_mixed<K::kDtFP16, false>(n, s, weight, rstd, dy, nullptr, ds, ds16, dweight, part, rows, dim, st);
  return e == hipSuccess ? ok() : fail((int)e, "launch failed: %s", hipGetErrorString(e));
}

int mt_swiglu_fwd(const void* gate, const void* up, void* out, int64_t n, int dtype, void* stream) {
  int rc;
  if ((rc = check_dtype(dtype, dtype))) return rc;
  if (n < 0) return fail(MT_E_SHAPE, "n must be >= 0 (got %lld)", (long long)n);
  if (n == 0) return ok();
  if ((rc = check_ptr("gate", gate)) || (rc = check_ptr("up", up)) || (rc = check_ptr("out", out))) return rc;
  hipStream_t st = (hipStream_t)stream;
  const dim3 grid(swiglu_blocks(n));
  if (dtype == MT_DTYPE_BF16) hipLaunchKernelGGL((K::swiglu_fwd_kernel<K::kDtBF16>), grid, dim3(256), 0, st, gate, up, out, n);
  else if (dtype == MT_DTYPE_FP16) hipLaunchKernelGGL((K::swiglu_fwd_kernel<K::kDtFP16>), grid, dim3(256), 0, st, gate, up, out, n);
  else hipLaunchKernelGGL((K::swiglu_fwd_kernel<K::kDtFP32>), grid, dim3(256), 0, st, gate, up, out, n);
  const hipError_t e = hipGetLastError();
  return e == hipSuccess ? ok() : fail((int)e, "launch failed: %s", hipGetErrorString(e));
}

int mt_swiglu_bwd(const void* gate, const void* up, const void* dout, void* dgate, void* dup, int64_t n, int dtype,
                  void* stream) {
  int rc;
  if ((rc = check_dtype(dtype, dtype))) return rc;
  if (n < 0) return fail(MT_E_SHAPE, "n must be >= 0 (got %lld)", (long long)n);
  if (n == 0) return ok();
  if ((rc = check_ptr("gate", gate)) || (rc = check_ptr("up", up)) || (rc = check_ptr("dout", dout)) ||
      (rc = check_ptr("dgate", dgate)) || (rc = check_ptr("dup", dup)))
    return rc;
  hipStream_t st = (hipStream_t)stream;
  const dim3 grid(swiglu_blocks(n));
  if (dtype == MT_DTYPE_BF16)
    hipLaunchKernelGGL((K::swiglu_bwd_kernel<K::kDtBF16>), grid, dim3(256), 0, st, gate, up, dout, dgate, dup, n);
  else if (dtype == MT_DTYPE_FP16)
    hipLaunchKernelGGL((K::swiglu_bwd_kernel<K::kDtFP16>), grid, dim3(256), 0, st, gate, up, dout, dgate, dup, n);
  else
    hipLaunchKernelGGL((K::swiglu_bwd_kernel<K::kDtFP32>), grid, dim3(256), 0, st, gate, up, dout, dgate, dup, n);
  const hipError_t e = hipGetLastError();
  return e == hipSuccess ? ok() : fail((int)e, "launch failed: %s", hipGetErrorString(e));
}

namespace {
int check_packed(int64_t rows, int64_t cols) {
  if (rows < 0 || cols < 0 || cols % 8)
    return fail(MT_E_SHAPE, "rows %lld and cols %lld must be >= 0 with cols a multiple of 8", (long long)rows,
                (long long)cols);
  if (rows * (cols / 8) >= (int64_t(1) << 31))
    return fail(MT_E_SHAPE, "rows * cols / 8 must be below 2^31 (got %lld)", (long long)(rows * (cols / 8)));
  return MT_OK;
}
}  // namespace

int mt_swiglu_packed_fwd(const void* gu, void* out, int64_t rows, int64_t cols, int dtype, void* stream) {
  int rc;
  if ((rc = check_dtype(dtype, dtype)) || (rc = check_packed(rows, cols))) return rc;
  if (rows == 0 || cols == 0) return ok();
  if ((rc = check_ptr("gu", gu)) || (rc = check_ptr("out", out))) return rc;
  hipStream_t st = (hipStream_t)stream;
  const int r = (int)rows, cpr = (int)(cols / 8);
  const dim3 grid(swiglu_blocks(rows * cols));
  if (dtype == MT_DTYPE_BF16) hipLaunchKernelGGL((K::swiglu_packed_fwd_kernel<K::kDtBF16>), grid, dim3(256), 0, st, gu, out, r, cpr);
  else if (dtype == MT_DTYPE_FP16) hipLaunchKernelGGL((K::swiglu_packed_fwd_kernel<K::kDtFP16>), grid, dim3(256), 0, st, gu, out, r, cpr);
  else hipLaunchKernelGGL((K::swiglu_packed_fwd_kernel<K::kDtFP32>), grid, dim3(256), 0, st, gu, out, r, cpr);
  const hipError_t e = hipGetLastError();
  return e == hipSuccess ? ok() : fail((int)e, "launch failed: %s", hipGetErrorString(e));
}

int mt_swiglu_packed_bwd(const void* gu, const void* dout, void* dgu, int64_t rows, int64_t cols, int dtype,
                         void* stream) {
  int rc;
  if ((rc = check_dtype(dtype, dtype)) || (rc = check_packed(rows, cols))) return rc;
  if (rows == 0 || cols == 0) return ok();
  if ((rc = check_ptr("gu", gu)) || (rc = check_ptr("dout", dout)) || (rc = check_ptr("dgu", dgu))) return rc;
  hipStream_t st = (hipStream_t)stream;
  const int r = (int)rows, cpr = (int)(cols / 8);
  const dim3 grid(swiglu_blocks(rows * cols));
  if (dtype == MT_DTYPE_BF16)
    hipLaunchKernelGGL((K::swiglu_packed_bwd_kernel<K::kDtBF16>), grid, dim3(256), 0, st, gu, dout, dgu, r, cpr);
  else if (dtype == MT_DTYPE_FP16)
    hipLaunchKernelGGL((K::swiglu_packed_bwd_kernel<K::kDtFP16>), grid, dim3(256), 0, st, gu, dout, dgu, r, cpr);
  else
    hipLaunchKernelGGL((K::swiglu_packed_bwd_kernel<K::kDtFP32>), grid, dim3(256), 0, st, gu, dout, dgu, r, cpr);
  const hipError_t e = hipGetLastError();
  return e == hipSuccess ? ok() : fail((int)e, "launch failed: %s", hipGetErrorString(e));
}

int mt_cross_entropy_rows(void* logits, int64_t row_stride, const int64_t* labels, int64_t rows, int vocab,
                          const int64_t* n_valid, int64_t ignore_index, float* loss_rows, int write_grad, int dtype,
                          void* stream) {
  int rc;
  if ((rc = check_dtype(dtype, dtype))) return rc;
  if (rows < 0 || rows > 0x7fffffffLL) return fail(MT_E_SHAPE, "rows must be in [0, 2^31) (got %lld)", (long long)rows);
  if (vocab < 1) return fail(MT_E_SHAPE, "vocab %d unsupported (positive)", vocab);
  if (rows == 0) return ok();
  // the row's last 8-value chunk may reach into the padding up to vocab rounded up to 8
  if ((rc = check_ptr("logits", logits)) || (rc = check_stride("logits", row_stride, (vocab + 7) / 8 * 8))) return rc;
  if (!labels || !n_valid || !loss_rows) return fail(MT_E_NULL, "labels, n_valid and loss_rows must be non-NULL");
  hipStream_t st = (hipStream_t)stream;
  const dim3 grid((unsigned)rows);
  const int nch = ((vocab + 7) / 8 + 255) / 256;  // 8-value chunks per thread
  if (dtype == MT_DTYPE_BF16) ce_dispatch<K::kDtBF16>(nch, write_grad != 0, grid, st, logits, row_stride, labels, vocab, n_valid, ignore_index, loss_rows);
  else if (dtype == MT_DTYPE_FP16) ce_dispatch<K::kDtFP16>(nch, write_grad != 0, grid, st, logits, row_stride, labels, vocab, n_valid, ignore_index, loss_rows);
  else ce_dispatch<K::kDtFP32>(nch, write_grad != 0, grid, st, logits, row_stride, labels, vocab, n_valid, ignore_index, loss_rows);
  const hipError_t e = hipGetLastError();
  return e == hipSuccess ? ok() : fail((int)e, "launch failed: %s", hipGetErrorString(e));
}

int mt_apply_rope(const void* q, const void* k, void* q_out, void* k_out, int B, int Hq, int Hkv, int T, int D,
                  const int64_t* strides, const float* rope_cos, const float* rope_sin, int64_t table_stride,
                  int table_rows, int inverse, int dtype, void* stream) {
  int rc;
  if ((rc = check_dtype(dtype, dtype))) return rc;
  if (B < 0 || Hq < 0 || Hkv < 0 || T < 0)
    return fail(MT_E_SHAPE, "B, Hq, Hkv and T must be >= 0 (got %d, %d, %d, %d)", B, Hq, Hkv, T);
  if (D < 2 || D % 2) return fail(MT_E_SHAPE, "RoPE requires an even head dimension (got %d)", D);
  if (table_rows < T) return fail(MT_E_ROPE, "RoPE tables have %d rows, fewer than T = %d", table_rows, T);
  if (table_stride < D / 2) return fail(MT_E_ROPE, "RoPE table row stride %lld below D / 2 = %d",
                                        (long long)table_stride, D / 2);
  const int64_t rows_q = (int64_t)B * Hq * T, rows_k = (int64_t)B * Hkv * T;
  if (rows_q + rows_k == 0) return ok();
  if (!strides || !rope_cos || !rope_sin) return fail(MT_E_NULL, "strides, rope_cos and rope_sin must be non-NULL");
  if ((rows_q && (!q || !q_out)) || (rows_k && (!k || !k_out))) return fail(MT_E_NULL, "q, k, q_out and k_out must be non-NULL");
  K::RopeArgs a;
  a.src[0] = q;
  a.src[1] = k;
  a.dst[0] = q_out;
  a.dst[1] = k_out;
  bool vec = D % 8 == 0 && aligned16(rope_cos) && aligned16(rope_sin) && table_stride % 4 == 0;
  for (int w = 0; w < 2; ++w)
    for (int j = 0; j < 4; ++j) {
      a.ss[w][j] = strides[8 * w + j];
      a.sd[w][j] = strides[8 * w + 4 + j];
    }
  for (int w = 0; w < 2; ++w) {
    if (w == 0 ? rows_q == 0 : rows_k == 0) continue;
    vec = vec && a.ss[w][3] == 1 && a.sd[w][3] == 1 && aligned16(a.src[w]) && aligned16(a.dst[w]);
    for (int j = 0; j < 3; ++j) vec = vec && a.ss[w][j] % 8 == 0 && a.sd[w][j] % 8 == 0;
  }
  a.heads[0] = Hq > 0 ? Hq : 1;
  a.heads[1] = Hkv > 0 ? Hkv : 1;
  a.T = T;
  a.half = D / 2;
  a.cos = rope_cos;
  a.sin = rope_sin;
  a.tstride = table_stride;
  a.sign = inverse ? -1.f : 1.f;
  const int per_row = vec ? D / 8 : D / 2;
  a.n0 = rows_q * per_row;
  a.n = a.n0 + rows_k * per_row;
  const int64_t blocks = (a.n + 255) / 256;
  if (blocks > 0x7fffffffLL) return fail(MT_E_SHAPE, "too many pairs (%lld)", (long long)(a.n));
  hipStream_t st = (hipStream_t)stream;
  const dim3 grid((unsigned)blocks);
  if (dtype == MT_DTYPE_BF16) rope_launch<K::kDtBF16>(vec, grid, st, a);
  else if (dtype == MT_DTYPE_FP16) rope_launch<K::kDtFP16>(vec, grid, st, a);
  else rope_launch<K::kDtFP32>(vec, grid, st, a);
  const hipError_t e = hipGetLastError();
  return e == hipSuccess ? ok() : fail((int)e, "launch failed: %s", hipGetErrorString(e));
}

int mt_linear_rows(const void* x, int64_t x_row_stride, const void* const* weights, const int* out_features,
                   const int64_t* w_row_strides, int groups, void* y, int64_t y_row_stride, int rows, int in_features,
                   int dtype, void* stream) {
  if (dtype != MT_DTYPE_FP32 && dtype != MT_DTYPE_BF16 && dtype != MT_DTYPE_FP16)
    return fail(MT_E_DTYPE, "x dtype code %d unsupported", dtype);
  if (groups < 1 || groups > mt::kLinGroups)
    return fail(MT_E_SHAPE, "groups must be in [1, %d] (got %d)", mt::kLinGroups, groups);
  if (rows < 1 || rows > mt::kLinMaxRows)
    return fail(MT_E_SHAPE, "rows must be in [1, %d] (got %d)", mt::kLinMaxRows, rows);
  if (in_features < 128 || in_features % 128)
    return fail(MT_E_SHAPE, "in_features must be a positive multiple of 128 (got %d)", in_features);
  if (!weights || !out_features || !w_row_strides) return fail(MT_E_NULL, "weights, out_features or w_row_strides is NULL");
  int rc;
  if (!x) return fail(MT_E_NULL, "x is NULL");
  if (reinterpret_cast<uintptr_t>(x) % (dtype == MT_DTYPE_FP32 ? 16 : 8))
    return fail(MT_E_STRIDE, "x must be %d-byte aligned", dtype == MT_DTYPE_FP32 ? 16 : 8);
  if (!y) return fail(MT_E_NULL, "y is NULL");
  if (x_row_stride < in_features || x_row_stride % 4)
    return fail(MT_E_STRIDE, "x row stride %lld must be >= in_features and a multiple of 4", (long long)x_row_stride);
  mt::LinearParams p{};
  p.x = x;
  p.y = static_cast<float*>(y);
  p.ldx = x_row_stride;
  p.ldy = y_row_stride;
  p.M = rows;
  p.K = in_features;
  p.groups = groups;
  int64_t cols = 0, tiles = 0;
  for (int g = 0; g < groups; ++g) {
    if ((rc = check_ptr("weights[g]", weights[g]))) return rc;
    if (out_features[g] < 1) return fail(MT_E_SHAPE, "out_features[%d] must be >= 1 (got %d)", g, out_features[g]);
    if (w_row_strides[g] < in_features || w_row_strides[g] % 4)
      return fail(MT_E_STRIDE, "weight %d row stride %lld must be >= in_features and a multiple of 4", g,
                  (long long)w_row_strides[g]);
    p.g[g].w = static_cast<const float*>(weights[g]);
    p.g[g].ldw = w_row_strides[g];
    p.g[g].n = out_features[g];
    p.g[g].col_off = (int)cols;
    p.g[g].tile0 = (int)tiles;
    cols += out_features[g];
    tiles += (out_features[g] + mt::kLinCols - 1) / mt::kLinCols;
  }
  if (cols > 0x7fffffffLL) return fail(MT_E_SHAPE, "too many output columns (%lld)", (long long)cols);
  if (y_row_stride < cols) return fail(MT_E_STRIDE, "y row stride %lld must be >= %lld", (long long)y_row_stride,
                                       (long long)cols);
  if (tiles * ((rows + 15) / 16) > 0x7fffffffLL) return fail(MT_E_SHAPE, "too many output tiles");
  hipStream_t st = (hipStream_t)stream;
  const dim3 grid((unsigned)(tiles * ((rows + 15) / 16))), block(64 * mt::kLinWaves);
  // every chunk of a lane in flight at once up to K = 1536 (12 chunks of 4 values per lane)
#define MT_LINEAR(XT)                                                                                        \
  if (in_features <= 128 * 12) hipLaunchKernelGGL((mt::linear_rows_f32_kernel<12, XT>), grid, block, 0, st, p); \
  else hipLaunchKernelGGL((mt::linear_rows_f32_kernel<4, XT>), grid, block, 0, st, p)
  if (dtype == MT_DTYPE_FP32) { MT_LINEAR(float); }
  else if (dtype == MT_DTYPE_BF16) { MT_LINEAR(mt::BF16); }
  else { MT_LINEAR(mt::FP16); }
#undef MT_LINEAR
  const hipError_t e = hipGetLastError();
  return e == hipSuccess ? ok() : fail((int)e, "launch failed: %s", hipGetErrorString(e));
}

int mt_topk_sample(const void* logits, int64_t row_stride, const void* noise, int64_t noise_row_stride, int rows,
                   int vocab, int k, int64_t* tokens, int dtype, void* stream) {
  if (dtype != MT_DTYPE_FP32) return fail(MT_E_DTYPE, "dtype code %d unsupported (fp32 only)", dtype);
  if (rows < 0) return fail(MT_E_SHAPE, "rows must be >= 0 (got %d)", rows);
  if (vocab < 1 || vocab > 32 * mt::kSampleThreads)
    return fail(MT_E_SHAPE, "vocab must be in [1, %d] (got %d)", 32 * mt::kSampleThreads, vocab);
  if (k < 1 || k > vocab) return fail(MT_E_SHAPE, "k must be in [1, vocab] (got %d)", k);
  if (row_stride < vocab || noise_row_stride < vocab)
    return fail(MT_E_STRIDE, "row strides (%lld, %lld) must be >= vocab", (long long)row_stride,
                (long long)noise_row_stride);
  if (rows == 0) return ok();
  if (!logits || !noise || !tokens) return fail(MT_E_NULL, "logits, noise or tokens is NULL");
  hipStream_t st = (hipStream_t)stream;
  const dim3 grid((unsigned)rows), block(mt::kSampleThreads);
  const float* x = static_cast<const float*>(logits);
  const float* e = static_cast<const float*>(noise);
  if (vocab <= 8 * mt::kSampleThreads)
    hipLaunchKernelGGL((mt::topk_sample_kernel<8>), grid, block, 0, st, x, row_stride, e, noise_row_stride, vocab, k, tokens);
  else if (vocab <= 16 * mt::kSampleThreads)
    hipLaunchKernelGGL((mt::topk_sample_kernel<16>), grid, block, 0, st, x, row_stride, e, noise_row_stride, vocab, k, tokens);
  else
    hipLaunchKernelGGL((mt::topk_sample_kernel<32>), grid, block, 0, st, x, row_stride, e, noise_row_stride, vocab, k, tokens);
  const hipError_t err = hipGetLastError();
  return err == hipSuccess ? ok() : fail((int)err, "launch failed: %s", hipGetErrorString(err));
}

}  // extern "C"
