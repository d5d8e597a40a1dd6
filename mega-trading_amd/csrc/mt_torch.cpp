// GPU kernels of the mega_trading_amd attention ops for PyTorch-ROCm.
//
// The op schemas, their fake (shape) implementations and their autograd are
// declared from Python (mega-trading_amd/attention.py); this library only
// registers what runs for ROCm tensors: argument preparation, output
// allocation through the caching allocator, the current HIP stream, and one
// call into the C ABI of libmt_attn.so (include/mt_attention.h).  Keeping that
// in C++ removes the Python dispatch work that bounds small shapes.
//
// The layout rules are those of the Python launchers they replace: a tensor is
// used in place when its last stride is 1, its outer strides are multiples of
// 8 elements and its base is 16-byte aligned, and is made contiguous
// otherwise.  Errors from the C ABI are raised as RuntimeError with
// mt_last_error()'s message.
#include <ATen/ATen.h>
#include <c10/core/DeviceGuard.h>
#include <c10/hip/HIPStream.h>
#include <torch/library.h>

#include <array>
#include <optional>
#include <tuple>

#include "../../include/mt_attention.h"

namespace {

bool kernel_ready(const at::Tensor& t) {
  if (t.dim() == 0 || t.stride(-1) != 1 || reinterpret_cast<uintptr_t>(t.data_ptr()) % 16) return false;
  for (int64_t i = 0; i + 1 < t.dim(); ++i)
    if (t.size(i) > 1 && t.stride(i) % 8) return false;
  return true;
}

at::Tensor ready(const at::Tensor& t) { return kernel_ready(t) ? t : t.contiguous(); }

// (b, h, t, d) element strides; size-1 dims report 0 (their stride is never used)
void put_strides(int64_t* dst, const at::Tensor& t) {
  for (int i = 0; i < 4; ++i) dst[i] = t.size(i) > 1 ? t.stride(i) : 0;
}

int dtype_code(const at::Tensor& t) {
  if (t.scalar_type() == at::kBFloat16) return MT_DTYPE_BF16;
  if (t.scalar_type() == at::kHalf) return MT_DTYPE_FP16;
  if (t.scalar_type() == at::kFloat) return MT_DTYPE_FP32;
  TORCH_CHECK(false, "hip attention kernels take bfloat16, float16 or float32 tensors (got ", t.scalar_type(), ")");
}

void check_rc(int rc, const char* what) {
  TORCH_CHECK(rc == 0, what, " failed (code ", rc, "): ", mt_last_error());
}

hipStream_t stream_of(const at::Tensor& t) { return c10::hip::getCurrentHIPStream(t.device().index()).stream(); }

const void* ptr_or_null(const std::optional<at::Tensor>& t) {
  return t.has_value() && t->defined() ? t->data_ptr() : nullptr;
}

// Forward: (out, lse, q_rot, k_rot).  `out_view`, when defined, is the output
// to write (any kernel-ready strides); q_rot / k_rot are empty without RoPE.
std::tuple<at::Tensor, at::Tensor, at::Tensor, at::Tensor> forward(
    const at::Tensor& q_in, const at::Tensor& k_in, const at::Tensor& v_in, const std::optional<at::Tensor>& cos,
    const std::optional<at::Tensor>& sin, double scale, at::Tensor out) {
  TORCH_CHECK(q_in.dim() == 4 && k_in.dim() == 4 && v_in.dim() == 4, "q, k, v must be [B, H, T, D]");
  const c10::DeviceGuard guard(q_in.device());
  const at::Tensor q = ready(q_in), k = ready(k_in), v = ready(v_in);
  const int64_t b = q.size(0), hq = q.size(1), t = q.size(2), d = q.size(3), hkv = k.size(1);
  // the returned output has the query's strides (empty_like of the caller's
  // q, as the reference allocates it); when those are not kernel-ready the
  // kernel writes a contiguous buffer that is copied into it afterwards
  at::Tensor result = out.defined() ? out : at::empty_like(q_in);
  out = ready(result);
  const at::Tensor lse = at::empty({b, hq, t}, q.options().dtype(at::kFloat));
  const bool rope = cos.has_value() && cos->defined();
  at::Tensor q_rot, k_rot;
  if (rope) {
    q_rot = at::empty({b, hq, t, d}, q.options());
    k_rot = at::empty({b, hkv, t, d}, q.options());
  } else {
    q_rot = at::empty({0}, q.options());
    k_rot = at::empty({0}, q.options());
  }
  std::array<int64_t, 16> s{};
  put_strides(s.data(), q);
  put_strides(s.data() + 4, k);
  put_strides(s.data() + 8, v);
  put_strides(s.data() + 12, out);
  check_rc(mt_gqa_attn_fwd(q.data_ptr(), k.data_ptr(), v.data_ptr(), out.data_ptr(), lse.data_ptr<float>(),
                           rope ? q_rot.data_ptr() : nullptr, rope ? k_rot.data_ptr() : nullptr, int(b), int(hq),
                           int(hkv), int(t), int(d), s.data(), float(scale), dtype_code(q),
                           static_cast<const float*>(ptr_or_null(cos)), static_cast<const float*>(ptr_or_null(sin)),
                           stream_of(q)),
           "mt_gqa_attn_fwd");
  if (!result.is_same(out)) result.copy_(out);
  return {result, lse, q_rot, k_rot};
}

// Backward into the given dq / dk / dv (shapes of q / k / v, kernel-ready strides).
void backward(const at::Tensor& q_in, const at::Tensor& k_in, const at::Tensor& v_in, const at::Tensor& o_in,
              const at::Tensor& lse_in, const at::Tensor& dout_in, const std::optional<at::Tensor>& cos,
              const std::optional<at::Tensor>& sin, double scale, const at::Tensor& dq, const at::Tensor& dk,
              const at::Tensor& dv) {
  const c10::DeviceGuard guard(q_in.device());
  const at::Tensor q = ready(q_in), k = ready(k_in), v = ready(v_in), o = ready(o_in);
  const at::Tensor dout = ready(dout_in.scalar_type() == q.scalar_type() ? dout_in : dout_in.to(q.scalar_type()));
  const at::Tensor lse = lse_in.contiguous();
  const int64_t b = q.size(0), hq = q.size(1), t = q.size(2), d = q.size(3), hkv = k.size(1);
  std::array<int64_t, 32> s{};
  const at::Tensor* ts[8] = {&q, &k, &v, &o, &dout, &dq, &dk, &dv};
  for (int i = 0; i < 8; ++i) put_strides(s.data() + 4 * i, *ts[i]);
  const size_t ws_bytes = mt_gqa_attn_bwd_workspace_size_dtype(int(b), int(hq), int(hkv), int(t), int(d), dtype_code(q));
  const at::Tensor ws = at::empty({int64_t(ws_bytes)}, q.options().dtype(at::kByte));
  check_rc(mt_gqa_attn_bwd(q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(), lse.data_ptr<float>(),
                           dout.data_ptr(), dq.data_ptr(), dk.data_ptr(), dv.data_ptr(), ws.data_ptr(), ws_bytes,
                           int(b), int(hq), int(hkv), int(t), int(d), s.data(), float(scale), dtype_code(q),
                           static_cast<const float*>(ptr_or_null(cos)), static_cast<const float*>(ptr_or_null(sin)),
                           stream_of(q)),
           "mt_gqa_attn_bwd");
}

// [B, H, T, D] views of the query, key and value heads of a packed [B, T, (Hq + 2 Hkv) D] tensor
std::array<at::Tensor, 3> packed_views(const at::Tensor& qkv, int64_t hq, int64_t hkv) {
  const int64_t b = qkv.size(0), t = qkv.size(1), d = qkv.size(2) / (hq + 2 * hkv);
  return {qkv.narrow(2, 0, hq * d).view({b, t, hq, d}).transpose(1, 2),
          qkv.narrow(2, hq * d, hkv * d).view({b, t, hkv, d}).transpose(1, 2),
          qkv.narrow(2, (hq + hkv) * d, hkv * d).view({b, t, hkv, d}).transpose(1, 2)};
}

// --- the op kernels (schemas in attention.py) -------------------------------

std::tuple<at::Tensor, at::Tensor> gqa_attn_fwd(const at::Tensor& q, const at::Tensor& k, const at::Tensor& v,
                                                double scale) {
  auto r = forward(q, k, v, std::nullopt, std::nullopt, scale, at::Tensor());
  return {std::get<0>(r), std::get<1>(r)};
}

std::tuple<at::Tensor, at::Tensor, at::Tensor, at::Tensor> gqa_rope_attn_fwd(const at::Tensor& q, const at::Tensor& k,
                                                                             const at::Tensor& v, const at::Tensor& cos,
                                                                             const at::Tensor& sin, double scale) {
  return forward(q, k, v, cos, sin, scale, at::Tensor());
}

std::tuple<at::Tensor, at::Tensor, at::Tensor> gqa_attn_bwd(const at::Tensor& q, const at::Tensor& k,
                                                            const at::Tensor& v, const at::Tensor& o,
                                                            const at::Tensor& lse, const at::Tensor& dout,
                                                            const std::optional<at::Tensor>& cos,
                                                            const std::optional<at::Tensor>& sin, double scale) {
  const at::Tensor dq = at::empty(q.sizes(), q.options());
  const at::Tensor dk = at::empty(k.sizes(), k.options());
  const at::Tensor dv = at::empty(v.sizes(), v.options());
  backward(q, k, v, o, lse, dout, cos, sin, scale, dq, dk, dv);
  return {dq, dk, dv};
}

std::tuple<at::Tensor, at::Tensor, at::Tensor, at::Tensor> gqa_rope_attn_packed_fwd(const at::Tensor& qkv,
                                                                                    const at::Tensor& cos,
                                                                                    const at::Tensor& sin, int64_t hq,
                                                                                    int64_t hkv, double scale) {
  TORCH_CHECK(qkv.dim() == 3, "qkv must be [B, T, (Hq + 2 Hkv) D]");
  const auto views = packed_views(qkv, hq, hkv);
  const int64_t b = qkv.size(0), t = qkv.size(1), d = views[0].size(3);
  const at::Tensor out = at::empty({b, t, hq, d}, qkv.options());
  auto r = forward(views[0], views[1], views[2], cos, sin, scale, out.transpose(1, 2));
  return {out.view({b, t, hq * d}), std::get<1>(r), std::get<2>(r), std::get<3>(r)};
}

at::Tensor gqa_attn_bwd_packed(const at::Tensor& q_rot, const at::Tensor& k_rot, const at::Tensor& qkv,
                               const at::Tensor& out, const at::Tensor& lse, const at::Tensor& dout,
                               const at::Tensor& cos, const at::Tensor& sin, int64_t hq, int64_t hkv, double scale) {
  const auto views = packed_views(qkv, hq, hkv);
  const int64_t b = qkv.size(0), t = qkv.size(1), d = views[2].size(3);
  const at::Tensor dqkv = at::empty(qkv.sizes(), qkv.options());
  const auto grads = packed_views(dqkv, hq, hkv);
  const at::Tensor o = out.view({b, t, hq, d}).transpose(1, 2);
  const at::Tensor dov = dout.reshape({b, t, hq, d}).transpose(1, 2);
  backward(q_rot, k_rot, views[2], o, lse, dov, cos, sin, scale, grads[0], grads[1], grads[2]);
  return dqkv;
}

}  // namespace

TORCH_LIBRARY_IMPL(mega_trading_amd, CUDA, m) {
  m.impl("gqa_attn_fwd", &gqa_attn_fwd);
  m.impl("gqa_rope_attn_fwd", &gqa_rope_attn_fwd);
  m.impl("gqa_attn_bwd", &gqa_attn_bwd);
  m.impl("gqa_rope_attn_packed_fwd", &gqa_rope_attn_packed_fwd);
  m.impl("gqa_attn_bwd_packed", &gqa_attn_bwd_packed);
}
