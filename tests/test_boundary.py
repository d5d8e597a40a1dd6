"""CPU tests of the drop-in boundary: the C ABI library and the Python operator.

No compute call is made here.  The C ABI checks run on arguments that fail
validation before any launch; the Python checks run under FakeTensorMode,
which yields "cuda" tensors without a GPU.
"""

from __future__ import annotations

import ctypes
import os
import re

import pytest
import torch
from torch._subclasses.fake_tensor import FakeTensorMode

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADERS = [os.path.join(ROOT, "include", h) for h in ("mt_attention.h", "mt_ops.h")]


def _header_functions() -> list[str]:
    text = "\n".join(open(h).read() for h in HEADERS)
    return sorted(set(re.findall(r"^\s*(?:int|size_t|const char\*)\s+(mt_\w+)\s*\(", text, flags=re.M)))


def test_library_exports_every_declared_symbol(mta):
    lib = mta._native.load()
    declared = _header_functions()
    assert declared == sorted(mta._native.EXPORTS)
    for name in declared:
        assert hasattr(lib, name), f"{name} declared in include/mt_attention.h but not exported"
    assert lib.mt_version() == (0 << 16) | 5


def test_noalloc_backward_rejects_shapes_beyond_its_scratch(mta):
    """mt_gqa_attn_bwd_noalloc: a shape whose delta / LSE vectors alone exceed
    the fixed 64 MiB scratch fails with MT_E_WORKSPACE before any device call
    (the pointers are never dereferenced)."""
    lib = mta._native.load()
    p = 0x10000
    s = (ctypes.c_int64 * 32)(*([0, 0, 64, 1] * 8))
    # 8 * B * Hq * T bytes of vectors: B=64, Hq=64, T=4096 -> 128 MiB
    rc = lib.mt_gqa_attn_bwd_noalloc(p, p, p, p, p, p, p, p, p, 64, 64, 16, 4096, 64, s, 0.125, 0, None, None, None)
    assert rc == -6
    assert b"at most 67108864" in lib.mt_last_error()
    # shape errors keep their own codes
    assert lib.mt_gqa_attn_bwd_noalloc(p, p, p, p, p, p, p, p, p, 1, 6, 4, 16, 64, s, 0.125, 0, None, None, None) == -2
    assert lib.mt_gqa_attn_bwd_noalloc(p, p, p, p, p, p, p, p, p, 1, 4, 2, 16, 48, s, 0.125, 0, None, None, None) == -2


def test_probe_library_exports_the_mfma_probe():
    # bench.py's sustained-MFMA probe lives in its own library, outside the attention ABI
    path = os.path.join(ROOT, "mega-trading_amd", "libmt_probe.so")
    assert os.path.exists(path), "run mega-trading_amd/build_lib.py"
    lib = ctypes.CDLL(path)
    assert hasattr(lib, "mt_probe_mfma")
    assert b"gfx950" in open(path, "rb").read()


def test_library_is_gfx950_only(mta):
    data = open(mta._native.library_path(), "rb").read()
    assert b"gfx950" in data
    for other in (b"gfx942", b"gfx90a", b"gfx1100", b"sm_"):
        assert b"amdgcn-amd-amdhsa--" + other not in data


def _fwd_call(lib, q=0x1000, k=0x1000, v=0x1000, o=0x1000, lse=0x1000, b=1, hq=4, hkv=2, t=16, d=64,
              strides=None, dtype=0, cos=None, sin=None, qrot=None, krot=None):
    if strides is None:
        strides = [hq * t * d, t * d, d, 1, hkv * t * d, t * d, d, 1, hkv * t * d, t * d, d, 1, hq * t * d, t * d, d, 1]
    arr = (ctypes.c_int64 * 16)(*strides)
    return lib.mt_gqa_attn_fwd(q, k, v, o, lse, qrot, krot, b, hq, hkv, t, d, arr, 0.125, dtype, cos, sin, None)


def test_ops_c_abi_rejects_bad_arguments_before_launch(mta):
    lib = mta._native.load()
    p = 0x10000  # aligned, never dereferenced: every call below fails validation first
    BF16, FP32 = mta._native.DTYPE_BF16, mta._native.DTYPE_FP32
    assert lib.mt_rms_norm_fwd(p, 16, p, p, p, 4, 12, 1e-5, FP32, FP32, None) == -2  # dim not a multiple of 8
    assert b"dim 12" in lib.mt_last_error()
    assert lib.mt_rms_norm_fwd(p, 8192, p, p, p, 4, 8192, 1e-5, FP32, FP32, None) == -2  # dim > 4096
    assert lib.mt_rms_norm_fwd(p, 16, p, p, p, 4, 16, 1e-5, 7, FP32, None) == -4
    assert lib.mt_rms_norm_fwd(p, 16, p, p, p, 4, 16, 1e-5, BF16, mta._native.DTYPE_FP16, None) == -4
    assert lib.mt_rms_norm_fwd(p + 2, 16, p, p, p, 4, 16, 1e-5, FP32, FP32, None) == -3  # misaligned x
    assert lib.mt_rms_norm_fwd(p, 12, p, p, p, 4, 16, 1e-5, FP32, FP32, None) == -3  # row stride < dim
    assert lib.mt_rms_norm_fwd(p, 16, None, p, p, 4, 16, 1e-5, FP32, FP32, None) == -1
    assert lib.mt_rms_norm_fwd(p, 16, p, p, p, 0, 16, 1e-5, FP32, FP32, None) == 0  # zero rows: nothing to do
    need = lib.mt_rms_norm_bwd_workspace_size(1000, 512)
    assert need >= 512 * 4 and need % 256 == 0
    assert lib.mt_rms_norm_bwd(p, p, p, p, p, p, p, need - 1, 1000, 512, FP32, FP32, None) == -6
    assert b"workspace" in lib.mt_last_error()
    assert lib.mt_add_rms_norm_fwd(p, 16, p, 8, p, p, p, p, 4, 16, 1e-5, FP32, FP32, None) == -3  # residual stride
    assert lib.mt_swiglu_fwd(p, p, p, -1, BF16, None) == -2
    assert lib.mt_swiglu_fwd(p, p + 8, p, 100, BF16, None) == -3
    assert lib.mt_swiglu_bwd(p, p, None, p, p, 100, BF16, None) == -1
    assert lib.mt_swiglu_fwd(None, None, None, 0, BF16, None) == 0  # n = 0: nothing to do
    assert lib.mt_cross_entropy_rows(p, 16, p, 4, 0, p, -100, p, 1, BF16, None) == -2  # vocab must be positive
    # an odd vocab needs a row stride of at least vocab rounded up to 8 (the last chunk reads the padding)
    assert lib.mt_cross_entropy_rows(p, 13, p, 4, 13, p, -100, p, 1, BF16, None) == -3
    assert lib.mt_cross_entropy_rows(p, 8, p, 4, 16, p, -100, p, 1, BF16, None) == -3  # row stride < vocab
    assert lib.mt_cross_entropy_rows(p, 16, None, 4, 16, p, -100, p, 1, BF16, None) == -1
    assert lib.mt_cross_entropy_rows(p, 16, p, -1, 16, p, -100, p, 1, BF16, None) == -2
    assert lib.mt_cross_entropy_rows(None, 16, None, 0, 16, None, -100, None, 1, BF16, None) == 0
    assert lib.mt_last_error() == b""
    # packed SwiGLU: cols a multiple of 8, 16-byte pointers, rows * cols / 8 < 2^31
    assert lib.mt_swiglu_packed_fwd(p, p, 4, 12, BF16, None) == -2
    assert lib.mt_swiglu_packed_fwd(p, p, 1 << 30, 1 << 10, BF16, None) == -2
    assert lib.mt_swiglu_packed_fwd(p + 8, p, 4, 16, BF16, None) == -3
    assert lib.mt_swiglu_packed_bwd(p, None, p, 4, 16, BF16, None) == -1
    assert lib.mt_swiglu_packed_fwd(None, None, 0, 16, BF16, None) == 0
    # mixed norms: 16-bit activations, fp32 weight; the same shape checks as the plain norms
    FP16 = mta._native.DTYPE_FP16
    assert lib.mt_rms_norm_fwd_mixed(p, 16, p, p, p, 4, 16, 1e-5, FP32, FP32, None) == -4  # y must be 16-bit
    assert lib.mt_rms_norm_fwd_mixed(p, 16, p, p, p, 4, 16, 1e-5, BF16, BF16, None) == -4  # weight must be fp32
    assert lib.mt_rms_norm_fwd_mixed(p, 16, p, p, p, 4, 12, 1e-5, BF16, FP32, None) == -2
    assert lib.mt_add_rms_norm_fwd_mixed(p, 16, p, 8, p, p, p, p, 4, 16, 1e-5, FP16, FP32, None) == -3
    assert lib.mt_rms_norm_bwd_mixed(p, p, p, None, p, p, None, p, p, need - 1, 1000, 512, BF16, FP32, None) == -6
    assert lib.mt_rms_norm_bwd_mixed(p, p, p, p + 4, p, p, None, p, p, need, 1000, 512, BF16, FP32, None) == -3
    assert lib.mt_rms_norm_fwd_mixed(p, 16, p, p, p, 0, 16, 1e-5, BF16, FP32, None) == 0
    # stand-alone RoPE: even D, tables of at least T rows and D/2 wide, non-NULL operands
    st = (ctypes.c_int64 * 16)(*([512, 64, 64, 1] * 4))
    assert lib.mt_apply_rope(p, p, p, p, 1, 4, 2, 8, 7, st, p, p, 4, 8, 0, BF16, None) == -2
    assert b"even head dimension" in lib.mt_last_error()
    assert lib.mt_apply_rope(p, p, p, p, 1, 4, 2, 8, 64, st, p, p, 32, 7, 0, BF16, None) == -5  # 7 rows < T
    assert lib.mt_apply_rope(p, p, p, p, 1, 4, 2, 8, 64, st, p, p, 16, 8, 0, BF16, None) == -5  # stride < D/2
    assert lib.mt_apply_rope(p, p, p, p, 1, 4, 2, 8, 64, st, None, p, 32, 8, 0, BF16, None) == -1
    assert lib.mt_apply_rope(p, None, p, p, 1, 4, 2, 8, 64, st, p, p, 32, 8, 0, BF16, None) == -1
    assert lib.mt_apply_rope(p, p, p, p, 1, 4, 2, 8, 64, st, p, p, 32, 8, 0, 9, None) == -4
    assert lib.mt_apply_rope(p, p, p, p, -1, 4, 2, 8, 64, st, p, p, 32, 8, 0, BF16, None) == -2
    assert lib.mt_apply_rope(None, None, None, None, 0, 4, 2, 8, 64, None, None, None, 32, 8, 0, BF16, None) == 0
    # few-row products against grouped weights: fp32, 1..4 groups, 1..64 rows, K a multiple of 128
    ws = (ctypes.c_void_p * 2)(p, p)
    ns = (ctypes.c_int * 2)(64, 32)
    ld = (ctypes.c_int64 * 2)(512, 512)
    assert lib.mt_linear_rows(p, 512, ws, ns, ld, 2, p, 96, 32, 512, 7, None) == -4
    assert lib.mt_linear_rows(p + 4, 512, ws, ns, ld, 2, p, 96, 32, 512, BF16, None) == -3  # 16-bit x: 8-byte aligned
    assert lib.mt_linear_rows(p, 512, ws, ns, ld, 0, p, 96, 32, 512, FP32, None) == -2
    assert lib.mt_linear_rows(p, 512, ws, ns, ld, 5, p, 96, 32, 512, FP32, None) == -2
    assert lib.mt_linear_rows(p, 512, ws, ns, ld, 2, p, 96, 65, 512, FP32, None) == -2
    assert lib.mt_linear_rows(p, 512, ws, ns, ld, 2, p, 96, 0, 512, FP32, None) == -2
    assert lib.mt_linear_rows(p, 512, ws, ns, ld, 2, p, 96, 32, 500, FP32, None) == -2
    assert b"multiple of 128" in lib.mt_last_error()
    assert lib.mt_linear_rows(p + 4, 512, ws, ns, ld, 2, p, 96, 32, 512, FP32, None) == -3  # misaligned x
    assert lib.mt_linear_rows(p, 510, ws, ns, ld, 2, p, 96, 32, 512, FP32, None) == -3  # x stride < K
    assert lib.mt_linear_rows(p, 512, ws, ns, ld, 2, p, 95, 32, 512, FP32, None) == -3  # y stride < 96 columns
    assert lib.mt_linear_rows(p, 512, ws, ns, (ctypes.c_int64 * 2)(512, 514), 2, p, 96, 32, 512, FP32, None) == -3
    assert lib.mt_linear_rows(p, 512, (ctypes.c_void_p * 2)(p, p + 8), ns, ld, 2, p, 96, 32, 512, FP32, None) == -3
    assert lib.mt_linear_rows(p, 512, ws, (ctypes.c_int * 2)(64, 0), ld, 2, p, 96, 32, 512, FP32, None) == -2
    assert lib.mt_linear_rows(p, 512, None, ns, ld, 2, p, 96, 32, 512, FP32, None) == -1
    assert lib.mt_linear_rows(p, 512, ws, ns, ld, 2, None, 96, 32, 512, FP32, None) == -1
    # top-k sampling: fp32, 1 <= k <= vocab <= 32768, row strides >= vocab
    assert lib.mt_topk_sample(p, 128, p, 128, 4, 128, 16, p, BF16, None) == -4
    assert lib.mt_topk_sample(p, 128, p, 128, 4, 0, 1, p, FP32, None) == -2
    assert lib.mt_topk_sample(p, 40000, p, 40000, 4, 40000, 16, p, FP32, None) == -2
    assert lib.mt_topk_sample(p, 128, p, 128, 4, 128, 129, p, FP32, None) == -2
    assert lib.mt_topk_sample(p, 128, p, 128, 4, 128, 0, p, FP32, None) == -2
    assert lib.mt_topk_sample(p, 127, p, 128, 4, 128, 16, p, FP32, None) == -3
    assert lib.mt_topk_sample(p, 128, p, 100, 4, 128, 16, p, FP32, None) == -3
    assert lib.mt_topk_sample(p, 128, None, 128, 4, 128, 16, p, FP32, None) == -1
    assert lib.mt_topk_sample(None, 128, None, 128, 0, 128, 16, None, FP32, None) == 0  # no rows: nothing to do


def test_ops_reject_cpu_tensors(mta):
    x = torch.zeros(4, 16)
    with pytest.raises(RuntimeError, match="ROCm GPU"):
        mta.rms_norm(x, torch.ones(16), eps=1e-5)
    with pytest.raises(RuntimeError, match="ROCm GPU"):
        mta.add_rms_norm(x, x, torch.ones(16), eps=1e-5)
    with pytest.raises(RuntimeError, match="ROCm GPU"):
        mta.swiglu_gate(x, x)
    with pytest.raises(RuntimeError, match="ROCm GPU"):
        mta.ops.fused_linear_cross_entropy(x, torch.zeros(8, 16), torch.zeros(4, dtype=torch.int64))
    with pytest.raises(ValueError, match="one entry per hidden row"):
        mta.ops.fused_linear_cross_entropy(x, torch.zeros(8, 16), torch.zeros(5, dtype=torch.int64))


def test_kernel_timer_arming(mta):
    lib = mta._native.load()
    assert lib.mt_time_next_kernel(0x1000, None) == -1
    assert b"both" in lib.mt_last_error()
    assert lib.mt_time_next_kernel(None, None) == 0  # disarm
    assert lib.mt_last_error() == b""
    # the process-wide queue: argument checks (no events are created here)
    arr = (ctypes.c_void_p * 2)(0x1000, None)
    assert lib.mt_time_kernel_queue(None, None, -1) == -2
    assert lib.mt_time_kernel_queue(None, None, 2) == -1
    assert lib.mt_time_kernel_queue(arr, arr, 2) == -1  # a NULL event in a pair
    assert lib.mt_time_kernel_queue(None, None, 0) == 0  # disarm


def test_c_abi_rejects_bad_arguments_before_launch(mta):
    lib = mta._native.load()
    E_NULL, E_SHAPE, E_STRIDE, E_DTYPE, E_ROPE = -1, -2, -3, -4, -5
    assert _fwd_call(lib, q=None) == E_NULL
    assert b"q is NULL" in lib.mt_last_error()
    assert _fwd_call(lib, lse=None) == E_NULL
    assert _fwd_call(lib, hq=5, hkv=2) == E_SHAPE
    assert b"repeats" in lib.mt_last_error()
    assert _fwd_call(lib, d=48) == E_SHAPE
    assert _fwd_call(lib, t=0) == E_SHAPE
    assert _fwd_call(lib, dtype=7) == E_DTYPE
    assert _fwd_call(lib, cos=0x1000, sin=None) == E_ROPE
    assert _fwd_call(lib, cos=0x1008, sin=0x1008) == E_ROPE  # misaligned tables
    assert _fwd_call(lib, cos=0x1000, sin=0x1000) == E_NULL  # RoPE needs q_rot / k_rot outputs
    assert b"q_rot" in lib.mt_last_error()
    bad = [4 * 16 * 64, 16 * 64, 64, 2] + [2 * 16 * 64, 16 * 64, 64, 1] * 2 + [4 * 16 * 64, 16 * 64, 64, 1]
    assert _fwd_call(lib, strides=bad) == E_STRIDE
    assert b"last-dim stride" in lib.mt_last_error()
    odd = [4 * 16 * 64, 16 * 64, 65, 1] + [2 * 16 * 64, 16 * 64, 64, 1] * 2 + [4 * 16 * 64, 16 * 64, 64, 1]
    assert _fwd_call(lib, strides=odd) == E_STRIDE
    assert _fwd_call(lib, q=0x1002) == E_STRIDE  # misaligned base
    arr = (ctypes.c_int64 * 32)(*([1] * 32))
    p = 0x1000
    assert lib.mt_gqa_attn_bwd(p, p, p, p, p, p, p, p, p, None, 1 << 20,
                               1, 4, 2, 16, 64, arr, 0.125, 0, None, None, None) == E_NULL
    assert b"workspace" in lib.mt_last_error()
    need = lib.mt_gqa_attn_bwd_workspace_size(1, 4, 2, 16, 64)
    assert need >= 4 * 16 * 4  # at least delta = [B, Hq, T] fp32
    assert lib.mt_gqa_attn_bwd_workspace_size(1, 5, 2, 16, 64) == 0
    assert lib.mt_gqa_attn_bwd(p, p, p, p, p, p, p, p, p, p, need - 1,
                               1, 4, 2, 16, 64, arr, 0.125, 0, None, None, None) == -6
    assert b"workspace too small" in lib.mt_last_error()
    assert lib.mt_gqa_attn_bwd(p, p, p, p, p, p, p, p, p, p + 16, need,
                               1, 4, 2, 16, 64, arr, 0.125, 0, None, None, None) == E_STRIDE
    for name in ("mt_gqa_attn_bwd_dq", "mt_gqa_attn_bwd_dkv"):
        fn = getattr(lib, name)
        assert fn(p, p, p, p, p, p, p, p, p, p, need, 1, 4, 2, 16, 33, arr, 0.125, 0, None, None, None) == E_SHAPE


def test_bwd_workspace_size_per_dtype(mta):
    """The fp32 backward never splits a key block's heads, so it needs only the
    delta / LSE vectors; the 16-bit backward of a group of 8 heads with a single
    key block splits them and needs the fp32 partials too.  The dtype-free size
    query is the upper bound (the 16-bit size), and mt_gqa_attn_bwd checks the
    given workspace against its dtype's exact size."""
    lib = mta._native.load()
    b, hq, hkv, t, d = 1, 8, 1, 64, 64
    vec = (b * hq * t * 4 + 255) // 256 * 256
    f32 = lib.mt_gqa_attn_bwd_workspace_size_dtype(b, hq, hkv, t, d, 2)
    bf16 = lib.mt_gqa_attn_bwd_workspace_size_dtype(b, hq, hkv, t, d, 0)
    assert f32 == 2 * vec
    assert bf16 > f32 and bf16 == lib.mt_gqa_attn_bwd_workspace_size(b, hq, hkv, t, d)
    assert lib.mt_gqa_attn_bwd_workspace_size_dtype(b, 5, 2, t, d, 2) == 0
    # a workspace of exactly the fp32 size passes the size check (the call then
    # stops at the deliberately bad q stride, before any device work); one byte
    # less is MT_E_WORKSPACE
    p = 0x1000
    arr = (ctypes.c_int64 * 32)(*([0, 0, 64, 2] + [0, 0, 64, 1] * 7))
    args = (b, hq, hkv, t, d, arr, 0.125, 2, None, None, None)
    assert lib.mt_gqa_attn_bwd(p, p, p, p, p, p, p, p, p, p, f32, *args) == -3  # MT_E_STRIDE
    assert lib.mt_gqa_attn_bwd(p, p, p, p, p, p, p, p, p, p, f32 - 1, *args) == -6


def test_error_codes_raise_python_errors(mta):
    with pytest.raises(mta._native.HipAttentionError, match="head_dim"):
        mta._native.check(_fwd_call(mta._native.load(), d=40), "mt_gqa_attn_fwd")


# ---------------------------------------------------------------------------
# Python operator validation: same checks, order and types as
# src/mega_trading/kernels/triton_attention.py:14-23
# ---------------------------------------------------------------------------
def test_cpu_tensors_are_rejected_like_the_reference(mta):
    q = torch.randn(1, 4, 8, 32)
    k = torch.randn(1, 2, 8, 32)
    with pytest.raises(RuntimeError, match="requires ROCm GPU tensors"):
        mta.attention(q, k, k, repeats=2)


def _fake(shape, dtype=torch.bfloat16):
    return torch.empty(shape, device="cuda", dtype=dtype)


def test_validation_errors_on_device_tensors(mta):
    with FakeTensorMode():
        q, k = _fake((1, 4, 8, 64)), _fake((1, 2, 8, 64))
        with pytest.raises(RuntimeError, match="float16, bfloat16, and float32"):
            mta.attention(_fake((1, 4, 8, 64), torch.int32), k, k, repeats=2)
        with pytest.raises(ValueError, match="multiplied by repeats"):
            mta.attention(q, k, k, repeats=4)
        with pytest.raises(ValueError, match="same shape"):
            mta.attention(q, k, _fake((1, 2, 9, 64)), repeats=2)
        with pytest.raises(ValueError, match="agree on batch"):
            mta.attention(q, _fake((1, 2, 9, 64)), _fake((1, 2, 9, 64)), repeats=2)
        with pytest.raises(ValueError, match="head_dim must be between 1 and 128"):
            mta.attention(_fake((1, 4, 8, 256)), _fake((1, 2, 8, 256)), _fake((1, 2, 8, 256)), repeats=2)
        # another head size is padded to the next kernel size: the result keeps its shape
        out48 = mta.attention(_fake((1, 4, 8, 48)), _fake((1, 2, 8, 48)), _fake((1, 2, 8, 48)), repeats=2)
        assert out48.shape == (1, 4, 8, 48)
        with pytest.raises(ValueError, match="even head dimension"):
            mta.rope_attention(_fake((1, 4, 8, 9)), _fake((1, 2, 8, 9)), _fake((1, 2, 8, 9)),
                               torch.empty(8, 4, device="cuda"), torch.empty(8, 4, device="cuda"), repeats=2)
        with pytest.raises(RuntimeError, match="share one dtype"):
            mta.attention(q, _fake((1, 2, 8, 64), torch.float16), k, repeats=2)
        cos = torch.empty(4, 32, device="cuda")
        with pytest.raises(ValueError, match="exceeds RoPE cache length"):
            mta.rope_attention(q, k, k, cos, cos, repeats=2)
        with pytest.raises(ValueError, match="head_dim/2"):
            mta.rope_attention(q, k, k, torch.empty(8, 31, device="cuda"), torch.empty(8, 31, device="cuda"), repeats=2)


def test_apply_rope_validation_like_the_reference_call(mta):
    """ops.apply_rope (triton_apply_rope, triton_ops.py:45-54): [B, H, T, D]
    query / key sharing B, T and D, even D, [1, 1, >= T, D/2] tables."""
    with FakeTensorMode():
        q, k = _fake((1, 4, 8, 64)), _fake((1, 2, 8, 64))
        cs = torch.empty(1, 1, 16, 32, device="cuda")
        qo, ko = mta.ops.apply_rope(q, k, cs, cs)
        assert qo.shape == q.shape and ko.shape == k.shape
        with pytest.raises(ValueError, match="even head dimension"):
            mta.ops.apply_rope(_fake((1, 4, 8, 9)), _fake((1, 2, 8, 9)), cs, cs)
        with pytest.raises(ValueError, match="B, T and D of query"):
            mta.ops.apply_rope(q, _fake((1, 2, 9, 64)), cs, cs)
        with pytest.raises(ValueError, match="fewer than the sequence length"):
            mta.ops.apply_rope(q, k, cs[:, :, :4], cs[:, :, :4])
        with pytest.raises(ValueError, match=r"D/2 = 32"):
            mta.ops.apply_rope(q, k, torch.empty(1, 1, 16, 31, device="cuda"), cs)
        with pytest.raises(RuntimeError, match="dtype and device of query"):
            mta.ops.apply_rope(q, _fake((1, 2, 8, 64), torch.float16), cs, cs)
    with pytest.raises(RuntimeError, match="ROCm GPU"):
        mta.ops.apply_rope(torch.zeros(1, 4, 8, 64), torch.zeros(1, 2, 8, 64), torch.zeros(1, 1, 8, 32),
                           torch.zeros(1, 1, 8, 32))


def test_fake_impls_give_shapes_for_tracing(mta):
    with FakeTensorMode():
        q, k = _fake((2, 8, 100, 64)), _fake((2, 2, 100, 64))
        out, lse = torch.ops.mega_trading_amd.gqa_attn_fwd(q, k, k, 0.125)
        assert out.shape == q.shape and lse.shape == (2, 8, 100) and lse.dtype == torch.float32
        cs = torch.empty(100, 32, device="cuda")
        out2, lse2, qr, kr = torch.ops.mega_trading_amd.gqa_rope_attn_fwd(q, k, k, cs, cs, 0.125)
        assert out2.shape == q.shape and qr.shape == q.shape and kr.shape == k.shape
        dq, dk, dv = torch.ops.mega_trading_amd.gqa_attn_bwd(q, k, k, out, lse, q, None, None, 0.125)
        assert dq.shape == q.shape and dk.shape == k.shape and dv.shape == k.shape
        qkv = _fake((2, 100, (8 + 2 + 2) * 64))
        o3, l3, qr3, kr3 = torch.ops.mega_trading_amd.gqa_rope_attn_packed_fwd(qkv, cs, cs, 8, 2, 0.125)
        assert o3.shape == (2, 100, 512) and l3.shape == (2, 8, 100) and qr3.shape == q.shape and kr3.shape == k.shape
        d3 = torch.ops.mega_trading_amd.gqa_attn_bwd_packed(qr3, kr3, qkv, o3, l3, o3, cs, cs, 8, 2, 0.125)
        assert d3.shape == qkv.shape
        y = torch.ops.mega_trading_amd.linear_rows(_fake((32, 512), torch.float32),
                                                   [_fake((768, 512), torch.float32), _fake((64, 512), torch.float32)])
        assert y.shape == (32, 832) and y.dtype == torch.float32
        tok = torch.ops.mega_trading_amd.topk_sample(_fake((32, 16384), torch.float32), _fake((32, 16384), torch.float32), 16)
        assert tok.shape == (32, 1) and tok.dtype == torch.int64


def test_kernel_ready_keeps_model_layout_views():
    """The [B,T,H,D]-physical views of model.py:220-222 pass through without a copy."""
    import importlib

    ops = importlib.import_module("mega-trading_amd.attention")
    x = torch.randn(2, 16, 8, 64).transpose(1, 2)  # [B, H, T, D] view
    assert ops._kernel_ready(x) is x
    y = torch.randn(2, 8, 16, 64)[..., ::2]  # non-unit last stride -> copy
    assert ops._kernel_ready(y).is_contiguous()
    arr = ops._strides(torch.empty(1, 1, 5, 32))
    assert list(arr) == [0, 0, 32, 1]  # size-1 dims pass stride 0


def test_decode_rope_append_bounds_pos_before_launch(mta):
    """mt_decode_rope_append rejects a position at or past the cache capacity or
    the RoPE table before any launch (pointers never dereferenced)."""
    lib = mta._native.load()
    p = 0x10000
    ins = (ctypes.c_int64 * 6)(512, 64, 128, 64, 128, 64)
    cst = (ctypes.c_int64 * 6)(2 * 40 * 64, 40 * 64, 64, 2 * 40 * 64, 40 * 64, 64)

    def call(table_rows, pos, capacity):
        return lib.mt_decode_rope_append(p, p, p, ins, p, p, table_rows, pos, None, p, p, p, cst, capacity,
                                         1, 8, 2, 64, 0, 0, None)

    assert call(64, 40, 40) == -2            # pos == capacity
    assert b"capacity 40" in lib.mt_last_error()
    assert call(20, 30, 40) == -2            # pos past the table
    assert call(64, -1, 40) == -2
    assert call(0, 0, 40) == -2
    assert lib.mt_decode_rope_append(p, p, p, ins, p, p, 64, 3, None, p, p, p, cst, 40, 1, 8, 2, 64, 0, 2,
                                     None) == -4  # fp32 caches
