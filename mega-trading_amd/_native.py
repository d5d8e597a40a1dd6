"""ctypes binding of libmt_attn.so (the C ABI declared in include/mt_attention.h and include/mt_ops.h).

The library is loaded lazily on first use.  There is no fallback: if the
library is missing the call raises, so a GPU run can never silently route
around the HIP kernels.
"""

from __future__ import annotations

import ctypes
import os
import threading

LIB_NAME = "libmt_attn.so"
LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), LIB_NAME)
# the GPU implementations of the mega_trading_amd attention ops (PyTorch-ROCm side, links libmt_attn.so)
TORCH_OPS_NAME = "libmt_torch.so"
TORCH_OPS_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), TORCH_OPS_NAME)

DTYPE_BF16 = 0
DTYPE_FP16 = 1
DTYPE_FP32 = 2

# Every symbol the header declares; tests check the library exports them all.
EXPORTS = (
    "mt_version",
    "mt_last_error",
    "mt_gqa_attn_bwd_workspace_size",
    "mt_gqa_attn_bwd_workspace_size_dtype",
    "mt_gqa_attn_fwd",
    "mt_gqa_attn_bwd",
    "mt_gqa_attn_bwd_dq",
    "mt_gqa_attn_bwd_dkv",
    "mt_gqa_attn_bwd_noalloc",
    "mt_time_next_kernel",
    "mt_time_kernel_queue",
    "mt_rms_norm_fwd",
    "mt_add_rms_norm_fwd",
    "mt_rms_norm_bwd_workspace_size",
    "mt_rms_norm_bwd",
    "mt_add_rms_norm_bwd",
    "mt_rms_norm_fwd_mixed",
    "mt_add_rms_norm_fwd_mixed",
    "mt_rms_norm_bwd_mixed",
    "mt_swiglu_fwd",
    "mt_swiglu_bwd",
    "mt_swiglu_packed_fwd",
    "mt_swiglu_packed_bwd",
    "mt_cross_entropy_rows",
    "mt_apply_rope",
    "mt_gqa_attn_decode_workspace_size",
    "mt_gqa_attn_decode",
    "mt_gqa_attn_decode_dev",
    "mt_decode_rope_append",
    "mt_linear_rows",
    "mt_topk_sample",
)

_lock = threading.Lock()
_lib: ctypes.CDLL | None = None

_P = ctypes.c_void_p
_I = ctypes.c_int
_F = ctypes.c_float
_S = ctypes.c_size_t
_FWD_ARGTYPES = [_P, _P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _P, _F, _I, _P, _P, _P]
_BWD_ARGTYPES = [_P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _S, _I, _I, _I, _I, _I, _P, _F, _I, _P, _P, _P]
_L = ctypes.c_int64
_OPS_SIGNATURES = {
    "mt_gqa_attn_bwd_workspace_size_dtype": (_S, [_I, _I, _I, _I, _I, _I]),
    "mt_time_kernel_queue": (_I, [_P, _P, _I]),
    "mt_gqa_attn_bwd_noalloc": (_I, [_P, _P, _P, _P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _P, _F, _I, _P, _P, _P]),
    "mt_rms_norm_fwd": (_I, [_P, _L, _P, _P, _P, _L, _I, _F, _I, _I, _P]),
    "mt_add_rms_norm_fwd": (_I, [_P, _L, _P, _L, _P, _P, _P, _P, _L, _I, _F, _I, _I, _P]),
    "mt_rms_norm_bwd_workspace_size": (_S, [_L, _I]),
    "mt_rms_norm_bwd": (_I, [_P, _P, _P, _P, _P, _P, _P, _S, _L, _I, _I, _I, _P]),
    "mt_add_rms_norm_bwd": (_I, [_P, _P, _P, _P, _P, _P, _P, _P, _S, _L, _I, _I, _I, _P]),
    "mt_rms_norm_fwd_mixed": (_I, [_P, _L, _P, _P, _P, _L, _I, _F, _I, _I, _P]),
    "mt_add_rms_norm_fwd_mixed": (_I, [_P, _L, _P, _L, _P, _P, _P, _P, _L, _I, _F, _I, _I, _P]),
    "mt_rms_norm_bwd_mixed": (_I, [_P, _P, _P, _P, _P, _P, _P, _P, _P, _S, _L, _I, _I, _I, _P]),
    "mt_swiglu_fwd": (_I, [_P, _P, _P, _L, _I, _P]),
    "mt_swiglu_bwd": (_I, [_P, _P, _P, _P, _P, _L, _I, _P]),
    "mt_swiglu_packed_fwd": (_I, [_P, _P, _L, _L, _I, _P]),
    "mt_swiglu_packed_bwd": (_I, [_P, _P, _P, _L, _L, _I, _P]),
    "mt_cross_entropy_rows": (_I, [_P, _L, _P, _L, _I, _P, _L, _P, _I, _I, _P]),
    "mt_apply_rope": (_I, [_P, _P, _P, _P, _I, _I, _I, _I, _I, _P, _P, _P, _L, _I, _I, _I, _P]),
    "mt_gqa_attn_decode_workspace_size": (_S, [_I, _I, _I, _I]),
    "mt_gqa_attn_decode": (_I, [_P, _P, _P, _P, _I, _I, _I, _I, _I, _P, _F, _I, _P, _S, _P]),
    "mt_gqa_attn_decode_dev": (_I, [_P, _P, _P, _P, _I, _I, _I, _I, _P, _I, _P, _F, _I, _P, _S, _P]),
    "mt_decode_rope_append": (_I, [_P, _P, _P, _P, _P, _P, _I, _I, _P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _I, _I,
                                   _P]),
    "mt_linear_rows": (_I, [_P, _L, _P, _P, _P, _I, _P, _L, _I, _I, _I, _P]),
    "mt_topk_sample": (_I, [_P, _L, _P, _L, _I, _I, _I, _P, _I, _P]),
}


class HipAttentionError(RuntimeError):
    """A non-zero return code from the C ABI."""


def library_path() -> str:
    return LIB_PATH


def torch_ops_path() -> str:
    return TORCH_OPS_PATH


def load() -> ctypes.CDLL:
    """Load libmt_attn.so (once) and declare the C signatures; also load
    libmt_torch.so, which registers the attention ops' GPU kernels with torch."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is not None:
            return _lib
        for path in (LIB_PATH, TORCH_OPS_PATH):
            if not os.path.exists(path):
                raise RuntimeError(
                    f"{path} is missing: build it with `python -c 'import __graft_entry__ as g; g.build()'` "
                    "(or python mega-trading_amd/build_lib.py) before using the HIP attention op"
                )
        lib = ctypes.CDLL(LIB_PATH)
        import torch

        torch.ops.load_library(TORCH_OPS_PATH)
        lib.mt_version.restype = _I
        lib.mt_version.argtypes = []
        lib.mt_last_error.restype = ctypes.c_char_p
        lib.mt_last_error.argtypes = []
        lib.mt_gqa_attn_bwd_workspace_size.restype = _S
        lib.mt_gqa_attn_bwd_workspace_size.argtypes = [_I, _I, _I, _I, _I]
        lib.mt_gqa_attn_fwd.restype = _I
        lib.mt_gqa_attn_fwd.argtypes = _FWD_ARGTYPES
        for name in ("mt_gqa_attn_bwd", "mt_gqa_attn_bwd_dq", "mt_gqa_attn_bwd_dkv"):
            fn = getattr(lib, name)
            fn.restype = _I
            fn.argtypes = _BWD_ARGTYPES
        lib.mt_time_next_kernel.restype = _I
        lib.mt_time_next_kernel.argtypes = [_P, _P]
        for name, (res, args) in _OPS_SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        _lib = lib
        return lib


def check(rc: int, what: str) -> None:
    if rc != 0:
        msg = load().mt_last_error().decode(errors="replace")
        raise HipAttentionError(f"{what} failed (code {rc}): {msg}")


def strides_array(*tensors) -> ctypes.Array:
    """Flatten (b, h, t, d) element strides of [B,H,T,D] tensors into int64[4 * n]."""
    flat: list[int] = []
    for t in tensors:
        flat.extend(int(s) for s in t.stride())
    return (ctypes.c_int64 * len(flat))(*flat)
