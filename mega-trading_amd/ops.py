"""The decoder's memory-bound operators on MI355X (gfx950) HIP kernels.

Drop-ins for the reference's operator functions in
``src/mega_trading/kernels/triton_ops.py``:

* ``rms_norm(hidden, weight, *, eps)``            <- ``triton_rms_norm`` (:11-15)
* ``add_rms_norm(hidden, residual, weight, *, eps)`` <- ``triton_add_rms_norm`` (:18-42)
* ``swiglu_gate(gate, up)``                       <- ``triton_swiglu_gate`` (:57-61)

Same argument meaning and results (fp32 arithmetic; outputs in the input
dtype; the roundings between steps as the reference performs them).  The
reference silently falls back to PyTorch for tensors it cannot handle; these
raise instead (``RuntimeError`` off the GPU or for an unsupported dtype,
``ValueError`` for shapes), so a run can never route around the kernels.

Each is a ``torch.library`` custom op with a fake implementation and a
registered backward, launched on the caller's current stream.
"""

from __future__ import annotations

import torch

from . import _native

__all__ = ["rms_norm", "add_rms_norm", "swiglu_gate", "MAX_NORM_DIM"]

MAX_NORM_DIM = 4096
_DT = {torch.bfloat16: _native.DTYPE_BF16, torch.float16: _native.DTYPE_FP16, torch.float32: _native.DTYPE_FP32}


# ---------------------------------------------------------------------------
# public functions
# ---------------------------------------------------------------------------
def rms_norm(hidden: torch.Tensor, weight: torch.Tensor, *, eps: float) -> torch.Tensor:
    """``hidden * rsqrt(mean(hidden^2, -1) + eps) * weight`` (``triton_ops.py:11``, kernel ``:528-539``)."""
    _check_norm(hidden, weight)
    y, _rstd = torch.ops.mega_trading_amd.rms_norm_fwd(hidden, weight, float(eps))
    return y


def add_rms_norm(
    hidden: torch.Tensor, residual: torch.Tensor, weight: torch.Tensor, *, eps: float
) -> tuple[torch.Tensor, torch.Tensor]:
    """``(new_residual, normed)`` with ``new_residual = hidden + residual`` and
    ``normed = RMSNorm(new_residual)`` from the unrounded sum (``triton_ops.py:18-42``)."""
    _check_norm(hidden, weight)
    if residual.shape != hidden.shape:
        raise ValueError("residual must have the same shape as hidden")
    if residual.dtype != hidden.dtype or residual.device != hidden.device:
        raise RuntimeError("residual must have the dtype and device of hidden")
    new_res, y, _rstd = torch.ops.mega_trading_amd.add_rms_norm_fwd(hidden, residual, weight, float(eps))
    return new_res, y


def swiglu_gate(gate: torch.Tensor, up: torch.Tensor) -> torch.Tensor:
    """``silu(gate) * up`` with silu rounded to the input dtype first (``triton_ops.py:57-61``)."""
    _check_device_dtype(gate, "gate")
    if up.shape != gate.shape:
        raise ValueError("gate and up must have the same shape")
    if up.dtype != gate.dtype or up.device != gate.device:
        raise RuntimeError("up must have the dtype and device of gate")
    return torch.ops.mega_trading_amd.swiglu_fwd(gate, up)


# ---------------------------------------------------------------------------
# helpers
# ---------------------------------------------------------------------------
def _check_device_dtype(t: torch.Tensor, name: str) -> None:
    if t.device.type != "cuda" or not torch.version.hip:
        raise RuntimeError(f"{name} must be on a ROCm GPU (got device {t.device})")
    if t.dtype not in _DT:
        raise RuntimeError(f"{name} dtype {t.dtype} unsupported (bfloat16, float16 or float32)")


def _check_norm(hidden: torch.Tensor, weight: torch.Tensor) -> None:
    _check_device_dtype(hidden, "hidden")
    d = hidden.shape[-1] if hidden.ndim else 0
    if hidden.ndim < 1 or weight.ndim != 1 or weight.numel() != d:
        raise ValueError("weight must be 1-D with hidden.shape[-1] elements")
    if d % 8 or d > MAX_NORM_DIM:
        raise ValueError(f"hidden_dim {d} unsupported: a multiple of 8 up to {MAX_NORM_DIM}")
    if weight.device != hidden.device:
        raise RuntimeError("weight must be on the device of hidden")


def _rows(x: torch.Tensor) -> tuple[torch.Tensor, int]:
    """[..., D] -> ([rows, D] usable in place or a contiguous copy, row stride)."""
    d = x.shape[-1]
    x2 = x.reshape(-1, d)
    if x2.stride(-1) != 1 or x2.data_ptr() % 16 or (x2.shape[0] > 1 and x2.stride(0) % 8):
        x2 = x2.contiguous()
        if x2.data_ptr() % 16:
            x2 = x2.clone()
    return x2, (x2.stride(0) if x2.shape[0] > 1 else d)


def _flat(t: torch.Tensor) -> torch.Tensor:
    t = t.contiguous()
    return t if t.data_ptr() % 16 == 0 else t.clone()


def _weight(w: torch.Tensor, x: torch.Tensor) -> torch.Tensor:
    """The weight as the kernels take it: x's dtype or fp32, contiguous, aligned."""
    if w.dtype != x.dtype and w.dtype != torch.float32:
        w = w.to(torch.float32)
    return _flat(w)


def _stream(t: torch.Tensor) -> int:
    return torch.cuda.current_stream(t.device).cuda_stream


# ---------------------------------------------------------------------------
# custom ops
# ---------------------------------------------------------------------------
@torch.library.custom_op("mega_trading_amd::rms_norm_fwd", mutates_args=(), device_types="cuda")
def rms_norm_fwd(x: torch.Tensor, weight: torch.Tensor, eps: float) -> tuple[torch.Tensor, torch.Tensor]:
    """Returns (y with x's shape, rstd fp32 [rows])."""
    lib = _native.load()
    x2, sx = _rows(x)
    w = _weight(weight, x)
    rows, d = x2.shape
    y = torch.empty((rows, d), device=x.device, dtype=x.dtype)
    rstd = torch.empty((rows,), device=x.device, dtype=torch.float32)
    with torch.cuda.device(x.device):
        rc = lib.mt_rms_norm_fwd(x2.data_ptr(), sx, w.data_ptr(), y.data_ptr(), rstd.data_ptr(), rows, d, eps,
                                 _DT[x.dtype], _DT[w.dtype], _stream(x))
    _native.check(rc, "mt_rms_norm_fwd")
    return y.view(x.shape), rstd


@rms_norm_fwd.register_fake
def _rms_norm_fwd_fake(x, weight, eps):
    return torch.empty_like(x, memory_format=torch.contiguous_format), x.new_empty(
        (x.numel() // max(x.shape[-1], 1),), dtype=torch.float32)


@torch.library.custom_op("mega_trading_amd::rms_norm_bwd", mutates_args=(), device_types="cuda")
def rms_norm_bwd(x: torch.Tensor, weight: torch.Tensor, rstd: torch.Tensor, dy: torch.Tensor
                 ) -> tuple[torch.Tensor, torch.Tensor]:
    """(dx with x's shape and dtype, dweight with weight's dtype)."""
    return _norm_bwd(x, weight, rstd, dy, None)


@rms_norm_bwd.register_fake
def _rms_norm_bwd_fake(x, weight, rstd, dy):
    return torch.empty_like(x, memory_format=torch.contiguous_format), torch.empty_like(weight)


@torch.library.custom_op("mega_trading_amd::add_rms_norm_fwd", mutates_args=(), device_types="cuda")
def add_rms_norm_fwd(x: torch.Tensor, residual: torch.Tensor, weight: torch.Tensor, eps: float
                     ) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """Returns (new_residual, y, rstd)."""
    lib = _native.load()
    x2, sx = _rows(x)
    r2, sr = _rows(residual)
    w = _weight(weight, x)
    rows, d = x2.shape
    new_res = torch.empty((rows, d), device=x.device, dtype=x.dtype)
    y = torch.empty((rows, d), device=x.device, dtype=x.dtype)
    rstd = torch.empty((rows,), device=x.device, dtype=torch.float32)
    with torch.cuda.device(x.device):
        rc = lib.mt_add_rms_norm_fwd(x2.data_ptr(), sx, r2.data_ptr(), sr, w.data_ptr(), new_res.data_ptr(),
                                     y.data_ptr(), rstd.data_ptr(), rows, d, eps, _DT[x.dtype], _DT[w.dtype],
                                     _stream(x))
    _native.check(rc, "mt_add_rms_norm_fwd")
    return new_res.view(x.shape), y.view(x.shape), rstd


@add_rms_norm_fwd.register_fake
def _add_rms_norm_fwd_fake(x, residual, weight, eps):
    rows = x.numel() // max(x.shape[-1], 1)
    return (torch.empty_like(x, memory_format=torch.contiguous_format),
            torch.empty_like(x, memory_format=torch.contiguous_format),
            x.new_empty((rows,), dtype=torch.float32))


@torch.library.custom_op("mega_trading_amd::add_rms_norm_bwd", mutates_args=(), device_types="cuda")
def add_rms_norm_bwd(new_residual: torch.Tensor, weight: torch.Tensor, rstd: torch.Tensor,
                     d_new_residual: torch.Tensor, dy: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """(d hidden = d residual, dweight)."""
    return _norm_bwd(new_residual, weight, rstd, dy, d_new_residual)


@add_rms_norm_bwd.register_fake
def _add_rms_norm_bwd_fake(new_residual, weight, rstd, d_new_residual, dy):
    return torch.empty_like(new_residual, memory_format=torch.contiguous_format), torch.empty_like(weight)


def _norm_bwd(s, weight, rstd, dy, dres):
    lib = _native.load()
    d = s.shape[-1]
    s2 = _flat(s.reshape(-1, d))
    dy2 = _flat(dy.to(s.dtype).reshape(-1, d))
    w = _weight(weight, s)
    rows = s2.shape[0]
    dx = torch.empty((rows, d), device=s.device, dtype=s.dtype)
    dw = torch.empty((d,), device=s.device, dtype=w.dtype)
    with torch.cuda.device(s.device):
        ws_bytes = lib.mt_rms_norm_bwd_workspace_size(rows, d)
        ws = torch.empty(max(ws_bytes, 256), device=s.device, dtype=torch.uint8)
        if dres is None:
            rc = lib.mt_rms_norm_bwd(s2.data_ptr(), w.data_ptr(), rstd.data_ptr(), dy2.data_ptr(), dx.data_ptr(),
                                     dw.data_ptr(), ws.data_ptr(), ws.numel(), rows, d, _DT[s.dtype], _DT[w.dtype],
                                     _stream(s))
            what = "mt_rms_norm_bwd"
        else:
            dr2 = _flat(dres.to(s.dtype).reshape(-1, d))
            rc = lib.mt_add_rms_norm_bwd(s2.data_ptr(), w.data_ptr(), rstd.data_ptr(), dr2.data_ptr(), dy2.data_ptr(),
                                         dx.data_ptr(), dw.data_ptr(), ws.data_ptr(), ws.numel(), rows, d,
                                         _DT[s.dtype], _DT[w.dtype], _stream(s))
            what = "mt_add_rms_norm_bwd"
    _native.check(rc, what)
    return dx.view(s.shape), dw.to(weight.dtype)


@torch.library.custom_op("mega_trading_amd::swiglu_fwd", mutates_args=(), device_types="cuda")
def swiglu_fwd(gate: torch.Tensor, up: torch.Tensor) -> torch.Tensor:
    lib = _native.load()
    g, u = _flat(gate), _flat(up)
    out = torch.empty(gate.shape, device=gate.device, dtype=gate.dtype)
    with torch.cuda.device(gate.device):
        rc = lib.mt_swiglu_fwd(g.data_ptr(), u.data_ptr(), out.data_ptr(), g.numel(), _DT[g.dtype], _stream(gate))
    _native.check(rc, "mt_swiglu_fwd")
    return out


@swiglu_fwd.register_fake
def _swiglu_fwd_fake(gate, up):
    return torch.empty_like(gate, memory_format=torch.contiguous_format)


@torch.library.custom_op("mega_trading_amd::swiglu_bwd", mutates_args=(), device_types="cuda")
def swiglu_bwd(gate: torch.Tensor, up: torch.Tensor, dout: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    lib = _native.load()
    g, u, dy = _flat(gate), _flat(up), _flat(dout.to(gate.dtype))
    dg = torch.empty(gate.shape, device=gate.device, dtype=gate.dtype)
    du = torch.empty(gate.shape, device=gate.device, dtype=gate.dtype)
    with torch.cuda.device(gate.device):
        rc = lib.mt_swiglu_bwd(g.data_ptr(), u.data_ptr(), dy.data_ptr(), dg.data_ptr(), du.data_ptr(), g.numel(),
                               _DT[g.dtype], _stream(gate))
    _native.check(rc, "mt_swiglu_bwd")
    return dg, du


@swiglu_bwd.register_fake
def _swiglu_bwd_fake(gate, up, dout):
    return (torch.empty_like(gate, memory_format=torch.contiguous_format),
            torch.empty_like(gate, memory_format=torch.contiguous_format))


# ---------------------------------------------------------------------------
# autograd
# ---------------------------------------------------------------------------
def _rms_setup(ctx, inputs, output):
    x, weight, _eps = inputs
    _y, rstd = output
    ctx.save_for_backward(x, weight, rstd)
    ctx.mark_non_differentiable(rstd)
    ctx.set_materialize_grads(False)


def _rms_backward(ctx, dy, _drstd):
    x, weight, rstd = ctx.saved_tensors
    if dy is None:
        return None, None, None
    dx, dw = torch.ops.mega_trading_amd.rms_norm_bwd(x, weight, rstd, dy)
    return dx, dw, None


def _add_rms_setup(ctx, inputs, output):
    _x, _r, weight, _eps = inputs
    new_res, _y, rstd = output
    ctx.save_for_backward(new_res, weight, rstd)
    ctx.mark_non_differentiable(rstd)
    ctx.set_materialize_grads(False)


def _add_rms_backward(ctx, d_new_res, dy, _drstd):
    new_res, weight, rstd = ctx.saved_tensors
    if d_new_res is None and dy is None:
        return None, None, None, None
    if dy is None:
        dy = torch.zeros_like(new_res)
    if d_new_res is None:
        d_new_res = torch.zeros_like(new_res)
    dx, dw = torch.ops.mega_trading_amd.add_rms_norm_bwd(new_res, weight, rstd, d_new_res, dy)
    # hidden and residual enter the add symmetrically: the same gradient for both (triton_ops.py:288-291)
    return dx, dx, dw, None


def _swiglu_setup(ctx, inputs, output):
    gate, up = inputs
    ctx.save_for_backward(gate, up)
    ctx.set_materialize_grads(False)


def _swiglu_backward(ctx, dout):
    gate, up = ctx.saved_tensors
    if dout is None:
        return None, None
    return torch.ops.mega_trading_amd.swiglu_bwd(gate, up, dout)


rms_norm_fwd.register_autograd(_rms_backward, setup_context=_rms_setup)
add_rms_norm_fwd.register_autograd(_add_rms_backward, setup_context=_add_rms_setup)
swiglu_fwd.register_autograd(_swiglu_backward, setup_context=_swiglu_setup)
