"""The decoder's memory-bound operators on MI355X (gfx950) HIP kernels.

Drop-ins for the reference's operator functions in
``src/mega_trading/kernels/triton_ops.py``:

* ``rms_norm(hidden, weight, *, eps)``            <- ``triton_rms_norm`` (:11-15)
* ``add_rms_norm(hidden, residual, weight, *, eps)`` <- ``triton_add_rms_norm`` (:18-42)
* ``swiglu_gate(gate, up)``                       <- ``triton_swiglu_gate`` (:57-61)
* ``apply_rope(query, key, cos, sin)``            <- ``triton_apply_rope`` (:45-54)
* ``fused_linear_cross_entropy(hidden, weight, labels, *, ignore_index)``
                                                  <- ``triton_fused_linear_cross_entropy`` (:64-92)

Same argument meaning and results (fp32 arithmetic; outputs in the input
dtype; the roundings between steps as the reference performs them).  The
reference silently falls back to PyTorch for tensors it cannot handle; these
raise instead (``RuntimeError`` off the GPU or for an unsupported dtype,
``ValueError`` for shapes), so a run can never route around the kernels.

Each is a ``torch.library`` custom op with a fake implementation and a
registered backward, launched on the caller's current stream.
"""

from __future__ import annotations

import ctypes
from typing import Optional

import torch

from . import _native
from .gemm_tuning import tuned_gemms

__all__ = ["rms_norm", "add_rms_norm", "rms_norm_mixed", "add_rms_norm_mixed", "swiglu_gate", "swiglu_gate_packed",
           "apply_rope", "fused_linear_cross_entropy", "topk_sample", "MAX_NORM_DIM", "MAX_SAMPLE_VOCAB"]

MAX_NORM_DIM = 4096
MAX_SAMPLE_VOCAB = 32768  # vocabulary of one topk_sample row (1024 threads x 32 values in registers)
_DT = {torch.bfloat16: _native.DTYPE_BF16, torch.float16: _native.DTYPE_FP16, torch.float32: _native.DTYPE_FP32}
_DTYPE_OF = {v: k for k, v in _DT.items()}


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


def rms_norm_mixed(hidden: torch.Tensor, weight: torch.Tensor, *, eps: float, out_dtype: torch.dtype) -> torch.Tensor:
    """``rms_norm`` of an fp32 residual stream with the result rounded once to
    the 16-bit ``out_dtype``: what the fp32 norm followed by the next
    projection's autocast cast gives, in one pass.  ``weight`` fp32."""
    _check_norm(hidden, weight)
    _check_mixed(hidden, weight, out_dtype)
    y, _rstd = torch.ops.mega_trading_amd.rms_norm_fwd_mixed(hidden, weight, float(eps), _DT[out_dtype])
    return y


def add_rms_norm_mixed(
    branch: torch.Tensor, residual: torch.Tensor, weight: torch.Tensor, *, eps: float
) -> tuple[torch.Tensor, torch.Tensor]:
    """``(new_residual, normed)``: ``new_residual = residual + branch`` in fp32
    (torch's promotion of an fp32 residual stream plus a 16-bit branch output)
    and ``normed = RMSNorm(new_residual)`` rounded once to the branch's dtype.
    ``residual`` and ``weight`` fp32, ``branch`` bf16 or fp16."""
    _check_norm(residual, weight)
    _check_mixed(residual, weight, branch.dtype)
    if branch.shape != residual.shape:
        raise ValueError("branch must have the shape of residual")
    if branch.device != residual.device:
        raise RuntimeError("branch must be on the device of residual")
    new_res, y, _rstd = torch.ops.mega_trading_amd.add_rms_norm_fwd_mixed(branch, residual, weight, float(eps))
    return new_res, y


def swiglu_gate(gate: torch.Tensor, up: torch.Tensor) -> torch.Tensor:
    """``silu(gate) * up`` with silu rounded to the input dtype first (``triton_ops.py:57-61``)."""
    _check_device_dtype(gate, "gate")
    if up.shape != gate.shape:
        raise ValueError("gate and up must have the same shape")
    if up.dtype != gate.dtype or up.device != gate.device:
        raise RuntimeError("up must have the dtype and device of gate")
    return torch.ops.mega_trading_amd.swiglu_fwd(gate, up)


def swiglu_gate_packed(gate_up: torch.Tensor) -> torch.Tensor:
    """``swiglu_gate(gate, up)`` on the packed [..., 2F] output of one GEMM
    against the stacked (w1; w3) weights: gate = the first F columns of each
    row, up = the last F.  Returns [..., F].  No reference counterpart (the
    reference gate takes the two products, ``triton_ops.py:57-61``); the
    arithmetic and roundings are ``swiglu_gate``'s."""
    _check_device_dtype(gate_up, "gate_up")
    if gate_up.ndim < 1 or gate_up.shape[-1] % 16:
        raise ValueError("gate_up's last dim must be 2F with F a multiple of 8")
    return torch.ops.mega_trading_amd.swiglu_packed_fwd(gate_up)


def apply_rope(
    query: torch.Tensor, key: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor
) -> tuple[torch.Tensor, torch.Tensor]:
    """``(rot(query), rot(key))`` (``triton_apply_rope``, ``triton_ops.py:45-54``).

    ``query`` [B, Hq, T, D] and ``key`` [B, Hkv, T, D] (any strides), tables
    [1, 1, >= T, D/2] as ``RotaryEmbedding`` keeps them (any float dtype, read
    as fp32; rows past T are ignored).  Each interleaved pair (e, o) of row t
    becomes (e cos - o sin, e sin + o cos) in fp32 with one rounding to the
    input dtype; outputs have the inputs' layout.  The backward rotates the
    gradients by -theta (``triton_ops.py:204-214``)."""
    _check_device_dtype(query, "query")
    if key.dtype != query.dtype or key.device != query.device:
        raise RuntimeError("key must have the dtype and device of query")
    if query.ndim != 4 or key.ndim != 4:
        raise ValueError("query and key must be [B, H, T, D]")
    b, _hq, t, d = query.shape
    if key.shape[0] != b or key.shape[2] != t or key.shape[3] != d:
        raise ValueError("key must be [B, Hkv, T, D] with the B, T and D of query")
    if d % 2:
        raise ValueError("RoPE requires an even head dimension")
    c = _rope_table(cos, "cos", t, d, query.device)
    s = _rope_table(sin, "sin", t, d, query.device)
    if s.shape != c.shape:
        raise ValueError("cos and sin must have the same shape")
    return torch.ops.mega_trading_amd.rope_fwd(query, key, c, s, False)


def fused_linear_cross_entropy(
    hidden: torch.Tensor, weight: torch.Tensor, labels: torch.Tensor, *, ignore_index: int = -100
) -> torch.Tensor:
    """Mean cross-entropy of ``hidden @ weight.T`` against ``labels`` without the
    [rows, vocab] logits ever existing at once (``triton_ops.py:64-92``).

    ``hidden`` [rows, H], ``weight`` [vocab, H] (``nn.Linear(bias=False).weight``),
    ``labels`` [rows] int32/int64; rows labelled ``ignore_index`` contribute
    nothing (all ignored: loss 0, zero gradients).  Rows are processed in chunks
    of at most 2 GB of logits: one GEMM for the chunk's logits, the HIP
    cross-entropy row kernel (loss and, in place, the logits gradient), then
    the two gradient GEMMs; the gradients are computed in the
    forward and scaled by the incoming gradient in the backward, as the
    reference does.  Under CUDA autocast the GEMMs run in the autocast dtype
    (what ``F.linear`` + ``F.cross_entropy`` do there); otherwise in hidden's
    dtype.  The loss is fp32.
    """
    if hidden.ndim != 2:
        raise ValueError("hidden must have shape [rows, hidden_dim]")
    if weight.ndim != 2 or weight.shape[1] != hidden.shape[1]:
        raise ValueError("weight must have shape [vocab, hidden_dim] matching hidden's last dim")
    if labels.ndim != 1 or labels.shape[0] != hidden.shape[0]:
        raise ValueError("labels must be a 1D tensor with one entry per hidden row")
    if labels.dtype not in (torch.int32, torch.int64):
        raise ValueError("labels must be an integer tensor")
    _check_device_dtype(hidden, "hidden")
    _check_device_dtype(weight, "weight")
    if torch.is_autocast_enabled("cuda"):
        compute = torch.get_autocast_dtype("cuda")
    else:
        compute = torch.promote_types(hidden.dtype, weight.dtype)
    need_grad = torch.is_grad_enabled() and (hidden.requires_grad or weight.requires_grad)
    with torch.autocast("cuda", enabled=False):
        loss, _gh, _gw = torch.ops.mega_trading_amd.fused_linear_ce(
            hidden, weight, labels, int(ignore_index), _DT[compute], need_grad)
    return loss


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


def _check_mixed(stream: torch.Tensor, weight: torch.Tensor, act: torch.dtype) -> None:
    if stream.dtype != torch.float32 or weight.dtype != torch.float32:
        raise RuntimeError("the residual stream and the weight must be float32")
    if act not in (torch.bfloat16, torch.float16):
        raise RuntimeError(f"activation dtype {act} unsupported (bfloat16 or float16)")


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


def _rope_table(table: torch.Tensor, name: str, t: int, d: int, device: torch.device) -> torch.Tensor:
    """A [..., rows, D/2] table (leading dims of size 1) as fp32 [rows, D/2] with unit d stride."""
    if table.ndim < 2 or any(n != 1 for n in table.shape[:-2]) or table.shape[-1] != d // 2:
        raise ValueError(f"{name} must be [1, 1, T, D/2] with D/2 = {d // 2} (got {tuple(table.shape)})")
    if table.shape[-2] < t:
        raise ValueError(f"{name} has {table.shape[-2]} rows, fewer than the sequence length {t}")
    if table.device != device:
        raise RuntimeError(f"{name} must be on the device of query")
    flat = table.reshape(table.shape[-2], table.shape[-1]).to(torch.float32)
    if flat.stride(-1) != 1:
        flat = flat.contiguous()
    return flat


def _ptr_or_none(t: Optional[torch.Tensor]) -> Optional[int]:
    return t.data_ptr() if t is not None else None


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


@torch.library.custom_op("mega_trading_amd::rms_norm_fwd_mixed", mutates_args=(), device_types="cuda")
def rms_norm_fwd_mixed(x: torch.Tensor, weight: torch.Tensor, eps: float, act: int
                       ) -> tuple[torch.Tensor, torch.Tensor]:
    """x fp32 -> (y in the 16-bit dtype of code ``act``, rstd fp32 [rows])."""
    lib = _native.load()
    x2, sx = _rows(x)
    w = _flat(weight)
    rows, d = x2.shape
    y = torch.empty((rows, d), device=x.device, dtype=_DTYPE_OF[act])
    rstd = torch.empty((rows,), device=x.device, dtype=torch.float32)
    with torch.cuda.device(x.device):
        rc = lib.mt_rms_norm_fwd_mixed(x2.data_ptr(), sx, w.data_ptr(), y.data_ptr(), rstd.data_ptr(), rows, d, eps,
                                       act, _DT[w.dtype], _stream(x))
    _native.check(rc, "mt_rms_norm_fwd_mixed")
    return y.view(x.shape), rstd


@rms_norm_fwd_mixed.register_fake
def _rms_norm_fwd_mixed_fake(x, weight, eps, act):
    return x.new_empty(x.shape, dtype=_DTYPE_OF[act]), x.new_empty((x.numel() // max(x.shape[-1], 1),),
                                                                  dtype=torch.float32)


@torch.library.custom_op("mega_trading_amd::add_rms_norm_fwd_mixed", mutates_args=(), device_types="cuda")
def add_rms_norm_fwd_mixed(x: torch.Tensor, residual: torch.Tensor, weight: torch.Tensor, eps: float
                           ) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """x 16-bit, residual fp32 -> (new_residual fp32, y in x's dtype, rstd)."""
    lib = _native.load()
    x2, sx = _rows(x)
    r2, sr = _rows(residual)
    w = _flat(weight)
    rows, d = x2.shape
    new_res = torch.empty((rows, d), device=x.device, dtype=torch.float32)
    y = torch.empty((rows, d), device=x.device, dtype=x.dtype)
    rstd = torch.empty((rows,), device=x.device, dtype=torch.float32)
    with torch.cuda.device(x.device):
        rc = lib.mt_add_rms_norm_fwd_mixed(x2.data_ptr(), sx, r2.data_ptr(), sr, w.data_ptr(), new_res.data_ptr(),
                                           y.data_ptr(), rstd.data_ptr(), rows, d, eps, _DT[x.dtype], _DT[w.dtype],
                                           _stream(x))
    _native.check(rc, "mt_add_rms_norm_fwd_mixed")
    return new_res.view(x.shape), y.view(x.shape), rstd


@add_rms_norm_fwd_mixed.register_fake
def _add_rms_norm_fwd_mixed_fake(x, residual, weight, eps):
    rows = x.numel() // max(x.shape[-1], 1)
    return (x.new_empty(x.shape, dtype=torch.float32), x.new_empty(x.shape),
            x.new_empty((rows,), dtype=torch.float32))


@torch.library.custom_op("mega_trading_amd::rms_norm_bwd_mixed", mutates_args=(), device_types="cuda")
def rms_norm_bwd_mixed(s: torch.Tensor, weight: torch.Tensor, rstd: torch.Tensor, d_new_residual: Optional[torch.Tensor],
                       dy: torch.Tensor, act: int, want16: bool) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """(ds fp32 [+ d_new_residual], ds rounded to ``act`` when ``want16`` (else
    an empty tensor), dweight fp32) for s fp32 and dy 16-bit."""
    lib = _native.load()
    d = s.shape[-1]
    s2 = _flat(s.reshape(-1, d))
    dy2 = _flat(dy.to(_DTYPE_OF[act]).reshape(-1, d))
    dr2 = _flat(d_new_residual.to(torch.float32).reshape(-1, d)) if d_new_residual is not None else None
    w = _flat(weight)
    rows = s2.shape[0]
    ds = torch.empty((rows, d), device=s.device, dtype=torch.float32)
    ds16 = torch.empty((rows, d) if want16 else (0,), device=s.device, dtype=_DTYPE_OF[act])
    dw = torch.empty((d,), device=s.device, dtype=torch.float32)
    with torch.cuda.device(s.device):
        ws_bytes = lib.mt_rms_norm_bwd_workspace_size(rows, d)
        ws = torch.empty(max(ws_bytes, 256), device=s.device, dtype=torch.uint8)
        rc = lib.mt_rms_norm_bwd_mixed(s2.data_ptr(), w.data_ptr(), rstd.data_ptr(), _ptr_or_none(dr2),
                                       dy2.data_ptr(), ds.data_ptr(), ds16.data_ptr() if want16 else None,
                                       dw.data_ptr(), ws.data_ptr(), ws.numel(), rows, d, act, _DT[w.dtype],
                                       _stream(s))
    _native.check(rc, "mt_rms_norm_bwd_mixed")
    return ds.view(s.shape), (ds16.view(s.shape) if want16 else ds16), dw


@rms_norm_bwd_mixed.register_fake
def _rms_norm_bwd_mixed_fake(s, weight, rstd, d_new_residual, dy, act, want16):
    return (s.new_empty(s.shape, dtype=torch.float32),
            s.new_empty(s.shape if want16 else (0,), dtype=_DTYPE_OF[act]), torch.empty_like(weight))


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


def topk_sample(logits: torch.Tensor, noise: torch.Tensor, k: int) -> torch.Tensor:
    """One token per row of fp32 ``logits`` [rows, vocab]: keep the values >=
    the k-th largest (ties included), p = softmax over them, return [rows, 1]
    int64 = the first index of the largest p / ``noise`` (Exponential(1)
    draws, same shape) -- the draw ``torch.multinomial(probs, 1)`` makes after
    the reference's top-k mask (``model.py:141-145``), in one launch
    (``mt_topk_sample``)."""
    if not logits.is_cuda or logits.dtype != torch.float32 or logits.ndim != 2:
        raise RuntimeError("topk_sample takes fp32 [rows, vocab] GPU logits")
    if noise.shape != logits.shape or noise.dtype != torch.float32 or noise.device != logits.device:
        raise ValueError("noise must be fp32 with the logits' shape and device")
    if not 1 <= k <= logits.shape[1] or logits.shape[1] > MAX_SAMPLE_VOCAB:
        raise ValueError(f"need 1 <= k <= vocab <= {MAX_SAMPLE_VOCAB} (k={k}, vocab={logits.shape[1]})")
    return torch.ops.mega_trading_amd.topk_sample(logits, noise, k)


@torch.library.custom_op("mega_trading_amd::topk_sample", mutates_args=(), device_types="cuda")
def _topk_sample_op(logits: torch.Tensor, noise: torch.Tensor, k: int) -> torch.Tensor:
    lib = _native.load()
    x = logits if logits.stride(1) == 1 else logits.contiguous()
    e = noise if noise.stride(1) == 1 else noise.contiguous()
    rows, vocab = x.shape
    out = torch.empty((rows, 1), device=x.device, dtype=torch.int64)
    with torch.cuda.device(x.device):
        rc = lib.mt_topk_sample(x.data_ptr(), x.stride(0), e.data_ptr(), e.stride(0), rows, vocab, k, out.data_ptr(),
                                _native.DTYPE_FP32, _stream(x))
    _native.check(rc, "mt_topk_sample")
    return out


@_topk_sample_op.register_fake
def _topk_sample_fake(logits, noise, k):
    return logits.new_empty((logits.shape[0], 1), dtype=torch.int64)


@torch.library.custom_op("mega_trading_amd::swiglu_packed_fwd", mutates_args=(), device_types="cuda")
def swiglu_packed_fwd(gate_up: torch.Tensor) -> torch.Tensor:
    lib = _native.load()
    gu = _flat(gate_up)
    cols = gu.shape[-1] // 2
    rows = gu.numel() // max(2 * cols, 1)
    out = torch.empty((*gu.shape[:-1], cols), device=gu.device, dtype=gu.dtype)
    with torch.cuda.device(gu.device):
        rc = lib.mt_swiglu_packed_fwd(gu.data_ptr(), out.data_ptr(), rows, cols, _DT[gu.dtype], _stream(gu))
    _native.check(rc, "mt_swiglu_packed_fwd")
    return out


@swiglu_packed_fwd.register_fake
def _swiglu_packed_fwd_fake(gate_up):
    return gate_up.new_empty((*gate_up.shape[:-1], gate_up.shape[-1] // 2))


@torch.library.custom_op("mega_trading_amd::swiglu_packed_bwd", mutates_args=(), device_types="cuda")
def swiglu_packed_bwd(gate_up: torch.Tensor, dout: torch.Tensor) -> torch.Tensor:
    lib = _native.load()
    gu, dy = _flat(gate_up), _flat(dout.to(gate_up.dtype))
    cols = gu.shape[-1] // 2
    rows = gu.numel() // max(2 * cols, 1)
    dgu = torch.empty(gu.shape, device=gu.device, dtype=gu.dtype)
    with torch.cuda.device(gu.device):
        rc = lib.mt_swiglu_packed_bwd(gu.data_ptr(), dy.data_ptr(), dgu.data_ptr(), rows, cols, _DT[gu.dtype],
                                      _stream(gu))
    _native.check(rc, "mt_swiglu_packed_bwd")
    return dgu


@swiglu_packed_bwd.register_fake
def _swiglu_packed_bwd_fake(gate_up, dout):
    return torch.empty_like(gate_up, memory_format=torch.contiguous_format)


# Stand-alone RoPE of query and key in one launch; `inverse` rotates by
# -theta (the backward).  Outputs take the inputs' layout (empty_like).
@torch.library.custom_op("mega_trading_amd::rope_fwd", mutates_args=(), device_types="cuda")
def rope_fwd(query: torch.Tensor, key: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor, inverse: bool
             ) -> tuple[torch.Tensor, torch.Tensor]:
    lib = _native.load()
    q_out, k_out = torch.empty_like(query), torch.empty_like(key)
    b, hq, t, d = query.shape
    strides = (ctypes.c_int64 * 16)(*query.stride(), *q_out.stride(), *key.stride(), *k_out.stride())
    with torch.cuda.device(query.device):
        rc = lib.mt_apply_rope(query.data_ptr(), key.data_ptr(), q_out.data_ptr(), k_out.data_ptr(), b, hq,
                               key.shape[1], t, d, strides, cos.data_ptr(), sin.data_ptr(), cos.stride(0),
                               cos.shape[0], int(inverse), _DT[query.dtype], _stream(query))
    _native.check(rc, "mt_apply_rope")
    return q_out, k_out


@rope_fwd.register_fake
def _rope_fwd_fake(query, key, cos, sin, inverse):
    return torch.empty_like(query), torch.empty_like(key)


# Logits bytes per chunk.  Measured at the C5 shape (32768 x 16384 bf16 logits,
# fwd + bwd): 64 MB chunks (cache-resident) 3.8 ms, 256 MB 2.7 ms, one 1 GB
# chunk 2.3 ms (the three GEMMs alone take 1.6 ms), against 4.4 ms for the eager
# F.linear + F.cross_entropy: on MI355X full-size GEMMs beat cache-resident
# chunks, and 288 GB of HBM leaves room for the whole logits tensor, so chunking
# only bounds memory for batches beyond 2 GB of logits.
_CE_CHUNK_BYTES = 2 << 30


@torch.library.custom_op("mega_trading_amd::fused_linear_ce", mutates_args=(), device_types="cuda")
def fused_linear_ce(hidden: torch.Tensor, weight: torch.Tensor, labels: torch.Tensor, ignore_index: int,
                    compute_dtype: int, need_grad: bool) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """(loss fp32 scalar, d loss / d hidden, d loss / d weight); the gradients are
    empty tensors when need_grad is False."""
    lib = _native.load()
    ct = _DTYPE_OF[compute_dtype]
    rows, h = hidden.shape
    vocab = weight.shape[0]
    # a vocab that is not a multiple of 8 (the reference tokenizer's always is
    # odd) gets zero weight rows up to the next multiple: the logits rows then
    # have a padded stride, and the row kernel ignores the pad columns and
    # writes them a zero gradient, so the pad rows contribute nothing
    vpad = (vocab + 7) // 8 * 8
    hc = hidden.to(ct).contiguous()
    if vpad == vocab:
        wc = weight.to(ct).contiguous()
    else:
        wc = torch.zeros((vpad, h), device=weight.device, dtype=ct)
        wc[:vocab].copy_(weight)
    lab = labels.to(torch.int64).contiguous()
    n_valid = (lab != ignore_index).sum()  # stays on the device: the kernel reads it
    loss_rows = torch.empty((rows,), device=hidden.device, dtype=torch.float32)
    if need_grad:
        gh = torch.empty((rows, h), device=hidden.device, dtype=ct)
        gw = torch.zeros((vpad, h), device=hidden.device, dtype=torch.float32)
    chunk = max(1, min(rows, _CE_CHUNK_BYTES // (vpad * ct.itemsize)))
    with torch.cuda.device(hidden.device), tuned_gemms():
        stream = _stream(hidden)
        for start in range(0, rows, chunk):
            end = min(rows, start + chunk)
            logits = torch.mm(hc[start:end], wc.t())  # [chunk, vocab] in ct, fp32 accumulation
            rc = lib.mt_cross_entropy_rows(logits.data_ptr(), logits.stride(0), lab[start:end].data_ptr(), end - start,
                                           vocab, n_valid.data_ptr(), ignore_index, loss_rows[start:end].data_ptr(),
                                           1 if need_grad else 0, compute_dtype, stream)
            _native.check(rc, "mt_cross_entropy_rows")
            if need_grad:  # logits now hold d loss / d logits
                torch.mm(logits, wc, out=gh[start:end])
                gw.add_(torch.mm(logits.t(), hc[start:end]))
    loss = loss_rows.sum()
    if not need_grad:
        return loss, hidden.new_empty((0,)), weight.new_empty((0,))
    return loss, gh.to(hidden.dtype), gw[:vocab].to(weight.dtype)


@fused_linear_ce.register_fake
def _fused_linear_ce_fake(hidden, weight, labels, ignore_index, compute_dtype, need_grad):
    loss = hidden.new_empty((), dtype=torch.float32)
    if not need_grad:
        return loss, hidden.new_empty((0,)), weight.new_empty((0,))
    return loss, torch.empty_like(hidden), torch.empty_like(weight)


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


def _rms_mixed_setup(ctx, inputs, output):
    x, weight, _eps, act = inputs
    _y, rstd = output
    ctx.act = act
    ctx.save_for_backward(x, weight, rstd)
    ctx.set_materialize_grads(False)


def _rms_mixed_backward(ctx, dy, _drstd):
    x, weight, rstd = ctx.saved_tensors
    if dy is None:
        return None, None, None, None
    dx, _ds16, dw = torch.ops.mega_trading_amd.rms_norm_bwd_mixed(x, weight, rstd, None, dy, ctx.act, False)
    return dx, dw, None, None


def _add_rms_mixed_setup(ctx, inputs, output):
    x, _residual, weight, _eps = inputs
    new_res, _y, rstd = output
    ctx.act = _DT[x.dtype]
    ctx.save_for_backward(new_res, weight, rstd)
    ctx.set_materialize_grads(False)


def _add_rms_mixed_backward(ctx, d_new_res, dy, _drstd):
    new_res, weight, rstd = ctx.saved_tensors
    if dy is None:
        if d_new_res is None:
            return None, None, None, None
        # only the sum is used: both inputs get its gradient (in their dtypes)
        return d_new_res.to(_DTYPE_OF[ctx.act]), d_new_res, None, None
    ds, ds16, dw = torch.ops.mega_trading_amd.rms_norm_bwd_mixed(new_res, weight, rstd, d_new_res, dy, ctx.act, True)
    return ds16, ds, dw, None


def _swiglu_setup(ctx, inputs, output):
    gate, up = inputs
    ctx.save_for_backward(gate, up)
    ctx.set_materialize_grads(False)


def _swiglu_backward(ctx, dout):
    gate, up = ctx.saved_tensors
    if dout is None:
        return None, None
    return torch.ops.mega_trading_amd.swiglu_bwd(gate, up, dout)


def _swiglu_packed_setup(ctx, inputs, output):
    ctx.save_for_backward(inputs[0])
    ctx.set_materialize_grads(False)


def _swiglu_packed_backward(ctx, dout):
    (gate_up,) = ctx.saved_tensors
    if dout is None:
        return None
    return torch.ops.mega_trading_amd.swiglu_packed_bwd(gate_up, dout)


def _rope_setup(ctx, inputs, output):
    _q, _k, cos, sin, inverse = inputs
    ctx.inverse = inverse
    ctx.save_for_backward(cos, sin)


def _rope_backward(ctx, dq, dk):
    # a rotation's gradient is the opposite rotation (an unused output's
    # gradient arrives as zeros: grads are materialized)
    cos, sin = ctx.saved_tensors
    gq, gk = torch.ops.mega_trading_amd.rope_fwd(dq, dk, cos, sin, not ctx.inverse)
    return gq, gk, None, None, None


def _ce_setup(ctx, inputs, output):
    _h, _w, _labels, _ignore, _dt, need_grad = inputs
    _loss, gh, gw = output
    ctx.need_grad = need_grad
    ctx.save_for_backward(gh, gw)
    ctx.mark_non_differentiable(gh, gw)
    ctx.set_materialize_grads(False)


def _ce_backward(ctx, dloss, _dgh, _dgw):
    gh, gw = ctx.saved_tensors
    if dloss is None or not ctx.need_grad:
        return None, None, None, None, None, None
    return gh * dloss.to(gh.dtype), gw * dloss.to(gw.dtype), None, None, None, None


rms_norm_fwd.register_autograd(_rms_backward, setup_context=_rms_setup)
fused_linear_ce.register_autograd(_ce_backward, setup_context=_ce_setup)
add_rms_norm_fwd.register_autograd(_add_rms_backward, setup_context=_add_rms_setup)
swiglu_fwd.register_autograd(_swiglu_backward, setup_context=_swiglu_setup)
swiglu_packed_fwd.register_autograd(_swiglu_packed_backward, setup_context=_swiglu_packed_setup)
rms_norm_fwd_mixed.register_autograd(_rms_mixed_backward, setup_context=_rms_mixed_setup)
add_rms_norm_fwd_mixed.register_autograd(_add_rms_mixed_backward, setup_context=_add_rms_mixed_setup)
rope_fwd.register_autograd(_rope_backward, setup_context=_rope_setup)
