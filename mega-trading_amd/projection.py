"""Decoder projections on the "hip" route: ``nn.Linear(bias=False)`` products
(``model.py:209-212`` q/k/v/o, ``model.py:243-245`` w1/w2/w3) with a split-K
weight gradient and optional weight grouping.

``project(x, weights)`` returns ``x @ w.T`` for every ``w`` in ``weights``
from ONE GEMM against the row-concatenated weights (the q/k/v projections
of a layer, or its w1/w3 pair, read the activations once), as views of the
packed [rows, sum(out)] result.  The dtype rules are ``F.linear``'s under
autocast: inside a CUDA autocast region the product runs in the autocast
dtype, otherwise in the promoted dtype of ``x`` and the weights; the
parameters stay in their own dtype and get gradients of that dtype.

Few rows without autograd (the decode step of generation: one token per
rollout, at most 64 rows, fp32 as the reference's eval runs the model):
``mt_linear_rows`` computes the packed result in one launch that reads every
weight in place, instead of concatenating the weights (a copy of each weight
per call) and running a library GEMM that is latency-bound at these sizes.

Backward:
* dX = dY W: one GEMM over the packed gradient.
* dW = dYᵀ X reduces over every token (batch x time rows, 32768 at the
  C5 shape) into a small output (128..2816 x 512).  A single library GEMM
  covers that output with a few dozen workgroups on 256 CUs; instead the
  rows are cut into S chunks of at least 1024 rows and the S chunk
  products run as one batched GEMM with fp32 outputs, summed in fp32.
  On MI355X this is 2.5-4x faster at the C5 shapes, and the gradient keeps
  fp32 accumulation until it reaches the fp32 parameter (the autocast
  ``F.linear`` backward rounds it to bf16 first).
"""

from __future__ import annotations

import ctypes
from typing import Sequence

import torch

from . import _native
from .gemm_tuning import tuned_gemms

__all__ = ["project", "project_packed", "split_k_chunks"]

_MIN_CHUNK_ROWS = 1024
_MAX_CHUNKS = 16


def split_k_chunks(rows: int) -> int:
    """Chunks of the weight-gradient reduction: the largest S in 16, 8, 4, 2
    that divides ``rows`` into chunks of at least 1024 rows, else 1."""
    s = _MAX_CHUNKS
    while s > 1 and (rows % s or rows // s < _MIN_CHUNK_ROWS):
        s //= 2
    return s


def _compute_dtype(x: torch.Tensor, weights: Sequence[torch.Tensor]) -> torch.dtype:
    if x.device.type == "cuda" and torch.is_autocast_enabled("cuda"):
        return torch.get_autocast_dtype("cuda")
    dt = x.dtype
    for w in weights:
        dt = torch.promote_types(dt, w.dtype)
    return dt


def _weight_grad(dy: torch.Tensor, x: torch.Tensor) -> torch.Tensor:
    """dYᵀ X for dY [rows, out], X [rows, in] (same dtype), accumulated and
    returned in fp32 (fp64 for fp64 inputs)."""
    rows, out = dy.shape
    s = split_k_chunks(rows)
    wide = dy.dtype in (torch.float32, torch.float64)
    if s > 1:
        dy, x = dy.view(s, rows // s, out).transpose(1, 2), x.view(s, rows // s, x.shape[1])
    else:
        dy = dy.t()
    mm = torch.bmm if s > 1 else torch.mm
    if wide:
        part = mm(dy, x)
    elif dy.device.type == "cuda":
        part = mm(dy, x, out_dtype=torch.float32)  # 16-bit operands, fp32 accumulate and output
    else:
        part = mm(dy.float(), x.float())
    return part.sum(0) if s > 1 else part


class _Project(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x, dtype, *weights):
        with torch.autocast("cuda", enabled=False):
            # one concatenation, then one cast (the same values as casting each weight)
            w = (weights[0] if len(weights) == 1 else torch.cat(weights)).to(dtype)
            x2 = x.reshape(-1, x.shape[-1]).to(dtype)
            with tuned_gemms():
                y = x2 @ w.t()
        ctx.save_for_backward(x2, w)
        ctx.outs = [v.shape[0] for v in weights]
        ctx.x_shape = x.shape
        ctx.w_dtypes = [v.dtype for v in weights]
        return y.view(*x.shape[:-1], w.shape[0])

    @staticmethod
    def backward(ctx, dy):
        x2, w = ctx.saved_tensors
        dy = dy.reshape(x2.shape[0], w.shape[0]).to(w.dtype)
        dx = None
        if ctx.needs_input_grad[0]:
            with tuned_gemms():
                dx = (dy @ w).view(ctx.x_shape)
        dws = [None] * len(ctx.outs)
        if any(ctx.needs_input_grad[2:]):
            dw = _weight_grad(dy, x2)
            dws = [g.to(dt) if need else None
                   for g, dt, need in zip(dw.split(ctx.outs, dim=0), ctx.w_dtypes, ctx.needs_input_grad[2:])]
        return (dx, None, *dws)


_ROWS_MAX = 64     # rows of one mt_linear_rows launch
_X_DTYPES = {torch.float32: _native.DTYPE_FP32, torch.bfloat16: _native.DTYPE_BF16, torch.float16: _native.DTYPE_FP16}
_ROWS_GROUPS = 4   # weights of one launch


def _rows_path(x2: torch.Tensor, weights: Sequence[torch.Tensor], dtype: torch.dtype) -> bool:
    """Whether ``mt_linear_rows`` takes the product: no autograd, fp32 weights
    and compute (x fp32, or 16-bit widened exactly as the promotion to fp32
    would), at most 64 rows and 4 weights, in_features a multiple of 128,
    aligned rows with unit last strides."""
    if dtype != torch.float32 or x2.dtype not in _X_DTYPES or x2.device.type != "cuda":
        return False
    if torch.is_grad_enabled() and (x2.requires_grad or any(w.requires_grad for w in weights)):
        return False
    rows, k = x2.shape
    if not 1 <= rows <= _ROWS_MAX or k % 128 or len(weights) > _ROWS_GROUPS:
        return False
    if x2.stride(1) != 1 or x2.stride(0) % 4 or x2.data_ptr() % (16 if x2.dtype == torch.float32 else 8):
        return False
    return all(w.dtype == torch.float32 and w.device == x2.device and w.stride(1) == 1 and w.stride(0) % 4 == 0
               and w.data_ptr() % 16 == 0 for w in weights)


@torch.library.custom_op("mega_trading_amd::linear_rows", mutates_args=(), device_types="cuda")
def linear_rows(x: torch.Tensor, weights: list[torch.Tensor]) -> torch.Tensor:
    """[rows, sum(out_i)] = cat([x.float() @ w.T for w in weights], -1), fp32,
    for x [rows <= 64, K] (fp32 or 16-bit) and fp32 weights [out_i, K]
    (``mt_linear_rows``)."""
    lib = _native.load()
    rows, k = x.shape
    outs = [w.shape[0] for w in weights]
    y = torch.empty((rows, sum(outs)), device=x.device, dtype=torch.float32)
    g = len(weights)
    ptrs = (ctypes.c_void_p * g)(*[w.data_ptr() for w in weights])
    ns = (ctypes.c_int * g)(*outs)
    lds = (ctypes.c_int64 * g)(*[w.stride(0) for w in weights])
    with torch.cuda.device(x.device):
        rc = lib.mt_linear_rows(x.data_ptr(), x.stride(0), ptrs, ns, lds, g, y.data_ptr(), y.stride(0), rows, k,
                                _X_DTYPES[x.dtype], torch.cuda.current_stream(x.device).cuda_stream)
    _native.check(rc, "mt_linear_rows")
    return y


@linear_rows.register_fake
def _linear_rows_fake(x, weights):
    return x.new_empty((x.shape[0], sum(w.shape[0] for w in weights)))


def _check(x: torch.Tensor, weights: Sequence[torch.Tensor]) -> None:
    if not weights:
        raise ValueError("weights must hold at least one matrix")
    d = x.shape[-1]
    for w in weights:
        if w.ndim != 2 or w.shape[1] != d:
            raise ValueError(f"every weight must have shape [out, {d}] (got {tuple(w.shape)})")
        if w.device != x.device:
            raise RuntimeError("weights must be on the device of x")


def project_packed(x: torch.Tensor, weights: Sequence[torch.Tensor]) -> torch.Tensor:
    """``cat([x @ w.T for w in weights], -1)`` from one GEMM: [..., sum(out_i)]."""
    _check(x, weights)
    dtype = _compute_dtype(x, weights)
    x2 = x.reshape(-1, x.shape[-1])
    if _rows_path(x2, weights, dtype):
        return linear_rows(x2, list(weights)).view(*x.shape[:-1], -1)
    return _Project.apply(x, dtype, *weights)


def project(x: torch.Tensor, weights: Sequence[torch.Tensor]) -> tuple[torch.Tensor, ...]:
    """``tuple(x @ w.T for w in weights)`` from one GEMM (see the module notes):
    [..., out_i] column views of the packed result."""
    return torch.split(project_packed(x, weights), [w.shape[0] for w in weights], dim=-1)
