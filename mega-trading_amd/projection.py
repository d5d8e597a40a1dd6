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

from typing import Sequence

import torch

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
    return _Project.apply(x, _compute_dtype(x, weights), *weights)


def project(x: torch.Tensor, weights: Sequence[torch.Tensor]) -> tuple[torch.Tensor, ...]:
    """``tuple(x @ w.T for w in weights)`` from one GEMM (see the module notes):
    [..., out_i] column views of the packed result."""
    return torch.split(project_packed(x, weights), [w.shape[0] for w in weights], dim=-1)
