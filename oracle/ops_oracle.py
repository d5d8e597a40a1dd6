"""CPU oracle for the decoder's memory-bound operators: RMSNorm, residual-add +
RMSNorm, and the SwiGLU gate (forward and backward).

TEST INFRASTRUCTURE ONLY.  Nothing in the shipped package imports this file:
only ``tests/`` (and ``__graft_entry__.smoke()`` / ``bench.py``'s
``cpu_baseline`` leg, should they need it) use it, and only as the checker.

Plain numpy restatements of the reference operators
(``src/mega_trading/kernels/triton_ops.py``), each citing the lines it follows:

* ``rms_norm_forward``      -- kernel ``:528-539``: ``y = x * rsqrt(mean(x^2) + eps) * w``,
                               ``rstd`` saved per row; output in the input dtype.
* ``rms_norm_backward``     -- kernel ``:633-666`` and ``:183``:
                               ``g = dy * w``, ``c = sum(g * x)``,
                               ``dx = rstd * (g - x * rstd^2 / D * c)``,
                               ``dw = sum_rows(dy * x * rstd)``.
* ``add_rms_norm_forward``  -- kernel ``:541-566``: ``s = x + r`` in fp32, ``s`` stored
                               in the input dtype, the norm taken of the unrounded ``s``.
* ``add_rms_norm_backward`` -- kernel ``:569-608``: the RMSNorm backward on the stored
                               ``s`` plus the direct residual gradient; the same
                               gradient for both add inputs (``:288-291``).
* ``swiglu_forward``        -- kernel ``:774-782``: ``silu(g) = g * sigmoid(g)`` in fp32
                               (evaluated as ``g / (1 + exp(-g))``, the form torch's
                               ``silu`` uses), rounded to the storage type, times
                               ``up``, rounded.
* ``swiglu_backward``       -- kernel ``:799-819``: ``t = round(dy * up)``,
                               ``dg = t * sig * (1 + g (1 - sig))``,
                               ``du = dy * round(silu(g))``.
* ``cross_entropy_rows``    -- kernel ``:822-887``: per row ``lse = logsumexp(logits)``,
                               ``loss = (lse - logits[label]) / n_valid`` and
                               ``grad = (softmax - onehot(label)) / n_valid``; rows labelled
                               ``ignore_index`` give 0 and a zero row.
* ``fused_linear_cross_entropy`` -- ``:294-412``: the mean loss of ``hidden @ weight.T`` and
                               its gradients ``grad_logits @ weight``, ``grad_logits.T @ hidden``,
                               with the compute-dtype roundings of the inputs and logits.

Arithmetic is float64 for the RMSNorm functions (compare with a tolerance) and
float32 with explicit storage roundings for the SwiGLU gate (so 16-bit results
can be compared value for value).  ``round_to`` emulates a store to bf16
(round to nearest even), fp16 or fp32.

How each part is pinned (tests/test_ops_oracle.py): against torch CPU
(``F.rms_norm`` + autograd, ``F.silu(g) * up`` + autograd -- the routines the
reference's eager path calls, ``model.py:254-255, 269``), in float64 and, for
the SwiGLU roundings, in bfloat16; against closed forms (scale invariance,
unit RMS of the output, ``silu(0) = 0``, ``silu'(0) = 1/2``,
``silu(-x) = silu(x) - x``, the ``dx . x`` identity, finite differences);
and against planted mistakes (eps outside the root, a dropped weight, a mean
over D - 1, a missing ``(1 - sig)`` term, no rounding of silu) that each fail
one of those checks.
"""

from __future__ import annotations

import numpy as np

__all__ = [
    "round_to",
    "rms_norm_forward",
    "rms_norm_backward",
    "add_rms_norm_forward",
    "add_rms_norm_backward",
    "swiglu_forward",
    "swiglu_backward",
    "cross_entropy_rows",
    "fused_linear_cross_entropy",
]


def round_to(x: np.ndarray, dtype: str) -> np.ndarray:
    """Value after a store to ``dtype`` ("bfloat16", "float16", "float32"), as float32."""
    x = np.asarray(x, dtype=np.float32)
    if dtype == "float32":
        return x.copy()
    if dtype == "float16":
        return x.astype(np.float16).astype(np.float32)
    if dtype != "bfloat16":
        raise ValueError(dtype)
    bits = x.view(np.uint32).astype(np.uint64)
    nan = np.isnan(x)
    bits = (bits + 0x7FFF + ((bits >> 16) & 1)) & 0xFFFF0000  # round to nearest even on the top 16 bits
    out = bits.astype(np.uint32).view(np.float32)
    return np.where(nan, np.float32(np.nan), out)


def rms_norm_forward(x: np.ndarray, w: np.ndarray, eps: float, out_dtype: str = "float32"):
    """(y, rstd) of ``triton_ops.py:528-539``; x [rows, D] (float64 arithmetic)."""
    x = np.asarray(x, dtype=np.float64)
    w = np.asarray(w, dtype=np.float64)
    rstd = 1.0 / np.sqrt(np.mean(x * x, axis=-1) + eps)
    y = x * rstd[:, None] * w[None, :]
    return round_to(y, out_dtype), rstd


def rms_norm_backward(x: np.ndarray, w: np.ndarray, rstd: np.ndarray, dy: np.ndarray):
    """(dx, dw) of ``triton_ops.py:633-666`` and ``:183`` (float64)."""
    x = np.asarray(x, dtype=np.float64)
    w = np.asarray(w, dtype=np.float64)
    dy = np.asarray(dy, dtype=np.float64)
    rstd = np.asarray(rstd, dtype=np.float64)
    d = x.shape[-1]
    g = dy * w[None, :]
    c = np.sum(g * x, axis=-1)
    dx = rstd[:, None] * (g - x * (rstd * rstd / d * c)[:, None])
    dw = np.sum(dy * x * rstd[:, None], axis=0)
    return dx, dw


def add_rms_norm_forward(x: np.ndarray, r: np.ndarray, w: np.ndarray, eps: float, dtype: str = "float32"):
    """(new_residual, y, rstd) of ``triton_ops.py:541-566``."""
    s32 = np.asarray(x, dtype=np.float32) + np.asarray(r, dtype=np.float32)  # fp32 sum, as the kernel
    y, rstd = rms_norm_forward(s32.astype(np.float64), w, eps, dtype)
    return round_to(s32, dtype), y, rstd


def add_rms_norm_backward(new_residual, w, rstd, d_new_residual, dy):
    """(d hidden = d residual, dw) of ``triton_ops.py:569-608``."""
    dx, dw = rms_norm_backward(new_residual, w, rstd, dy)
    return dx + np.asarray(d_new_residual, dtype=np.float64), dw


def _silu32(g: np.ndarray) -> np.ndarray:
    g = np.asarray(g, dtype=np.float32)
    with np.errstate(over="ignore"):
        return (g / (np.float32(1) + np.exp(-g))).astype(np.float32)


def swiglu_forward(g: np.ndarray, up: np.ndarray, dtype: str = "bfloat16") -> np.ndarray:
    """``round(round(silu(g)) * up)`` (``triton_ops.py:774-782``), float32 arithmetic."""
    silu = round_to(_silu32(g), dtype)
    return round_to(silu * np.asarray(up, dtype=np.float32), dtype)


def swiglu_backward(g: np.ndarray, up: np.ndarray, dy: np.ndarray, dtype: str = "bfloat16"):
    """(dg, du) of ``triton_ops.py:799-819``, float32 arithmetic with storage roundings."""
    g = np.asarray(g, dtype=np.float32)
    up = np.asarray(up, dtype=np.float32)
    dy = np.asarray(dy, dtype=np.float32)
    with np.errstate(over="ignore"):
        sig = (np.float32(1) / (np.float32(1) + np.exp(-g))).astype(np.float32)
    t = round_to(dy * up, dtype)
    dg = round_to((t * sig) * (np.float32(1) + g * (np.float32(1) - sig)), dtype)
    du = round_to(dy * round_to(_silu32(g), dtype), dtype)
    return dg, du


def cross_entropy_rows(logits: np.ndarray, labels: np.ndarray, ignore_index: int = -100):
    """(loss per row, d loss / d logits) of ``triton_ops.py:822-887`` (float64)."""
    x = np.asarray(logits, dtype=np.float64)
    labels = np.asarray(labels, dtype=np.int64)
    keep = labels != ignore_index
    n_valid = int(keep.sum())
    inv_n = 1.0 / n_valid if n_valid else 0.0
    m = np.max(x, axis=-1, keepdims=True)
    lse = (m + np.log(np.sum(np.exp(x - m), axis=-1, keepdims=True)))[:, 0]
    rows = np.arange(x.shape[0])
    safe = np.where(keep, labels, 0)
    loss = np.where(keep, (lse - x[rows, safe]) * inv_n, 0.0)
    grad = np.exp(x - lse[:, None])
    grad[rows, safe] -= 1.0
    grad *= inv_n
    grad[~keep] = 0.0
    return loss, grad


def fused_linear_cross_entropy(hidden, weight, labels, ignore_index: int = -100, compute: str = "bfloat16"):
    """(mean loss, d/d hidden, d/d weight) of ``triton_ops.py:294-412`` in float64 on
    compute-dtype-rounded hidden and weight, with the logits rounded to that dtype
    (the GEMM's output type) before the cross-entropy."""
    h = round_to(np.asarray(hidden, dtype=np.float32), compute).astype(np.float64)
    w = round_to(np.asarray(weight, dtype=np.float32), compute).astype(np.float64)
    logits = round_to((h @ w.T).astype(np.float32), compute)
    loss_rows, grad = cross_entropy_rows(logits, labels, ignore_index)
    return float(np.sum(loss_rows)), grad @ w, grad.T @ h
