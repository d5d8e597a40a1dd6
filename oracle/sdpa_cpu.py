"""The reference's eager attention path, run through torch on the CPU.

TEST INFRASTRUCTURE ONLY (tests, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py``).

The reference's non-Triton branch is one library call,
``F.scaled_dot_product_attention(q, k, v, dropout_p, is_causal=True,
enable_gqa=repeats > 1)`` (``src/mega_trading/model.py:228-235``), with autograd
for the backward.  This module restates that call site so the numpy oracle can
be pinned against the library routine itself (torch is the third-party
dependency; the reference pins ``torch==2.11.0`` in ``uv.lock``, this image has
2.10.0), and so ``bench.py`` can time the reference's CPU attention on the host
cores as the CPU baseline.
"""

from __future__ import annotations

import torch
import torch.nn.functional as F


def sdpa_forward(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, repeats: int) -> torch.Tensor:
    """``model.py:228-235``: causal SDPA with native GQA."""
    return F.scaled_dot_product_attention(q, k, v, dropout_p=0.0, is_causal=True, enable_gqa=repeats > 1)


def sdpa_forward_backward(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    do: torch.Tensor,
    repeats: int,
) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor, torch.Tensor]:
    """Forward plus ``autograd.grad`` into (q, k, v), as the reference benchmark's
    ``_attention_step`` (``scripts/benchmark_triton_attention.py:133-146``)."""
    q = q.detach().requires_grad_(True)
    k = k.detach().requires_grad_(True)
    v = v.detach().requires_grad_(True)
    with torch.enable_grad():
        out = sdpa_forward(q, k, v, repeats)
        dq, dk, dv = torch.autograd.grad(out, (q, k, v), do)
    return out.detach(), dq, dk, dv


def masked_logsumexp(q: torch.Tensor, k: torch.Tensor, repeats: int) -> torch.Tensor:
    """Natural-log LSE of the causal scaled scores, ``triton_attention.py:346-349``.

    Computed with ``torch.logsumexp`` on the dense masked score matrix (small
    inputs only)."""
    d = q.shape[-1]
    kk = k.repeat_interleave(repeats, dim=1) if repeats > 1 else k
    s = torch.matmul(q, kk.transpose(-2, -1)) / (d ** 0.5)
    t = q.shape[-2]
    mask = torch.ones((t, t), dtype=torch.bool).tril()
    s = s.masked_fill(~mask, float("-inf"))
    return torch.logsumexp(s, dim=-1)


def rope_tables_torch(seq_len: int, head_dim: int, theta: float) -> tuple[torch.Tensor, torch.Tensor]:
    """fp32 tables exactly as ``RotaryEmbedding.__init__`` builds them (``model.py:279-284``)."""
    positions = torch.arange(seq_len, dtype=torch.float32)
    inv_freq = 1.0 / (theta ** (torch.arange(0, head_dim, 2, dtype=torch.float32) / head_dim))
    freqs = torch.outer(positions, inv_freq)
    return freqs.cos(), freqs.sin()
