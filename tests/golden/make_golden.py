"""Write the golden vectors in this directory.

The reference holds no stored vectors for its attention path: its own parity
tests compare live against ``torch.nn.functional.scaled_dot_product_attention``
(``tests/test_training.py:519-600``), the routine its eager path calls at
``src/mega_trading/model.py:228-235``.  These fixtures freeze that routine's
output (torch on the CPU, fp32, this image's torch 2.10.0) so the oracle is
pinned to concrete numbers that do not depend on re-running torch:

* ``c1_sdpa_fp32.npz``  -- BASELINE config 1: B=2, T=256, Hq=4, Hkv=2, D=32,
  Q/K/V/dO ~ N(0,1) drawn in that order from ``torch.Generator().manual_seed(0)``.
  Holds O, LSE (natural log), dQ, dK, dV and the SHA-256 of the regenerated
  inputs (the inputs themselves are re-drawn from the seed by the tests).
* ``t17_sdpa_fp32.npz`` -- the reference's small parity shape
  (``test_training.py:519-548``: B=1, Hq=4, Hkv=2, T=17, D=32, seed 11), with
  its inputs stored.
* ``rope_t17_fp32.npz`` -- RoPE tables for theta 1e4 and 5e5 built exactly as
  ``RotaryEmbedding.__init__`` (``model.py:279-284``), and the gradient of
  ``SDPA(rope(q), rope(k), v)`` w.r.t. the un-rotated q, k via autograd through
  the interleaved rotation of ``model.py:312-316`` (theta 1e4, T=17).

Run from the repository root:  ``python tests/golden/make_golden.py``
"""

from __future__ import annotations

import hashlib
import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

from oracle.sdpa_cpu import masked_logsumexp, rope_tables_torch, sdpa_forward_backward  # noqa: E402


def c1_inputs() -> tuple[torch.Tensor, ...]:
    """BASELINE config 1 inputs (seeded draw order Q, K, V, dO)."""
    g = torch.Generator().manual_seed(0)
    q = torch.randn(2, 4, 256, 32, generator=g)
    k = torch.randn(2, 2, 256, 32, generator=g)
    v = torch.randn(2, 2, 256, 32, generator=g)
    do = torch.randn(2, 4, 256, 32, generator=g)
    return q, k, v, do


def input_digest(*tensors: torch.Tensor) -> str:
    h = hashlib.sha256()
    for t in tensors:
        h.update(t.contiguous().numpy().astype("<f4").tobytes())
    return h.hexdigest()


def t17_inputs() -> tuple[torch.Tensor, ...]:
    g = torch.Generator().manual_seed(11)
    q = torch.randn(1, 4, 17, 32, generator=g)
    k = torch.randn(1, 2, 17, 32, generator=g)
    v = torch.randn(1, 2, 17, 32, generator=g)
    do = torch.randn(1, 4, 17, 32, generator=g)
    return q, k, v, do


def _rotate(x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor) -> torch.Tensor:
    even, odd = x[..., 0::2], x[..., 1::2]
    return torch.stack((even * cos - odd * sin, even * sin + odd * cos), dim=-1).flatten(start_dim=-2)


def main() -> None:
    torch.set_num_threads(min(8, os.cpu_count() or 1))

    q, k, v, do = c1_inputs()
    o, dq, dk, dv = sdpa_forward_backward(q, k, v, do, repeats=2)
    lse = masked_logsumexp(q, k, repeats=2)
    np.savez_compressed(
        os.path.join(HERE, "c1_sdpa_fp32.npz"),
        o=o.numpy(), lse=lse.numpy(), dq=dq.numpy(), dk=dk.numpy(), dv=dv.numpy(),
        input_sha256=np.array(input_digest(q, k, v, do)),
    )

    q, k, v, do = t17_inputs()
    o, dq, dk, dv = sdpa_forward_backward(q, k, v, do, repeats=2)
    lse = masked_logsumexp(q, k, repeats=2)
    np.savez_compressed(
        os.path.join(HERE, "t17_sdpa_fp32.npz"),
        q=q.numpy(), k=k.numpy(), v=v.numpy(), do=do.numpy(),
        o=o.numpy(), lse=lse.numpy(), dq=dq.numpy(), dk=dk.numpy(), dv=dv.numpy(),
    )

    cos4, sin4 = rope_tables_torch(17, 32, 10_000.0)
    cos5, sin5 = rope_tables_torch(17, 32, 500_000.0)
    qr = q.clone().requires_grad_(True)
    kr = k.clone().requires_grad_(True)
    vr = v.clone().requires_grad_(True)
    out = torch.nn.functional.scaled_dot_product_attention(
        _rotate(qr, cos4, sin4), _rotate(kr, cos4, sin4), vr, is_causal=True, enable_gqa=True
    )
    gq, gk, gv = torch.autograd.grad(out, (qr, kr, vr), do)
    np.savez_compressed(
        os.path.join(HERE, "rope_t17_fp32.npz"),
        cos_1e4=cos4.numpy(), sin_1e4=sin4.numpy(), cos_5e5=cos5.numpy(), sin_5e5=sin5.numpy(),
        o=out.detach().numpy(), dq=gq.numpy(), dk=gk.numpy(), dv=gv.numpy(),
    )
    for name in sorted(os.listdir(HERE)):
        if name.endswith(".npz"):
            print(name, os.path.getsize(os.path.join(HERE, name)))


if __name__ == "__main__":
    main()
