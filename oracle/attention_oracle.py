"""CPU oracle for causal grouped-query attention with interleaved RoPE.

TEST INFRASTRUCTURE ONLY.  Nothing in the shipped package imports this file:
only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` use it, and only as the checker.

This is a plain numpy restatement (float64 by default) of the reference's
attention algorithm.  Every function cites the reference line it follows
(paths relative to the duoan/mega-trading source tree):

* ``rope_tables``      -- ``src/mega_trading/model.py:279-284``
                          (fp32 tables, ``inv_freq = theta ** (-2i/D)``).
* ``apply_rope``       -- ``src/mega_trading/model.py:312-316``
                          (interleaved pairs ``(x[2i], x[2i+1])``).
* ``rope_inverse``     -- ``src/mega_trading/kernels/triton_ops.py:205-214,740``
                          (the RoPE backward is the same rotation with ``-sin``).
* ``attention_forward``  -- ``src/mega_trading/kernels/triton_attention.py:28-38,
                          329-349`` (scale ``1/sqrt(D)``, causal mask ``j <= i``,
                          GQA map ``kv = h // repeats``, ``LSE = m + ln(l)``,
                          natural log).
* ``attention_backward`` -- ``src/mega_trading/kernels/triton_attention.py:88-111``
                          (dense fp32 backward: ``dS = P * (dP - rowsum(dP * P))``,
                          ``dQ = scale dS K``, ``dK = scale dS^T Q``, ``dV = P^T dO``,
                          dK/dV summed over the ``repeats`` query heads of a group)
                          and ``:561-583`` (``delta = rowsum(O * dO)``, which equals
                          ``rowsum(dP * P)``).
* ``rope_attention_forward/backward`` -- ``model.py:223-226`` (RoPE on q and k,
                          then attention), with the chain rule through the rotation.
* ``decode_attention``   -- the last query row of ``attention_forward`` over the
                          ``length`` cached positions: what ``TradingModel.generate``
                          (``model.py:134-147``) computes for each new token by
                          re-running the whole context.

How each part is pinned (tests/test_oracle.py):

* forward/backward: against ``torch.nn.functional.scaled_dot_product_attention``
  (``is_causal=True, enable_gqa=True``) + autograd on the CPU -- the library
  routine the reference's eager path calls (``model.py:228-235``) -- against the
  committed golden vectors in ``tests/golden/`` (written by
  ``tests/golden/make_golden.py`` from that routine), against a brute-force
  per-element triple loop on tiny inputs, and against invariants (row 0 of O is
  v_0, LSE of row 0 is ``scale q_0.k_0``, future keys do not change O, the GQA
  result equals the MHA result on ``repeat_interleave``-expanded K/V, dK/dV are
  group sums, finite-difference gradients).
* RoPE: closed form at position 0 (identity) and a hand-computed pair, norm
  preservation, inverse-rotation round trip, and torch-computed tables.

No function here is left "parity unpinned".
"""

from __future__ import annotations

import numpy as np

__all__ = [
    "rope_tables",
    "apply_rope",
    "rope_inverse",
    "attention_forward",
    "attention_backward",
    "rope_attention_forward",
    "rope_attention_backward",
]


def rope_tables(seq_len: int, head_dim: int, theta: float) -> tuple[np.ndarray, np.ndarray]:
    """fp32 cos/sin tables of shape [T, D/2] (``model.py:279-284``).

    ``inv_freq_i = 1 / theta ** (2i / D)``, ``freqs[t, i] = t * inv_freq_i``,
    all in float32 as the reference registers them.
    """
    if head_dim % 2:
        raise ValueError("RoPE requires an even head dimension")
    positions = np.arange(seq_len, dtype=np.float32)
    exponent = np.arange(0, head_dim, 2, dtype=np.float32) / np.float32(head_dim)
    inv_freq = (np.float32(1.0) / (np.float32(theta) ** exponent)).astype(np.float32)
    freqs = np.outer(positions, inv_freq).astype(np.float32)
    return np.cos(freqs).astype(np.float32), np.sin(freqs).astype(np.float32)


def apply_rope(x: np.ndarray, cos: np.ndarray, sin: np.ndarray) -> np.ndarray:
    """Rotate interleaved pairs of the last axis (``model.py:312-316``).

    ``x``: [..., T, D]; ``cos``/``sin``: [T, D/2] (broadcast over leading axes).
    ``(e, o) -> (e cos - o sin, e sin + o cos)`` for ``e = x[..., 0::2]``,
    ``o = x[..., 1::2]``.
    """
    even = x[..., 0::2]
    odd = x[..., 1::2]
    out = np.empty(np.broadcast_shapes(x.shape), dtype=np.result_type(x, cos))
    out[..., 0::2] = even * cos - odd * sin
    out[..., 1::2] = even * sin + odd * cos
    return out


def rope_inverse(g: np.ndarray, cos: np.ndarray, sin: np.ndarray) -> np.ndarray:
    """Rotation by ``-theta``: the RoPE backward (``triton_ops.py:205-214``, ``NEGATE_SIN``)."""
    return apply_rope(g, cos, -sin)


def _check_shapes(q: np.ndarray, k: np.ndarray, v: np.ndarray, repeats: int) -> tuple[int, int, int, int, int]:
    if q.ndim != 4 or k.ndim != 4 or v.ndim != 4:
        raise ValueError("q, k and v must be [B, H, T, D]")
    b, hq, t, d = q.shape
    if k.shape != v.shape:
        raise ValueError("key and value must have the same shape")
    if k.shape[1] * repeats != hq:
        raise ValueError("query heads must equal key/value heads multiplied by repeats")
    if k.shape[0] != b or k.shape[2:] != q.shape[2:]:
        raise ValueError("query, key, and value must agree on batch, sequence, and head dimensions")
    return b, hq, k.shape[1], t, d


def _row_chunks(t: int, chunk: int):
    for r0 in range(0, t, chunk):
        yield r0, min(t, r0 + chunk)


def attention_forward(
    q: np.ndarray,
    k: np.ndarray,
    v: np.ndarray,
    repeats: int,
    scale: float | None = None,
    dtype=np.float64,
    chunk: int = 1024,
) -> tuple[np.ndarray, np.ndarray]:
    """Causal GQA forward: returns (O [B,Hq,T,D], LSE [B,Hq,T]) in ``dtype``.

    ``S = scale Q K^T`` with column ``j`` allowed for row ``i`` iff ``j <= i``;
    ``O = softmax(S) V``; ``LSE = max_j S + ln(sum_j exp(S - max))`` (natural log,
    ``triton_attention.py:346-349``).  Query head ``h`` reads KV head
    ``h // repeats`` (``triton_attention.py:299``).  Rows are processed in chunks
    so a T=4096 slab never holds more than ``chunk x T`` scores.
    """
    b, hq, _hkv, t, d = _check_shapes(q, k, v, repeats)
    if scale is None:
        scale = 1.0 / np.sqrt(d)
    o = np.empty((b, hq, t, d), dtype=dtype)
    lse = np.empty((b, hq, t), dtype=dtype)
    cols = np.arange(t)
    for bi in range(b):
        for h in range(hq):
            kh = h // repeats
            kk = k[bi, kh].astype(dtype)
            vv = v[bi, kh].astype(dtype)
            qq = q[bi, h].astype(dtype)
            for r0, r1 in _row_chunks(t, chunk):
                s = (qq[r0:r1] @ kk[:r1].T) * dtype(scale)
                rows = np.arange(r0, r1)
                s[cols[None, :r1] > rows[:, None]] = -np.inf
                m = s.max(axis=1)
                p = np.exp(s - m[:, None])
                l = p.sum(axis=1)
                o[bi, h, r0:r1] = (p @ vv[:r1]) / l[:, None]
                lse[bi, h, r0:r1] = m + np.log(l)
    return o, lse


def attention_backward(
    q: np.ndarray,
    k: np.ndarray,
    v: np.ndarray,
    do: np.ndarray,
    repeats: int,
    scale: float | None = None,
    dtype=np.float64,
    chunk: int = 1024,
) -> tuple[np.ndarray, np.ndarray, np.ndarray]:
    """Causal GQA backward (``triton_attention.py:88-111``): returns (dQ, dK, dV).

    ``P = softmax(S)``, ``dP = dO V^T``, ``dS = P * (dP - rowsum(dP * P))``,
    ``dQ = scale dS K``, ``dK = scale dS^T Q``, ``dV = P^T dO``; dK and dV are
    summed over the ``repeats`` query heads that share a KV head
    (``triton_attention.py:107-110``).  ``rowsum(dP * P)`` equals
    ``rowsum(O * dO)`` (the ``delta`` of ``:561``); the closed form is used here.
    """
    b, hq, hkv, t, d = _check_shapes(q, k, v, repeats)
    if do.shape != q.shape:
        raise ValueError("grad_output must match query")
    if scale is None:
        scale = 1.0 / np.sqrt(d)
    dq = np.zeros((b, hq, t, d), dtype=dtype)
    dk = np.zeros((b, hkv, t, d), dtype=dtype)
    dv = np.zeros((b, hkv, t, d), dtype=dtype)
    cols = np.arange(t)
    for bi in range(b):
        for h in range(hq):
            kh = h // repeats
            kk = k[bi, kh].astype(dtype)
            vv = v[bi, kh].astype(dtype)
            qq = q[bi, h].astype(dtype)
            gg = do[bi, h].astype(dtype)
            for r0, r1 in _row_chunks(t, chunk):
                s = (qq[r0:r1] @ kk[:r1].T) * dtype(scale)
                rows = np.arange(r0, r1)
                mask = cols[None, :r1] > rows[:, None]
                s[mask] = -np.inf
                m = s.max(axis=1)
                p = np.exp(s - m[:, None])
                p /= p.sum(axis=1)[:, None]
                dp = gg[r0:r1] @ vv[:r1].T
                ds = p * (dp - (dp * p).sum(axis=1)[:, None])
                dq[bi, h, r0:r1] = (ds @ kk[:r1]) * dtype(scale)
                dk[bi, kh, :r1] += (ds.T @ qq[r0:r1]) * dtype(scale)
                dv[bi, kh, :r1] += p.T @ gg[r0:r1]
    return dq, dk, dv


def rope_attention_forward(
    q: np.ndarray,
    k: np.ndarray,
    v: np.ndarray,
    cos: np.ndarray,
    sin: np.ndarray,
    repeats: int,
    scale: float | None = None,
    dtype=np.float64,
) -> tuple[np.ndarray, np.ndarray]:
    """RoPE on q and k (``model.py:223``) followed by attention (``model.py:226``).

    The rotation runs in ``dtype`` on the (already rounded) inputs, i.e. the
    fp32-or-better RoPE the fused kernel is specified against.
    """
    t = q.shape[2]
    c = cos[:t].astype(dtype)
    s = sin[:t].astype(dtype)
    return attention_forward(apply_rope(q.astype(dtype), c, s), apply_rope(k.astype(dtype), c, s), v, repeats, scale, dtype)


def rope_attention_backward(
    q: np.ndarray,
    k: np.ndarray,
    v: np.ndarray,
    do: np.ndarray,
    cos: np.ndarray,
    sin: np.ndarray,
    repeats: int,
    scale: float | None = None,
    dtype=np.float64,
) -> tuple[np.ndarray, np.ndarray, np.ndarray]:
    """Gradients of the RoPE+attention composite w.r.t. the *un-rotated* q and k.

    dQ/dK are the attention gradients rotated back by ``-theta``
    (``triton_ops.py:205-214``); dV is unchanged.
    """
    t = q.shape[2]
    c = cos[:t].astype(dtype)
    s = sin[:t].astype(dtype)
    qr = apply_rope(q.astype(dtype), c, s)
    kr = apply_rope(k.astype(dtype), c, s)
    dq, dk, dv = attention_backward(qr, kr, v, do, repeats, scale, dtype)
    return rope_inverse(dq, c, s), rope_inverse(dk, c, s), dv


def decode_attention(q: np.ndarray, k: np.ndarray, v: np.ndarray, length: int, repeats: int,
                     scale: float | None = None, dtype=np.float64) -> np.ndarray:
    """One query per (batch, head) at position ``length - 1`` against keys/values
    0 .. length-1: ``softmax(scale q k^T) v`` (no mask is needed: every cached
    position precedes the query).  q [B, Hq, D]; k, v [B, Hkv, >= length, D];
    returns [B, Hq, D]."""
    b, hq, d = q.shape
    if k.shape[1] * repeats != hq:
        raise ValueError("query heads must equal key/value heads multiplied by repeats")
    if scale is None:
        scale = 1.0 / np.sqrt(d)
    out = np.empty((b, hq, d), dtype=dtype)
    for bi in range(b):
        for h in range(hq):
            kk = k[bi, h // repeats, :length].astype(dtype)
            s = (kk @ q[bi, h].astype(dtype)) * dtype(scale)
            p = np.exp(s - s.max())
            out[bi, h] = (p @ v[bi, h // repeats, :length].astype(dtype)) / p.sum()
    return out
