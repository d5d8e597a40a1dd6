"""Input generation and comparison helpers shared by the GPU parity tests and bench.

Inputs follow the measurement recipe of the BASELINE configs: one CPU
``torch.Generator`` seeded once, drawing Q, K, V, dO in that order;
Q/K/V ~ N(0, sigma^2), dO ~ N(0, 1); rounded to the kernel dtype on the CPU so
the oracle sees exactly the values the GPU sees.
"""

from __future__ import annotations

import numpy as np
import torch

from oracle import attention_oracle as orc

# Tolerances from BASELINE.json's north star.
TOL_OUT_MAXABS = 2e-2   # bf16/fp16 output vs the fp32-or-better oracle, max-abs
TOL_GRAD_REL = 3e-2     # gradients, ||got - ref||_2 / ||ref||_2
TOL_LSE_MAXABS = 1e-2   # fp32 LSE from 16-bit inputs

CONFIGS = {
    # name: (B, T, Hq, Hkv, D, sigma, theta)
    "C1": (2, 256, 4, 2, 32, 1.0, 10_000.0),
    "C2": (16, 1024, 8, 2, 64, 0.5, 10_000.0),
    "C3": (4, 4096, 16, 4, 64, 0.5, 10_000.0),
    "C4": (8, 2048, 32, 8, 128, 0.5, 10_000.0),
}


def make_inputs(b, t, hq, hkv, d, sigma=0.5, seed=0, dtype=torch.bfloat16):
    g = torch.Generator().manual_seed(seed)
    q = (torch.randn(b, hq, t, d, generator=g) * sigma).to(dtype)
    k = (torch.randn(b, hkv, t, d, generator=g) * sigma).to(dtype)
    v = (torch.randn(b, hkv, t, d, generator=g) * sigma).to(dtype)
    do = torch.randn(b, hq, t, d, generator=g).to(dtype)
    return q, k, v, do


def run_hip(pkg, q, k, v, do, repeats, cos=None, sin=None, device="cuda:0"):
    """Forward + backward through the public op; returns CPU fp32 numpy arrays."""
    qd, kd, vd = (x.to(device).requires_grad_(True) for x in (q, k, v))
    if cos is None:
        out, lse = pkg.attention_forward(qd, kd, vd, repeats=repeats)
    else:
        out, lse = pkg.attention_forward(
            qd, kd, vd, repeats=repeats, cos=torch.from_numpy(cos).to(device), sin=torch.from_numpy(sin).to(device)
        )
    dq, dk, dv = torch.autograd.grad(out, (qd, kd, vd), do.to(device))
    torch.cuda.synchronize()
    f = lambda x: x.detach().float().cpu().numpy()  # noqa: E731
    return f(out), f(lse), f(dq), f(dk), f(dv)


def oracle(q, k, v, do, repeats, cos=None, sin=None):
    f = lambda x: x.float().numpy()  # noqa: E731
    if cos is None:
        o, lse = orc.attention_forward(f(q), f(k), f(v), repeats)
        dq, dk, dv = orc.attention_backward(f(q), f(k), f(v), f(do), repeats)
    else:
        o, lse = orc.rope_attention_forward(f(q), f(k), f(v), cos, sin, repeats)
        dq, dk, dv = orc.rope_attention_backward(f(q), f(k), f(v), f(do), cos, sin, repeats)
    return o, lse, dq, dk, dv


def rel(a, b):
    """||a - b|| / ||b||, with ||b|| floored at an RMS of 1e-3 per element: where
    the exact gradient vanishes (T = 1 gives dQ = dK = 0) the ratio is otherwise
    meaningless, and 1e-3 is far below the O(0.1-1) gradients of these inputs."""
    floor = 1e-3 * np.sqrt(b.size)
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), floor))


def compare(got, ref, out_tol=TOL_OUT_MAXABS, grad_tol=TOL_GRAD_REL, lse_tol=TOL_LSE_MAXABS):
    """Assert BASELINE tolerances; returns the error figures for reporting."""
    o, lse, dq, dk, dv = got
    eo, e_lse, edq, edk, edv = ref
    errs = {
        "o_maxabs": float(np.abs(o - eo).max()),
        "lse_maxabs": float(np.abs(lse - e_lse).max()),
        "dq_rel": rel(dq, edq),
        "dk_rel": rel(dk, edk),
        "dv_rel": rel(dv, edv),
    }
    assert np.isfinite(o).all() and np.isfinite(dq).all() and np.isfinite(dk).all() and np.isfinite(dv).all()
    assert errs["o_maxabs"] <= out_tol, errs
    assert errs["lse_maxabs"] <= lse_tol, errs
    assert errs["dq_rel"] <= grad_tol and errs["dk_rel"] <= grad_tol and errs["dv_rel"] <= grad_tol, errs
    return errs


def slice_group(arrs, b, kvg, repeats):
    """Restrict (o, lse, dq, dk, dv) or (q, k, v, do) style tuples to batch b, KV group kvg."""
    hs = slice(kvg * repeats, (kvg + 1) * repeats)
    o, lse, dq, dk, dv = arrs
    return o[b : b + 1, hs], lse[b : b + 1, hs], dq[b : b + 1, hs], dk[b : b + 1, kvg : kvg + 1], dv[b : b + 1, kvg : kvg + 1]
