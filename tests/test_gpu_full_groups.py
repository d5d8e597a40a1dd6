"""Every (batch, KV group) of BASELINE configs 2-4 against a reference value.

The oracle comparisons in ``test_gpu_parity.py`` run the float64 oracle on a
few (batch, KV group) slices per config, because the oracle needs seconds per
slice at full T.  Here the HIP op's O, LSE, dQ, dK and dV for the WHOLE
config are compared group by group with a dense float32 reference computed on
the GPU: S = scale * Q K^T over the group's query heads (K/V repeated per
query head, ``triton_attention.py:88-89``), the causal mask, softmax, O = P V,
LSE = logsumexp(S) (``:346-349``), and autograd for the gradients (RoPE in
float32 on the bf16-rounded inputs, as the oracle applies it).  The dense
reference itself is pinned to the float64 oracle on one group per config
(agreement to float32 rounding), so every group is checked against a value
that the oracle vouches for.  BASELINE tolerances apply per group.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import attention_oracle as orc
from tests.gpu_cases import CONFIGS, TOL_GRAD_REL, TOL_LSE_MAXABS, TOL_OUT_MAXABS, make_inputs, oracle

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda:0")


def _rot(x, c, s):
    """Interleaved-pair rotation (model.py:312-316) in float32."""
    e, o = x[..., 0::2], x[..., 1::2]
    return torch.stack((e * c - o * s, e * s + o * c), dim=-1).flatten(-2)


def dense_reference(q, k, v, do, repeats, cos=None, sin=None):
    """float32 dense causal GQA forward + autograd backward of one batch element
    (q, do [1, Hq, T, D]; k, v [1, Hkv, T, D], bf16 on the GPU).  Returns
    (o, lse, dq, dk, dv) as float32 GPU tensors."""
    t, d = q.shape[2], q.shape[3]
    qf, kf, vf = (x.float().requires_grad_(True) for x in (q, k, v))
    qr, kr = qf, kf
    if cos is not None:
        qr, kr = _rot(qf, cos, sin), _rot(kf, cos, sin)
    kk = kr.repeat_interleave(repeats, dim=1)
    vv = vf.repeat_interleave(repeats, dim=1)
    scores = torch.matmul(qr, kk.transpose(-2, -1).contiguous()) * (1.0 / d ** 0.5)
    mask = torch.ones(t, t, dtype=torch.bool, device=q.device).triu(1)
    scores = scores.masked_fill(mask, float("-inf"))
    lse = torch.logsumexp(scores, dim=-1)
    out = torch.matmul(torch.softmax(scores, dim=-1), vv)
    dq, dk, dv = torch.autograd.grad(out, (qf, kf, vf), do.float())
    return out.detach(), lse.detach(), dq, dk, dv


def _hip(mta, q, k, v, do, repeats, cos, sin):
    qd, kd, vd = (x.requires_grad_(True) for x in (q.clone(), k.clone(), v.clone()))
    if cos is None:
        out, lse = mta.attention_forward(qd, kd, vd, repeats=repeats)
    else:
        out, lse = mta.attention_forward(qd, kd, vd, repeats=repeats, cos=cos, sin=sin)
    dq, dk, dv = torch.autograd.grad(out, (qd, kd, vd), do)
    return out.detach().float(), lse.detach(), dq.float(), dk.float(), dv.float()


def _group_errors(got, ref, g, r):
    """Per-group error figures of (o, lse, dq, dk, dv) tensors of one batch element."""
    hs = slice(g * r, (g + 1) * r)
    o, lse, dq, dk, dv = got
    eo, else_, edq, edk, edv = ref

    def relg(a, b):
        floor = 1e-3 * b.numel() ** 0.5
        return float((a - b).norm() / max(float(b.norm()), floor))

    return {
        "o_maxabs": float((o[:, hs] - eo[:, hs]).abs().max()),
        "lse_maxabs": float((lse[:, hs] - else_[:, hs]).abs().max()),
        "dq_rel": relg(dq[:, hs], edq[:, hs]),
        "dk_rel": relg(dk[:, g : g + 1], edk[:, g : g + 1]),
        "dv_rel": relg(dv[:, g : g + 1], edv[:, g : g + 1]),
    }


def test_dense_reference_matches_the_oracle():
    """The float32 dense reference against the float64 oracle on one (batch,
    KV group) per config, plain and with RoPE: agreement to float32 rounding
    (far inside the BASELINE tolerances), so it is a valid stand-in for the
    oracle on the groups the oracle is too slow to cover."""
    for name in ("C2", "C3", "C4"):
        b, t, hq, hkv, d, sigma, theta = CONFIGS[name]
        r = hq // hkv
        q, k, v, do = make_inputs(b, t, hq, hkv, d, sigma=sigma, seed=0)
        bi, g = b - 1, hkv - 1  # the last group in issue order
        hs = slice(g * r, (g + 1) * r)
        qs, ks, vs, dos = q[bi : bi + 1, hs], k[bi : bi + 1, g : g + 1], v[bi : bi + 1, g : g + 1], do[bi : bi + 1, hs]
        for rope in (False, True):
            cos = sin = None
            if rope:
                cos, sin = orc.rope_tables(t, d, theta)
            ref = oracle(qs, ks, vs, dos, r, cos, sin)
            cd = sd = None
            if rope:
                cd, sd = torch.from_numpy(cos).to(DEV), torch.from_numpy(sin).to(DEV)
            got = dense_reference(qs.to(DEV), ks.to(DEV), vs.to(DEV), dos.to(DEV), r, cd, sd)
            got = [x.cpu().numpy() for x in got]
            err_o = float(np.abs(got[0] - ref[0]).max())
            err_l = float(np.abs(got[1] - ref[1]).max())
            rels = [float(np.linalg.norm(a - e) / np.linalg.norm(e)) for a, e in zip(got[2:], ref[2:])]
            print(name, "rope" if rope else "plain", f"o {err_o:.1e} lse {err_l:.1e} grads {max(rels):.1e}", flush=True)
            assert err_o <= 1e-4 and err_l <= 1e-4 and max(rels) <= 1e-4, (name, rope, err_o, err_l, rels)


@pytest.mark.parametrize("rope", [False, True], ids=["plain", "rope"])
@pytest.mark.parametrize("name", ["C2", "C3", "C4"])
def test_every_group_against_dense_reference(mta, name, rope):
    b, t, hq, hkv, d, sigma, theta = CONFIGS[name]
    r = hq // hkv
    print(f"case {name} {'rope' if rope else 'plain'}: {b * hkv} groups", flush=True)
    q, k, v, do = (x.to(DEV) for x in make_inputs(b, t, hq, hkv, d, sigma=sigma, seed=0))
    cos = sin = None
    if rope:
        c, s = orc.rope_tables(t, d, theta)
        cos, sin = torch.from_numpy(c).to(DEV), torch.from_numpy(s).to(DEV)
    got = _hip(mta, q, k, v, do, r, cos, sin)
    torch.cuda.synchronize()
    for x in got:
        assert bool(torch.isfinite(x).all())
    worst = {}
    for bi in range(b):
        ref = dense_reference(q[bi : bi + 1], k[bi : bi + 1], v[bi : bi + 1], do[bi : bi + 1], r, cos, sin)
        mine = tuple(x[bi : bi + 1] for x in got)
        for g in range(hkv):
            errs = _group_errors(mine, ref, g, r)
            for key, val in errs.items():
                worst[key] = max(worst.get(key, 0.0), val)
            assert errs["o_maxabs"] <= TOL_OUT_MAXABS, (bi, g, errs)
            assert errs["lse_maxabs"] <= TOL_LSE_MAXABS, (bi, g, errs)
            assert max(errs["dq_rel"], errs["dk_rel"], errs["dv_rel"]) <= TOL_GRAD_REL, (bi, g, errs)
        del ref
    print(name, "rope" if rope else "plain", "worst over all groups",
          {k_: f"{v_:.2e}" for k_, v_ in worst.items()}, flush=True)
