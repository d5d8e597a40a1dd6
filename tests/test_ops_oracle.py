"""Pinning the operator oracle (oracle/ops_oracle.py) on the CPU.

Against torch (``F.rms_norm`` / ``F.silu`` + autograd: the routines the
reference's eager path calls, ``model.py:254-255, 269``), closed forms and
finite differences, and with planted mistakes that each fail a check.
"""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import ops_oracle as oo


def _rand(shape, seed, scale=1.0):
    return np.random.default_rng(seed).standard_normal(shape) * scale


# ---------------------------------------------------------------------------
# RMSNorm
# ---------------------------------------------------------------------------
def _torch_rms(x, w, eps, dy):
    xt = torch.tensor(x, dtype=torch.float64, requires_grad=True)
    wt = torch.tensor(w, dtype=torch.float64, requires_grad=True)
    y = F.rms_norm(xt, (x.shape[-1],), wt, eps=eps)
    y.backward(torch.tensor(dy, dtype=torch.float64))
    return y.detach().numpy(), xt.grad.numpy(), wt.grad.numpy()


@pytest.mark.parametrize("rows,d,eps", [(7, 8, 1e-5), (33, 512, 1e-5), (5, 1000, 1e-6), (3, 4096, 1e-5)])
def test_rms_norm_matches_torch(rows, d, eps):
    x, w, dy = _rand((rows, d), 1), _rand(d, 2, 0.5) + 1.0, _rand((rows, d), 3)
    y, rstd = oo.rms_norm_forward(x, w, eps, "float32")
    dx, dw = oo.rms_norm_backward(x, w, rstd, dy)
    ty, tdx, tdw = _torch_rms(x, w, eps, dy)
    np.testing.assert_allclose(y, ty, rtol=1e-6, atol=1e-6)  # y is rounded to fp32
    np.testing.assert_allclose(dx, tdx, rtol=1e-10, atol=1e-10)
    np.testing.assert_allclose(dw, tdw, rtol=1e-10, atol=1e-10)


def test_rms_norm_closed_forms():
    x = _rand((4, 64), 5)
    w = np.ones(64)
    y, rstd = oo.rms_norm_forward(x, w, 0.0, "float32")
    np.testing.assert_allclose(np.sqrt(np.mean(y.astype(np.float64) ** 2, -1)), 1.0, rtol=1e-6)  # unit RMS
    y2, _ = oo.rms_norm_forward(3.5 * x, w, 0.0, "float32")
    np.testing.assert_allclose(y2, y, rtol=1e-6)  # scale invariance
    np.testing.assert_allclose(rstd, 1.0 / np.sqrt(np.mean(x * x, -1)), rtol=1e-12)
    # constant row c: y = sign(c) * |c| / sqrt(c^2 + eps)
    yc, _ = oo.rms_norm_forward(np.full((1, 16), -2.0), w[:16], 1e-2, "float32")
    np.testing.assert_allclose(yc, -2.0 / math.sqrt(4.0 + 1e-2), rtol=1e-6)
    # with w = 1 and eps = 0 the input gradient is orthogonal to x (the norm is scale-free)
    dx, _ = oo.rms_norm_backward(x, w, rstd, _rand((4, 64), 6))
    assert np.max(np.abs(np.sum(dx * x, -1))) < 1e-10


def test_rms_norm_finite_differences():
    x, w, dy = _rand((3, 16), 7), _rand(16, 8) + 1.0, _rand((3, 16), 9)
    eps = 1e-3
    _, rstd = oo.rms_norm_forward(x, w, eps)
    dx, dw = oo.rms_norm_backward(x, w, rstd, dy)

    def loss(xx, ww):
        rs = 1.0 / np.sqrt(np.mean(xx * xx, -1) + eps)
        return np.sum(xx * rs[:, None] * ww[None, :] * dy)

    h = 1e-6
    for (i, j) in [(0, 0), (1, 5), (2, 15)]:
        xp, xm = x.copy(), x.copy()
        xp[i, j] += h
        xm[i, j] -= h
        assert abs((loss(xp, w) - loss(xm, w)) / (2 * h) - dx[i, j]) < 1e-6
    for j in (0, 9):
        wp, wm = w.copy(), w.copy()
        wp[j] += h
        wm[j] -= h
        assert abs((loss(x, wp) - loss(x, wm)) / (2 * h) - dw[j]) < 1e-6


def test_add_rms_norm_matches_torch_and_reuses_norm():
    x, r, w = _rand((9, 64), 10), _rand((9, 64), 11), _rand(64, 12) + 1.0
    dy, dres = _rand((9, 64), 13), _rand((9, 64), 14)
    s, y, rstd = oo.add_rms_norm_forward(x, r, w, 1e-5, "float32")
    xt = torch.tensor(x, dtype=torch.float32, requires_grad=True)
    rt = torch.tensor(r, dtype=torch.float32, requires_grad=True)
    wt = torch.tensor(w, dtype=torch.float32, requires_grad=True)
    st = xt + rt
    yt = F.rms_norm(st, (64,), wt, eps=1e-5)
    torch.autograd.backward([st, yt], [torch.tensor(dres, dtype=torch.float32), torch.tensor(dy, dtype=torch.float32)])
    np.testing.assert_array_equal(s, st.detach().numpy())
    np.testing.assert_allclose(y, yt.detach().numpy(), rtol=2e-6, atol=2e-6)
    dx, dw = oo.add_rms_norm_backward(s, w, rstd, dres, dy)
    np.testing.assert_allclose(dx, xt.grad.numpy(), rtol=1e-4, atol=1e-5)
    np.testing.assert_allclose(dx, rt.grad.numpy(), rtol=1e-4, atol=1e-5)
    np.testing.assert_allclose(dw, wt.grad.numpy(), rtol=1e-4, atol=1e-4)


def test_rms_norm_planted_mistakes_fail():
    x, w, dy = _rand((6, 32), 20), _rand(32, 21) + 1.0, _rand((6, 32), 22)
    eps = 0.1  # large, so its placement matters
    ty, tdx, tdw = _torch_rms(x, w, eps, dy)

    def fwd_eps_outside(x, w, eps):
        rstd = 1.0 / (np.sqrt(np.mean(x * x, -1)) + eps)
        return x * rstd[:, None] * w

    def fwd_no_weight(x, w, eps):
        return x / np.sqrt(np.mean(x * x, -1) + eps)[:, None]

    def fwd_mean_d_minus_1(x, w, eps):
        return x / np.sqrt(np.sum(x * x, -1) / (x.shape[-1] - 1) + eps)[:, None] * w

    for bad in (fwd_eps_outside, fwd_no_weight, fwd_mean_d_minus_1):
        assert not np.allclose(bad(x, w, eps), ty, rtol=1e-4, atol=1e-4), bad.__name__
    _, rstd = oo.rms_norm_forward(x, w, eps)
    # backward without the projection term is wrong
    bad_dx = rstd[:, None] * dy * w
    assert not np.allclose(bad_dx, tdx, rtol=1e-4, atol=1e-4)


# ---------------------------------------------------------------------------
# SwiGLU gate
# ---------------------------------------------------------------------------
def _bf16(a):
    return torch.tensor(np.asarray(a, dtype=np.float32)).to(torch.bfloat16)


def test_round_to_bf16_matches_torch():
    v = _rand(100_000, 30, 3.0).astype(np.float32)
    v[:4] = [np.inf, -np.inf, 0.0, -0.0]
    ours = oo.round_to(v, "bfloat16")
    ref = torch.tensor(v).to(torch.bfloat16).float().numpy()
    np.testing.assert_array_equal(ours, ref)
    np.testing.assert_array_equal(oo.round_to(v, "float16"), torch.tensor(v).half().float().numpy())


@pytest.mark.parametrize("dtype", ["bfloat16", "float16", "float32"])
def test_swiglu_matches_torch_eager(dtype):
    n = 50_000
    tdt = {"bfloat16": torch.bfloat16, "float16": torch.float16, "float32": torch.float32}[dtype]
    g = torch.tensor(_rand(n, 31, 3.0), dtype=torch.float32).to(tdt)
    u = torch.tensor(_rand(n, 32), dtype=torch.float32).to(tdt)
    dy = torch.tensor(_rand(n, 33), dtype=torch.float32).to(tdt)
    gg, uu = g.clone().requires_grad_(True), u.clone().requires_grad_(True)
    out = F.silu(gg) * uu
    out.backward(dy)
    ours = oo.swiglu_forward(g.float().numpy(), u.float().numpy(), dtype)
    dg, du = oo.swiglu_backward(g.float().numpy(), u.float().numpy(), dy.float().numpy(), dtype)
    # torch CPU follows the same rounding sequence; its exp may differ in the last
    # fp32 ulp, which 16-bit storage almost always absorbs
    for name, a, b in (("out", ours, out.detach().float().numpy()), ("dgate", dg, gg.grad.float().numpy()),
                       ("dup", du, uu.grad.float().numpy())):
        if dtype != "float32":
            same = np.mean(a == b)
            assert same > 0.999, f"{name}: only {same:.5f} bit-equal"
        tol = {"bfloat16": 2 ** -7, "float16": 2 ** -10, "float32": 2 ** -19}[dtype]
        np.testing.assert_allclose(a, b, rtol=tol, atol=tol)


def test_swiglu_closed_forms():
    g = np.array([0.0, 1.0, -1.0, 20.0, -20.0, 3.25], dtype=np.float32)
    one = np.ones_like(g)
    out = oo.swiglu_forward(g, one, "float32")
    assert out[0] == 0.0
    np.testing.assert_allclose(out[3], 20.0, rtol=1e-6)  # silu(x) -> x
    np.testing.assert_allclose(out[4], 0.0, atol=1e-6)   # silu(-x) -> 0
    np.testing.assert_allclose(oo.swiglu_forward(-g, one, "float32"), out - g, rtol=1e-5, atol=1e-6)  # silu(-x) = silu(x) - x
    dg, du = oo.swiglu_backward(g, one, one, "float32")
    np.testing.assert_allclose(dg[0], 0.5)  # silu'(0) = 1/2
    np.testing.assert_array_equal(du, out)  # d/d up = silu(g) when dy = 1
    # central differences of silu
    h = 1e-3
    fd = (oo.swiglu_forward(g.astype(np.float64) + h, one, "float32") -
          oo.swiglu_forward(g.astype(np.float64) - h, one, "float32")) / (2 * h)
    np.testing.assert_allclose(dg, fd, rtol=2e-3, atol=2e-3)


def test_swiglu_planted_mistakes_fail():
    n = 20_000
    g = _rand(n, 40, 3.0).astype(np.float32)
    u = _rand(n, 41).astype(np.float32)
    dy = _rand(n, 42).astype(np.float32)
    gt, ut, dyt = _bf16(g), _bf16(u), _bf16(dy)
    gg, uu = gt.clone().requires_grad_(True), ut.clone().requires_grad_(True)
    (F.silu(gg) * uu).backward(dyt)
    ref_out = (F.silu(gt) * ut).float().numpy()
    gb, ub, dyb = gt.float().numpy(), ut.float().numpy(), dyt.float().numpy()
    # no rounding of silu before the product
    no_round = oo.round_to(oo._silu32(gb) * ub, "bfloat16")
    assert np.mean(no_round == ref_out) < 0.995
    # silu' without the (1 - sig) factor
    sig = 1 / (1 + np.exp(-gb))
    bad_dg = oo.round_to(oo.round_to(dyb * ub, "bfloat16") * sig * (1 + gb), "bfloat16")
    assert not np.allclose(bad_dg, gg.grad.float().numpy(), rtol=1e-2, atol=1e-2)


# ---------------------------------------------------------------------------
# cross-entropy rows / fused linear cross-entropy
# ---------------------------------------------------------------------------
def _torch_ce(x, labels, ignore):
    xt = torch.tensor(x, dtype=torch.float64, requires_grad=True)
    loss = F.cross_entropy(xt, torch.tensor(labels), ignore_index=ignore)
    loss.backward()
    return loss.item(), xt.grad.numpy()


@pytest.mark.parametrize("ignore_frac", [0.0, 0.3])
def test_cross_entropy_rows_match_torch(ignore_frac):
    rng = np.random.default_rng(50)
    x = rng.standard_normal((64, 40)) * 3
    labels = rng.integers(0, 40, 64)
    labels[rng.random(64) < ignore_frac] = -100
    loss, grad = oo.cross_entropy_rows(x, labels, -100)
    tl, tg = _torch_ce(x, labels, -100)
    assert abs(loss.sum() - tl) < 1e-12
    np.testing.assert_allclose(grad, tg, rtol=1e-12, atol=1e-14)


def test_cross_entropy_closed_forms():
    v = 24
    loss, grad = oo.cross_entropy_rows(np.zeros((3, v)), np.array([0, 5, 23]))
    np.testing.assert_allclose(loss.sum(), math.log(v))  # uniform logits: mean loss = log V
    np.testing.assert_allclose(grad.sum(-1), 0.0, atol=1e-15)  # softmax minus onehot sums to 0
    np.testing.assert_allclose(grad[1, 5], (1 / v - 1) / 3)
    loss, grad = oo.cross_entropy_rows(np.ones((2, v)), np.array([-100, -100]))
    assert loss.sum() == 0.0 and not grad.any()  # everything ignored: zeros
    # shifting a row by a constant changes nothing
    x = np.random.default_rng(51).standard_normal((4, v))
    a = oo.cross_entropy_rows(x, np.array([1, 2, 3, 4]))
    b = oo.cross_entropy_rows(x + 7.5, np.array([1, 2, 3, 4]))
    np.testing.assert_allclose(a[0], b[0], rtol=1e-12)
    np.testing.assert_allclose(a[1], b[1], rtol=1e-12, atol=1e-15)


def test_cross_entropy_planted_mistakes_fail():
    rng = np.random.default_rng(52)
    x = rng.standard_normal((32, 16))
    labels = rng.integers(0, 16, 32)
    labels[:5] = -100
    tl, tg = _torch_ce(x, labels, -100)
    keep = labels != -100
    lse = np.log(np.exp(x).sum(-1))
    safe = np.where(keep, labels, 0)
    by_rows = np.where(keep, lse - x[np.arange(32), safe], 0).sum() / 32  # normalised by all rows
    assert abs(by_rows - tl) > 1e-3
    shifted = np.where(keep, lse - x[np.arange(32), (safe + 1) % 16], 0).sum() / keep.sum()  # wrong column
    assert abs(shifted - tl) > 1e-3
    _, grad = oo.cross_entropy_rows(x, labels)
    assert not np.allclose(np.exp(x - lse[:, None]) / keep.sum(), tg)  # no onehot term


def test_fused_linear_ce_matches_torch_linear_plus_ce():
    rng = np.random.default_rng(53)
    h = rng.standard_normal((48, 32)).astype(np.float32)
    w = (rng.standard_normal((64, 32)) * 0.2).astype(np.float32)
    labels = rng.integers(0, 64, 48)
    labels[::7] = -100
    loss, gh, gw = oo.fused_linear_cross_entropy(h, w, labels, -100, "float32")
    ht = torch.tensor(h, dtype=torch.float64, requires_grad=True)
    wt = torch.tensor(w, dtype=torch.float64, requires_grad=True)
    tl = F.cross_entropy(F.linear(ht, wt), torch.tensor(labels), ignore_index=-100)
    tl.backward()
    assert abs(loss - tl.item()) < 1e-6
    np.testing.assert_allclose(gh, ht.grad.numpy(), rtol=1e-5, atol=1e-7)
    np.testing.assert_allclose(gw, wt.grad.numpy(), rtol=1e-5, atol=1e-7)
