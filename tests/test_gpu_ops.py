"""GPU parity of the operator kernels (RMSNorm, add + RMSNorm, SwiGLU gate,
stand-alone RoPE) against the CPU oracle (oracle/ops_oracle.py,
oracle/attention_oracle.py) and torch's eager routines.

Tolerances: fp32 outputs rel 2e-5 (rsqrt and summation order), 16-bit outputs
within one storage ulp of the oracle (RMSNorm) or value-for-value equal to it
for >= 99.9 % of the elements (SwiGLU, whose roundings the kernels
reproduce; the rest differ by a last-ulp exp difference carried through one
rounding step, within 4 ulps), gradients rel 1e-5 in fp32.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import attention_oracle as ao
from oracle import ops_oracle as oo

pytestmark = pytest.mark.gpu

_NP = {torch.bfloat16: "bfloat16", torch.float16: "float16", torch.float32: "float32"}
_ULP = {torch.bfloat16: 2 ** -8, torch.float16: 2 ** -11, torch.float32: 2 ** -23}


def _gen(shape, seed, dtype, scale=1.0):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(shape, generator=g) * scale).to(dtype)


def _rel(a, b):
    a, b = np.asarray(a, np.float64), np.asarray(b, np.float64)
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-30))


def _within_ulps(got, ref, dtype, ulps=1.0):
    got, ref = np.asarray(got, np.float64), np.asarray(ref, np.float64)
    tol = ulps * _ULP[dtype] * np.maximum(np.abs(ref), 2.0 ** -14) * 2.0
    bad = np.abs(got - ref) > tol
    assert not bad.any(), f"{bad.sum()} values off by more than {ulps} ulp; worst {np.abs(got - ref).max():.3e}"


# ---------------------------------------------------------------------------
# RMSNorm
# ---------------------------------------------------------------------------
NORM_CASES = [
    # (rows shape, D, x dtype, weight dtype)
    ((32, 1024), 512, torch.float32, torch.float32),    # BASELINE config 5 residual stream
    ((7,), 8, torch.float32, torch.float32),
    ((1000,), 1000, torch.bfloat16, torch.float32),
    ((3,), 4096, torch.float16, torch.float16),
    ((5, 3), 2048, torch.bfloat16, torch.bfloat16),
    ((0,), 64, torch.float32, torch.float32),
]


@pytest.mark.parametrize("rows,d,dt,wdt", NORM_CASES)
def test_rms_norm_forward_backward_vs_oracle(mta, rows, d, dt, wdt):
    x = _gen(rows + (d,), 1, dt)
    w = (1.0 + 0.5 * _gen((d,), 2, torch.float32)).to(wdt)
    dy = _gen(rows + (d,), 3, dt)
    eps = 1e-5
    xg = x.cuda().requires_grad_(True)
    wg = w.cuda().requires_grad_(True)
    y = mta.rms_norm(xg, wg, eps=eps)
    y.backward(dy.cuda())
    torch.cuda.synchronize()
    assert y.dtype == dt and y.shape == x.shape and wg.grad.dtype == wdt
    x2, dy2 = x.float().numpy().reshape(-1, d), dy.float().numpy().reshape(-1, d)
    ry, rstd = oo.rms_norm_forward(x2, w.float().numpy(), eps, _NP[dt])
    rdx, rdw = oo.rms_norm_backward(x2, w.float().numpy(), rstd, dy2)
    gy = y.detach().float().cpu().numpy().reshape(-1, d)
    gdx = xg.grad.float().cpu().numpy().reshape(-1, d)
    if x2.shape[0] == 0:
        assert gy.size == 0 and not wg.grad.any()
        return
    if dt == torch.float32:
        np.testing.assert_allclose(gy, ry, rtol=2e-5, atol=2e-5)
        assert _rel(gdx, rdx) < 1e-5
    else:
        _within_ulps(gy, ry, dt)
        assert _rel(gdx, oo.round_to(rdx, _NP[dt])) < 4 * _ULP[dt]
    assert _rel(wg.grad.float().cpu().numpy(), rdw) < (1e-5 if wdt == torch.float32 else 4 * _ULP[wdt])


def test_rms_norm_strided_rows_and_torch_autograd(mta):
    # x is a column slice of a wider buffer: read in place with its row stride
    base = _gen((600, 768), 4, torch.float32).cuda()
    x = base[:, 128:640].requires_grad_(False)
    assert x.stride() == (768, 1)
    w = (1.0 + 0.1 * _gen((512,), 5, torch.float32)).cuda()
    xa = x.clone().requires_grad_(True)
    wa = w.clone().requires_grad_(True)
    xb = x.clone().requires_grad_(True)
    wb = w.clone().requires_grad_(True)
    dy = _gen((600, 512), 6, torch.float32).cuda()
    ya = mta.rms_norm(x, w, eps=1e-6)
    yb = F.rms_norm(xb, (512,), wb, eps=1e-6)
    torch.testing.assert_close(ya, yb.detach(), rtol=2e-5, atol=2e-5)
    mta.rms_norm(xa, wa, eps=1e-6).backward(dy)
    yb.backward(dy)
    torch.testing.assert_close(xa.grad, xb.grad, rtol=1e-4, atol=1e-5)
    torch.testing.assert_close(wa.grad, wb.grad, rtol=1e-4, atol=1e-3)


@pytest.mark.parametrize("dt", [torch.float32, torch.bfloat16])
def test_add_rms_norm_vs_oracle(mta, dt):
    rows, d = 777, 512
    x, r = _gen((rows, d), 7, dt), _gen((rows, d), 8, dt)
    w = 1.0 + 0.5 * _gen((d,), 9, torch.float32)
    dres, dy = _gen((rows, d), 10, dt), _gen((rows, d), 11, dt)
    xg, rg, wg = x.cuda().requires_grad_(True), r.cuda().requires_grad_(True), w.cuda().requires_grad_(True)
    s, y = mta.add_rms_norm(xg, rg, wg, eps=1e-5)
    torch.autograd.backward([s, y], [dres.cuda(), dy.cuda()])
    rs, ry, rstd = oo.add_rms_norm_forward(x.float().numpy(), r.float().numpy(), w.numpy(), 1e-5, _NP[dt])
    np.testing.assert_array_equal(s.detach().float().cpu().numpy(), rs)
    rdx, rdw = oo.add_rms_norm_backward(rs, w.numpy(), rstd, dres.float().numpy(), dy.float().numpy())
    if dt == torch.float32:
        np.testing.assert_allclose(y.detach().cpu().numpy(), ry, rtol=2e-5, atol=2e-5)
        assert _rel(xg.grad.cpu().numpy(), rdx) < 1e-5
    else:
        _within_ulps(y.detach().float().cpu().numpy(), ry, dt)
        assert _rel(xg.grad.float().cpu().numpy(), rdx) < 4 * _ULP[dt]
    assert torch.equal(xg.grad, rg.grad)
    assert _rel(wg.grad.cpu().numpy(), rdw) < 1e-5


def test_norm_errors_on_device_tensors(mta):
    x = torch.zeros(4, 12, device="cuda")
    with pytest.raises(ValueError, match="multiple of 8"):
        mta.rms_norm(x, torch.ones(12, device="cuda"), eps=1e-5)
    with pytest.raises(ValueError, match="weight must be 1-D"):
        mta.rms_norm(torch.zeros(4, 16, device="cuda"), torch.ones(8, device="cuda"), eps=1e-5)
    with pytest.raises(ValueError, match="same shape"):
        mta.add_rms_norm(torch.zeros(4, 16, device="cuda"), torch.zeros(4, 8, device="cuda"),
                         torch.ones(16, device="cuda"), eps=1e-5)


# ---------------------------------------------------------------------------
# SwiGLU gate
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("shape,dt", [((32, 1024, 1408), torch.bfloat16), ((1,), torch.bfloat16), ((7,), torch.float16),
                                      ((9,), torch.float32), ((1_000_003,), torch.bfloat16),
                                      ((333, 1408), torch.float16), ((1000, 24), torch.float32)])
def test_swiglu_vs_oracle(mta, shape, dt):
    g, u, dy = _gen(shape, 12, dt, 3.0), _gen(shape, 13, dt), _gen(shape, 14, dt)
    gg, ug = g.cuda().requires_grad_(True), u.cuda().requires_grad_(True)
    out = mta.swiglu_gate(gg, ug)
    out.backward(dy.cuda())
    torch.cuda.synchronize()
    n = g.numel()
    sl = slice(0, min(n, 4_000_000))  # the oracle on the first 4M values of the full-size launch
    gf, uf, dyf = (t.float().numpy().reshape(-1)[sl] for t in (g, u, dy))
    ro = oo.swiglu_forward(gf, uf, _NP[dt])
    rdg, rdu = oo.swiglu_backward(gf, uf, dyf, _NP[dt])
    for name, got, ref in (("out", out.detach(), ro), ("dgate", gg.grad, rdg), ("dup", ug.grad, rdu)):
        got = got.float().cpu().numpy().reshape(-1)[sl]
        if dt == torch.float32:
            np.testing.assert_allclose(got, ref, rtol=2e-6, atol=2e-6, err_msg=name)
        else:
            same = float(np.mean(got == ref))
            assert same >= 0.999, f"{name}: {same:.5f} equal"
            # the rest differ through a last-ulp exp difference that one rounding step
            # (e.g. round(silu) times dy) can carry into a few ulps of the result
            _within_ulps(got, ref, dt, ulps=4)


def test_swiglu_matches_torch_eager_on_gpu(mta):
    g, u, dy = (_gen((4096, 1408), s, torch.bfloat16).cuda() for s in (15, 16, 17))
    ga, ua = g.clone().requires_grad_(True), u.clone().requires_grad_(True)
    gb, ub = g.clone().requires_grad_(True), u.clone().requires_grad_(True)
    oa = mta.swiglu_gate(ga, ua)
    ob = F.silu(gb) * ub
    oa.backward(dy)
    ob.backward(dy)
    for a, b in ((oa, ob), (ga.grad, gb.grad), (ua.grad, ub.grad)):
        assert float((a == b).float().mean()) >= 0.999
        torch.testing.assert_close(a.float(), b.float(), rtol=2 ** -7, atol=2 ** -7)


@pytest.mark.parametrize("rows,d,act", [(32768, 512, torch.bfloat16), (1, 8, torch.bfloat16), (333, 1024, torch.float16),
                                        (77, 4096, torch.bfloat16), (5, 24, torch.float16)])
def test_mixed_norms_equal_the_fp32_kernels_rounded(mta, rows, d, act):
    # fp32 residual stream + 16-bit activations: the same fp32 arithmetic as the
    # single-dtype fp32 kernels, with the 16-bit outputs rounded once
    from importlib import import_module
    ops = import_module("mega-trading_amd.ops")
    branch = _gen((rows, d), 31, act).cuda()
    res = _gen((rows, d), 32, torch.float32).cuda()
    w = (1.0 + 0.1 * _gen((d,), 33, torch.float32)).cuda()
    dy = _gen((rows, d), 34, act).cuda()
    dres = _gen((rows, d), 35, torch.float32).cuda()
    # add + norm
    a_b, a_r, a_w = (t.clone().requires_grad_(True) for t in (branch, res, w))
    new_a, y_a = ops.add_rms_norm_mixed(a_b, a_r, a_w, eps=1e-5)
    torch.autograd.backward((new_a, y_a), (dres, dy))
    b_b, b_r, b_w = branch.float().requires_grad_(True), res.clone().requires_grad_(True), w.clone().requires_grad_(True)
    new_b, y_b = mta.add_rms_norm(b_b, b_r, b_w, eps=1e-5)
    torch.autograd.backward((new_b, y_b), (dres, dy.float()))
    torch.cuda.synchronize()
    assert new_a.dtype == torch.float32 and y_a.dtype == act and a_b.grad.dtype == act
    assert torch.equal(new_a, new_b) and torch.equal(y_a, y_b.to(act))
    assert torch.equal(a_r.grad, b_r.grad) and torch.equal(a_b.grad, b_b.grad.to(act))
    assert torch.equal(a_w.grad, b_w.grad)
    # plain norm of the fp32 stream
    c_x, c_w = res.clone().requires_grad_(True), w.clone().requires_grad_(True)
    y_c = ops.rms_norm_mixed(c_x, c_w, eps=1e-5, out_dtype=act)
    y_c.backward(dy)
    d_x, d_w = res.clone().requires_grad_(True), w.clone().requires_grad_(True)
    y_d = mta.rms_norm(d_x, d_w, eps=1e-5)
    y_d.backward(dy.float())
    torch.cuda.synchronize()
    assert y_c.dtype == act and torch.equal(y_c, y_d.to(act))
    assert torch.equal(c_x.grad, d_x.grad) and torch.equal(c_w.grad, d_w.grad)


def test_mixed_norm_errors():
    from importlib import import_module
    ops = import_module("mega-trading_amd.ops")
    x = torch.zeros(4, 16, device="cuda")
    w = torch.ones(16, device="cuda")
    with pytest.raises(RuntimeError, match="float32"):
        ops.rms_norm_mixed(x.bfloat16(), w, eps=1e-5, out_dtype=torch.bfloat16)
    with pytest.raises(RuntimeError, match="unsupported"):
        ops.rms_norm_mixed(x, w, eps=1e-5, out_dtype=torch.float32)
    with pytest.raises(ValueError, match="shape"):
        ops.add_rms_norm_mixed(torch.zeros(2, 16, device="cuda", dtype=torch.bfloat16), x, w, eps=1e-5)


@pytest.mark.parametrize("rows,cols,dt", [(32768, 1408, torch.bfloat16), (1, 8, torch.bfloat16), (333, 24, torch.float16),
                                          (1000, 1408, torch.float32), (7, 704, torch.bfloat16)])
def test_swiglu_packed_equals_the_pair_gate(rows, cols, dt):
    # same kernel arithmetic on the packed (gate | up) rows: bit-identical to
    # swiglu_gate on the two halves, forward and backward
    from importlib import import_module
    ops = import_module("mega-trading_amd.ops")
    gu, dy = _gen((rows, 2 * cols), 21, dt, 3.0).cuda(), _gen((rows, cols), 22, dt).cuda()
    a = gu.clone().requires_grad_(True)
    out = ops.swiglu_gate_packed(a)
    out.backward(dy)
    g, u = gu[:, :cols].contiguous().requires_grad_(True), gu[:, cols:].contiguous().requires_grad_(True)
    ref = ops.swiglu_gate(g, u)
    ref.backward(dy)
    torch.cuda.synchronize()
    assert out.shape == (rows, cols) and out.dtype == dt
    assert torch.equal(out, ref)
    assert torch.equal(a.grad[:, :cols], g.grad) and torch.equal(a.grad[:, cols:], u.grad)


def test_swiglu_packed_errors():
    from importlib import import_module
    ops = import_module("mega-trading_amd.ops")
    with pytest.raises(ValueError, match="multiple of 8"):
        ops.swiglu_gate_packed(torch.zeros(4, 24, device="cuda", dtype=torch.bfloat16))


@pytest.mark.parametrize("outs,rows", [((512, 128, 128), 32768), ((1408, 1408), 32768), ((512,), 32768),
                                       ((64, 32), 1000), ((96,), 3 * 1024)])
def test_projection_split_k_vs_fp64(outs, rows):
    # bf16 autocast product (one GEMM over the stacked weights) and fp32 split-K
    # weight gradients against fp64 products of the same bf16-rounded operands
    from importlib import import_module
    pj = import_module("mega-trading_amd.projection")
    g = torch.Generator().manual_seed(rows + sum(outs))
    x = torch.randn(rows, 512, generator=g).cuda().requires_grad_(True)
    ws = [(torch.randn(o, 512, generator=g) * 0.02).cuda().requires_grad_(True) for o in outs]
    with torch.autocast("cuda", dtype=torch.bfloat16):
        ys = pj.project(x, ws)
    dys = [torch.randn(rows, o, generator=g).cuda().bfloat16() for o in outs]
    torch.autograd.backward(ys, dys)
    xb = x.detach().bfloat16().double()
    for y, w, dy in zip(ys, ws, dys):
        wb = w.detach().bfloat16().double()
        assert y.dtype == torch.bfloat16 and w.grad.dtype == torch.float32
        ref = xb @ wb.t()
        assert ((y.double() - ref).norm() / ref.norm()).item() < 2 ** -8
        ref_dw = dy.double().t() @ xb
        assert ((w.grad.double() - ref_dw).norm() / ref_dw.norm()).item() < 1e-5  # fp32 accumulation
    ref_dx = sum(dy.double() @ w.detach().bfloat16().double() for dy, w in zip(dys, ws))
    assert ((x.grad.double() - ref_dx).norm() / ref_dx.norm()).item() < 2 ** -8


def test_swiglu_errors(mta):
    with pytest.raises(ValueError, match="same shape"):
        mta.swiglu_gate(torch.zeros(4, device="cuda"), torch.zeros(5, device="cuda"))
    with pytest.raises(RuntimeError, match="dtype"):
        mta.swiglu_gate(torch.zeros(4, device="cuda", dtype=torch.float64), torch.zeros(4, device="cuda", dtype=torch.float64))


# ---------------------------------------------------------------------------
# fused linear cross-entropy (HIP cross-entropy rows between hipBLASLt GEMMs)
# ---------------------------------------------------------------------------
def _ce_case(rows, hdim, vocab, seed, ignore_every=0):
    h = _gen((rows, hdim), seed, torch.float32)
    w = _gen((vocab, hdim), seed + 1, torch.float32, 0.05)
    g = torch.Generator().manual_seed(seed + 2)
    labels = torch.randint(0, vocab, (rows,), generator=g)
    if ignore_every:
        labels[::ignore_every] = -100
    return h, w, labels


@pytest.mark.parametrize("compute", ["bfloat16", "float32"])
def test_fused_linear_ce_vs_oracle(mta, compute):
    h, w, labels = _ce_case(1000, 512, 16384, 60, ignore_every=9)
    hg, wg = h.cuda().requires_grad_(True), w.cuda().requires_grad_(True)
    with torch.autocast("cuda", dtype=torch.bfloat16, enabled=compute == "bfloat16"):
        loss = mta.ops.fused_linear_cross_entropy(hg, wg, labels.cuda())
    loss.backward()
    assert loss.dtype == torch.float32 and hg.grad.dtype == torch.float32 and wg.grad.dtype == torch.float32
    rl, rgh, rgw = oo.fused_linear_cross_entropy(h.numpy(), w.numpy(), labels.numpy(), -100, compute)
    assert abs(loss.item() - rl) <= 1e-4 * abs(rl), (loss.item(), rl)
    tol = 1e-2 if compute == "bfloat16" else 1e-4
    assert _rel(hg.grad.cpu().numpy(), rgh) < tol
    assert _rel(wg.grad.cpu().numpy(), rgw) < tol


def test_fused_linear_ce_matches_eager_autocast_route_at_c5_rows(mta):
    # the reference's eager loss head under bf16 autocast: F.linear + F.cross_entropy
    # (model.py:124-129) on the C5 shape: 32 x 1024 rows, hidden 512, vocab 16384
    h, w, labels = _ce_case(32 * 1024, 512, 16384, 61)
    h, w, labels = h.cuda(), w.cuda(), labels.cuda()
    ha, wa = h.clone().requires_grad_(True), w.clone().requires_grad_(True)
    hb, wb = h.clone().requires_grad_(True), w.clone().requires_grad_(True)
    with torch.autocast("cuda", dtype=torch.bfloat16):
        la = mta.ops.fused_linear_cross_entropy(ha, wa, labels)
        lb = F.cross_entropy(F.linear(hb, wb), labels)
    la.backward()
    lb.backward()
    assert abs(la.item() - lb.item()) <= 1e-3 * abs(lb.item()), (la.item(), lb.item())
    assert _rel(ha.grad.cpu().numpy(), hb.grad.cpu().numpy()) < 2e-2
    assert _rel(wa.grad.cpu().numpy(), wb.grad.cpu().numpy()) < 2e-2


def test_fused_linear_ce_edge_cases(mta):
    h, w, labels = _ce_case(37, 64, 96, 62)
    hg, wg = h.cuda().requires_grad_(True), w.cuda().requires_grad_(True)
    # every row ignored: zero loss and zero gradients, as the reference
    loss = mta.ops.fused_linear_cross_entropy(hg, wg, torch.full((37,), -100, device="cuda"))
    loss.backward()
    assert loss.item() == 0.0 and not hg.grad.any() and not wg.grad.any()
    # int32 labels and a custom ignore_index; no-grad path returns the same loss
    lab32 = labels.to(torch.int32).cuda()
    lab32[3] = 7
    with torch.no_grad():
        l0 = mta.ops.fused_linear_cross_entropy(h.cuda(), w.cuda(), lab32, ignore_index=7)
    l1 = mta.ops.fused_linear_cross_entropy(h.cuda().requires_grad_(True), w.cuda(), lab32, ignore_index=7)
    assert torch.equal(l0, l1.detach())
    rl, _, _ = oo.fused_linear_cross_entropy(h.numpy(), w.numpy(), lab32.cpu().numpy(), 7, "float32")
    assert abs(l0.item() - rl) <= 1e-4 * abs(rl)
    # a label outside [0, vocab) gives a NaN loss rather than a read out of bounds
    bad = labels.clone().cuda()
    bad[0] = 96
    assert torch.isnan(mta.ops.fused_linear_cross_entropy(h.cuda(), w.cuda(), bad))


@pytest.mark.parametrize("vocab,compute", [(16387, "bfloat16"), (16387, "float32"), (97, "float32"), (13, "bfloat16"),
                                           (20003, "float32")])
def test_fused_linear_ce_odd_vocab(mta, vocab, compute):
    """Vocabularies that are not a multiple of 8: the reference tokenizer's size is
    3 specials plus a product with a 2-way side factor, always odd
    (tokenizer.py:103-107).  The logits get a padded row stride; the pad columns
    must not enter the softmax or the gradients.  20003 also takes the kernel's
    streaming path (more than 16384 logits per row)."""
    h, w, labels = _ce_case(300, 64, vocab, 65 + vocab % 7, ignore_every=11)
    labels[1] = vocab - 1  # the last real column, inside the padded chunk
    labels[2] = 0
    hg, wg = h.cuda().requires_grad_(True), w.cuda().requires_grad_(True)
    with torch.autocast("cuda", dtype=torch.bfloat16, enabled=compute == "bfloat16"):
        loss = mta.ops.fused_linear_cross_entropy(hg, wg, labels.cuda())
    loss.backward()
    assert wg.grad.shape == (vocab, 64)
    rl, rgh, rgw = oo.fused_linear_cross_entropy(h.numpy(), w.numpy(), labels.numpy(), -100, compute)
    assert abs(loss.item() - rl) <= 1e-4 * abs(rl), (loss.item(), rl)
    tol = 1e-2 if compute == "bfloat16" else 1e-4
    assert _rel(hg.grad.cpu().numpy(), rgh) < tol
    assert _rel(wg.grad.cpu().numpy(), rgw) < tol
    # and the eager route the model uses for requested logits (model.py:124-129)
    he, we = h.cuda().requires_grad_(True), w.cuda().requires_grad_(True)
    with torch.autocast("cuda", dtype=torch.bfloat16, enabled=compute == "bfloat16"):
        le = F.cross_entropy(F.linear(he, we), labels.cuda())
    le.backward()
    assert abs(loss.item() - le.item()) <= 1e-3 * abs(le.item())


def test_fused_linear_ce_chunked_equals_single_chunk(mta, monkeypatch):
    # batches beyond the chunk budget are processed in row chunks: same loss and gradients
    h, w, labels = _ce_case(3000, 128, 4096, 63, ignore_every=5)
    outs = []
    for budget in (2 << 30, 700 * 4096 * 2):  # one chunk; chunks of 700 rows (5 chunks, ragged last)
        monkeypatch.setattr(mta.ops, "_CE_CHUNK_BYTES", budget)
        hg, wg = h.cuda().requires_grad_(True), w.cuda().requires_grad_(True)
        with torch.autocast("cuda", dtype=torch.bfloat16):
            loss = mta.ops.fused_linear_cross_entropy(hg, wg, labels.cuda())
        loss.backward()
        outs.append((loss.detach(), hg.grad, wg.grad))
    (l1, gh1, gw1), (l2, gh2, gw2) = outs
    torch.testing.assert_close(l2, l1, rtol=1e-6, atol=1e-6)
    # rows are independent, but the GEMM library may pick other tilings for other row counts
    # (another accumulation order): equal to about a bf16 ulp
    assert _rel(gh2.cpu().numpy(), gh1.cpu().numpy()) < 2e-3
    assert _rel(gw2.cpu().numpy(), gw1.cpu().numpy()) < 5e-3  # summed per chunk in fp32 from bf16 products


def test_cross_entropy_rows_streaming_vocab(mta):
    # vocab above 16384 logits per row: the kernel streams the row twice instead of holding it in registers
    h, w, labels = _ce_case(64, 64, 20000, 64, ignore_every=6)
    hg, wg = h.cuda().requires_grad_(True), w.cuda().requires_grad_(True)
    loss = mta.ops.fused_linear_cross_entropy(hg, wg, labels.cuda())
    loss.backward()
    rl, rgh, rgw = oo.fused_linear_cross_entropy(h.numpy(), w.numpy(), labels.numpy(), -100, "float32")
    assert abs(loss.item() - rl) <= 1e-4 * abs(rl)
    assert _rel(hg.grad.cpu().numpy(), rgh) < 1e-4
    assert _rel(wg.grad.cpu().numpy(), rgw) < 1e-4


def test_tuned_gemm_replay_is_scoped_and_the_results_file_applies():
    # the committed results match this runtime (else TunableOp ignores them) and
    # the replay is switched on only inside tuned_gemms(), with tuning off,
    # leaving the process-wide TunableOp state as it was
    from importlib import import_module
    gt = import_module("mega-trading_amd.gemm_tuning")
    tun = torch.cuda.tunable
    assert gt._load(), "tuned/gemm_gfx950.csv does not validate against this runtime"
    before = (tun.is_enabled(), tun.tuning_is_enabled())
    with gt.tuned_gemms():
        assert tun.is_enabled() and not tun.tuning_is_enabled()
        a = torch.randn(32768, 512, device="cuda").bfloat16()
        w = torch.randn(768, 512, device="cuda").bfloat16()
        y = a @ w.t()
    assert (tun.is_enabled(), tun.tuning_is_enabled()) == before
    ref = a.double() @ w.double().t()
    assert ((y.double() - ref).norm() / ref.norm()).item() < 2 ** -8


# ---------------------------------------------------------------------------
# stand-alone RoPE (ops.apply_rope <- triton_apply_rope)
# ---------------------------------------------------------------------------
def _rope_layout(x, layout):
    """A [B, H, T, D] tensor with x's values in the given memory layout."""
    if layout == "bthd":  # the model's projection views
        return x.transpose(1, 2).contiguous().transpose(1, 2)
    if layout == "dstride2":  # every other element of a twice-as-wide buffer
        wide = torch.zeros(*x.shape[:-1], 2 * x.shape[-1], dtype=x.dtype, device=x.device)
        wide[..., ::2] = x
        return wide[..., ::2]
    return x


def _check_rotation(got, x, cos, sin, dt, inverse=False):
    """got == rot(x) (or rot^-1) from the fp64 oracle: one rounding to dt plus fp32 arithmetic error."""
    xf = x.double().cpu().numpy()
    c, s = cos.double().cpu().numpy(), sin.double().cpu().numpy()
    ref = ao.rope_inverse(xf, c, s) if inverse else ao.apply_rope(xf, c, s)
    pair = np.abs(xf[..., 0::2]) + np.abs(xf[..., 1::2])
    mag = np.repeat(pair, 2, axis=-1)
    tol = _ULP[dt] * np.abs(ref) + 2.0 ** -21 * mag
    err = np.abs(got.double().cpu().numpy() - ref)
    assert (err <= tol).all(), f"{(err > tol).sum()} values off; worst {err.max():.3e}"


ROPE_CASES = [
    # the reference's own parity shape (tests/test_training.py:627-647)
    ((1, 16, 4, 512, 64), torch.bfloat16, "contig"),
    ((2, 8, 2, 1024, 64), torch.bfloat16, "bthd"),    # the C5 layer's layout
    ((1, 4, 2, 17, 128), torch.float16, "bthd"),
    ((2, 4, 2, 33, 6), torch.float32, "contig"),      # D % 8 != 0: one pair per lane
    ((1, 2, 1, 9, 8), torch.bfloat16, "dstride2"),    # d stride 2
    ((1, 3, 3, 1, 32), torch.float32, "contig"),      # T = 1, R = 1
]


@pytest.mark.parametrize("shape,dt,layout", ROPE_CASES)
def test_apply_rope_vs_oracle(mta, shape, dt, layout):
    b, hq, hkv, t, d = shape
    rope = mta.model.RotaryEmbedding(d, max(t, 8) + 5, theta=500_000.0).cuda()
    q = _rope_layout(_gen((b, hq, t, d), 31, dt).cuda(), layout).requires_grad_(True)
    k = _rope_layout(_gen((b, hkv, t, d), 32, dt).cuda(), layout).requires_grad_(True)
    gq, gk = _gen((b, hq, t, d), 33, dt).cuda(), _gen((b, hkv, t, d), 34, dt).cuda()
    # tables cast to the activation dtype and sliced to T, as RotaryEmbedding.forward passes them
    cos = rope.cos[:, :, :t].to(dt)
    sin = rope.sin[:, :, :t].to(dt)
    qo, ko = mta.ops.apply_rope(q, k, cos, sin)
    torch.autograd.backward((qo, ko), (gq, gk))
    torch.cuda.synchronize()
    assert qo.stride() == q.stride() or layout == "dstride2"
    c2, s2 = cos[0, 0], sin[0, 0]
    _check_rotation(qo.detach(), q.detach(), c2, s2, dt)
    _check_rotation(ko.detach(), k.detach(), c2, s2, dt)
    _check_rotation(q.grad, gq, c2, s2, dt, inverse=True)
    _check_rotation(k.grad, gk, c2, s2, dt, inverse=True)


def test_apply_rope_matches_the_torch_rotation_and_inverts(mta):
    """Against the model's torch rotation (model.py:312-316) on fp32 tables,
    and rot^-1(rot(x)) == x to fp32 rounding."""
    rope = mta.model.RotaryEmbedding(64, 1024, theta=10_000.0).cuda()
    q = _gen((2, 8, 1024, 64), 35, torch.float32).cuda()
    k = _gen((2, 2, 1024, 64), 36, torch.float32).cuda()
    qo, ko = mta.ops.apply_rope(q, k, rope.cos, rope.sin)
    torch.testing.assert_close(qo, mta.model.rotate(q, rope.cos, rope.sin), rtol=1e-6, atol=1e-6)
    torch.testing.assert_close(ko, mta.model.rotate(k, rope.cos, rope.sin), rtol=1e-6, atol=1e-6)
    back_q, back_k = torch.ops.mega_trading_amd.rope_fwd(qo, ko, rope.cos[0, 0], rope.sin[0, 0], True)
    torch.testing.assert_close(back_q, q, rtol=1e-5, atol=1e-5)
    torch.testing.assert_close(back_k, k, rtol=1e-5, atol=1e-5)


def test_rotary_embedding_hip_route_vs_torch_route(mta):
    """RotaryEmbedding(operator_backend="triton") (model.py:292-293) against the
    torch route on the same module tables, bf16, gradients included."""
    hip = mta.model.RotaryEmbedding(64, 512, theta=500_000.0, operator_backend="triton").cuda()
    ref = mta.model.RotaryEmbedding(64, 512, theta=500_000.0).cuda()
    q = _gen((1, 16, 300, 64), 37, torch.bfloat16).cuda()
    k = _gen((1, 4, 300, 64), 38, torch.bfloat16).cuda()
    qa, ka = q.clone().requires_grad_(True), k.clone().requires_grad_(True)
    qb, kb = q.clone().requires_grad_(True), k.clone().requires_grad_(True)
    oa, pa = hip(qa, ka)
    ob, pb = ref(qb, kb)
    g1, g2 = torch.randn_like(oa), torch.randn_like(pa)
    torch.autograd.backward((oa, pa), (g1, g2))
    torch.autograd.backward((ob, pb), (g1, g2))
    # the torch route rounds each product to bf16 before the sum; the kernel rounds
    # once.  The reference's own bar for this comparison (tests/test_training.py:643-646)
    for got, want in ((oa, ob), (pa, pb)):
        torch.testing.assert_close(got.float(), want.float(), rtol=6e-2, atol=6e-2)
    for got, want in ((qa.grad, qb.grad), (ka.grad, kb.grad)):
        torch.testing.assert_close(got.float(), want.float(), rtol=8e-2, atol=8e-2)
