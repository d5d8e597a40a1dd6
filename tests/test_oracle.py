"""Pin the CPU oracle (oracle/attention_oracle.py) before trusting it.

Every oracle function is checked against something that does not restate its
own formula: the committed golden vectors (torch SDPA, the routine the
reference's eager path calls), live torch SDPA + autograd, a brute-force
per-element loop, closed forms and invariants, and finite differences.  The
``test_mutation_*`` tests plant plausible mistakes in a copy of the oracle and
show that at least one of these checks rejects each of them.
"""

from __future__ import annotations

import os

import numpy as np
import pytest
import torch

from oracle import attention_oracle as orc
from oracle.sdpa_cpu import masked_logsumexp, rope_tables_torch, sdpa_forward_backward

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def _rand(shape, seed, scale=1.0):
    return np.random.default_rng(seed).standard_normal(shape) * scale


def _rel(a, b):
    return float(np.linalg.norm(np.asarray(a) - np.asarray(b)) / max(np.linalg.norm(np.asarray(b)), 1e-30))


# ---------------------------------------------------------------------------
# golden vectors
# ---------------------------------------------------------------------------
def test_golden_c1_config():
    """BASELINE config 1 (B2 T256 Hq4 Hkv2 D32, seed 0) against frozen SDPA output."""
    from tests.golden.make_golden import c1_inputs, input_digest

    g = np.load(os.path.join(GOLDEN, "c1_sdpa_fp32.npz"))
    q, k, v, do = c1_inputs()
    assert input_digest(q, k, v, do) == str(g["input_sha256"]), "torch RNG changed: inputs differ from the golden draw"
    q, k, v, do = (t.numpy() for t in (q, k, v, do))
    o, lse = orc.attention_forward(q, k, v, repeats=2)
    dq, dk, dv = orc.attention_backward(q, k, v, do, repeats=2)
    np.testing.assert_allclose(o, g["o"], atol=2e-5, rtol=1e-4)
    np.testing.assert_allclose(lse, g["lse"], atol=2e-5, rtol=1e-5)
    for got, key in ((dq, "dq"), (dk, "dk"), (dv, "dv")):
        np.testing.assert_allclose(got, g[key], atol=5e-5, rtol=1e-4)


def test_golden_reference_t17_shape():
    """The reference's own small parity shape (test_training.py:519-548)."""
    g = np.load(os.path.join(GOLDEN, "t17_sdpa_fp32.npz"))
    o, lse = orc.attention_forward(g["q"], g["k"], g["v"], repeats=2)
    dq, dk, dv = orc.attention_backward(g["q"], g["k"], g["v"], g["do"], repeats=2)
    np.testing.assert_allclose(o, g["o"], atol=1e-5, rtol=1e-5)
    np.testing.assert_allclose(lse, g["lse"], atol=1e-5, rtol=1e-5)
    np.testing.assert_allclose(dq, g["dq"], atol=2e-5, rtol=1e-4)
    np.testing.assert_allclose(dk, g["dk"], atol=2e-5, rtol=1e-4)
    np.testing.assert_allclose(dv, g["dv"], atol=2e-5, rtol=1e-4)


def test_golden_rope_tables_and_rope_attention():
    g = np.load(os.path.join(GOLDEN, "rope_t17_fp32.npz"))
    t17 = np.load(os.path.join(GOLDEN, "t17_sdpa_fp32.npz"))
    for theta, tag in ((10_000.0, "1e4"), (500_000.0, "5e5")):
        cos, sin = orc.rope_tables(17, 32, theta)
        np.testing.assert_allclose(cos, g[f"cos_{tag}"], atol=2e-6, rtol=0)
        np.testing.assert_allclose(sin, g[f"sin_{tag}"], atol=2e-6, rtol=0)
    cos, sin = g["cos_1e4"], g["sin_1e4"]
    o, _ = orc.rope_attention_forward(t17["q"], t17["k"], t17["v"], cos, sin, repeats=2)
    dq, dk, dv = orc.rope_attention_backward(t17["q"], t17["k"], t17["v"], t17["do"], cos, sin, repeats=2)
    np.testing.assert_allclose(o, g["o"], atol=1e-5, rtol=1e-5)
    np.testing.assert_allclose(dq, g["dq"], atol=2e-5, rtol=1e-4)
    np.testing.assert_allclose(dk, g["dk"], atol=2e-5, rtol=1e-4)
    np.testing.assert_allclose(dv, g["dv"], atol=2e-5, rtol=1e-4)


# ---------------------------------------------------------------------------
# live torch SDPA (float64) over ragged shapes and GQA ratios
# ---------------------------------------------------------------------------
@pytest.mark.parametrize(
    "b,hq,hkv,t,d",
    [(1, 1, 1, 1, 8), (1, 2, 1, 2, 8), (2, 4, 2, 17, 16), (1, 8, 2, 65, 32), (1, 3, 1, 33, 8), (2, 4, 4, 31, 8)],
)
def test_against_torch_sdpa_float64(b, hq, hkv, t, d):
    r = hq // hkv
    q, k, v, do = (_rand(s, i) for i, s in enumerate([(b, hq, t, d), (b, hkv, t, d), (b, hkv, t, d), (b, hq, t, d)]))
    o, lse = orc.attention_forward(q, k, v, repeats=r)
    dq, dk, dv = orc.attention_backward(q, k, v, do, repeats=r)
    tq, tk, tv, tdo = (torch.from_numpy(x) for x in (q, k, v, do))
    eo, edq, edk, edv = sdpa_forward_backward(tq, tk, tv, tdo, repeats=r)
    e_lse = masked_logsumexp(tq, tk, repeats=r)
    np.testing.assert_allclose(o, eo.numpy(), atol=1e-12, rtol=1e-10)
    np.testing.assert_allclose(lse, e_lse.numpy(), atol=1e-12, rtol=1e-10)
    np.testing.assert_allclose(dq, edq.numpy(), atol=1e-11, rtol=1e-9)
    np.testing.assert_allclose(dk, edk.numpy(), atol=1e-11, rtol=1e-9)
    np.testing.assert_allclose(dv, edv.numpy(), atol=1e-11, rtol=1e-9)


def test_row_chunking_does_not_change_results():
    q, k, v, do = (_rand(s, 40 + i) for i, s in enumerate([(1, 2, 50, 8), (1, 1, 50, 8), (1, 1, 50, 8), (1, 2, 50, 8)]))
    a = orc.attention_forward(q, k, v, repeats=2, chunk=7)
    b = orc.attention_forward(q, k, v, repeats=2, chunk=1024)
    np.testing.assert_allclose(a[0], b[0], atol=1e-14)
    ga = orc.attention_backward(q, k, v, do, repeats=2, chunk=7)
    gb = orc.attention_backward(q, k, v, do, repeats=2, chunk=1024)
    for x, y in zip(ga, gb):
        np.testing.assert_allclose(x, y, atol=1e-13)


# ---------------------------------------------------------------------------
# brute force and closed forms
# ---------------------------------------------------------------------------
def _brute_force(q, k, v, r):
    b, hq, t, d = q.shape
    o = np.zeros_like(q)
    lse = np.zeros((b, hq, t))
    for bi in range(b):
        for h in range(hq):
            for i in range(t):
                s = [sum(q[bi, h, i, x] * k[bi, h // r, j, x] for x in range(d)) / np.sqrt(d) for j in range(i + 1)]
                mx = max(s)
                w = [np.exp(x - mx) for x in s]
                z = sum(w)
                lse[bi, h, i] = mx + np.log(z)
                for x in range(d):
                    o[bi, h, i, x] = sum(w[j] * v[bi, h // r, j, x] for j in range(i + 1)) / z
    return o, lse


def test_brute_force_tiny():
    q, k, v = _rand((1, 4, 6, 4), 1), _rand((1, 2, 6, 4), 2), _rand((1, 2, 6, 4), 3)
    o, lse = orc.attention_forward(q, k, v, repeats=2)
    eo, e_lse = _brute_force(q, k, v, 2)
    np.testing.assert_allclose(o, eo, atol=1e-13)
    np.testing.assert_allclose(lse, e_lse, atol=1e-13)


def test_closed_form_first_row_and_lse():
    q, k, v = _rand((2, 4, 9, 8), 4), _rand((2, 2, 9, 8), 5), _rand((2, 2, 9, 8), 6)
    o, lse = orc.attention_forward(q, k, v, repeats=2)
    for h in range(4):
        np.testing.assert_allclose(o[:, h, 0], v[:, h // 2, 0], atol=1e-14)
        np.testing.assert_allclose(lse[:, h, 0], (q[:, h, 0] * k[:, h // 2, 0]).sum(-1) / np.sqrt(8), atol=1e-13)
    # LSE bounds: max_j s_ij <= LSE_i <= max_j s_ij + ln(i + 1)
    s = np.einsum("bhid,bhjd->bhij", q, np.repeat(k, 2, axis=1)) / np.sqrt(8)
    s = np.where(np.tril(np.ones((9, 9), bool)), s, -np.inf)
    m = s.max(-1)
    assert np.all(lse >= m - 1e-12)
    assert np.all(lse <= m + np.log(np.arange(1, 10)) + 1e-12)


def test_causality_future_keys_do_not_matter():
    q, k, v = _rand((1, 2, 12, 8), 7), _rand((1, 1, 12, 8), 8), _rand((1, 1, 12, 8), 9)
    o, _ = orc.attention_forward(q, k, v, repeats=2)
    k2, v2 = k.copy(), v.copy()
    k2[:, :, 7:] += 5.0
    v2[:, :, 7:] -= 3.0
    o2, _ = orc.attention_forward(q, k2, v2, repeats=2)
    np.testing.assert_allclose(o[:, :, :7], o2[:, :, :7], atol=1e-14)
    assert not np.allclose(o[:, :, 7:], o2[:, :, 7:])
    # gradient of a single early row reaches no later key/value
    do = np.zeros_like(q)
    do[:, :, 3] = _rand((1, 2, 8), 10)
    _, dk, dv = orc.attention_backward(q, k, v, do, repeats=2)
    assert np.abs(dk[:, :, 4:]).max() == 0 and np.abs(dv[:, :, 4:]).max() == 0


def test_gqa_equals_mha_on_expanded_kv_and_grads_are_group_sums():
    r = 4
    q, k, v, do = (_rand(s, 20 + i) for i, s in enumerate([(2, 8, 11, 8), (2, 2, 11, 8), (2, 2, 11, 8), (2, 8, 11, 8)]))
    ke, ve = np.repeat(k, r, axis=1), np.repeat(v, r, axis=1)
    o, lse = orc.attention_forward(q, k, v, repeats=r)
    o1, lse1 = orc.attention_forward(q, ke, ve, repeats=1)
    np.testing.assert_allclose(o, o1, atol=1e-14)
    np.testing.assert_allclose(lse, lse1, atol=1e-14)
    dq, dk, dv = orc.attention_backward(q, k, v, do, repeats=r)
    dq1, dk1, dv1 = orc.attention_backward(q, ke, ve, do, repeats=1)
    np.testing.assert_allclose(dq, dq1, atol=1e-13)
    np.testing.assert_allclose(dk, dk1.reshape(2, 2, r, 11, 8).sum(2), atol=1e-13)
    np.testing.assert_allclose(dv, dv1.reshape(2, 2, r, 11, 8).sum(2), atol=1e-13)


def test_backward_matches_finite_differences():
    rng = np.random.default_rng(31)
    q, k, v = rng.standard_normal((1, 2, 5, 4)), rng.standard_normal((1, 1, 5, 4)), rng.standard_normal((1, 1, 5, 4))
    w = rng.standard_normal((1, 2, 5, 4))

    def loss(q_, k_, v_):
        return float((orc.attention_forward(q_, k_, v_, repeats=2)[0] * w).sum())

    dq, dk, dv = orc.attention_backward(q, k, v, w, repeats=2)
    eps = 1e-6
    for arr, grad in ((q, dq), (k, dk), (v, dv)):
        it = np.nditer(arr, flags=["multi_index"])
        for _ in it:
            idx = it.multi_index
            save = arr[idx]
            arr[idx] = save + eps
            up = loss(q, k, v)
            arr[idx] = save - eps
            dn = loss(q, k, v)
            arr[idx] = save
            assert abs((up - dn) / (2 * eps) - grad[idx]) < 1e-7


def test_delta_identity_rowsum_o_do_equals_rowsum_dp_p():
    """triton_attention.py:561 uses rowsum(O*dO) where :99 uses rowsum(dP*P)."""
    q, k, v, do = (_rand(s, 50 + i) for i, s in enumerate([(1, 2, 10, 8), (1, 1, 10, 8), (1, 1, 10, 8), (1, 2, 10, 8)]))
    o, _ = orc.attention_forward(q, k, v, repeats=2)
    s = np.einsum("hid,jd->hij", q[0], k[0, 0]) / np.sqrt(8)
    s = np.where(np.tril(np.ones((10, 10), bool)), s, -np.inf)
    p = np.exp(s - s.max(-1, keepdims=True))
    p /= p.sum(-1, keepdims=True)
    dp = np.einsum("hid,jd->hij", do[0], v[0, 0])
    np.testing.assert_allclose((o[0] * do[0]).sum(-1), (dp * p).sum(-1), atol=1e-13)


# ---------------------------------------------------------------------------
# RoPE
# ---------------------------------------------------------------------------
def test_rope_closed_forms():
    cos, sin = orc.rope_tables(16, 8, 10_000.0)
    assert np.all(cos[0] == 1.0) and np.all(sin[0] == 0.0)
    x = _rand((2, 3, 16, 8), 60)
    y = orc.apply_rope(x, cos, sin)
    np.testing.assert_allclose(y[..., 0, :], x[..., 0, :], atol=0)
    # norm of every pair is preserved
    np.testing.assert_allclose(
        y[..., 0::2] ** 2 + y[..., 1::2] ** 2, x[..., 0::2] ** 2 + x[..., 1::2] ** 2, rtol=1e-6
    )
    # hand-computed pair: position 3, pair 1 (dims 2,3), inv_freq = 1e4 ** (-2/8)
    ang = 3 * 10_000.0 ** (-2 / 8)
    e, o = x[0, 0, 3, 2], x[0, 0, 3, 3]
    np.testing.assert_allclose(y[0, 0, 3, 2], e * np.cos(ang) - o * np.sin(ang), rtol=1e-6)
    np.testing.assert_allclose(y[0, 0, 3, 3], e * np.sin(ang) + o * np.cos(ang), rtol=1e-6)
    # the backward rotation inverts the forward one
    np.testing.assert_allclose(orc.rope_inverse(y, cos, sin), x, atol=1e-12)


def test_rope_tables_match_torch_formula():
    for t, d, theta in ((64, 32, 10_000.0), (4096, 64, 10_000.0), (512, 64, 500_000.0), (2048, 128, 10_000.0)):
        c, s = orc.rope_tables(t, d, theta)
        tc, ts = rope_tables_torch(t, d, theta)
        # identical fp32 formula; numpy's and torch's fp32 pow may differ by one
        # ulp in inv_freq, which position t amplifies to ~t * 6e-8 rad
        np.testing.assert_allclose(c, tc.numpy(), atol=1e-6 + 1e-7 * t, rtol=0)
        np.testing.assert_allclose(s, ts.numpy(), atol=1e-6 + 1e-7 * t, rtol=0)


def test_rope_attention_backward_matches_autograd():
    rng = np.random.default_rng(70)
    q, k, v, do = (rng.standard_normal(s) for s in [(2, 4, 13, 8), (2, 2, 13, 8), (2, 2, 13, 8), (2, 4, 13, 8)])
    cos, sin = orc.rope_tables(13, 8, 10_000.0)
    dq, dk, dv = orc.rope_attention_backward(q, k, v, do, cos, sin, repeats=2)
    tq, tk, tv = (torch.from_numpy(x).requires_grad_(True) for x in (q, k, v))
    tc, ts = torch.from_numpy(cos.astype(np.float64)), torch.from_numpy(sin.astype(np.float64))

    def rot(x):
        e, o = x[..., 0::2], x[..., 1::2]
        return torch.stack((e * tc - o * ts, e * ts + o * tc), dim=-1).flatten(-2)

    out = torch.nn.functional.scaled_dot_product_attention(rot(tq), rot(tk), tv, is_causal=True, enable_gqa=True)
    gq, gk, gv = torch.autograd.grad(out, (tq, tk, tv), torch.from_numpy(do))
    np.testing.assert_allclose(dq, gq.numpy(), atol=1e-11)
    np.testing.assert_allclose(dk, gk.numpy(), atol=1e-11)
    np.testing.assert_allclose(dv, gv.numpy(), atol=1e-11)


# ---------------------------------------------------------------------------
# planted mistakes: each must be caught by one of the checks above
# ---------------------------------------------------------------------------
def _fwd_check(fwd):
    """Golden t17 forward check as a predicate (True = passes)."""
    g = np.load(os.path.join(GOLDEN, "t17_sdpa_fp32.npz"))
    o, lse = fwd(g["q"], g["k"], g["v"], 2)
    return np.allclose(o, g["o"], atol=1e-5) and np.allclose(lse, g["lse"], atol=1e-5)


def _bwd_check(bwd):
    g = np.load(os.path.join(GOLDEN, "t17_sdpa_fp32.npz"))
    dq, dk, dv = bwd(g["q"], g["k"], g["v"], g["do"], 2)
    return all(np.allclose(a, g[n], atol=2e-5, rtol=1e-4) for a, n in ((dq, "dq"), (dk, "dk"), (dv, "dv")))


def test_mutation_checks_are_sensitive():
    ok_f = lambda q, k, v, r: orc.attention_forward(q, k, v, repeats=r)  # noqa: E731
    ok_b = lambda q, k, v, do, r: orc.attention_backward(q, k, v, do, repeats=r)  # noqa: E731
    assert _fwd_check(ok_f) and _bwd_check(ok_b)

    # wrong scale (1/D instead of 1/sqrt(D))
    assert not _fwd_check(lambda q, k, v, r: orc.attention_forward(q, k, v, repeats=r, scale=1.0 / q.shape[-1]))
    # strided instead of contiguous GQA map (kv = h % Hkv)
    perm = lambda x: x[:, [0, 2, 1, 3]]  # noqa: E731
    assert not _fwd_check(lambda q, k, v, r: (lambda o: (perm(o[0]), perm(o[1])))(orc.attention_forward(perm(q), k, v, repeats=r)))
    # missing causal mask: attend to every key
    def no_mask(q, k, v, r):
        b, h, t, d = q.shape
        s = np.einsum("bhid,bhjd->bhij", q, np.repeat(k, r, 1)) / np.sqrt(d)
        m = s.max(-1, keepdims=True)
        p = np.exp(s - m)
        z = p.sum(-1, keepdims=True)
        return (p / z) @ np.repeat(v, r, 1), (m + np.log(z))[..., 0]
    assert not _fwd_check(no_mask)
    # LSE in log2 instead of natural log
    assert not _fwd_check(lambda q, k, v, r: (lambda o: (o[0], o[1] / np.log(2)))(orc.attention_forward(q, k, v, repeats=r)))
    # backward: dK not scaled / dV transposed roles / delta dropped
    assert not _bwd_check(lambda q, k, v, do, r: (lambda g: (g[0], g[1] / (1 / np.sqrt(32)), g[2]))(ok_b(q, k, v, do, r)))
    assert not _bwd_check(lambda q, k, v, do, r: (lambda g: (g[0], g[2], g[1]))(ok_b(q, k, v, do, r)))
    # dK/dV not summed over the group (first head only)
    def first_head_only(q, k, v, do, r):
        do2 = do.copy()
        do2[:, 1::2] = 0
        dq, dk, dv = ok_b(q, k, v, do2, r)
        return ok_b(q, k, v, do, r)[0], dk, dv
    assert not _bwd_check(first_head_only)
    # RoPE pairs half-split instead of interleaved
    cos, sin = orc.rope_tables(8, 8, 10_000.0)
    x = _rand((1, 1, 8, 8), 80)
    half = np.concatenate([x[..., :4] * cos - x[..., 4:] * sin, x[..., :4] * sin + x[..., 4:] * cos], -1)
    ang = 3 * 10_000.0 ** (-2 / 8)
    assert not np.isclose(half[0, 0, 3, 2], x[0, 0, 3, 2] * np.cos(ang) - x[0, 0, 3, 3] * np.sin(ang))



def test_decode_oracle_is_the_last_row_of_the_causal_forward():
    # pinned by the (already pinned) causal forward: the new token's output is the
    # last row of attention over all cached positions, for every prefix length
    rng = np.random.default_rng(70)
    b, hq, hkv, t, d = 2, 8, 2, 19, 32
    q = rng.standard_normal((b, hq, t, d))
    k = rng.standard_normal((b, hkv, t, d))
    v = rng.standard_normal((b, hkv, t, d))
    for length in (1, 2, 7, 19):
        full, _ = orc.attention_forward(q[:, :, :length], k[:, :, :length], v[:, :, :length], 4)
        dec = orc.decode_attention(q[:, :, length - 1], k, v, length, 4)
        np.testing.assert_allclose(dec, full[:, :, -1], rtol=1e-12, atol=1e-12)
    # length 1: the output is v_0 exactly (one key)
    np.testing.assert_allclose(orc.decode_attention(q[:, :, 0], k, v, 1, 4)[:, 0], v[:, 0, 0], rtol=1e-15)
