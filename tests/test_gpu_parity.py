"""GPU parity of the HIP kernels against the CPU oracle (BASELINE tolerances).

Every test runs the public op on cuda:0 and compares with
``oracle/attention_oracle.py`` on the same seeded, already-rounded inputs:
output max-abs <= 2e-2, gradient relative L2 <= 3e-2, LSE max-abs <= 1e-2.
Full-size configs are checked on sampled (batch, KV group) slices plus
size-independent properties (causality, determinism, GQA expansion).
"""

from __future__ import annotations

import os

import numpy as np
import pytest
import torch

from oracle import attention_oracle as orc
from tests.gpu_cases import (
    CONFIGS,
    TOL_GRAD_REL,
    TOL_OUT_MAXABS,
    compare,
    make_inputs,
    oracle,
    rel,
    run_hip,
    slice_group,
)

pytestmark = pytest.mark.gpu
GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")

# (batch, kv group) slices checked against the oracle at full size.  The grids
# issue (batch 0, group 0) first and (last batch, last group) last -- in every
# kernel the workgroup index runs over (batch, group) fastest, longest causal
# work first -- so those two slices hold the first and the last workgroups in
# issue order; the others are interior.
SAMPLES = {"C1": [(0, 0), (1, 1)], "C2": [(0, 0), (15, 1), (7, 0)],
           "C3": [(0, 0), (3, 3), (1, 2), (3, 1)], "C4": [(0, 0), (7, 7), (3, 4), (7, 5)]}


@pytest.mark.parametrize("rope", [False, True], ids=["plain", "rope"])
@pytest.mark.parametrize("name", ["C1", "C2", "C3", "C4"])
def test_baseline_config_parity(mta, name, rope):
    b, t, hq, hkv, d, sigma, theta = CONFIGS[name]
    r = hq // hkv
    q, k, v, do = make_inputs(b, t, hq, hkv, d, sigma=sigma, seed=0)
    cos = sin = None
    if rope:
        cos, sin = orc.rope_tables(t, d, theta)
    got = run_hip(mta, q, k, v, do, r, cos, sin)
    for bi, g in SAMPLES[name]:
        hs = slice(g * r, (g + 1) * r)
        ref = oracle(q[bi : bi + 1, hs], k[bi : bi + 1, g : g + 1], v[bi : bi + 1, g : g + 1], do[bi : bi + 1, hs], r, cos, sin)
        errs = compare(slice_group(got, bi, g, r), ref)
        print(name, "rope" if rope else "plain", (bi, g), {k_: f"{v_:.2e}" for k_, v_ in errs.items()}, flush=True)


@pytest.mark.parametrize("b,hkv,t", [(9, 2, 960), (10, 2, 960), (16, 2, 1024)])
def test_one_round_forward_grids(mta, b, hkv, t):
    """Forward grids of one resident round (256 < workgroups <= 512 on the
    MI355X's 256 CUs) run their second half lightest first: 270 and 300
    workgroups (the tail reversed workgroup by workgroup) and BASELINE
    config 2's 512 (reversed in chunks of 8).  Every row of the forward is
    checked against the oracle, so a task left out or run twice shows; the
    backward on the first and the last (batch, group) slice."""
    hq, d = 4 * hkv, 64
    q, k, v, do = make_inputs(b, t, hq, hkv, d, sigma=0.5, seed=b * 31 + t)
    got = run_hip(mta, q, k, v, do, 4)
    o_ref, lse_ref = orc.attention_forward(q.float().numpy(), k.float().numpy(), v.float().numpy(), 4)
    assert np.abs(got[0] - o_ref).max() <= TOL_OUT_MAXABS
    assert np.abs(got[1] - lse_ref).max() <= 1e-2
    for bi, g in ((0, 0), (b - 1, hkv - 1)):
        hs = slice(g * 4, (g + 1) * 4)
        ref = oracle(q[bi : bi + 1, hs], k[bi : bi + 1, g : g + 1], v[bi : bi + 1, g : g + 1], do[bi : bi + 1, hs], 4)
        compare(slice_group(got, bi, g, 4), ref)


@pytest.mark.parametrize("t", [1, 2, 17, 63, 64, 65, 127, 200, 333])
@pytest.mark.parametrize("hq,hkv", [(4, 4), (4, 2), (8, 2), (16, 2), (6, 2)])
def test_ragged_lengths_and_group_sizes(mta, t, hq, hkv):
    d = 64
    r = hq // hkv
    q, k, v, do = make_inputs(2, t, hq, hkv, d, sigma=0.5, seed=t * 100 + hq)
    cos, sin = orc.rope_tables(t, d, 10_000.0)
    compare(run_hip(mta, q, k, v, do, r), oracle(q, k, v, do, r))
    compare(run_hip(mta, q, k, v, do, r, cos, sin), oracle(q, k, v, do, r, cos, sin))


@pytest.mark.parametrize("t", [1, 31, 33, 65, 127, 129, 200])
@pytest.mark.parametrize("hq,hkv", [(4, 4), (6, 2), (8, 2)])
@pytest.mark.parametrize("d", [32, 128])
def test_ragged_lengths_other_head_dims(mta, d, t, hq, hkv):
    """Ragged T and every workgroup shape (R = 1, 3, 4) at D = 32 and D = 128;
    at D = 128 the forward and dQ split each 64-row block into two 32-row
    waves, so T just below / above a 32- or 64-row boundary matters."""
    r = hq // hkv
    q, k, v, do = make_inputs(2, t, hq, hkv, d, sigma=0.5, seed=t * 10 + hq + d)
    cos, sin = orc.rope_tables(t, d, 10_000.0)
    compare(run_hip(mta, q, k, v, do, r), oracle(q, k, v, do, r))
    compare(run_hip(mta, q, k, v, do, r, cos, sin), oracle(q, k, v, do, r, cos, sin))


@pytest.mark.parametrize("d", [32, 64, 128])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16], ids=["bf16", "fp16"])
def test_head_dims_and_dtypes(mta, d, dtype):
    t = 150
    q, k, v, do = make_inputs(2, t, 8, 2, d, sigma=0.5, seed=d, dtype=dtype)
    cos, sin = orc.rope_tables(t, d, 500_000.0)
    compare(run_hip(mta, q, k, v, do, 4), oracle(q, k, v, do, 4))
    compare(run_hip(mta, q, k, v, do, 4, cos, sin), oracle(q, k, v, do, 4, cos, sin))


@pytest.mark.parametrize("pattern", ["ramp", "spike"])
@pytest.mark.parametrize("d", [32, 64, 128])
def test_online_softmax_rescales(mta, d, pattern):
    """Running row max raised in the middle of tiles.

    "ramp" grows the key magnitudes along the sequence, so the row max of
    nearly every 32-key quarter exceeds the previous one by more than the
    kernels' lazy-rescale slack; "spike" puts one dominant key in the third
    quarter of the first tile and another in the second tile.  Both make the
    forward rescale while the next quarter's scores are already in flight.
    """
    b, t, hq, hkv = 1, 300, 8, 2
    q, k, v, do = make_inputs(b, t, hq, hkv, d, sigma=0.5, seed=7 + d)
    if pattern == "ramp":
        k = (k.float() * torch.linspace(1.0, 12.0, t).view(1, 1, t, 1)).to(k.dtype)
    else:
        k = k.float()
        k[:, :, 70] *= 24.0
        k[:, :, 190] *= 48.0
        k = k.to(q.dtype)
    compare(run_hip(mta, q, k, v, do, hq // hkv), oracle(q, k, v, do, hq // hkv))


def test_reference_small_case_fp16(mta):
    """test_training.py:519-548: fp16, B=1, Hq=4, Hkv=2, T=17, D=32, seed 11,
    against the frozen SDPA output at the reference's own tolerance (5e-2/6e-2),
    and against the oracle on the rounded inputs at ours."""
    g = np.load(os.path.join(GOLDEN, "t17_sdpa_fp32.npz"))
    q, k, v, do = (torch.from_numpy(g[n]).to(torch.float16) for n in ("q", "k", "v", "do"))
    got = run_hip(mta, q, k, v, do, 2)
    np.testing.assert_allclose(got[0], g["o"], atol=5e-2, rtol=5e-2)
    for i, n in ((2, "dq"), (3, "dk"), (4, "dv")):
        np.testing.assert_allclose(got[i], g[n], atol=6e-2, rtol=6e-2)
    compare(got, oracle(q, k, v, do, 2))


def test_reference_server_shape(mta):
    """test_training.py:550-600: bf16, B=1, Hq=16, Hkv=4, T=512, D=64, N(0,1) inputs."""
    q, k, v, do = make_inputs(1, 512, 16, 4, 64, sigma=1.0, seed=13)
    compare(run_hip(mta, q, k, v, do, 4), oracle(q, k, v, do, 4))


def test_model_layout_views_and_strided_grad(mta):
    """q/k/v as the [B,T,H,D]-physical views of model.py:220-222; dO non-contiguous."""
    b, t, hq, hkv, d = 2, 300, 8, 2, 64
    q, k, v, do = make_inputs(b, t, hq, hkv, d, seed=5)
    dev = "cuda:0"
    qv = q.transpose(1, 2).contiguous().to(dev).transpose(1, 2).requires_grad_(True)
    kv = k.transpose(1, 2).contiguous().to(dev).transpose(1, 2).requires_grad_(True)
    vv = v.transpose(1, 2).contiguous().to(dev).transpose(1, 2).requires_grad_(True)
    out = mta.attention(qv, kv, vv, repeats=4)
    assert out.stride() == qv.stride(), "output must keep the query's layout"
    dod = do.transpose(1, 2).contiguous().to(dev).transpose(1, 2)
    dq, dk, dv = torch.autograd.grad(out, (qv, kv, vv), dod)
    f = lambda x: x.detach().float().cpu().numpy()  # noqa: E731
    eo, _, edq, edk, edv = oracle(q, k, v, do, 4)
    assert np.abs(f(out) - eo).max() <= TOL_OUT_MAXABS
    assert max(rel(f(dq), edq), rel(f(dk), edk), rel(f(dv), edv)) <= TOL_GRAD_REL
    # an expanded (stride-0) upstream gradient, as out.sum().backward() produces
    qd = q.to(dev).requires_grad_(True)
    kd, vd = k.to(dev).requires_grad_(True), v.to(dev).requires_grad_(True)
    mta.attention(qd, kd, vd, repeats=4).float().sum().backward()
    ones = torch.ones_like(do)
    _, _, edq1, edk1, edv1 = oracle(q, k, v, ones, 4)
    assert max(rel(f(qd.grad), edq1), rel(f(kd.grad), edk1), rel(f(vd.grad), edv1)) <= TOL_GRAD_REL


@pytest.mark.parametrize("b,t,hq,hkv,d,dt", [(2, 1024, 8, 2, 64, torch.bfloat16), (1, 333, 4, 4, 128, torch.float16),
                                            (3, 200, 6, 2, 32, torch.bfloat16)])
def test_packed_qkv_equals_the_head_views(mta, b, t, hq, hkv, d, dt):
    """rope_attention_packed on one [B, T, (Hq + 2 Hkv) D] projection output: the
    same kernels with other strides, so output and packed gradient equal
    rope_attention on the three head views bit for bit."""
    from importlib import import_module
    attn = import_module("mega-trading_amd.attention")
    model_mod = import_module("mega-trading_amd.model")
    g = torch.Generator().manual_seed(t + d)
    qkv = (torch.randn(b, t, (hq + 2 * hkv) * d, generator=g) * 0.5).to(dt).cuda()
    dout = torch.randn(b, t, hq * d, generator=g).to(dt).cuda()
    rope = model_mod.RotaryEmbedding(d, 1024, theta=10_000.0).cuda()
    a = qkv.clone().requires_grad_(True)
    out = attn.rope_attention_packed(a, rope.cos, rope.sin, heads=hq, kv_heads=hkv)
    out.backward(dout)
    q, k, v = (x.detach().clone().requires_grad_(True) for x in attn._packed_views(qkv, hq, hkv))
    ref = attn.rope_attention(q, k, v, rope.cos, rope.sin, repeats=hq // hkv)
    ref.backward(dout.view(b, t, hq, d).transpose(1, 2))
    torch.cuda.synchronize()
    assert out.shape == (b, t, hq * d) and out.is_contiguous()
    assert torch.equal(out, ref.transpose(1, 2).reshape(b, t, hq * d))
    dq, dk, dv = attn._packed_views(a.grad, hq, hkv)
    assert torch.equal(dq, q.grad) and torch.equal(dk, k.grad) and torch.equal(dv, v.grad)


@pytest.mark.parametrize("t,rope", [(16384, False), (12345, True)])
def test_long_sequences_against_fp32_torch(mta, t, rope):
    """T four times BASELINE config 3's (and a ragged one): row indices, tile
    offsets and the causal loops at lengths the oracle is too slow for,
    against a float32 torch reference on the GPU (the dense softmax
    formula; the group's K/V repeated per query head).  BASELINE tolerances."""
    b, hq, hkv, d = 1, 4, 1, 64
    q, k, v, do = make_inputs(b, t, hq, hkv, d, sigma=0.5, seed=t)
    cos = sin = None
    if rope:
        cos, sin = orc.rope_tables(t, d, 10_000.0)
    got = run_hip(mta, q, k, v, do, hq // hkv, cos, sin)
    dev = torch.device("cuda:0")
    qf, kf, vf = (x.float().to(dev).requires_grad_(True) for x in (q, k, v))
    qr, kr = qf, kf
    if rope:
        c = torch.from_numpy(cos).to(dev)
        s_ = torch.from_numpy(sin).to(dev)

        def rot(x):
            e, o = x[..., 0::2], x[..., 1::2]
            return torch.stack((e * c - o * s_, e * s_ + o * c), dim=-1).flatten(-2)

        qr, kr = rot(qf), rot(kf)
    kk = kr.repeat_interleave(hq // hkv, dim=1)
    vv = vf.repeat_interleave(hq // hkv, dim=1)
    scores = torch.matmul(qr, kk.transpose(-2, -1).contiguous()) / d ** 0.5
    mask = torch.ones(t, t, dtype=torch.bool, device=dev).triu(1)
    scores = scores.masked_fill(mask, float("-inf"))
    lse = torch.logsumexp(scores, dim=-1)
    out = torch.matmul(torch.softmax(scores, dim=-1), vv)
    dq, dk, dv = torch.autograd.grad(out, (qf, kf, vf), do.float().to(dev))
    f = lambda x: x.detach().float().cpu().numpy()  # noqa: E731
    errs = compare(got, (f(out), f(lse), f(dq), f(dk), f(dv)))
    print(t, "rope" if rope else "plain", {k_: f"{v_:.2e}" for k_, v_ in errs.items()}, flush=True)


def test_causality_and_determinism_at_full_size(mta):
    """C3 shape: changing keys/values at positions >= t0 leaves output rows < t0
    bit-identical, and repeated runs are bit-identical (no atomics anywhere)."""
    b, t, hq, hkv, d, sigma, _ = CONFIGS["C3"]
    q, k, v, do = make_inputs(b, t, hq, hkv, d, sigma=sigma, seed=1)
    r = hq // hkv
    a = run_hip(mta, q, k, v, do, r)
    a2 = run_hip(mta, q, k, v, do, r)
    for x, y in zip(a, a2):
        assert np.array_equal(x, y)
    t0 = 2500
    k2, v2 = k.clone(), v.clone()
    k2[:, :, t0:] = (k2[:, :, t0:].float() * -3.0).to(k.dtype)
    v2[:, :, t0:] = (v2[:, :, t0:].float() + 1.0).to(v.dtype)
    c = run_hip(mta, q, k2, v2, do, r)
    assert np.array_equal(a[0][:, :, :t0], c[0][:, :, :t0])
    assert np.array_equal(a[1][:, :, :t0], c[1][:, :, :t0])
    assert not np.array_equal(a[0][:, :, t0:], c[0][:, :, t0:])


def test_gqa_matches_expanded_mha(mta):
    b, t, hq, hkv, d = 2, 777, 16, 4, 64
    r = hq // hkv
    q, k, v, do = make_inputs(b, t, hq, hkv, d, seed=9)
    g = run_hip(mta, q, k, v, do, r)
    e = run_hip(mta, q, k.repeat_interleave(r, 1), v.repeat_interleave(r, 1), do, 1)
    assert np.array_equal(g[0], e[0]), "forward per (head, row block) work is identical"
    assert np.array_equal(g[2], e[2]), "dQ per (head, row block) work is identical"
    assert rel(g[3], e[3].reshape(b, hkv, r, t, d).sum(2)) <= 1e-2
    assert rel(g[4], e[4].reshape(b, hkv, r, t, d).sum(2)) <= 1e-2


# fp32 inputs run on full-fp32 MFMA kernels (exact fp32 products, fp32
# accumulation, fp32 P and dS), so they are held to fp32-level tolerances
# against the float64 oracle -- far inside the 16-bit bars, and tighter than
# what the reference's own fp32 path (TF32 forward dots) would meet.
TOL_F32_OUT = 1e-4    # O max-abs
TOL_F32_LSE = 1e-4    # LSE max-abs
TOL_F32_GRAD = 1e-4   # ||dg|| / ||g|| for dQ, dK, dV


def test_fp32_config1_against_the_golden_sdpa_output(mta):
    """BASELINE config 1 in fp32 (B2 T256 Hq4 Hkv2 D32, N(0,1), seed 0): against the
    frozen torch-SDPA fp32 output (the golden fixture) and the oracle."""
    from tests.golden.make_golden import c1_inputs, input_digest

    g = np.load(os.path.join(GOLDEN, "c1_sdpa_fp32.npz"))
    q, k, v, do = c1_inputs()
    assert input_digest(q, k, v, do) == str(g["input_sha256"])
    got = run_hip(mta, q, k, v, do, 2)
    np.testing.assert_allclose(got[0], g["o"], atol=5e-5, rtol=1e-4)
    np.testing.assert_allclose(got[1], g["lse"], atol=5e-5, rtol=1e-5)
    for i, key in ((2, "dq"), (3, "dk"), (4, "dv")):
        np.testing.assert_allclose(got[i], g[key], atol=1e-4, rtol=1e-4)
    errs = compare(got, oracle(q, k, v, do, 2), out_tol=TOL_F32_OUT, grad_tol=TOL_F32_GRAD, lse_tol=TOL_F32_LSE)
    print("C1 fp32", {k_: f"{v_:.2e}" for k_, v_ in errs.items()}, flush=True)


@pytest.mark.parametrize("t", [1, 33, 100, 257])
@pytest.mark.parametrize("hq,hkv", [(4, 4), (6, 2), (8, 2)])
@pytest.mark.parametrize("d", [32, 64, 128])
def test_fp32_ragged_lengths_head_dims_and_rope(mta, d, t, hq, hkv):
    r = hq // hkv
    q, k, v, do = make_inputs(2, t, hq, hkv, d, sigma=1.0, seed=t + 7 * d + hq, dtype=torch.float32)
    cos, sin = orc.rope_tables(t, d, 10_000.0)
    for c, s_ in ((None, None), (cos, sin)):
        got = run_hip(mta, q, k, v, do, r, c, s_)
        ref = oracle(q, k, v, do, r, c, s_)
        if t == 1:
            # one key per row: P = 1, so dQ = dK = 0 exactly; fp32 leaves rounding noise
            assert np.abs(got[2]).max() <= 1e-5 and np.abs(got[3]).max() <= 1e-5
            got, ref = (got[0], got[1], ref[2], ref[3], got[4]), ref
        compare(got, ref, out_tol=TOL_F32_OUT, grad_tol=TOL_F32_GRAD, lse_tol=TOL_F32_LSE)


def test_fp32_model_layout_views(mta):
    """fp32 q/k/v as the [B,T,H,D]-physical views of model.py:220-222, output in q's layout."""
    b, t, hq, hkv, d = 2, 130, 8, 2, 64
    q, k, v, do = make_inputs(b, t, hq, hkv, d, sigma=1.0, seed=21, dtype=torch.float32)
    dev = "cuda:0"
    qv, kv, vv = (x.transpose(1, 2).contiguous().to(dev).transpose(1, 2).requires_grad_(True) for x in (q, k, v))
    out = mta.attention(qv, kv, vv, repeats=4)
    assert out.dtype == torch.float32 and out.stride() == qv.stride()
    dq, dk, dv = torch.autograd.grad(out, (qv, kv, vv), do.to(dev))
    f = lambda x: x.detach().cpu().numpy()  # noqa: E731
    eo, _, edq, edk, edv = oracle(q, k, v, do, 4)
    assert np.abs(f(out) - eo).max() <= TOL_F32_OUT
    assert max(rel(f(dq), edq), rel(f(dk), edk), rel(f(dv), edv)) <= TOL_F32_GRAD


def test_native_library_is_loaded(mta):
    mta._native.load()
    maps = open("/proc/self/maps").read()
    assert mta._native.library_path() in maps
    assert mta._native.torch_ops_path() in maps


@pytest.mark.parametrize("d", [8, 16, 40, 48, 80, 100, 17])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32], ids=["bf16", "fp32"])
def test_other_head_dims_are_padded_to_a_kernel_size(mta, d, dtype):
    """Head sizes the kernels are not built for (the reference's forward takes any
    D, triton_attention.py:36; its demo ablation uses D = 8, configs/ablations/
    demo.yaml:24-31) run zero-padded to the next of 32 / 64 / 128 with the scale of
    the real D.  RoPE needs an even D (17 runs without it)."""
    t, hq, hkv = 150, 6, 2
    q, k, v, do = make_inputs(2, t, hq, hkv, d, sigma=0.5, seed=d, dtype=dtype)
    tol = dict(out_tol=1e-4, grad_tol=1e-4, lse_tol=1e-4) if dtype == torch.float32 else {}
    compare(run_hip(mta, q, k, v, do, 3), oracle(q, k, v, do, 3), **tol)
    if d % 2 == 0:
        cos, sin = orc.rope_tables(t, d, 10_000.0)
        compare(run_hip(mta, q, k, v, do, 3, cos, sin), oracle(q, k, v, do, 3, cos, sin), **tol)


def test_padded_head_dim_keeps_the_query_layout(mta):
    b, t, hq, hkv, d = 2, 64, 4, 2, 8
    q, k, v, do = make_inputs(b, t, hq, hkv, d, seed=3)
    dev = "cuda:0"
    qv = q.transpose(1, 2).contiguous().to(dev).transpose(1, 2).requires_grad_(True)
    out = mta.attention(qv, k.to(dev), v.to(dev), repeats=2)
    assert out.shape == qv.shape and out.stride() == qv.stride()
