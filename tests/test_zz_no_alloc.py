"""GPU test of the allocation-free backward, mt_gqa_attn_bwd_noalloc, through
the C ABI: its dQ/dK/dV against mt_gqa_attn_bwd's (caller workspace) on the
same forward outputs, for two calls in a row with the second smaller, and for
a shape whose standard dK/dV partial sums exceed the fixed scratch (a smaller
head split is used there, so only the summation order differs)."""

from __future__ import annotations

import ctypes
import math

import pytest
import torch

from oracle import attention_oracle as orc
from tests.gpu_cases import TOL_GRAD_REL, make_inputs, rel

pytestmark = pytest.mark.gpu

DTYPES = {torch.bfloat16: 0, torch.float16: 1}


def _backward_both_ways(mta, b, t, hq, hkv, d, dtype, rope, seed):
    native = mta._native
    lib = native.load()
    dev = torch.device("cuda:0")
    q, k, v, do = (x.to(dev) for x in make_inputs(b, t, hq, hkv, d, sigma=0.5, seed=seed, dtype=dtype))
    o = torch.empty_like(q)
    lse = torch.empty((b, hq, t), device=dev, dtype=torch.float32)
    cos = sin = None
    q_rot = k_rot = None
    if rope:
        c, s = orc.rope_tables(t, d, 10_000.0)
        cos, sin = torch.from_numpy(c).to(dev), torch.from_numpy(s).to(dev)
        q_rot, k_rot = torch.empty_like(q), torch.empty_like(k)
    ptr = lambda x: None if x is None else x.data_ptr()  # noqa: E731
    stream = torch.cuda.current_stream(dev).cuda_stream
    scale = 1.0 / math.sqrt(d)
    print(f"case B={b} T={t} Hq={hq} Hkv={hkv} D={d} {dtype} rope={rope}", flush=True)
    native.check(lib.mt_gqa_attn_fwd(q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(), lse.data_ptr(),
                                     ptr(q_rot), ptr(k_rot), b, hq, hkv, t, d, native.strides_array(q, k, v, o),
                                     scale, DTYPES[dtype], ptr(cos), ptr(sin), stream), "mt_gqa_attn_fwd")
    qs, ks = (q_rot, k_rot) if rope else (q, k)
    outs = []
    for noalloc in (False, True):
        dq, dk, dv = torch.empty_like(q), torch.empty_like(k), torch.empty_like(v)
        strides = native.strides_array(qs, ks, v, o, do, dq, dk, dv)
        args_in = (qs.data_ptr(), ks.data_ptr(), v.data_ptr(), o.data_ptr(), lse.data_ptr(), do.data_ptr(),
                   dq.data_ptr(), dk.data_ptr(), dv.data_ptr())
        tail = (b, hq, hkv, t, d, strides, scale, DTYPES[dtype], ptr(cos), ptr(sin), stream)
        if noalloc:
            native.check(lib.mt_gqa_attn_bwd_noalloc(*args_in, *tail), "mt_gqa_attn_bwd_noalloc")
        else:
            ws_bytes = lib.mt_gqa_attn_bwd_workspace_size(b, hq, hkv, t, d)
            ws = torch.empty(ws_bytes, device=dev, dtype=torch.uint8)
            native.check(lib.mt_gqa_attn_bwd(*args_in, ws.data_ptr(), ws_bytes, *tail), "mt_gqa_attn_bwd")
        torch.cuda.synchronize()
        outs.append((dq, dk, dv))
    return outs, lib.mt_gqa_attn_bwd_workspace_size(b, hq, hkv, t, d)


def test_noalloc_backward_equals_the_workspace_backward_on_two_calls(mta):
    # first call, then a smaller second one: the scratch keeps the first call's
    # contents, which the second must not read
    for case in ((2, 1024, 8, 2, 64, torch.bfloat16, True, 1), (1, 300, 4, 1, 32, torch.float16, False, 2)):
        (ref, got), ws_bytes = _backward_both_ways(mta, *case)
        assert ws_bytes <= 64 << 20, "the standard head split fits the scratch: same kernels, same split"
        for name, a, e in zip(("dq", "dk", "dv"), got, ref):
            assert torch.isfinite(a).all(), name
            assert torch.equal(a, e), f"{name}: max diff {(a.float() - e.float()).abs().max().item()}"


def test_noalloc_backward_with_a_smaller_head_split(mta):
    # one long D = 128 sequence: the standard dK/dV head split's fp32 partials
    # exceed the 64 MiB scratch, so the allocation-free call sums the heads in
    # fewer workgroups; the gradients agree to the summation order
    (ref, got), ws_bytes = _backward_both_ways(mta, 1, 8192, 16, 4, 128, torch.bfloat16, True, 3)
    assert ws_bytes > 64 << 20
    for name, a, e in zip(("dq", "dk", "dv"), got, ref):
        err = rel(a.float().cpu().numpy(), e.float().cpu().numpy())
        print(name, f"rel {err:.2e}", flush=True)
        if name == "dq":
            assert torch.equal(a, e), "dQ does not depend on the dK/dV split"
        assert err <= TOL_GRAD_REL / 10
