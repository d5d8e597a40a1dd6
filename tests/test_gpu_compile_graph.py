"""The op under torch.compile and inside a captured HIP graph.

The reference's training config compiles the model (configs/rtx.yaml:75-77)
and the attention must be re-entrant on the caller's stream, so: the custom
ops trace with fullgraph=True (fake implementations, registered autograd),
and a captured forward + backward replays to the eager results, replay after
replay, with eager work on the same tensors in between.
"""

from __future__ import annotations

import gc

import importlib

import pytest
import torch

from tests.gpu_cases import make_inputs

pytestmark = pytest.mark.gpu

mta = importlib.import_module("mega-trading_amd")


def _rope_tables(t, d, theta=10_000.0):
    pos = torch.arange(t, dtype=torch.float32)
    inv = 1.0 / (theta ** (torch.arange(0, d, 2, dtype=torch.float32) / d))
    f = torch.outer(pos, inv)
    return f.cos().cuda(), f.sin().cuda()


def _case(b=2, t=300, hq=8, hkv=2, d=64, seed=3):
    q, k, v, do = make_inputs(b, t, hq, hkv, d, seed=seed)
    q, k, v, do = (x.cuda() for x in (q, k, v, do))
    cos, sin = _rope_tables(t, d)
    return q, k, v, do, cos, sin


def _fwd_bwd(fn, q, k, v, do, cos, sin):
    q, k, v = (x.detach().requires_grad_(True) for x in (q, k, v))
    out = fn(q, k, v, cos, sin)
    dq, dk, dv = torch.autograd.grad(out, (q, k, v), do)
    return out.detach(), dq, dk, dv


@pytest.mark.parametrize("backend", ["aot_eager", "inductor"])
def test_torch_compile_fullgraph_matches_eager(backend):
    if backend == "inductor":
        pytest.importorskip("triton")
    q, k, v, do, cos, sin = _case()

    def f(q, k, v, cos, sin):
        return mta.rope_attention(q, k, v, cos, sin, repeats=4) * 1.0

    eager = _fwd_bwd(f, q, k, v, do, cos, sin)
    torch._dynamo.reset()
    compiled = torch.compile(f, backend=backend, fullgraph=True)
    got = _fwd_bwd(compiled, q, k, v, do, cos, sin)
    for name, a, b in zip(("O", "dQ", "dK", "dV"), got, eager):
        assert torch.equal(a, b), f"{name} differs under torch.compile({backend})"


def test_torch_compile_plain_op_fullgraph():
    q, k, v, do, _, _ = _case(t=129, hq=4, hkv=4)

    def f(q, k, v, cos, sin):
        return mta.attention(q, k, v, repeats=1)

    eager = _fwd_bwd(f, q, k, v, do, None, None)
    torch._dynamo.reset()
    got = _fwd_bwd(torch.compile(f, backend="aot_eager", fullgraph=True), q, k, v, do, None, None)
    for a, b in zip(got, eager):
        assert torch.equal(a, b)


def test_hip_graph_replays_match_eager():
    q0, k0, v0, do0, cos, sin = _case(b=2, t=512, hq=16, hkv=4, seed=7)
    eager = _fwd_bwd(lambda q, k, v, c, s: mta.rope_attention(q, k, v, c, s, repeats=4), q0, k0, v0, do0, cos, sin)

    # static inputs the graph reads
    q = q0.clone().requires_grad_(True)
    k = k0.clone().requires_grad_(True)
    v = v0.clone().requires_grad_(True)
    do = do0.clone()

    def step():
        out = mta.rope_attention(q, k, v, cos, sin, repeats=4)
        return (out,) + torch.autograd.grad(out, (q, k, v), do)

    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(2):
            step()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()

    # dead reference cycles holding GPU objects are freed before the capture and
    # the cyclic collector is paused during it: destroying a graph or stream
    # while a capture is under way is an error
    gc.collect()
    gc.disable()
    try:
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            static = step()
    finally:
        gc.enable()
    torch.cuda.synchronize()

    for replay in range(3):
        # eager work on the same tensors between replays
        _ = mta.rope_attention(q.detach(), k.detach(), v.detach(), cos, sin, repeats=4)
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        for name, a, b in zip(("O", "dQ", "dK", "dV"), static, eager):
            assert torch.equal(a, b), f"replay {replay}: {name} differs from eager"

    # new input values flow through the captured graph
    with torch.no_grad():
        q.mul_(0.5)
    graph.replay()
    torch.cuda.synchronize()
    ref = _fwd_bwd(lambda q_, k_, v_, c, s: mta.rope_attention(q_, k_, v_, c, s, repeats=4), q.detach(), k0, v0, do0,
                   cos, sin)
    for a, b in zip(static, ref):
        assert torch.equal(a, b)
