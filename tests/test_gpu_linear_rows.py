"""GPU tests of the few-row grouped products (mt_linear_rows) that the decode
step's projections use: against float64 products of the same fp32 operands,
through the C ABI's torch op and through projection.project_packed, which
routes to it only without autograd (the training path keeps its own GEMM)."""

from __future__ import annotations

import importlib

import pytest
import torch

pytestmark = pytest.mark.gpu

mta = importlib.import_module("mega-trading_amd")
proj = importlib.import_module("mega-trading_amd.projection")

CASES = [
    # (rows, K, out_features of each group)
    (1, 128, [16]),
    (5, 512, [512, 128, 128]),          # a layer's q | k | v at 5 rollouts
    (32, 512, [1408, 1408]),            # BASELINE config 5 w1 | w3 at 32 rollouts
    (32, 1408, [512]),                  # ... and w2
    (16, 256, [33, 100, 7, 2]),         # four groups, widths not multiples of 16
    (17, 384, [48]),                    # two 16-row tiles
    (40, 128, [20, 300]),               # four 16-row tiles
    (64, 1024, [64]),
]


def _ref(x, ws):
    return torch.cat([x.double() @ w.double().t() for w in ws], dim=-1)


@pytest.mark.parametrize("rows,k,outs", CASES)
def test_linear_rows_against_float64(rows, k, outs):
    g = torch.Generator().manual_seed(rows * 1000 + k)
    x = torch.randn(rows, k, generator=g).cuda()
    ws = [(torch.randn(n, k, generator=g) / k ** 0.5).cuda() for n in outs]
    y = proj.linear_rows(x, ws)
    torch.cuda.synchronize()
    ref = _ref(x, ws)
    assert y.shape == (rows, sum(outs)) and y.dtype == torch.float32
    err = (y.double() - ref).abs().max().item()
    assert err <= 1e-5 * ref.abs().max().item() + 1e-6, err


@pytest.mark.parametrize("dt", [torch.bfloat16, torch.float16])
def test_linear_rows_widens_16bit_x_exactly(dt):
    g = torch.Generator().manual_seed(17)
    x = torch.randn(32, 512, generator=g).to(dt).cuda()
    ws = [(torch.randn(n, 512, generator=g) / 22.6).cuda() for n in (512, 64)]
    y = proj.linear_rows(x, ws)
    assert (y.double() - _ref(x.float(), ws)).abs().max().item() <= 1e-5
    with torch.no_grad():  # the promotion path of project_packed: 16-bit x, fp32 weights
        z = proj.project_packed(x.view(32, 1, 512), ws)
    assert torch.equal(z.view(32, -1), y)


def test_linear_rows_reads_strided_rows_in_place():
    # x rows with a larger stride, weights that are row blocks of a wider matrix
    g = torch.Generator().manual_seed(7)
    base_x = torch.randn(24, 640, generator=g).cuda()
    x = base_x[:, :512]
    wide = torch.randn(300, 768, generator=g).cuda()
    ws = [wide[:200, :512], wide[200:, 128:640]]
    y = proj.linear_rows(x, ws)
    assert (y.double() - _ref(x, ws)).abs().max().item() <= 1e-4


def test_project_packed_routes_few_rows_without_autograd():
    g = torch.Generator().manual_seed(11)
    x = torch.randn(32, 1, 512, generator=g).cuda()
    ws = [torch.nn.Parameter((torch.randn(n, 512, generator=g) / 22.6).cuda()) for n in (512, 128, 128)]
    with torch.no_grad():
        y = proj.project_packed(x, ws)
    ref = _ref(x.view(32, 512), ws).view(32, 1, 768)
    assert (y.double() - ref).abs().max().item() <= 1e-4
    # with autograd the library path runs, and gradients flow
    y2 = proj.project_packed(x, ws)
    y2.sum().backward()
    assert (y2.detach().double() - ref).abs().max().item() <= 1e-3
    assert all(w.grad is not None and w.grad.shape == w.shape for w in ws)


def test_linear_rows_in_a_recorded_graph_matches_eager():
    g = torch.Generator().manual_seed(13)
    x = torch.randn(32, 512, generator=g).cuda()
    ws = [torch.randn(n, 512, generator=g).cuda() for n in (1408, 1408)]
    eager = proj.linear_rows(x, ws)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        proj.linear_rows(x, ws)
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        static = proj.linear_rows(x, ws)
    for _ in range(3):
        proj.linear_rows(x * 2, ws)  # eager work between replays
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(static, eager)
    with torch.no_grad():
        ws[0].mul_(0.5)  # the recorded launch reads the weights in place
    graph.replay()
    torch.cuda.synchronize()
    assert torch.equal(static, proj.linear_rows(x, ws))
