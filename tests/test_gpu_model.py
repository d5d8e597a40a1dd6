"""GPU tests of the decoder with the HIP attention swapped into every layer:
same weights and batch through the HIP route and the reference's SDPA route
(model.py:225-235), a few optimisation steps, and one step at the full
8-layer BASELINE config 5 shape."""

from __future__ import annotations

import importlib
import math

import pytest
import torch

pytestmark = pytest.mark.gpu

workload = importlib.import_module("mega-trading_amd.workload")

SMALL = dict(vocab_size=512, block_size=512, hidden_dim=256, layers=2, attention_heads=4, kv_heads=2,
             intermediate_dim=704, dropout=0.0, rope_theta=10_000.0)

# HIP vs SDPA route, both under bf16 autocast: only the attention differs
TOL_LOSS_REL = 1e-2
TOL_GRAD_REL = 3e-2


def _loss_and_grads(backend, ids, labels, fuse_rope=True):
    m = workload.build_model(backend, seed=0, device="cuda", fuse_rope=fuse_rope, **SMALL)
    with torch.autocast(device_type="cuda", dtype=torch.bfloat16):
        loss, _ = m.forward_with_loss(ids, labels, return_logits=False)
    loss.backward()
    grads = {n: p.grad.detach().float().clone() for n, p in m.named_parameters()}
    return loss.detach().float(), grads


def _rel(a, b):
    return ((a - b).norm() / b.norm().clamp_min(1e-12)).item()


@pytest.mark.parametrize("backend,fuse", [("hip", True), ("triton", True), ("hip", False), ("attention_only", True)])
def test_hip_route_matches_sdpa_route(backend, fuse):
    ids, labels = workload.zipf_batch(2, 384, SMALL["vocab_size"], seed=1)
    ids, labels = ids.cuda(), labels.cuda()
    loss_ref, g_ref = _loss_and_grads("auto", ids, labels)
    loss, g = _loss_and_grads(backend, ids, labels, fuse_rope=fuse)
    print(f"loss hip={loss.item():.5f} sdpa={loss_ref.item():.5f}")
    assert abs(loss.item() - loss_ref.item()) <= TOL_LOSS_REL * abs(loss_ref.item())
    worst = max(((_rel(g[n], g_ref[n]), n) for n in g_ref))
    print(f"worst grad rel err {worst[0]:.3e} ({worst[1]})")
    assert worst[0] <= TOL_GRAD_REL


def test_train_steps_reduce_loss():
    ids, labels = workload.zipf_batch(4, 256, SMALL["vocab_size"], seed=2)
    m = workload.build_model("hip", seed=0, device="cuda", **SMALL)
    step = workload.TrainStep(m, ids, labels, lr=1e-3)
    losses = [float(step()) for _ in range(8)]
    print("losses", [round(x, 4) for x in losses])
    assert all(math.isfinite(x) for x in losses)
    assert losses[-1] < losses[0] - 0.5


def test_c5_full_shape_step_runs_through_hip_kernels():
    ids, labels = workload.zipf_batch(workload.C5_BATCH, workload.C5_SEQ, workload.C5_MODEL["vocab_size"])
    m = workload.build_model("hip", seed=0, device="cuda")
    step = workload.TrainStep(m, ids, labels)
    loss = float(step())
    # tied N(0, 0.02) embeddings start near the uniform-prediction loss ln(16384) = 9.70
    assert abs(loss - math.log(16384)) < 0.5, loss
    loss2 = float(step())
    assert math.isfinite(loss2) and loss2 < loss


@pytest.mark.parametrize("autocast", [False, True])
def test_fused_residual_chain_equals_the_block_loop(autocast):
    # the "hip" model fuses each residual add into the next norm; the values
    # equal model.py:184-187's block loop bit for bit (same fp32 adds, same
    # norm kernel, one rounding to the autocast dtype), the gradients to rounding
    ids, _ = workload.zipf_batch(2, 256, SMALL["vocab_size"], seed=3)
    ids = ids.cuda()
    m = workload.build_model("hip", seed=0, device="cuda", **SMALL)
    params = [p for p in m.parameters()]
    with torch.autocast(device_type="cuda", dtype=torch.bfloat16, enabled=autocast):
        fused = m._hidden(ids)
        h = m.token_embedding(ids)
        for block in m.blocks:
            h = block(h)
        ref = m.norm(h)
    assert fused.dtype == (torch.bfloat16 if autocast else torch.float32)
    assert torch.equal(fused, ref.to(fused.dtype))
    g = torch.randn(fused.shape, generator=torch.Generator().manual_seed(4)).cuda()
    ga = torch.autograd.grad((fused.float() * g).sum(), params, allow_unused=True)
    gb = torch.autograd.grad((ref.to(fused.dtype).float() * g).sum(), params, allow_unused=True)
    for a, b in zip(ga, gb):
        if a is None or b is None:
            assert a is None and b is None
            continue
        # the fused backward adds the residual gradient inside the norm kernel
        # (possibly contracted into an fma): last-ulp fp32 differences that can
        # flip bf16 roundings in the attention backward, which runs in bf16
        assert _rel(a.float(), b.float()) <= 1e-3


def test_workload_cli_runs_the_c5_step(capsys):
    # python -m mega-trading_amd.workload: the command the committed C5 profile was made with
    assert workload.main(["--route", "hip", "--steps", "1", "--warmup", "1"]) == 0
    out = capsys.readouterr().out
    assert "C5 train step, route hip:" in out and "tokens/s" in out


@pytest.mark.parametrize("backend,op", [("math", "aten::_scaled_dot_product_attention_math"),
                                        ("efficient", "aten::_scaled_dot_product_efficient_attention")])
def test_forced_sdpa_backend_dispatches_that_kernel(backend, op):
    """trainer.py:977-1001 restated: inside the context SDPA runs the forced kernel
    (seen in the dispatched aten op), or raises when that kernel cannot serve the
    call; outside it torch chooses freely again."""
    from torch.profiler import ProfilerActivity, profile

    q = torch.randn(2, 8, 256, 64, device="cuda", dtype=torch.bfloat16)
    k = torch.randn(2, 2, 256, 64, device="cuda", dtype=torch.bfloat16)
    try:
        with workload.attention_kernel_context(backend, "cuda"), profile(activities=[ProfilerActivity.CPU]) as prof:
            torch.nn.functional.scaled_dot_product_attention(q, k, k, is_causal=True, enable_gqa=True)
            torch.cuda.synchronize()
    except RuntimeError as exc:
        pytest.skip(f"{backend} SDPA kernel refuses a causal GQA bf16 call on this build: {exc}")
    names = {e.name for e in prof.events()}
    assert op in names, sorted(n for n in names if "scaled_dot" in n)


def test_attention_only_train_step_runs_with_the_trainer_loss():
    ids, labels = workload.zipf_batch(2, 256, SMALL["vocab_size"], seed=5)
    losses = {}
    for route in ("auto", "attention_only"):
        m = workload.build_model(route, seed=0, device="cuda", **SMALL)
        step = workload.TrainStep(m, ids, labels)
        assert step.loss_kind == "trainer"
        losses[route] = [float(step()) for _ in range(3)]
    print("losses", losses)
    for a, b in zip(losses["attention_only"], losses["auto"]):
        assert abs(a - b) <= TOL_LOSS_REL * abs(b)


def test_fp32_model_without_autocast_matches_the_sdpa_route():
    """A fp32 decoder without autocast (the reference trainer's precision "fp32":
    no mixed precision, trainer.py:940-945,1009-1010) sends fp32 q/k/v to the
    attention op, which computes in fp32: loss and gradients agree with the SDPA
    route (fp32) to fp32 rounding."""
    ids, labels = workload.zipf_batch(2, 300, SMALL["vocab_size"], seed=6)
    ids, labels = ids.cuda(), labels.cuda()
    out = {}
    for route in ("auto", "triton"):
        m = workload.build_model(route, seed=0, device="cuda", **SMALL)
        loss, _ = m.forward_with_loss(ids, labels, return_logits=True)
        loss.backward()
        out[route] = (loss.detach(), {n: p.grad.detach().clone() for n, p in m.named_parameters()})
    (l_ref, g_ref), (l_hip, g_hip) = out["auto"], out["triton"]
    print(f"fp32 loss hip={l_hip.item():.7f} sdpa={l_ref.item():.7f}")
    assert abs(l_hip.item() - l_ref.item()) <= 1e-5 * abs(l_ref.item())
    worst = max(_rel(g_hip[n], g_ref[n]) for n in g_ref)
    print(f"worst fp32 grad rel err {worst:.3e}")
    assert worst <= 1e-4


def test_demo_ablation_model_with_head_dim_8():
    """The reference's demo ablation sizes (configs/ablations/demo.yaml:24-31:
    hidden 16 with 2 heads, head_dim 8) on the "triton" route: the attention runs
    zero-padded to the 32-wide kernels, loss and gradients match the SDPA route,
    and generate (the reference's recompute loop at this head size) runs."""
    cfg = dict(vocab_size=64, block_size=128, hidden_dim=16, layers=1, attention_heads=2, kv_heads=2,
               intermediate_dim=48, dropout=0.0, rope_theta=10_000.0)
    ids, labels = workload.zipf_batch(4, 96, cfg["vocab_size"], seed=8)
    ids, labels = ids.cuda(), labels.cuda()
    out = {}
    for route in ("auto", "triton"):
        m = workload.build_model(route, seed=0, device="cuda", **cfg)
        with torch.autocast(device_type="cuda", dtype=torch.bfloat16):
            loss, _ = m.forward_with_loss(ids, labels, return_logits=True)
        loss.backward()
        out[route] = (loss.detach().float(), {n: p.grad.detach().float().clone() for n, p in m.named_parameters()})
    (l_ref, g_ref), (l_hip, g_hip) = out["auto"], out["triton"]
    assert abs(l_hip.item() - l_ref.item()) <= TOL_LOSS_REL * abs(l_ref.item())
    assert max(_rel(g_hip[n], g_ref[n]) for n in g_ref) <= TOL_GRAD_REL
    m = workload.build_model("triton", seed=0, device="cuda", **cfg)
    gen = m.generate(ids[:2, :20], max_new_tokens=8, top_k=4)
    assert gen.shape == (2, 28)
