"""CPU tests of the restated decoder: attention routing (as the reference's
tests/test_training.py:421-461 checks it), RoPE tables, init, the C5 shape and
its synthetic data."""

from __future__ import annotations

import importlib
import math
from unittest.mock import patch

import numpy as np
import pytest
import torch
import torch.nn.functional as F

model_mod = importlib.import_module("mega-trading_amd.model")
workload = importlib.import_module("mega-trading_amd.workload")
RotaryEmbedding = model_mod.RotaryEmbedding
rotate = model_mod.rotate


def _attn(backend="auto", **kw):
    args = dict(hidden_dim=16, block_size=8, attention_heads=4, kv_heads=2, dropout=0.0, rope_theta=10_000.0)
    args.update(kw)
    return model_mod.LlamaAttention(attention_backend=backend, **args)


def test_backend_values_validated():
    with pytest.raises(ValueError, match="attention_backend must be one of"):
        _attn("cuda")
    for b in ("auto", "flash", "efficient", "math", "triton", "hip"):
        _attn(b)


def test_sdpa_route_uses_native_gqa():
    attention = _attn("auto")
    hidden = torch.randn(1, 8, 16)
    with patch("mega-trading_amd.model.F.scaled_dot_product_attention", return_value=torch.zeros(1, 4, 8, 4)) as sdpa:
        attention(hidden)
    _q, key, value = sdpa.call_args.args[:3]
    assert key.shape[1] == 2 and value.shape[1] == 2
    assert sdpa.call_args.kwargs["enable_gqa"] is True
    assert sdpa.call_args.kwargs["is_causal"] is True


@pytest.mark.parametrize("backend", ["triton", "hip"])
def test_hip_backend_calls_local_kernel(backend):
    attention = _attn(backend, fuse_rope=False)
    hidden = torch.randn(1, 8, 16)
    # the RoPE kernel stand-in rotates in torch, so the attention sees rotated q / k
    with patch("mega-trading_amd.model._hip_apply_rope",
               side_effect=lambda q, k, c, s: (rotate(q, c, s), rotate(k, c, s))) as rope_op, \
            patch("mega-trading_amd.model._kernel_operands", return_value=True), \
            patch("mega-trading_amd.model._hip_attention", return_value=torch.zeros(1, 4, 8, 4)) as op:
        out = attention(hidden)
    rope_op.assert_called_once()
    query, key, value = op.call_args.args[:3]
    assert out.shape == hidden.shape
    assert query.shape == (1, 4, 8, 4) and key.shape[1] == 2 and value.shape[1] == 2
    assert op.call_args.kwargs["repeats"] == 2
    # RoPE was applied before the call, as model.py:223 does
    raw_q = attention.q_proj(hidden).view(1, 8, 4, 4).transpose(1, 2)
    cos, sin = attention.rope.cos[:, :, :8], attention.rope.sin[:, :, :8]
    assert torch.allclose(query, rotate(raw_q, cos, sin))


@pytest.mark.parametrize("backend,kernel", [("triton", True), ("hip", True), ("auto", False), ("math", False)])
def test_rotary_embedding_routes_by_operator_backend(backend, kernel):
    # as the reference test patches _triton_apply_rope (tests/test_training.py:470-475)
    rope = RotaryEmbedding(head_dim=4, max_sequence_length=8, theta=10_000.0, operator_backend=backend)
    query, key = torch.randn(1, 4, 8, 4), torch.randn(1, 2, 8, 4)
    with patch("mega-trading_amd.model._hip_apply_rope", return_value=(query, key)) as rope_kernel, \
            patch("mega-trading_amd.model._kernel_operands", return_value=True):
        out_q, _out_k = rope(query, key)
    assert rope_kernel.call_count == (1 if kernel else 0)
    assert out_q.shape == query.shape
    if kernel:
        _q, _k, cos, sin = rope_kernel.call_args.args
        assert cos.shape == (1, 1, 8, 2) and cos.dtype == query.dtype  # cast as model.py:290-291


def test_fused_rope_route_passes_fp32_tables_and_raw_qk():
    attention = _attn("hip")
    hidden = torch.randn(1, 8, 16)
    with patch("mega-trading_amd.model._hip_rope_attention", return_value=torch.zeros(1, 4, 8, 4)) as op:
        attention(hidden)
    query, key, value, cos, sin = op.call_args.args[:5]
    assert op.call_args.kwargs["repeats"] == 2
    assert cos is attention.rope.cos and sin is attention.rope.sin and cos.dtype == torch.float32
    raw_q = attention.q_proj(hidden).view(1, 8, 4, 4).transpose(1, 2)
    torch.testing.assert_close(query, raw_q)  # un-rotated: the kernel rotates on load
    # strided views of the one packed q|k|v product (rows of 16 + 8 + 8) are passed as is
    assert query.stride() == (256, 4, 32, 1) and key.stride() == (256, 4, 32, 1)
    assert key.data_ptr() == query.data_ptr() + 16 * 4 and value.data_ptr() == key.data_ptr() + 8 * 4


def test_hip_route_passes_the_packed_qkv_product_in_16_bits():
    # 16-bit activations (the autocast case) and a kernel head size: one q|k|v
    # GEMM whose packed output goes to the packed fused-RoPE op; fp32 keeps the
    # head views, and so does a head size the kernels pad (head_dim 4 here)
    attention = _attn("hip", hidden_dim=128).to(torch.bfloat16)  # 4 heads of 32
    hidden = torch.randn(1, 8, 128).to(torch.bfloat16)
    with patch("mega-trading_amd.model._hip_rope_attention_packed",
               return_value=torch.zeros(1, 8, 128, dtype=torch.bfloat16)) as op:
        out = attention(hidden)
    qkv, cos, sin = op.call_args.args[:3]
    assert out.shape == hidden.shape and qkv.shape == (1, 8, 128 + 64 + 64)
    assert op.call_args.kwargs == {"heads": 4, "kv_heads": 2}
    assert cos is attention.rope.cos and sin is attention.rope.sin
    want = torch.cat([attention.q_proj(hidden), attention.k_proj(hidden), attention.v_proj(hidden)], dim=-1)
    torch.testing.assert_close(qkv, want)
    small = _attn("hip").to(torch.bfloat16)  # head_dim 4
    with patch("mega-trading_amd.model._hip_rope_attention",
               return_value=torch.zeros(1, 4, 8, 4, dtype=torch.bfloat16)) as op2:
        small(torch.randn(1, 8, 16).to(torch.bfloat16))
    assert op2.call_args.args[0].shape == (1, 4, 8, 4)


def test_dropout_in_training_falls_back_to_sdpa():
    attention = _attn("hip", dropout=0.1)
    attention.train()
    hidden = torch.randn(1, 8, 16)
    with patch("mega-trading_amd.model.F.scaled_dot_product_attention", return_value=torch.zeros(1, 4, 8, 4)) as sdpa, \
            patch("mega-trading_amd.model._hip_rope_attention") as op, \
            patch("mega-trading_amd.model._kernel_operands", return_value=True), \
            patch("mega-trading_amd.model._hip_apply_rope", side_effect=lambda q, k, c, s: (q, k)) as rope_op:
        attention(hidden)
    assert sdpa.call_args.kwargs["dropout_p"] == 0.1
    op.assert_not_called()
    rope_op.assert_called_once()  # the RoPE still takes the backend (model.py:213, 223)
    attention.eval()
    with patch("mega-trading_amd.model._hip_rope_attention", return_value=torch.zeros(1, 4, 8, 4)) as op:
        attention(hidden)
    op.assert_called_once()


def test_rope_tables_and_rotation_closed_form():
    rope = model_mod.RotaryEmbedding(8, 16, theta=10_000.0)
    assert rope.cos.shape == (1, 1, 16, 4)
    pos, i = 5, 3
    ang = pos * 10_000.0 ** (-2 * i / 8)
    assert math.isclose(rope.cos[0, 0, pos, i].item(), math.cos(ang), rel_tol=1e-5, abs_tol=1e-6)
    x = torch.randn(1, 2, 16, 8)
    rq, rk = rope(x, x)
    assert torch.allclose(rq[..., 0, :], x[..., 0, :])  # position 0 is the identity
    assert torch.allclose(rq.norm(dim=-1), x.norm(dim=-1), atol=1e-5)  # rotations keep the norm
    c, s = rope.cos[0, 0, pos, i], rope.sin[0, 0, pos, i]
    x0, x1 = x[0, 0, pos, 2 * i], x[0, 0, pos, 2 * i + 1]
    assert torch.allclose(rq[0, 0, pos, 2 * i], x0 * c - x1 * s, atol=1e-6)
    assert torch.allclose(rq[0, 0, pos, 2 * i + 1], x0 * s + x1 * c, atol=1e-6)
    with pytest.raises(ValueError, match="exceeds RoPE cache length"):
        rope(torch.randn(1, 1, 17, 8), torch.randn(1, 1, 17, 8))


def test_model_init_tying_and_c5_parameter_count():
    m = model_mod.TradingModel(attention_backend="auto", **workload.C5_MODEL)
    assert m.output.weight is m.token_embedding.weight
    emb = m.token_embedding.weight.numel()
    total = sum(p.numel() for p in m.parameters())
    assert emb == 16384 * 512
    # per layer: q, o 512x512; k, v 512x128; SwiGLU 3 x 512x1408; two norms of 512
    per_layer = 2 * 512 * 512 + 2 * 512 * 128 + 3 * 512 * 1408 + 2 * 512
    assert total == emb + 8 * per_layer + 512
    w = m.blocks[0].attention.q_proj.weight
    assert abs(w.std().item() - 0.02) < 1e-3
    assert model_mod._llama_intermediate_dim(512) == 1376


def test_model_forward_shapes_and_errors():
    m = model_mod.TradingModel(vocab_size=32, block_size=8, hidden_dim=16, layers=2, attention_heads=4, kv_heads=2,
                               dropout=0.0, rope_theta=10_000.0)
    ids = torch.randint(0, 32, (2, 8))
    assert m(ids).shape == (2, 8, 32)
    loss, logits = m.forward_with_loss(ids, ids, return_logits=True)
    assert logits.shape == (2, 8, 32) and loss.ndim == 0
    assert abs(loss.item() - math.log(32)) < 0.5
    with pytest.raises(ValueError, match="block_size"):
        m(torch.randint(0, 32, (1, 9)))
    with pytest.raises(ValueError, match="batch, time"):
        m(torch.randint(0, 32, (8,)))


def test_triton_operators_compute_with_torch_where_the_reference_does():
    # triton_ops.py:51-52, 59-60, 87-88: the reference's triton_* operators take
    # torch's path for tensors their kernels do not take (here: CPU tensors, as in
    # a "triton" model training with dropout > 0 on the CPU), so the same model
    # runs here and equals the "auto" model with the same weights
    kw = dict(vocab_size=32, block_size=8, hidden_dim=16, layers=1, attention_heads=4, kv_heads=2, dropout=0.1,
              rope_theta=10_000.0)
    tri = model_mod.TradingModel(attention_backend="triton", **kw)
    ref = model_mod.TradingModel(attention_backend="auto", **kw)
    ref.load_state_dict(tri.state_dict())
    ids = torch.randint(0, 32, (2, 8))
    for m in (tri, ref):
        m.train()
    torch.manual_seed(3)
    loss_t, _ = tri.forward_with_loss(ids, ids, return_logits=False)
    torch.manual_seed(3)
    loss_r, _ = ref.forward_with_loss(ids, ids, return_logits=False)
    torch.testing.assert_close(loss_t, loss_r)
    rope = RotaryEmbedding(head_dim=4, max_sequence_length=8, theta=10_000.0, operator_backend="triton")
    q, k = torch.randn(1, 4, 8, 4, dtype=torch.float64), torch.randn(1, 2, 8, 4, dtype=torch.float64)
    cos, sin = rope.cos.to(torch.float64), rope.sin.to(torch.float64)
    rq, rk = rope(q, k)
    torch.testing.assert_close(rq, rotate(q, cos, sin))
    torch.testing.assert_close(rk, rotate(k, cos, sin))
    # every label ignored: a zero loss (the reference's torch form of the fused loss), not NaN
    loss0, _ = tri.forward_with_loss(ids, torch.full_like(ids, -100), return_logits=False)
    assert float(loss0.detach()) == 0.0


def test_hip_route_on_cpu_tensors_raises():
    m = model_mod.TradingModel(vocab_size=32, block_size=8, hidden_dim=256, layers=1, attention_heads=4, kv_heads=2,
                               dropout=0.0, rope_theta=10_000.0, attention_backend="hip")
    with pytest.raises(RuntimeError, match="ROCm GPU"):
        m(torch.randint(0, 32, (1, 8)))


def test_zipf_batch_is_seeded_shifted_and_heavy_headed():
    x, y = workload.zipf_batch(4, 256, 16384)
    x2, y2 = workload.zipf_batch(4, 256, 16384)
    assert torch.equal(x, x2) and torch.equal(y, y2)
    assert x.shape == y.shape == (4, 256) and x.dtype == torch.int64
    assert torch.equal(x[:, 1:], y[:, :-1])
    assert int(x.min()) >= 0 and int(x.max()) < 16384
    counts = np.bincount(x.flatten().numpy(), minlength=16384)
    p1 = 1.0 / sum(k ** -1.1 for k in range(1, 16385))
    assert abs(counts[0] / x.numel() - p1) < 0.03  # rank 1 carries ~10% of the mass
    assert counts[0] > counts[1] > counts[10]


@pytest.mark.parametrize("backend,gate,norm_hip", [("auto", None, False), ("triton", "pair", False),
                                                   ("hip", "packed", True)])
def test_operator_routing_follows_the_reference(backend, gate, norm_hip):
    # SwiGLU takes the attention backend (reference model.py:179-183); the reference's
    # norms have none (model.py:166,176), so only this package's "hip" value moves them
    m = model_mod.TradingModel(vocab_size=32, block_size=8, hidden_dim=16, layers=1, attention_heads=4, kv_heads=2,
                               dropout=0.0, rope_theta=10_000.0, attention_backend=backend)
    assert m.blocks[0].feed_forward.operator_backend == backend
    assert m.blocks[0].attention_norm.operator_backend == ("hip" if norm_hip else "auto")
    assert m.norm.operator_backend == m.blocks[0].ffn_norm.operator_backend
    hidden = torch.randn(1, 8, 16)
    ffn = m.blocks[0].feed_forward
    ref = ffn.w2(F.silu(ffn.w1(hidden)) * ffn.w3(hidden))
    with patch("mega-trading_amd.model._hip_swiglu_gate", side_effect=lambda g, u: F.silu(g) * u) as pair, \
         patch("mega-trading_amd.model._kernel_operands", return_value=True), \
         patch("mega-trading_amd.model._hip_swiglu_gate_packed",
               side_effect=lambda gu: F.silu(gu[..., :gu.shape[-1] // 2]) * gu[..., gu.shape[-1] // 2:]) as packed:
        out = ffn(hidden)
    assert pair.called == (gate == "pair") and packed.called == (gate == "packed")
    torch.testing.assert_close(out, ref, rtol=1e-5, atol=1e-6)
    norm = m.blocks[0].attention_norm
    with patch("mega-trading_amd.model._hip_rms_norm", side_effect=lambda x, w, eps: x) as rms:
        norm(hidden)
    assert rms.called == norm_hip
    if norm_hip:
        assert rms.call_args.kwargs["eps"] == 1e-5 and rms.call_args.args[1] is norm.weight



@pytest.mark.parametrize("backend,fused", [("auto", False), ("triton", True), ("hip", True)])
def test_loss_head_routing(backend, fused):
    # model.py:113-123: the fused linear cross-entropy for the Triton route when logits are not requested
    m = model_mod.TradingModel(vocab_size=32, block_size=8, hidden_dim=16, layers=1, attention_heads=4, kv_heads=2,
                               dropout=0.0, rope_theta=10_000.0, attention_backend="auto")
    m.operator_backend = backend  # keep the rest of the network on torch ops (CPU)
    ids = torch.randint(0, 32, (2, 8))
    with patch("mega-trading_amd.model._hip_fused_linear_cross_entropy", return_value=torch.tensor(1.5)) as ce, \
            patch("mega-trading_amd.model._kernel_operands", return_value=True):
        loss, logits = m.forward_with_loss(ids, ids, return_logits=False)
    assert ce.called == fused and logits is None
    if fused:
        hidden, weight, labels = ce.call_args.args
        assert hidden.shape == (16, 16) and weight is m.output.weight and labels.shape == (16,)
        assert ce.call_args.kwargs["ignore_index"] == -100 and loss.item() == 1.5
    with patch("mega-trading_amd.model._hip_fused_linear_cross_entropy") as ce:
        loss, logits = m.forward_with_loss(ids, ids, return_logits=True)  # logits requested: torch head
    ce.assert_not_called()
    assert logits.shape == (2, 8, 32)


def test_generate_reference_loop_on_cpu():
    # the "auto" route keeps the reference's recompute loop (model.py:134-147), window included
    m = model_mod.TradingModel(vocab_size=32, block_size=8, hidden_dim=16, layers=1, attention_heads=4, kv_heads=2,
                               dropout=0.1, rope_theta=10_000.0)
    ids = torch.randint(0, 32, (3, 5))
    torch.manual_seed(0)
    a = m.generate(ids, max_new_tokens=6, top_k=4)  # crosses block_size: the window slides
    torch.manual_seed(0)
    b = m._generate_recompute(ids, 6, 4)
    assert a.shape == (3, 11) and torch.equal(a[:, :5], ids) and torch.equal(a, b)
    assert int(a.max()) < 32 and not m.training
    # top_k = 1 is greedy: the first new token is the argmax of the prompt's last logits
    g = m.generate(ids, max_new_tokens=1, top_k=1)
    assert torch.equal(g[:, -1], m(ids)[:, -1, :].argmax(-1))


def test_hip_route_projections_match_the_linear_modules():
    # "hip": q/k/v from one GEMM against the stacked weights, o through the same
    # function; values and every weight's gradient equal the nn.Linear products
    m = model_mod.TradingModel(vocab_size=32, block_size=16, hidden_dim=32, layers=1, attention_heads=4, kv_heads=2,
                               dropout=0.0, rope_theta=10_000.0, attention_backend="hip").double()
    attn = m.blocks[0].attention
    hidden = torch.randn(2, 16, 32, dtype=torch.float64, requires_grad=True)
    q, k, v = attn._heads(hidden)
    ref = [p(hidden) for p in (attn.q_proj, attn.k_proj, attn.v_proj)]
    for got, want, h in zip((q, k, v), ref, (4, 2, 2)):
        assert got.shape == (2, h, 16, 8)
        torch.testing.assert_close(got.transpose(1, 2).reshape(2, 16, -1), want)
    o = attn._out(hidden)
    torch.testing.assert_close(o, attn.o_proj(hidden))
    gs = [torch.randn_like(t) for t in (q, k, v, o)]
    got = torch.autograd.grad((q, k, v, o), [hidden, attn.q_proj.weight, attn.k_proj.weight, attn.v_proj.weight,
                                             attn.o_proj.weight], gs)
    want = torch.autograd.grad(ref + [attn.o_proj(hidden)],
                               [hidden, attn.q_proj.weight, attn.k_proj.weight, attn.v_proj.weight,
                                attn.o_proj.weight],
                               [g.transpose(1, 2).reshape(2, 16, -1) for g in gs[:3]] + [gs[3]])
    for a, b in zip(got, want):
        torch.testing.assert_close(a, b)


def test_tuned_gemm_context_is_inert_without_a_gpu():
    gt = importlib.import_module("mega-trading_amd.gemm_tuning")
    if torch.cuda.is_available():
        pytest.skip("a GPU is present")
    with gt.tuned_gemms():
        x = torch.randn(4, 8) @ torch.randn(8, 3)
    assert x.shape == (4, 3) and gt._load() is False


def test_split_k_chunking_and_weight_gradient_on_cpu():
    pj = importlib.import_module("mega-trading_amd.projection")
    # the largest of 16, 8, 4, 2 that divides the rows into chunks of >= 1024, else 1
    assert [pj.split_k_chunks(r) for r in (32768, 16384, 8192, 4096, 3072, 2048, 1024, 1000, 0)] == \
        [16, 16, 8, 4, 2, 2, 1, 1, 1]
    g = torch.Generator().manual_seed(7)
    x = torch.randn(3, 1024, 48, generator=g, dtype=torch.float64, requires_grad=True)   # 3072 rows: 2 chunks
    ws = [torch.randn(o, 48, generator=g, dtype=torch.float64, requires_grad=True) for o in (16, 8)]
    a, b = pj.project(x, ws)
    ga, gb = torch.randn_like(a), torch.randn_like(b)
    torch.autograd.backward((a, b), (ga, gb))
    x2 = x.detach().reshape(-1, 48)
    torch.testing.assert_close(ws[0].grad, ga.reshape(-1, 16).t() @ x2)
    torch.testing.assert_close(ws[1].grad, gb.reshape(-1, 8).t() @ x2)
    torch.testing.assert_close(x.grad, (ga @ ws[0].detach() + gb @ ws[1].detach()))
