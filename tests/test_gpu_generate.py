"""GPU tests of decode attention and KV-cached generation.

The decode kernel against the oracle (the last row of the causal forward over
the cached positions; bf16 O max-abs <= 2e-2 as for the forward), and the
cached ``generate`` of the HIP routes against the reference's full-recompute
loop on the same weights: teacher-forced logits within 2e-2 relative (both
run the attention in bf16 through different kernels), greedy tokens equal
wherever the recompute's top-2 logit gap is clear of that tolerance.
"""

from __future__ import annotations

import importlib

import numpy as np
import pytest
import torch

from oracle import attention_oracle as orc

pytestmark = pytest.mark.gpu

mta = importlib.import_module("mega-trading_amd")
model_mod = importlib.import_module("mega-trading_amd.model")

DECODE_CASES = [
    # (B, Hq, Hkv, L, D, dtype, capacity)
    (2, 8, 2, 1, 64, torch.bfloat16, 16),
    (3, 16, 4, 255, 64, torch.bfloat16, 300),
    (1, 4, 4, 256, 128, torch.float16, 256),
    (2, 8, 1, 1000, 64, torch.bfloat16, 1024),
    (1, 32, 8, 4096, 128, torch.bfloat16, 4096),
    (4, 6, 3, 517, 32, torch.float16, 600),
    (32, 8, 2, 1024, 64, torch.bfloat16, 1024),  # BASELINE config 5 layer at the end of the window
]


@pytest.mark.parametrize("b,hq,hkv,length,d,dt,cap", DECODE_CASES)
def test_decode_attention_vs_oracle(b, hq, hkv, length, d, dt, cap):
    g = torch.Generator().manual_seed(length + d)
    q = (torch.randn(b, hq, 1, d, generator=g) * 0.5).to(dt)
    kc = (torch.randn(b, hkv, cap, d, generator=g) * 0.5).to(dt)
    vc = torch.randn(b, hkv, cap, d, generator=g).to(dt)
    kc[:, :, length:] = float("nan")  # past the length: never read
    out = mta.decode_attention(q.cuda(), kc.cuda(), vc.cuda(), length, repeats=hq // hkv)
    torch.cuda.synchronize()
    ref = orc.decode_attention(q[:, :, 0].double().numpy(), kc.double().numpy(), vc.double().numpy(), length, hq // hkv)
    err = np.abs(out[:, :, 0].double().cpu().numpy() - ref).max()
    assert out.shape == (b, hq, 1, d) and out.dtype == dt
    assert err <= 2e-2, err


def test_decode_attention_strided_views_and_errors():
    # the caches are views of a [B, T, H, D] buffer (the projections' layout)
    g = torch.Generator().manual_seed(5)
    base = (torch.randn(2, 64, 2, 64, generator=g) * 0.5).to(torch.bfloat16).cuda()
    kc, vc = base.transpose(1, 2), (base * 0.5).transpose(1, 2)
    q = (torch.randn(2, 8, 1, 64, generator=g) * 0.5).to(torch.bfloat16).cuda()
    out = mta.decode_attention(q, kc, vc, 40, repeats=4)
    ref = orc.decode_attention(q[:, :, 0].double().cpu().numpy(), kc.double().cpu().numpy(),
                               vc.double().cpu().numpy(), 40, 4)
    assert np.abs(out[:, :, 0].double().cpu().numpy() - ref).max() <= 2e-2
    with pytest.raises(ValueError, match="length"):
        mta.decode_attention(q, kc, vc, 65, repeats=4)
    with pytest.raises(ValueError, match="repeats"):
        mta.decode_attention(torch.zeros(1, 32, 1, 64, device="cuda", dtype=torch.bfloat16),
                             torch.zeros(1, 2, 8, 64, device="cuda", dtype=torch.bfloat16),
                             torch.zeros(1, 2, 8, 64, device="cuda", dtype=torch.bfloat16), 4, repeats=16)
    with pytest.raises(RuntimeError, match="float16 and bfloat16"):
        mta.decode_attention(q.float(), kc, vc, 4, repeats=4)


def _model(backend, block_size=64, seed=0, **kw):
    torch.manual_seed(seed)
    cfg = dict(vocab_size=128, block_size=block_size, hidden_dim=512, layers=2, attention_heads=8, kv_heads=2,
               dropout=0.0, rope_theta=10_000.0, attention_backend=backend)
    cfg.update(kw)
    return model_mod.TradingModel(**cfg).cuda().eval()


def _rel(a, b):
    return ((a - b).norm() / b.norm()).item()


@pytest.mark.parametrize("backend", ["hip", "triton"])
def test_cached_logits_match_full_recompute(backend):
    m = _model(backend)
    g = torch.Generator().manual_seed(11)
    tokens = torch.randint(0, 128, (3, 40), generator=g).cuda()
    with torch.no_grad():
        logits, cache = m._prefill(tokens[:, :10])
        assert _rel(logits, m(tokens[:, :10])[:, -1, :]) < 2e-2
        for pos in range(10, 40):  # teacher forcing: feed the true next token
            step = m._decode(tokens[:, pos:pos + 1], cache, pos)
            full = m(tokens[:, :pos + 1])[:, -1, :]
            assert _rel(step, full) < 2e-2, pos


def test_generate_greedy_matches_recompute_and_crosses_the_window():
    m = _model("hip", block_size=32)
    for p in m.output.parameters():  # sharper logits: fewer near-ties between top-2 tokens
        p.data.mul_(25.0)
    g = torch.Generator().manual_seed(12)
    prompt = torch.randint(0, 128, (4, 12), generator=g).cuda()
    out = m.generate(prompt, max_new_tokens=30, top_k=1)  # 12 + 30 > 32: the window slides
    assert out.shape == (4, 42) and torch.equal(out[:, :12], prompt)
    with torch.no_grad():
        for t in range(12, 42):
            full = m(out[:, max(0, t - 32):t])[:, -1, :]
            top2 = full.topk(2, dim=-1).values
            clear = (top2[:, 0] - top2[:, 1]) > 5e-2 * top2[:, 0].abs().clamp_min(1.0)
            assert torch.equal(out[clear, t], full.argmax(-1)[clear]), t


def test_generate_sampling_runs_at_c5_shape():
    wl = importlib.import_module("mega-trading_amd.workload")
    m = wl.build_model("hip", seed=0, device="cuda").eval()
    ids, _ = wl.zipf_batch(8, 256, wl.C5_MODEL["vocab_size"])
    torch.manual_seed(0)
    out = m.generate(ids.cuda(), max_new_tokens=16, top_k=16)
    assert out.shape == (8, 272) and int(out.max()) < wl.C5_MODEL["vocab_size"] and int(out.min()) >= 0
