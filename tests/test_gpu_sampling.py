"""GPU tests of the one-launch top-k draw (mt_topk_sample) that generation
uses after each decode step, against the library formulation of the same draw
(topk, mask, softmax, p / E, argmax) on the same logits and noise: every token
must match.  Ties at the k-th value, k = 1 and k = vocab, and vocabularies on
both sides of each register-tile size are covered."""

from __future__ import annotations

import importlib

import pytest
import torch

pytestmark = pytest.mark.gpu

ops = importlib.import_module("mega-trading_amd.ops")
model_mod = importlib.import_module("mega-trading_amd.model")


def _torch_draw(logits, noise, k):
    values, _ = torch.topk(logits, k)
    masked = logits.masked_fill(logits < values[:, -1:], float("-inf"))
    probs = torch.softmax(masked, dim=-1)
    return torch.argmax(probs / noise, dim=-1, keepdim=True)


@pytest.mark.parametrize("rows,vocab,k,scale", [
    (32, 16384, 16, 3.0),     # BASELINE config 5 generation: 32 rollouts, vocab 16384, top-k 16
    (5, 128, 16, 3.0),
    (3, 1, 1, 1.0),
    (4, 7, 3, 1.0),
    (6, 8192, 50, 0.5),
    (6, 8193, 50, 0.5),
    (2, 32768, 16, 4.0),
    (8, 1000, 1, 2.0),
    (8, 300, 300, 1.0),       # k = vocab: every logit kept
])
def test_topk_sample_matches_the_library_draw(rows, vocab, k, scale):
    g = torch.Generator(device="cuda").manual_seed(rows * 7 + vocab + k)
    for _ in range(4):
        logits = torch.randn(rows, vocab, device="cuda", generator=g) * scale
        noise = torch.empty_like(logits).exponential_(1, generator=g)
        got = ops.topk_sample(logits, noise, k)
        assert got.shape == (rows, 1) and got.dtype == torch.int64
        assert torch.equal(got, _torch_draw(logits, noise, k))


def test_topk_sample_keeps_every_tie_at_the_kth_value():
    # integer-valued logits: many ties at the k-th value, all of which stay candidates
    g = torch.Generator(device="cuda").manual_seed(3)
    for _ in range(8):
        logits = torch.randint(-3, 4, (16, 512), device="cuda", generator=g).float()
        noise = torch.empty_like(logits).exponential_(1, generator=g)
        for k in (1, 5, 16, 200):
            assert torch.equal(ops.topk_sample(logits, noise, k), _torch_draw(logits, noise, k)), k


def test_recorded_sampling_uses_one_launch_and_the_same_noise():
    # the model's draw after a decode step: same tokens as torch.multinomial for the same seed
    g = torch.Generator().manual_seed(8)
    logits = (torch.randn(32, 16384, generator=g) * 3).cuda()
    for k in (16, 1):
        torch.manual_seed(21)
        ref = model_mod._sample_next(logits, k)
        torch.manual_seed(21)
        got = model_mod._sample_recorded(logits, k)
        assert torch.equal(ref, got), k


def test_topk_sample_rejects_bad_arguments():
    x = torch.zeros(2, 64, device="cuda")
    with pytest.raises(ValueError):
        ops.topk_sample(x, x, 65)
    with pytest.raises(ValueError):
        ops.topk_sample(x, x[:, :32], 4)
    with pytest.raises(RuntimeError):
        ops.topk_sample(x.double(), x.double(), 4)
