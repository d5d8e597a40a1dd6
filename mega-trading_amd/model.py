"""Llama-style decoder restated around the HIP attention op.

The module tree, argument names and routing follow the reference model
(``src/mega_trading/model.py:20-131`` TradingModel, ``:150-187`` decoder block,
``:189-237`` LlamaAttention, ``:240-269`` SwiGLU / RMSNorm, ``:272-316`` RoPE,
``:319-330`` init), so the train step the reference measures in tokens/sec
(``trainer.py:333-346``) can run on MI355X with either attention path:

* ``attention_backend`` in {"auto", "flash", "efficient", "math"}: RoPE in
  torch (tables cast to the activation dtype, ``model.py:290-291``) then
  ``F.scaled_dot_product_attention(is_causal=True, enable_gqa=...)``
  (``model.py:228-235``) -- the reference's eager path;
* ``"triton"`` (the reference's value, kept so its configs work unchanged) or
  ``"hip"`` with ``dropout_p == 0`` (``model.py:225``): the gfx950 kernels.  By
  default RoPE is fused into them (``rope_attention`` with the fp32 tables);
  ``fuse_rope=False`` keeps the reference's two calls, ``self.rope`` (on
  the HIP RoPE kernel, ``ops.apply_rope``, as the reference's RotaryEmbedding
  takes the attention backend) then ``attention(query, key, value,
  repeats=...)`` (``model.py:213,223,226``).

The other operators follow the reference's routing too: the SwiGLU gate
takes the attention backend (``model.py:179-183, 252-253``), so "triton" /
"hip" use the HIP gate (``ops.swiglu_gate``); the reference builds its RMSNorm
modules without a backend (``model.py:166, 176``, torch ``F.rms_norm``), which
"triton" keeps, while "hip" -- this package's own value -- also runs them on
the HIP RMSNorm kernels (``ops.rms_norm``).  The loss head follows
``model.py:113-123``: "triton" / "hip" without requested logits use the fused
linear cross-entropy (``ops.fused_linear_cross_entropy``), everything else the
torch ``F.linear`` + ``F.cross_entropy``.
"""

from __future__ import annotations

import gc
import itertools
import math
import weakref

import torch
import torch.nn.functional as F
from torch import nn

from . import _native
from .attention import KERNEL_HEAD_DIMS, _rope_tables
from .attention import attention as _hip_attention
from .attention import decode_attention as _hip_decode_attention
from .attention import decode_rope_append as _hip_decode_rope_append
from .attention import rope_attention as _hip_rope_attention
from .attention import rope_attention_packed as _hip_rope_attention_packed
from .ops import fused_linear_cross_entropy as _hip_fused_linear_cross_entropy
from .ops import add_rms_norm as _hip_add_rms_norm
from .ops import apply_rope as _hip_apply_rope
from .ops import add_rms_norm_mixed as _hip_add_rms_norm_mixed
from .ops import rms_norm as _hip_rms_norm
from .ops import rms_norm_mixed as _hip_rms_norm_mixed
from .ops import swiglu_gate as _hip_swiglu_gate
from .ops import swiglu_gate_packed as _hip_swiglu_gate_packed
from .ops import MAX_SAMPLE_VOCAB as _MAX_SAMPLE_VOCAB
from .ops import topk_sample as _hip_topk_sample
from .projection import project as _project
from .projection import project_packed as _project_packed

__all__ = ["TradingModel", "LlamaDecoderBlock", "LlamaAttention", "SwiGLU", "RMSNorm", "RotaryEmbedding",
           "ATTENTION_BACKENDS", "HIP_BACKENDS"]

ATTENTION_BACKENDS = ("auto", "flash", "efficient", "math", "triton", "hip")
HIP_BACKENDS = ("triton", "hip")
_KERNEL_DTYPES = (torch.float16, torch.bfloat16, torch.float32)


def _kernel_operands(*tensors: torch.Tensor) -> bool:
    """The operator kernels' precondition, as the reference's ``_can_use_triton``
    (``triton_ops.py:95-96``): GPU tensors of a 16- or 32-bit float dtype.  Where
    it fails the reference's triton_* operators compute with torch instead, and
    so do the operator routes here (the attention op itself has no such path)."""
    return all(t.is_cuda and t.dtype in _KERNEL_DTYPES for t in tensors)


class TradingModel(nn.Module):
    """Causal decoder with tied embeddings and next-token cross entropy (``model.py:20-131``)."""

    def __init__(
        self,
        vocab_size: int,
        block_size: int,
        hidden_dim: int = 128,
        layers: int = 4,
        attention_heads: int = 4,
        kv_heads: int | None = None,
        intermediate_dim: int | None = None,
        dropout: float = 0.1,
        rope_theta: float = 500_000.0,
        norm_eps: float = 1e-5,
        attention_backend: str = "auto",
        fuse_rope: bool = True,
    ) -> None:
        super().__init__()
        if hidden_dim % attention_heads != 0:
            raise ValueError("hidden_dim must be divisible by attention_heads")
        kv_heads = kv_heads or attention_heads
        if attention_heads % kv_heads != 0:
            raise ValueError("attention_heads must be divisible by kv_heads")
        self.vocab_size = vocab_size
        self.block_size = block_size
        self.hidden_dim = hidden_dim
        self.attention_heads = attention_heads
        self.kv_heads = kv_heads
        self.operator_backend = attention_backend
        self.token_embedding = nn.Embedding(vocab_size, hidden_dim)
        self.blocks = nn.ModuleList(
            [
                LlamaDecoderBlock(
                    hidden_dim=hidden_dim,
                    block_size=block_size,
                    attention_heads=attention_heads,
                    kv_heads=kv_heads,
                    intermediate_dim=intermediate_dim,
                    dropout=dropout,
                    rope_theta=rope_theta,
                    norm_eps=norm_eps,
                    attention_backend=attention_backend,
                    fuse_rope=fuse_rope,
                )
                for _ in range(layers)
            ]
        )
        self.norm = RMSNorm(hidden_dim, eps=norm_eps, operator_backend=_norm_backend(attention_backend))
        self.output = nn.Linear(hidden_dim, vocab_size, bias=False)
        self.apply(_init_weights)
        self.output.weight = self.token_embedding.weight  # tied after init, as model.py:71

    # KV-cached generate on the HIP routes replays one recorded HIP graph per token
    decode_graphs = True
    # (key, per-layer KV caches, recorded decode step) kept between generate
    # calls so later calls with the same key reuse the recording; the key is
    # (batch, device, top_k, _recording_fingerprint())
    _gen_state = None

    def forward(self, input_ids: torch.Tensor) -> torch.Tensor:
        return self.output(self._hidden(input_ids))

    def forward_with_loss(
        self,
        input_ids: torch.Tensor,
        labels: torch.Tensor,
        *,
        return_logits: bool,
        ignore_index: int = -100,
    ) -> tuple[torch.Tensor, torch.Tensor | None]:
        """Network plus next-token cross entropy (``model.py:84-131``)."""
        if labels.shape != input_ids.shape:
            raise ValueError("labels must match input_ids shape")
        normalized = self._hidden(input_ids)
        if self.operator_backend in HIP_BACKENDS and not return_logits and _kernel_operands(normalized,
                                                                                           self.output.weight):
            loss = _hip_fused_linear_cross_entropy(normalized.reshape(-1, normalized.shape[-1]), self.output.weight,
                                                   labels.reshape(-1), ignore_index=ignore_index)
            return loss, None
        if self.operator_backend in HIP_BACKENDS and not return_logits and not bool((labels != ignore_index).any()):
            # the reference's torch form of the fused loss returns a zero loss
            # when every label is ignored, where F.cross_entropy gives NaN
            # (triton_ops.py:107-110)
            return (normalized.sum() + self.output.weight.sum()) * 0.0, None
        logits = self.output(normalized)
        loss = F.cross_entropy(logits.reshape(-1, logits.shape[-1]), labels.reshape(-1), ignore_index=ignore_index)
        return loss, (logits if return_logits else None)

    @torch.no_grad()
    def generate(self, input_ids: torch.Tensor, max_new_tokens: int, top_k: int = 16) -> torch.Tensor:
        """Sample ``max_new_tokens`` tokens (top-k, multinomial) after ``input_ids``
        (``model.py:134-147``).

        The reference re-runs the whole context (the last ``block_size`` tokens)
        through the model for every new token.  The HIP routes ("triton" / "hip")
        instead keep a KV cache: one prefill over the prompt records every
        layer's rotated keys and values, then each new token runs through the
        model alone and attends to the cache (``decode_attention``).  The logits
        are those of the full recompute (same causal attention, computed once).
        When the sequence outgrows ``block_size`` the reference's window slides
        and renumbers the RoPE positions, so from then on these routes recompute
        the window as the reference does.  Other backends run the reference loop.
        """
        self.eval()
        if self.operator_backend not in HIP_BACKENDS or self.hidden_dim // self.attention_heads not in KERNEL_HEAD_DIMS:
            # the decode kernels are built for head_dim 32 / 64 / 128; other sizes
            # (padded in the prefill-free forward) use the reference's loop
            return self._generate_recompute(input_ids, max_new_tokens, top_k)
        tokens = input_ids
        cache = step = None
        key = (tokens.shape[0], tokens.device, top_k, self._recording_fingerprint())
        if self._gen_state is not None and self._gen_state[0] != key:
            self._gen_state = None  # recorded against other weights, dtypes or autocast state
        for _ in range(max_new_tokens):
            t = tokens.shape[1]
            if t > self.block_size:
                cache = step = None
                nxt = _sample_next(self(tokens[:, -self.block_size:])[:, -1, :], top_k)
            elif cache is None:
                # prefill into the kept caches when a recording for this batch exists
                state = self._gen_state if self.decode_graphs else None
                reuse = state is not None and state[0] == key
                logits, cache, reused = self._prefill(tokens, state[1] if reuse else None)
                step = state[2] if reuse and reused else None
                if reuse and not reused:
                    self._gen_state = None
                nxt = _sample_next(logits, top_k)
            elif self.decode_graphs:
                if step is None:
                    step = _DecodeGraph(self, cache, tokens.shape[0], tokens.device, top_k=top_k)
                    self._gen_state = (key, cache, step)
                nxt = step(tokens[:, -1:], t - 1)  # replays the recorded step, then samples
            else:
                nxt = _sample_next(self._decode(tokens[:, -1:], cache, t - 1), top_k)
            tokens = torch.cat([tokens, nxt], dim=1)
        return tokens

    def _recording_fingerprint(self):
        """What a recorded decode step has built in besides its shapes: the
        storage address and dtype of every parameter and buffer (the recorded
        kernels read them by address, so ``.to(dtype)`` or
        ``load_state_dict(assign=True)`` must not replay an old recording) and
        the autocast state (it fixes which precision path was recorded)."""
        tensors = tuple((t.data_ptr(), t.dtype) for t in itertools.chain(self.parameters(), self.buffers()))
        return tensors, torch.is_autocast_enabled("cuda"), torch.get_autocast_dtype("cuda")

    @torch.no_grad()
    def _generate_recompute(self, input_ids: torch.Tensor, max_new_tokens: int, top_k: int) -> torch.Tensor:
        """The reference's loop (``model.py:136-147``): the whole window per token."""
        self.eval()
        tokens = input_ids
        for _ in range(max_new_tokens):
            logits = self(tokens[:, -self.block_size:])[:, -1, :]
            tokens = torch.cat([tokens, _sample_next(logits, top_k)], dim=1)
        return tokens

    def _prefill(self, tokens: torch.Tensor, into=None):
        """Forward over the prompt that also fills per-layer KV caches of capacity
        block_size: the caches given in ``into`` when their shape and dtype fit
        (then ``reused`` is True), else new ones.  Returns (logits, caches, reused)."""
        cache = []
        reused = into is not None

        def attend(i, block, normed):
            nonlocal reused
            attended, k_cache, v_cache = block.attention.prefill(normed, self.block_size,
                                                                 into[i] if into is not None else None)
            reused = reused and k_cache is into[i][0]
            cache.append((k_cache, v_cache))
            return attended

        normed = self._residual_chain(self.token_embedding(tokens), attend)
        # the loss head on the last position only: the logits generate samples from
        return self.output(normed[:, -1, :]), cache, reused

    def _decode(self, token: torch.Tensor, cache, pos) -> torch.Tensor:
        """Logits after the token at position ``pos`` (its K/V are appended to the
        caches).  ``pos`` is an int, or a one-element int32 GPU tensor that the
        kernels read when they run (the form a recorded HIP graph replays)."""
        length = pos + 1

        def attend(i, block, normed):
            k_cache, v_cache = cache[i]
            return block.attention.decode(normed, k_cache, v_cache, pos, length)

        return self.output(self._residual_chain(self.token_embedding(token), attend))[:, -1, :]

    def _residual_chain(self, hidden: torch.Tensor, attend) -> torch.Tensor:
        """The blocks (``model.py:184-187`` each) and the final norm over the
        residual stream ``hidden``, with ``attend(i, block, normed)`` for the
        attention call (training, prefill and decode differ only there);
        returns the final norm's output.  With the norms on HIP ("hip") every residual add is fused
        into the norm that reads its sum (the block's FFN norm, the next
        block's attention norm, or the final norm): ``ops.add_rms_norm`` when
        the branch and the stream share a dtype, ``ops.add_rms_norm_mixed``
        for a 16-bit branch on an fp32 stream under autocast, whose norms then
        write the autocast dtype that the next projection would cast to.
        Both are bit-identical to the add followed by the norm (and the cast)."""
        if self.norm.operator_backend != "hip":
            for i, block in enumerate(self.blocks):
                hidden = hidden + attend(i, block, block.attention_norm(hidden))
                hidden = hidden + block.feed_forward(block.ffn_norm(hidden))
            return self.norm(hidden)
        act = None
        if (hidden.is_cuda and hidden.dtype == torch.float32 and torch.is_autocast_enabled("cuda")
                and torch.get_autocast_dtype("cuda") in (torch.bfloat16, torch.float16)
                and self.norm.weight.dtype == torch.float32):
            act = torch.get_autocast_dtype("cuda")
        first = self.blocks[0].attention_norm if len(self.blocks) else self.norm
        normed = _hip_rms_norm_mixed(hidden, first.weight, eps=first.eps, out_dtype=act) if act else first(hidden)
        for i, block in enumerate(self.blocks):
            nxt = self.blocks[i + 1].attention_norm if i + 1 < len(self.blocks) else self.norm
            hidden, normed = _add_norm(attend(i, block, normed), hidden, block.ffn_norm)
            hidden, normed = _add_norm(block.feed_forward(normed), hidden, nxt)
        return normed

    def _hidden(self, input_ids: torch.Tensor) -> torch.Tensor:
        if input_ids.ndim != 2:
            raise ValueError("input_ids must have shape [batch, time]")
        if input_ids.shape[1] > self.block_size:
            raise ValueError(f"sequence length {input_ids.shape[1]} exceeds block_size {self.block_size}")
        hidden = self.token_embedding(input_ids)
        if self.norm.operator_backend == "hip":
            return self._residual_chain(hidden, lambda i, block, normed: block.attention(normed))
        for block in self.blocks:
            hidden = block(hidden)
        return self.norm(hidden)


class LlamaDecoderBlock(nn.Module):
    """Pre-norm block: x + attn(norm(x)), then + ffn(norm(x)) (``model.py:150-187``)."""

    def __init__(
        self,
        hidden_dim: int,
        block_size: int,
        attention_heads: int,
        kv_heads: int,
        intermediate_dim: int | None,
        dropout: float,
        rope_theta: float,
        norm_eps: float,
        attention_backend: str,
        fuse_rope: bool = True,
    ) -> None:
        super().__init__()
        norm_backend = _norm_backend(attention_backend)
        self.attention_norm = RMSNorm(hidden_dim, eps=norm_eps, operator_backend=norm_backend)
        self.attention = LlamaAttention(
            hidden_dim=hidden_dim,
            block_size=block_size,
            attention_heads=attention_heads,
            kv_heads=kv_heads,
            dropout=dropout,
            rope_theta=rope_theta,
            attention_backend=attention_backend,
            fuse_rope=fuse_rope,
        )
        self.ffn_norm = RMSNorm(hidden_dim, eps=norm_eps, operator_backend=norm_backend)
        self.feed_forward = SwiGLU(hidden_dim, intermediate_dim or _llama_intermediate_dim(hidden_dim), dropout,
                                   operator_backend=attention_backend)

    def forward(self, hidden: torch.Tensor) -> torch.Tensor:
        hidden = hidden + self.attention(self.attention_norm(hidden))
        return hidden + self.feed_forward(self.ffn_norm(hidden))


class LlamaAttention(nn.Module):
    """Causal GQA self-attention with RoPE (``model.py:189-237``)."""

    def __init__(
        self,
        hidden_dim: int,
        block_size: int,
        attention_heads: int,
        kv_heads: int,
        dropout: float,
        rope_theta: float,
        attention_backend: str = "auto",
        fuse_rope: bool = True,
    ) -> None:
        super().__init__()
        if attention_backend not in ATTENTION_BACKENDS:
            raise ValueError("attention_backend must be one of: " + ", ".join(ATTENTION_BACKENDS))
        self.attention_heads = attention_heads
        self.kv_heads = kv_heads
        self.head_dim = hidden_dim // attention_heads
        self.repeats = attention_heads // kv_heads
        self.q_proj = nn.Linear(hidden_dim, attention_heads * self.head_dim, bias=False)
        self.k_proj = nn.Linear(hidden_dim, kv_heads * self.head_dim, bias=False)
        self.v_proj = nn.Linear(hidden_dim, kv_heads * self.head_dim, bias=False)
        self.o_proj = nn.Linear(hidden_dim, hidden_dim, bias=False)
        self.rope = RotaryEmbedding(self.head_dim, block_size, theta=rope_theta, operator_backend=attention_backend)
        self.dropout = dropout
        self.rope_theta = rope_theta
        self.attention_backend = attention_backend
        self.fuse_rope = fuse_rope

    def forward(self, hidden: torch.Tensor) -> torch.Tensor:
        batch_size, sequence_length, hidden_dim = hidden.shape
        dropout_p = self.dropout if self.training else 0.0
        if self.attention_backend == "hip" and self.fuse_rope and dropout_p == 0.0 and self.head_dim in KERNEL_HEAD_DIMS:
            # one q|k|v GEMM whose packed output the fused-RoPE kernels read in
            # place; they write the output in the o-projection's layout and
            # the backward writes one packed q|k|v gradient
            qkv = _project_packed(hidden, (self.q_proj.weight, self.k_proj.weight, self.v_proj.weight))
            if qkv.dtype in (torch.bfloat16, torch.float16):
                return self._out(_hip_rope_attention_packed(qkv, self.rope.cos, self.rope.sin,
                                                            heads=self.attention_heads, kv_heads=self.kv_heads))
            d = self.head_dim
            query, key, value = self._head_views(*torch.split(
                qkv, [self.attention_heads * d, self.kv_heads * d, self.kv_heads * d], dim=-1))
        else:
            query, key, value = self._heads(hidden)
        if self.attention_backend in HIP_BACKENDS and dropout_p == 0.0:
            if self.fuse_rope:
                attended = _hip_rope_attention(query, key, value, self.rope.cos, self.rope.sin, repeats=self.repeats)
            else:
                query, key = self.rope(query, key)
                attended = _hip_attention(query, key, value, repeats=self.repeats)
        else:
            query, key = self.rope(query, key)
            attended = F.scaled_dot_product_attention(
                query, key, value, dropout_p=dropout_p, is_causal=True, enable_gqa=self.repeats > 1
            )
        attended = attended.transpose(1, 2).contiguous().view(batch_size, sequence_length, hidden_dim)
        return self._out(attended)

    def _heads(self, hidden: torch.Tensor):
        """[B, T, H*D] projections -> [B, H, T, D] strided views, as model.py:220-222.
        On "hip" the three products come from one GEMM (``projection.project``)."""
        if self.attention_backend == "hip":
            return self._head_views(*_project(hidden, (self.q_proj.weight, self.k_proj.weight, self.v_proj.weight)))
        return self._head_views(self.q_proj(hidden), self.k_proj(hidden), self.v_proj(hidden))

    def _head_views(self, query: torch.Tensor, key: torch.Tensor, value: torch.Tensor):
        b, t, _ = query.shape
        query = query.view(b, t, self.attention_heads, self.head_dim).transpose(1, 2)
        key = key.view(b, t, self.kv_heads, self.head_dim).transpose(1, 2)
        value = value.view(b, t, self.kv_heads, self.head_dim).transpose(1, 2)
        return query, key, value

    def _out(self, attended: torch.Tensor) -> torch.Tensor:
        if self.attention_backend == "hip":
            return _project_packed(attended, (self.o_proj.weight,))
        return self.o_proj(attended)

    def prefill(self, hidden: torch.Tensor, capacity: int, into=None):
        """Attention over the prompt (fused-RoPE HIP kernels) plus KV caches
        [B, Hkv, capacity, D] holding its rotated keys and values (16-bit);
        ``into`` = (k_cache, v_cache) to fill instead of allocating, used when
        its shape and dtype match."""
        b, t, hidden_dim = hidden.shape
        query, key, value = self._heads(hidden)
        kdt = query.dtype if query.dtype in (torch.bfloat16, torch.float16) else torch.bfloat16
        q16, k16, v16 = query.to(kdt), key.to(kdt), value.to(kdt)
        cos, sin = _rope_tables(self.rope.cos, self.rope.sin, q16)
        _native.load()
        out, _lse, _q_rot, k_rot = torch.ops.mega_trading_amd.gqa_rope_attn_fwd(
            q16, k16, v16, cos, sin, 1.0 / math.sqrt(self.head_dim))
        shape = (b, self.kv_heads, capacity, self.head_dim)
        if into is not None and into[0].shape == shape and into[0].dtype == kdt and into[0].device == hidden.device:
            k_cache, v_cache = into
        else:
            k_cache = torch.empty(shape, device=hidden.device, dtype=kdt)
            v_cache = torch.empty_like(k_cache)
        k_cache[:, :, :t] = k_rot
        v_cache[:, :, :t] = v16
        attended = out.to(hidden.dtype).transpose(1, 2).contiguous().view(b, t, hidden_dim)
        return self._out(attended), k_cache, v_cache

    def decode(self, hidden: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor, pos, length=None):
        """One token at position ``pos`` (int or device int32 tensor): rotate its
        q/k (fp32 from the 16-bit values, as the fused kernels do), append k/v to
        the caches, attend over positions 0..pos."""
        b, _, hidden_dim = hidden.shape
        query, key, value = self._heads(hidden)
        q_rot = _hip_decode_rope_append(query, key, value, self.rope.cos, self.rope.sin, pos, k_cache, v_cache)
        out = _hip_decode_attention(q_rot, k_cache, v_cache, pos + 1 if length is None else length,
                                    repeats=self.repeats)
        if self.attention_backend != "hip":
            out = out.to(hidden.dtype)
        # on "hip" o_proj takes the 16-bit output as it is (the few-row product
        # widens it on load: the same values as casting first)
        attended = out.transpose(1, 2).reshape(b, 1, hidden_dim)
        return self._out(attended)


class SwiGLU(nn.Module):
    """w2(silu(w1 x) * w3 x) (``model.py:240-256``); the gate on HIP for "triton" / "hip"."""

    def __init__(self, hidden_dim: int, intermediate_dim: int, dropout: float, operator_backend: str = "auto") -> None:
        super().__init__()
        self.w1 = nn.Linear(hidden_dim, intermediate_dim, bias=False)
        self.w2 = nn.Linear(intermediate_dim, hidden_dim, bias=False)
        self.w3 = nn.Linear(hidden_dim, intermediate_dim, bias=False)
        self.dropout = nn.Dropout(dropout)
        self.operator_backend = operator_backend

    def forward(self, hidden: torch.Tensor) -> torch.Tensor:
        if self.operator_backend == "hip":
            # one GEMM for w1 and w3, the gate on its packed output, split-K dW
            gated = _hip_swiglu_gate_packed(_project_packed(hidden, (self.w1.weight, self.w3.weight)))
            return _project_packed(self.dropout(gated), (self.w2.weight,))
        gate = self.w1(hidden)
        up = self.w3(hidden)
        if self.operator_backend in HIP_BACKENDS and _kernel_operands(gate, up) and gate.shape == up.shape:
            gated = _hip_swiglu_gate(gate, up)
        else:
            gated = F.silu(gate) * up
        return self.w2(self.dropout(gated))


class RMSNorm(nn.Module):
    """``F.rms_norm`` with a learned scale (``model.py:259-269``); HIP kernels for "hip"."""

    def __init__(self, hidden_dim: int, eps: float = 1e-5, operator_backend: str = "auto") -> None:
        super().__init__()
        self.weight = nn.Parameter(torch.ones(hidden_dim))
        self.eps = eps
        self.operator_backend = operator_backend

    def forward(self, hidden: torch.Tensor) -> torch.Tensor:
        if self.operator_backend == "hip":
            return _hip_rms_norm(hidden, self.weight, eps=self.eps)
        return F.rms_norm(hidden, (hidden.shape[-1],), self.weight, eps=self.eps)


def _norm_backend(attention_backend: str) -> str:
    """The reference builds its norms without a backend (torch); "hip" moves them to HIP."""
    return "hip" if attention_backend == "hip" else "auto"


class RotaryEmbedding(nn.Module):
    """fp32 tables cos/sin [1, 1, T_max, D/2] of pos * theta^(-2i/D) (``model.py:272-294``).

    ``operator_backend`` "triton" or "hip" rotates with the HIP RoPE kernel
    (``ops.apply_rope``, in place of ``triton_apply_rope``, ``model.py:292-293``);
    any other value with torch.  Both take the tables cast to the activation
    dtype, as the reference does."""

    def __init__(self, head_dim: int, max_sequence_length: int, theta: float, operator_backend: str = "auto") -> None:
        super().__init__()
        if head_dim % 2 != 0:
            raise ValueError("RoPE requires an even head dimension")
        self.operator_backend = operator_backend
        positions = torch.arange(max_sequence_length, dtype=torch.float32)
        inv_freq = 1.0 / (theta ** (torch.arange(0, head_dim, 2, dtype=torch.float32) / head_dim))
        freqs = torch.outer(positions, inv_freq)
        self.register_buffer("cos", freqs.cos().view(1, 1, max_sequence_length, head_dim // 2), persistent=False)
        self.register_buffer("sin", freqs.sin().view(1, 1, max_sequence_length, head_dim // 2), persistent=False)

    def forward(self, query: torch.Tensor, key: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
        sequence_length = query.shape[-2]
        if sequence_length > self.cos.shape[-2]:
            raise ValueError(f"sequence length {sequence_length} exceeds RoPE cache length {self.cos.shape[-2]}")
        cos = self.cos[:, :, :sequence_length].to(dtype=query.dtype)
        sin = self.sin[:, :, :sequence_length].to(dtype=query.dtype)
        # the reference's triton_apply_rope computes with torch for tensors its
        # kernel does not take, and when query and key differ in head size
        # (triton_ops.py:51-52)
        if (self.operator_backend in HIP_BACKENDS and _kernel_operands(query, key)
                and query.shape[-1] == key.shape[-1]):
            return _hip_apply_rope(query, key, cos, sin)
        return rotate(query, cos, sin), rotate(key, cos, sin)


class _DecodeGraph:
    """One decode step of ``TradingModel._decode`` recorded as a HIP graph and
    replayed for every new token.  The token and its position live in device
    buffers that the recorded kernels read (the decode kernels take the length
    from device memory and cover the cache capacity), so one recording serves
    every position; the host only writes the next token and position before
    each replay.  Replaying a step again for the same position rewrites the
    same cache row with the same values, so the first call (warm-up, record,
    replay) is harmless.  The result is the graph's static logits buffer,
    valid until the next call, or with ``top_k`` set the sampled next tokens
    [batch, 1] (``_sample_recorded``: the reference's top-k multinomial draw
    without its host-side validity check, so no host synchronisation).  The
    sampling runs after the replay, outside the recording: ``torch.topk``
    over a large vocabulary clears its counters with ``hipMemsetAsync``, and
    memset nodes are kept out of recorded graphs (their replays are not
    reliable); every recorded kernel writes its outputs in full.

    The model is held by a weak reference: the model keeps its recording in
    ``_gen_state``, and a strong reference back would make every generating
    model a reference cycle that only Python's cyclic garbage collector frees,
    at an arbitrary later moment -- possibly in the middle of another graph
    capture, where destroying a graph or a stream is an error.  For the same
    reason the capture runs with the cyclic collector paused, after one
    collection of whatever dead cycles exist."""

    def __init__(self, model: "TradingModel", cache, batch: int, device: torch.device, top_k=None):
        self._model = weakref.ref(model)
        self.cache = cache
        self.top_k = top_k
        self.tok = torch.zeros((batch, 1), dtype=torch.long, device=device)
        self.pos = torch.zeros((1,), dtype=torch.int32, device=device)
        self.graph = None
        self.out = None

    def __call__(self, token: torch.Tensor, pos: int) -> torch.Tensor:
        model = self._model()
        if model is None:
            raise RuntimeError("the model of this recorded decode step no longer exists")
        self.tok.copy_(token)
        self.pos.fill_(pos)
        if self.graph is None:
            side = torch.cuda.Stream(device=self.tok.device)
            side.wait_stream(torch.cuda.current_stream(self.tok.device))
            with torch.cuda.stream(side):  # warm-up: allocator and library state outside the recording
                model._decode(self.tok, self.cache, self.pos)
            torch.cuda.current_stream(self.tok.device).wait_stream(side)
            gc.collect()
            was_enabled = gc.isenabled()
            gc.disable()
            try:
                self.graph = torch.cuda.CUDAGraph()
                with torch.cuda.graph(self.graph):
                    self.out = model._decode(self.tok, self.cache, self.pos)
            finally:
                if was_enabled:
                    gc.enable()
        self.graph.replay()
        if self.top_k is not None:
            return _sample_recorded(self.out, self.top_k)
        return self.out


def _add_norm(branch: torch.Tensor, hidden: torch.Tensor, norm: "RMSNorm") -> tuple[torch.Tensor, torch.Tensor]:
    """(hidden + branch, norm(hidden + branch)) with the add fused into the HIP norm."""
    if branch.dtype == hidden.dtype:
        return _hip_add_rms_norm(branch, hidden, norm.weight, eps=norm.eps)
    if (hidden.dtype == torch.float32 and branch.dtype in (torch.bfloat16, torch.float16)
            and norm.weight.dtype == torch.float32):
        return _hip_add_rms_norm_mixed(branch, hidden, norm.weight, eps=norm.eps)
    hidden = hidden + branch
    return hidden, norm(hidden)


def _sample_next(logits: torch.Tensor, top_k: int) -> torch.Tensor:
    """Top-k filtered multinomial sample of one token per row (``model.py:141-145``)."""
    if top_k > 0:
        values, _ = torch.topk(logits, min(top_k, logits.shape[-1]))
        logits = logits.masked_fill(logits < values[:, [-1]], float("-inf"))
    probs = torch.softmax(logits, dim=-1)
    return torch.multinomial(probs, num_samples=1)


def _sample_recorded(logits: torch.Tensor, top_k: int) -> torch.Tensor:
    """``_sample_next`` without a host synchronisation.  For one sample
    ``torch.multinomial`` draws argmax(p / E) with E ~ Exponential(1) from the
    same generator, after a host-synchronising check that p holds no inf, NaN
    or negative value; this is that draw without the check (same tokens for
    the same generator state).  For fp32 GPU logits it is one HIP launch
    (``ops.topk_sample``) after the same noise draw; the kernel's fp32 sums
    run in its own order, so only a p / E tie within a rounding error could
    pick another token than the library kernels."""
    k = min(top_k, logits.shape[-1])
    if (top_k > 0 and logits.is_cuda and logits.dtype == torch.float32 and logits.ndim == 2
            and logits.shape[-1] <= _MAX_SAMPLE_VOCAB):
        return _hip_topk_sample(logits, torch.empty_like(logits).exponential_(1), k)
    if top_k > 0:
        values, _ = torch.topk(logits, min(top_k, logits.shape[-1]))
        logits = logits.masked_fill(logits < values[:, -1:], float("-inf"))  # a slice: no host index tensor
    probs = torch.softmax(logits, dim=-1)
    return torch.argmax(probs / torch.empty_like(probs).exponential_(1), dim=-1, keepdim=True)


def rotate(value: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor) -> torch.Tensor:
    """Interleaved-pair rotation (x0, x1) -> (x0 c - x1 s, x0 s + x1 c) (``model.py:312-316``)."""
    even = value[..., 0::2]
    odd = value[..., 1::2]
    return torch.stack((even * cos - odd * sin, even * sin + odd * cos), dim=-1).flatten(start_dim=-2)


def _init_weights(module: nn.Module) -> None:
    """N(0, 0.02) weights, zero biases (``model.py:319-326``)."""
    if isinstance(module, nn.Linear):
        nn.init.normal_(module.weight, mean=0.0, std=0.02)
        if module.bias is not None:
            nn.init.zeros_(module.bias)
    elif isinstance(module, nn.Embedding):
        nn.init.normal_(module.weight, mean=0.0, std=0.02)


def _llama_intermediate_dim(hidden_dim: int) -> int:
    """8/3 d_model rounded up to a multiple of 16 (``model.py:329-331``)."""
    return int(math.ceil((8 * hidden_dim / 3) / 16) * 16)
