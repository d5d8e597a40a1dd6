"""Causal grouped-query attention on MI355X (gfx950) HIP kernels.

Drop-in for the reference operator
``mega_trading.kernels.triton_attention.triton_attention(query, key, value, *, repeats)``
(``src/mega_trading/kernels/triton_attention.py:12-24``): same argument
meaning, same validation order and exception types, output with the query's
layout, LSE saved for the backward.  ``rope_attention`` additionally fuses the
interleaved RoPE that ``model.py:223`` applies right before the attention call
(``triton_apply_rope``, ``src/mega_trading/kernels/triton_ops.py:45-54``) into
the kernels' Q/K tile loads.

The attention ops are ``torch.library`` ops (``mega_trading_amd::gqa_attn_fwd``,
``::gqa_rope_attn_fwd``, ``::gqa_attn_bwd`` and the packed q|k|v pair) whose
schemas, fake implementations and autograd are declared here, so
``torch.compile`` treats them as opaque nodes; their GPU implementations live
in ``libmt_torch.so`` (``csrc/mt_torch.cpp``), which prepares the arguments,
allocates the outputs and calls the C ABI of ``libmt_attn.so`` on the
caller's current stream.  They never synchronise and never fall back to
another implementation: without the HIP libraries they raise.
"""

from __future__ import annotations

import math
from typing import Optional

import torch

from . import _native

__all__ = ["attention", "rope_attention", "rope_attention_packed", "attention_forward", "decode_attention",
           "SUPPORTED_HEAD_DIMS", "KERNEL_HEAD_DIMS", "MAX_HEAD_DIM", "MAX_DECODE_REPEATS"]

# query heads per KV head one decode launch serves; larger groups run as several launches
MAX_DECODE_REPEATS = 8

# head sizes the kernels are built for; any other head_dim up to MAX_HEAD_DIM is
# zero-padded to the next one (the reference's forward takes any D, rounding its
# tile to the next power of two, triton_attention.py:36)
KERNEL_HEAD_DIMS = (32, 64, 128)
SUPPORTED_HEAD_DIMS = KERNEL_HEAD_DIMS
MAX_HEAD_DIM = 128
_KERNEL_DTYPES = {torch.bfloat16: _native.DTYPE_BF16, torch.float16: _native.DTYPE_FP16}


def attention(query: torch.Tensor, key: torch.Tensor, value: torch.Tensor, *, repeats: int) -> torch.Tensor:
    """Causal GQA attention (``triton_attention.py:12``).

    ``query`` [B, Hq, T, D]; ``key``/``value`` [B, Hkv, T, D] with
    ``Hq == Hkv * repeats``; query head ``h`` attends to KV head ``h // repeats``.
    Scale ``1/sqrt(D)``, top-left causal mask.  Any strides with a unit last
    stride are used in place.  bf16 / fp16 inputs run on the 16-bit MFMA
    kernels (fp32 accumulation and softmax); fp32 inputs run on full-fp32
    MFMA kernels, at least as precise as the reference's fp32 path (TF32
    forward dots, dense fp32 backward, ``triton_attention.py:88-111``).
    """
    _validate(query, key, value, repeats)
    out, _lse = _forward(query, key, value, None, None)
    return out


def rope_attention(
    query: torch.Tensor,
    key: torch.Tensor,
    value: torch.Tensor,
    cos: torch.Tensor,
    sin: torch.Tensor,
    *,
    repeats: int,
) -> torch.Tensor:
    """RoPE(query), RoPE(key), then causal GQA attention, in one fused op.

    Equivalent to ``model.py:223`` + ``:226``: ``query, key = rope(query, key)``
    then ``triton_attention(query, key, value, repeats=repeats)``, with the
    rotation done in fp32 inside the kernels' tile loads.  ``cos``/``sin`` are
    the RotaryEmbedding tables (``model.py:279-284``): fp32, last dim D/2,
    leading singleton dims allowed, at least T rows; row t rotates position t.
    Gradients w.r.t. query and key are returned in the un-rotated basis.
    """
    _validate(query, key, value, repeats)
    c, s = _rope_tables(cos, sin, query)
    out, _lse = _forward(query, key, value, c, s)
    return out


def rope_attention_packed(
    qkv: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor, *, heads: int, kv_heads: int
) -> torch.Tensor:
    """``rope_attention`` on the packed output of one q|k|v projection GEMM.

    ``qkv`` [B, T, (heads + 2 kv_heads) * D] holds, per token, the query
    heads, then the key heads, then the value heads (``model.py:220-222``'s
    three products side by side), bf16 or fp16.  Returns the attention output
    as [B, T, heads * D], the layout the output projection reads
    (``model.py:236``), written there directly by the kernel; the backward
    writes dQ, dK and dV into one gradient of qkv's layout.  Results equal
    ``rope_attention`` on the three head views."""
    if qkv.ndim != 3:
        raise ValueError("qkv must have shape [batch, time, (heads + 2 kv_heads) * head_dim]")
    if heads <= 0 or kv_heads <= 0 or heads % kv_heads:
        raise ValueError("heads must be a positive multiple of kv_heads")
    if qkv.shape[-1] % (heads + 2 * kv_heads):
        raise ValueError("qkv's last dim must be (heads + 2 kv_heads) * head_dim")
    if qkv.dtype not in (torch.bfloat16, torch.float16):
        raise RuntimeError(f"qkv dtype {qkv.dtype} unsupported (bfloat16 or float16)")
    q, k, v = _packed_views(qkv, heads, kv_heads)
    _validate(q, k, v, heads // kv_heads)
    c, s = _rope_tables(cos, sin, q)
    d = q.shape[-1]
    if d not in KERNEL_HEAD_DIMS:
        raise ValueError(f"the packed form needs head_dim {KERNEL_HEAD_DIMS} (got {d}); use rope_attention")
    _native.load()
    out, _lse, _q_rot, _k_rot = torch.ops.mega_trading_amd.gqa_rope_attn_packed_fwd(
        qkv, c, s, heads, kv_heads, 1.0 / math.sqrt(d))
    return out


def _packed_views(qkv: torch.Tensor, heads: int, kv_heads: int):
    """[B, H, T, D] views of the query, key and value heads of a packed qkv."""
    b, t, width = qkv.shape
    d = width // (heads + 2 * kv_heads)
    q = qkv[..., : heads * d].view(b, t, heads, d).transpose(1, 2)
    k = qkv[..., heads * d:(heads + kv_heads) * d].view(b, t, kv_heads, d).transpose(1, 2)
    v = qkv[..., (heads + kv_heads) * d:].view(b, t, kv_heads, d).transpose(1, 2)
    return q, k, v


def attention_forward(
    query: torch.Tensor,
    key: torch.Tensor,
    value: torch.Tensor,
    *,
    repeats: int,
    cos: Optional[torch.Tensor] = None,
    sin: Optional[torch.Tensor] = None,
) -> tuple[torch.Tensor, torch.Tensor]:
    """Forward returning ``(output, logsumexp)``; LSE is fp32 [B, Hq, T], natural log
    (``triton_attention.py:346-349``).  Differentiable in the output."""
    _validate(query, key, value, repeats)
    c = s = None
    if cos is not None or sin is not None:
        if cos is None or sin is None:
            raise ValueError("cos and sin must be given together")
        c, s = _rope_tables(cos, sin, query)
    return _forward(query, key, value, c, s)


def decode_attention(
    query: torch.Tensor, key_cache: torch.Tensor, value_cache: torch.Tensor, length, *, repeats: int
) -> torch.Tensor:
    """One new query token per sequence against a KV cache (inference only).

    ``query`` [B, Hq, 1, D] is the new token's (rotated) query at position
    ``length - 1``; ``key_cache`` / ``value_cache`` [B, Hkv, >= length, D] hold
    the rotated keys and the values of positions 0 .. length-1 (the new token's
    own included).  Returns [B, Hq, 1, D]: the last row of the causal GQA
    attention over those positions (what ``TradingModel.generate``,
    ``model.py:134-147``, obtains by recomputing the whole context).  16-bit
    inputs; query head h reads KV head h // repeats; head_dim 32, 64 or 128.
    A group of more than 8 query heads per KV head runs as several launches.

    ``length`` is an int, or a one-element int32 tensor on the GPU that the
    kernels read when they run (clamped to [1, capacity]): the launch then
    covers the whole cache capacity and can be recorded once in a HIP graph
    and replayed for every step.
    """
    if query.device.type != "cuda":
        raise RuntimeError("hip attention backend requires ROCm GPU tensors")
    if query.dtype not in _KERNEL_DTYPES:
        raise RuntimeError("decode attention supports float16 and bfloat16 tensors")
    if query.ndim != 4 or key_cache.ndim != 4 or value_cache.ndim != 4 or query.shape[2] != 1:
        raise ValueError("query must be [batch, heads, 1, head_dim] and the caches [batch, heads, capacity, head_dim]")
    if key_cache.shape != value_cache.shape:
        raise ValueError("key and value caches must have the same shape")
    if key_cache.shape[1] * repeats != query.shape[1]:
        raise ValueError("query heads must equal key/value heads multiplied by repeats")
    if key_cache.shape[0] != query.shape[0] or key_cache.shape[3] != query.shape[3]:
        raise ValueError("query and caches must agree on batch and head_dim")
    dev_length = isinstance(length, torch.Tensor)
    if dev_length:
        if length.dtype != torch.int32 or length.numel() != 1 or length.device != query.device:
            raise ValueError("a tensor length must be a one-element int32 tensor on the query's device")
    elif not 1 <= length <= key_cache.shape[2]:
        raise ValueError(f"length {length} outside [1, cache capacity {key_cache.shape[2]}]")
    if key_cache.dtype != query.dtype or value_cache.dtype != query.dtype:
        raise RuntimeError("query and caches must share one dtype")
    if query.shape[-1] not in KERNEL_HEAD_DIMS:
        raise ValueError(f"head_dim must be one of {KERNEL_HEAD_DIMS} (got {query.shape[-1]})")
    scale = 1.0 / math.sqrt(query.shape[-1])
    if repeats > MAX_DECODE_REPEATS:
        # the group's query heads in even sub-groups of at most MAX_DECODE_REPEATS,
        # each one launch over the same cache (a sub-group is a GQA group of its own)
        b, hq, _, d = query.shape
        hkv = key_cache.shape[1]
        n = -(-repeats // MAX_DECODE_REPEATS)
        bounds = [repeats * j // n for j in range(n + 1)]
        grouped = query.reshape(b, hkv, repeats, d)
        parts = [decode_attention(grouped[:, :, lo:hi].reshape(b, hkv * (hi - lo), 1, d), key_cache, value_cache,
                                  length, repeats=hi - lo).view(b, hkv, hi - lo, d)
                 for lo, hi in zip(bounds[:-1], bounds[1:])]
        return torch.cat(parts, dim=2).view(b, hq, 1, d)
    if dev_length:
        return torch.ops.mega_trading_amd.gqa_attn_decode_dev(query, key_cache, value_cache, length, scale)
    return torch.ops.mega_trading_amd.gqa_attn_decode(query, key_cache, value_cache, int(length), scale)


def decode_rope_append(query: torch.Tensor, key: torch.Tensor, value: torch.Tensor, cos: torch.Tensor,
                       sin: torch.Tensor, pos, key_cache: torch.Tensor, value_cache: torch.Tensor) -> torch.Tensor:
    """The decode step's RoPE and cache append in one launch: returns the
    rotated query [B, Hq, 1, D] (cache dtype) and writes the rotated key and the
    value of the new token into ``key_cache[:, :, pos]`` / ``value_cache[:, :, pos]``.
    ``query`` [B, Hq, 1, D], ``key`` / ``value`` [B, Hkv, 1, D] (any float dtype:
    fp32 is rounded to the cache dtype first, as the fused forward does);
    ``cos`` / ``sin`` the fp32 RotaryEmbedding tables (row ``pos`` is used).
    ``pos`` is an int or a one-element int32 GPU tensor read when the kernel
    runs (clamped to the cache and table)."""
    if query.device.type != "cuda":
        raise RuntimeError("hip attention backend requires ROCm GPU tensors")
    for t in (key, value, key_cache, value_cache, cos, sin):
        if t.device != query.device:
            raise RuntimeError("query, key, value, the caches and the RoPE tables must be on one device")
    if key_cache.dtype not in _KERNEL_DTYPES or value_cache.dtype != key_cache.dtype:
        raise RuntimeError("the caches must be float16 or bfloat16 and share one dtype")
    if query.dtype not in (key_cache.dtype, torch.float32) or key.dtype != query.dtype or value.dtype != query.dtype:
        raise RuntimeError("query, key and value must share one dtype: the cache dtype or float32")
    if query.ndim != 4 or key.ndim != 4 or value.ndim != 4 or key_cache.ndim != 4 or key_cache.shape != value_cache.shape:
        raise ValueError("query [B, Hq, 1, D], key / value [B, Hkv, 1, D], caches [B, Hkv, capacity, D]")
    d = query.shape[-1]
    if key.shape[-1] != d or value.shape[-1] != d or key_cache.shape[-1] != d:
        raise ValueError("query, key, value and the caches must share head_dim")
    for name, t in (("query", query), ("key", key), ("value", value), ("key_cache", key_cache),
                    ("value_cache", value_cache)):
        if t.stride(-1) != 1:
            raise ValueError(f"{name} must have a unit last-dim stride")
    for name, tab in (("cos", cos), ("sin", sin)):
        if tab.shape[-1] != d // 2 or not tab.is_floating_point():
            raise ValueError(f"RoPE {name} table must be floating point with last dimension head_dim/2 = {d // 2}")
    # the kernel reads fp32 tables (a model cast with .to(dtype) casts its RoPE buffers too)
    cos, sin = cos.to(torch.float32), sin.to(torch.float32)
    last = min(key_cache.shape[2], cos.reshape(-1, cos.shape[-1]).shape[0]) - 1
    if isinstance(pos, torch.Tensor):
        if pos.dtype != torch.int32 or pos.numel() != 1 or pos.device != query.device:
            raise ValueError("a tensor pos must be a one-element int32 tensor on the query's device")
        return torch.ops.mega_trading_amd.decode_rope_append(query, key, value, cos, sin, last, pos, key_cache,
                                                             value_cache)
    if not 0 <= pos <= last:
        raise ValueError(f"pos {pos} outside the cache / RoPE table")
    return torch.ops.mega_trading_amd.decode_rope_append(query, key, value, cos, sin, int(pos), None, key_cache,
                                                         value_cache)


# ---------------------------------------------------------------------------
# validation (triton_attention.py:14-23) and argument preparation
# ---------------------------------------------------------------------------
def _validate(query: torch.Tensor, key: torch.Tensor, value: torch.Tensor, repeats: int) -> None:
    if query.device.type != "cuda":
        raise RuntimeError("hip attention backend requires ROCm GPU tensors")
    if query.dtype not in {torch.float16, torch.bfloat16, torch.float32}:
        raise RuntimeError("hip attention supports float16, bfloat16, and float32 tensors")
    if query.ndim != 4 or key.ndim != 4 or value.ndim != 4:
        raise ValueError("query, key, and value must be [batch, heads, sequence, head_dim]")
    if key.shape[1] * repeats != query.shape[1]:
        raise ValueError("query heads must equal key/value heads multiplied by repeats")
    if key.shape != value.shape:
        raise ValueError("key and value must have the same shape")
    if query.shape[0] != key.shape[0] or query.shape[2:] != key.shape[2:]:
        raise ValueError("query, key, and value must agree on batch, sequence, and head dimensions")
    if key.dtype != query.dtype or value.dtype != query.dtype:
        raise RuntimeError("query, key, and value must share one dtype")
    if key.device != query.device or value.device != query.device:
        raise RuntimeError("query, key, and value must be on one device")
    if not 1 <= query.shape[-1] <= MAX_HEAD_DIM:
        raise ValueError(f"head_dim must be between 1 and {MAX_HEAD_DIM} (got {query.shape[-1]})")
    if query.shape[2] < 1 or query.shape[0] < 1:
        raise ValueError("batch and sequence length must be positive")


def _rope_tables(cos: torch.Tensor, sin: torch.Tensor, query: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    t, d = query.shape[2], query.shape[3]
    if d % 2:
        raise ValueError("RoPE requires an even head dimension")
    out = []
    for name, tab in (("cos", cos), ("sin", sin)):
        if tab.shape[-1] != d // 2:
            raise ValueError(f"RoPE {name} table must have last dimension head_dim/2 = {d // 2}")
        tab2 = tab.reshape(-1, d // 2)
        if tab2.shape[0] < t:
            raise ValueError(f"sequence length {t} exceeds RoPE cache length {tab2.shape[0]}")
        out.append(tab2[:t].to(device=query.device, dtype=torch.float32).contiguous())
    return out[0], out[1]


def _kernel_ready(t: torch.Tensor) -> torch.Tensor:
    """Unit last stride, 8-element-aligned outer strides and a 16-byte-aligned base."""
    ok = t.stride(-1) == 1 and t.data_ptr() % 16 == 0
    if ok:
        for size, stride in zip(t.shape[:-1], t.stride()[:-1]):
            if size > 1 and stride % 8:
                ok = False
                break
    return t if ok else t.contiguous()


def _strides(*tensors: torch.Tensor):
    flat = []
    for t in tensors:
        flat.extend(int(st) if sz > 1 else 0 for sz, st in zip(t.shape, t.stride()))
    import ctypes

    return (ctypes.c_int64 * len(flat))(*flat)


def _ptr(t: Optional[torch.Tensor]) -> Optional[int]:
    return None if t is None else t.data_ptr()


def _kernel_head_dim(d: int) -> int:
    return next(x for x in KERNEL_HEAD_DIMS if x >= d)


def _forward(q, k, v, cos, sin):
    d = q.shape[-1]
    dk = _kernel_head_dim(d)
    if dk != d:
        return _forward_padded(q, k, v, cos, sin, dk)
    _native.load()
    scale = 1.0 / math.sqrt(d)
    if cos is None:
        return torch.ops.mega_trading_amd.gqa_attn_fwd(q, k, v, scale)
    out, lse, _q_rot, _k_rot = torch.ops.mega_trading_amd.gqa_rope_attn_fwd(q, k, v, cos, sin, scale)
    return out, lse


def _forward_padded(q, k, v, cos, sin, dk):
    """A head_dim the kernels are not built for, zero-padded to ``dk``: the padded
    q / k columns add nothing to QK^T, the padded v columns produce zero output
    columns that are dropped, the pad pairs rotate by the identity (cos 1, sin
    0), and the scale stays 1/sqrt(head_dim).  Gradients flow back through the
    padding.  The output keeps the query's layout."""
    import torch.nn.functional as F

    d = q.shape[-1]
    pad = (0, dk - d)
    qp, kp, vp = F.pad(q, pad), F.pad(k, pad), F.pad(v, pad)
    _native.load()
    scale = 1.0 / math.sqrt(d)
    if cos is None:
        out, lse = torch.ops.mega_trading_amd.gqa_attn_fwd(qp, kp, vp, scale)
    else:
        half = (dk - d) // 2
        cos = F.pad(cos, (0, half), value=1.0)
        sin = F.pad(sin, (0, half), value=0.0)
        out, lse, _q_rot, _k_rot = torch.ops.mega_trading_amd.gqa_rope_attn_fwd(qp, kp, vp, cos, sin, scale)
    result = torch.empty_like(q)
    result.copy_(out[..., :d])
    return result, lse


# ---------------------------------------------------------------------------
# the attention ops: schemas and shapes here, GPU kernels in libmt_torch.so
# ---------------------------------------------------------------------------
_LIB = torch.library.Library("mega_trading_amd", "FRAGMENT")
_LIB.define("gqa_attn_fwd(Tensor q, Tensor k, Tensor v, float scale) -> (Tensor, Tensor)")
# returns (out, lse, q_rot, k_rot); q_rot / k_rot feed the backward
_LIB.define("gqa_rope_attn_fwd(Tensor q, Tensor k, Tensor v, Tensor cos, Tensor sin, float scale) "
            "-> (Tensor, Tensor, Tensor, Tensor)")
# gradients w.r.t. (q, k, v); with RoPE tables q and k are the forward's
# rotated tensors and dQ / dK come back in the un-rotated basis
_LIB.define("gqa_attn_bwd(Tensor q, Tensor k, Tensor v, Tensor o, Tensor lse, Tensor dout, Tensor? cos, "
            "Tensor? sin, float scale) -> (Tensor, Tensor, Tensor)")
# (out [B, T, Hq*D], lse, q_rot, k_rot) for a packed qkv
_LIB.define("gqa_rope_attn_packed_fwd(Tensor qkv, Tensor cos, Tensor sin, int hq, int hkv, float scale) "
            "-> (Tensor, Tensor, Tensor, Tensor)")
# gradient w.r.t. the packed qkv (un-rotated basis), in qkv's layout
_LIB.define("gqa_attn_bwd_packed(Tensor q_rot, Tensor k_rot, Tensor qkv, Tensor out, Tensor lse, Tensor dout, "
            "Tensor cos, Tensor sin, int hq, int hkv, float scale) -> Tensor")


@torch.library.register_fake("mega_trading_amd::gqa_attn_fwd")
def _gqa_attn_fwd_fake(q, k, v, scale):
    return torch.empty_like(q), q.new_empty((q.shape[0], q.shape[1], q.shape[2]), dtype=torch.float32)


@torch.library.register_fake("mega_trading_amd::gqa_rope_attn_fwd")
def _gqa_rope_attn_fwd_fake(q, k, v, cos, sin, scale):
    b, hq, t, d = q.shape
    return (
        torch.empty_like(q),
        q.new_empty((b, hq, t), dtype=torch.float32),
        q.new_empty((b, hq, t, d)),
        q.new_empty((b, k.shape[1], t, d)),
    )


@torch.library.register_fake("mega_trading_amd::gqa_attn_bwd")
def _gqa_attn_bwd_fake(q, k, v, o, lse, dout, cos, sin, scale):
    return q.new_empty(q.shape), k.new_empty(k.shape), v.new_empty(v.shape)


@torch.library.register_fake("mega_trading_amd::gqa_rope_attn_packed_fwd")
def _gqa_rope_attn_packed_fwd_fake(qkv, cos, sin, hq, hkv, scale):
    b, t, width = qkv.shape
    d = width // (hq + 2 * hkv)
    return (qkv.new_empty((b, t, hq * d)), qkv.new_empty((b, hq, t), dtype=torch.float32),
            qkv.new_empty((b, hq, t, d)), qkv.new_empty((b, hkv, t, d)))


@torch.library.register_fake("mega_trading_amd::gqa_attn_bwd_packed")
def _gqa_attn_bwd_packed_fake(q_rot, k_rot, qkv, out, lse, dout, cos, sin, hq, hkv, scale):
    return qkv.new_empty(qkv.shape)


@torch.library.custom_op("mega_trading_amd::gqa_attn_decode", mutates_args=(), device_types="cuda")
def gqa_attn_decode(q: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor, length: int,
                    scale: float) -> torch.Tensor:
    lib = _native.load()
    q, k_cache, v_cache = _kernel_ready(q), _kernel_ready(k_cache), _kernel_ready(v_cache)
    b, hq, _, d = q.shape
    hkv = k_cache.shape[1]
    out = torch.empty((b, hq, 1, d), device=q.device, dtype=q.dtype)
    strides = _strides(q, k_cache, v_cache, out)
    with torch.cuda.device(q.device):
        ws_bytes = lib.mt_gqa_attn_decode_workspace_size(b, hq, length, d)
        ws = torch.empty(ws_bytes, device=q.device, dtype=torch.uint8)
        rc = lib.mt_gqa_attn_decode(q.data_ptr(), k_cache.data_ptr(), v_cache.data_ptr(), out.data_ptr(), b, hq, hkv,
                                    length, d, strides, scale, _KERNEL_DTYPES[q.dtype], ws.data_ptr(), ws_bytes,
                                    torch.cuda.current_stream(q.device).cuda_stream)
    _native.check(rc, "mt_gqa_attn_decode")
    return out


@torch.library.custom_op("mega_trading_amd::decode_rope_append", mutates_args=("k_cache", "v_cache"),
                         device_types="cuda")
def decode_rope_append_op(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor,
                          pos: int, pos_dev: Optional[torch.Tensor], k_cache: torch.Tensor,
                          v_cache: torch.Tensor) -> torch.Tensor:
    import ctypes

    lib = _native.load()
    b, hq, _, d = q.shape
    hkv = k.shape[1]
    q_rot = torch.empty((b, hq, 1, d), device=q.device, dtype=k_cache.dtype)
    cs = cos.reshape(-1, d // 2).contiguous()
    sn = sin.reshape(-1, d // 2).contiguous()
    ins = (ctypes.c_int64 * 6)(q.stride(0), q.stride(1), k.stride(0), k.stride(1), v.stride(0), v.stride(1))
    cst = (ctypes.c_int64 * 6)(*k_cache.stride()[:3], *v_cache.stride()[:3])
    in_dt = _native.DTYPE_FP32 if q.dtype == torch.float32 else _KERNEL_DTYPES[q.dtype]
    with torch.cuda.device(q.device):
        rc = lib.mt_decode_rope_append(q.data_ptr(), k.data_ptr(), v.data_ptr(), ins, cs.data_ptr(), sn.data_ptr(),
                                       min(cs.shape[0], sn.shape[0]), pos, _ptr(pos_dev), q_rot.data_ptr(),
                                       k_cache.data_ptr(), v_cache.data_ptr(), cst, k_cache.shape[2],
                                       b, hq, hkv, d,
                                       in_dt, _KERNEL_DTYPES[k_cache.dtype],
                                       torch.cuda.current_stream(q.device).cuda_stream)
    _native.check(rc, "mt_decode_rope_append")
    return q_rot


@decode_rope_append_op.register_fake
def _decode_rope_append_fake(q, k, v, cos, sin, pos, pos_dev, k_cache, v_cache):
    return q.new_empty(q.shape, dtype=k_cache.dtype)


@torch.library.custom_op("mega_trading_amd::gqa_attn_decode_dev", mutates_args=(), device_types="cuda")
def gqa_attn_decode_dev(q: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor, length: torch.Tensor,
                        scale: float) -> torch.Tensor:
    lib = _native.load()
    q, k_cache, v_cache = _kernel_ready(q), _kernel_ready(k_cache), _kernel_ready(v_cache)
    b, hq, _, d = q.shape
    hkv, cap = k_cache.shape[1], k_cache.shape[2]
    out = torch.empty((b, hq, 1, d), device=q.device, dtype=q.dtype)
    strides = _strides(q, k_cache, v_cache, out)
    with torch.cuda.device(q.device):
        ws_bytes = lib.mt_gqa_attn_decode_workspace_size(b, hq, cap, d)
        ws = torch.empty(ws_bytes, device=q.device, dtype=torch.uint8)
        rc = lib.mt_gqa_attn_decode_dev(q.data_ptr(), k_cache.data_ptr(), v_cache.data_ptr(), out.data_ptr(), b, hq,
                                        hkv, cap, length.data_ptr(), d, strides, scale, _KERNEL_DTYPES[q.dtype],
                                        ws.data_ptr(), ws_bytes, torch.cuda.current_stream(q.device).cuda_stream)
    _native.check(rc, "mt_gqa_attn_decode_dev")
    return out


@gqa_attn_decode_dev.register_fake
def _gqa_attn_decode_dev_fake(q, k_cache, v_cache, length, scale):
    return q.new_empty(q.shape)


@gqa_attn_decode.register_fake
def _gqa_attn_decode_fake(q, k_cache, v_cache, length, scale):
    return q.new_empty(q.shape)


def _fwd_setup_context(ctx, inputs, output):
    q, k, v, scale = inputs
    out, lse = output
    ctx.save_for_backward(q, k, v, out, lse)
    ctx.scale = scale
    ctx.mark_non_differentiable(lse)
    ctx.set_materialize_grads(False)


def _fwd_backward(ctx, grad_out, _grad_lse):
    q, k, v, out, lse = ctx.saved_tensors
    dq, dk, dv = torch.ops.mega_trading_amd.gqa_attn_bwd(q, k, v, out, lse, grad_out, None, None, ctx.scale)
    return dq, dk, dv, None


def _rope_fwd_setup_context(ctx, inputs, output):
    _q, _k, v, cos, sin, scale = inputs
    out, lse, q_rot, k_rot = output
    ctx.save_for_backward(q_rot, k_rot, v, out, lse, cos, sin)
    ctx.scale = scale
    ctx.mark_non_differentiable(lse, q_rot, k_rot)
    ctx.set_materialize_grads(False)


def _rope_fwd_backward(ctx, grad_out, _grad_lse, _grad_q_rot, _grad_k_rot):
    q_rot, k_rot, v, out, lse, cos, sin = ctx.saved_tensors
    dq, dk, dv = torch.ops.mega_trading_amd.gqa_attn_bwd(q_rot, k_rot, v, out, lse, grad_out, cos, sin, ctx.scale)
    return dq, dk, dv, None, None, None


def _packed_setup_context(ctx, inputs, output):
    qkv, cos, sin, hq, hkv, scale = inputs
    out, lse, q_rot, k_rot = output
    ctx.save_for_backward(q_rot, k_rot, qkv, out, lse, cos, sin)
    ctx.hq, ctx.hkv, ctx.scale = hq, hkv, scale
    ctx.mark_non_differentiable(lse, q_rot, k_rot)
    ctx.set_materialize_grads(False)


def _packed_backward(ctx, grad_out, _grad_lse, _grad_q_rot, _grad_k_rot):
    if grad_out is None:
        return None, None, None, None, None, None
    q_rot, k_rot, qkv, out, lse, cos, sin = ctx.saved_tensors
    dqkv = torch.ops.mega_trading_amd.gqa_attn_bwd_packed(q_rot, k_rot, qkv, out, lse, grad_out, cos, sin, ctx.hq,
                                                          ctx.hkv, ctx.scale)
    return dqkv, None, None, None, None, None


torch.library.register_autograd("mega_trading_amd::gqa_attn_fwd", _fwd_backward, setup_context=_fwd_setup_context)
torch.library.register_autograd("mega_trading_amd::gqa_rope_attn_packed_fwd", _packed_backward,
                                setup_context=_packed_setup_context)
torch.library.register_autograd("mega_trading_amd::gqa_rope_attn_fwd", _rope_fwd_backward,
                                setup_context=_rope_fwd_setup_context)
