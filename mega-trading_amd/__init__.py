"""MI355X-native causal grouped-query attention for the mega-trading decoder.

Import with ``importlib.import_module("mega-trading_amd")`` (the directory
name carries a hyphen).  Public API:

* ``attention(query, key, value, *, repeats)`` -- drop-in for the reference's
  ``triton_attention`` (``src/mega_trading/kernels/triton_attention.py:12``).
* ``rope_attention(query, key, value, cos, sin, *, repeats)`` -- the same with
  the interleaved RoPE of ``model.py:223`` fused into the kernels.
* ``attention_forward(...)`` -- forward returning ``(output, logsumexp)``.
* ``decode_attention(query, key_cache, value_cache, length, *, repeats)`` --
  one new token against a KV cache (KV-cached ``generate``).
* ``rms_norm``, ``add_rms_norm``, ``swiglu_gate`` -- the decoder's
  memory-bound operators (``triton_ops.py:11-61``) on HIP kernels (``ops``).
* ``model`` -- the Llama-style order-flow decoder that calls them
  (``attention_backend="triton"`` or ``"hip"``), and ``workload`` -- its
  8-layer train step on synthetic Zipf tokens (the tokens/sec benchmark).
"""

from . import model, ops, workload
from .attention import SUPPORTED_HEAD_DIMS, attention, attention_forward, decode_attention, rope_attention
from .ops import add_rms_norm, rms_norm, swiglu_gate

__all__ = ["attention", "rope_attention", "attention_forward", "decode_attention", "SUPPORTED_HEAD_DIMS",
           "rms_norm", "add_rms_norm",
           "swiglu_gate", "model", "ops", "workload"]
