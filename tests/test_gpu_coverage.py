"""GPU tests that every gradient row is written by the backward's task order.

The one-launch backward deals its dQ and dK/dV tasks to workgroups through a
host-computed longest-first order (a head of one kind, a proportional middle,
a tail of the other kind), rotated in blocks over the shader engines, and the
dK/dV tasks take 128 or 64 keys depending on the shape.  A task that no
workgroup ran would leave its rows unwritten, and the slice-wise oracle
comparisons elsewhere sample only some (batch, KV head) groups.  Here the
outputs are filled with NaN before each backward call through the C ABI and
must come back finite everywhere, equal to a second call into zero-filled
outputs, and (on a sample of rows) to the fp64 oracle, for shapes that
exercise each arrangement: 64- and 128-key dK/dV tasks, head splits with
partial sums, group sizes without the 4-head peel, D = 32 and the separate
D = 128 kernels, and the half-backward entry points.
"""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from oracle import attention_oracle as orc
from tests.gpu_cases import TOL_GRAD_REL, make_inputs, rel

pytestmark = pytest.mark.gpu

# (B, T, Hq, Hkv, D): 64-key tasks with a 1:1 dQ / dK/dV interleave (BASELINE
# config 2), 128-key tasks with a dK/dV head (config 3), R = 8 (head split 2),
# R = 3 and R = 1 (no peel), D = 32, D = 128, and a ragged T
SHAPES = [
    (16, 1024, 8, 2, 64),
    (4, 4096, 16, 4, 64),
    (2, 2048, 16, 2, 64),
    (3, 1000, 12, 4, 64),
    (2, 777, 8, 8, 64),
    (4, 2048, 8, 2, 32),
    (2, 1500, 16, 4, 128),
]


def _run(mta, shape, rope, fill, entry="mt_gqa_attn_bwd"):
    b, t, hq, hkv, d = shape
    native = mta._native
    lib = native.load()
    dev = torch.device("cuda:0")
    q, k, v, do = (x.to(dev) for x in make_inputs(b, t, hq, hkv, d, sigma=0.5, seed=t + hq + d))
    o = torch.empty_like(q)
    lse = torch.empty((b, hq, t), device=dev, dtype=torch.float32)
    cos = sin = q_rot = k_rot = None
    if rope:
        c, s = orc.rope_tables(t, d, 10_000.0)
        cos, sin = torch.from_numpy(c).to(dev), torch.from_numpy(s).to(dev)
        q_rot, k_rot = torch.empty_like(q), torch.empty_like(k)
    ptr = lambda x: None if x is None else x.data_ptr()  # noqa: E731
    stream = torch.cuda.current_stream(dev).cuda_stream
    scale = 1.0 / math.sqrt(d)
    print(f"case {shape} rope={rope} fill={fill} {entry}", flush=True)
    native.check(lib.mt_gqa_attn_fwd(q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(), lse.data_ptr(),
                                     ptr(q_rot), ptr(k_rot), b, hq, hkv, t, d, native.strides_array(q, k, v, o),
                                     scale, 0, ptr(cos), ptr(sin), stream), "mt_gqa_attn_fwd")
    qs, ks = (q_rot, k_rot) if rope else (q, k)
    dq, dk, dv = (torch.full_like(x, fill) for x in (q, k, v))
    ws_bytes = lib.mt_gqa_attn_bwd_workspace_size(b, hq, hkv, t, d)
    ws = torch.empty(ws_bytes, device=dev, dtype=torch.uint8)
    strides = native.strides_array(qs, ks, v, o, do, dq, dk, dv)
    args = (qs.data_ptr(), ks.data_ptr(), v.data_ptr(), o.data_ptr(), lse.data_ptr(), do.data_ptr(),
            dq.data_ptr(), dk.data_ptr(), dv.data_ptr(), ws.data_ptr(), ws_bytes,
            b, hq, hkv, t, d, strides, scale, 0, ptr(cos), ptr(sin), stream)
    if entry == "halves":
        # the half-backward entry points, dQ (with delta) first, on one stream
        native.check(lib.mt_gqa_attn_bwd_dq(*args), "mt_gqa_attn_bwd_dq")
        native.check(lib.mt_gqa_attn_bwd_dkv(*args), "mt_gqa_attn_bwd_dkv")
    else:
        native.check(lib.mt_gqa_attn_bwd(*args), "mt_gqa_attn_bwd")
    torch.cuda.synchronize()
    return (q, k, v, do, cos, sin), (dq, dk, dv)


@pytest.mark.parametrize("shape", SHAPES, ids=lambda s: "x".join(map(str, s)))
def test_every_gradient_row_is_written(mta, shape):
    rope = shape[4] != 32
    _, got = _run(mta, shape, rope, float("nan"))
    _, again = _run(mta, shape, rope, 0.0)
    for name, a, e in zip(("dq", "dk", "dv"), got, again):
        bad = (~torch.isfinite(a)).nonzero()
        assert bad.numel() == 0, f"{name}: {bad.shape[0]} entries not written, first at {bad[0].tolist()}"
        assert torch.equal(a, e), f"{name}: the two calls differ"


@pytest.mark.parametrize("shape", [SHAPES[0], SHAPES[3]], ids=lambda s: "x".join(map(str, s)))
def test_half_backward_entry_points_write_every_row(mta, shape):
    (q, k, v, do, cos, sin), got = _run(mta, shape, True, float("nan"), entry="halves")
    _, full = _run(mta, shape, True, 0.0)
    for name, a, e in zip(("dq", "dk", "dv"), got, full):
        assert torch.isfinite(a).all(), name
        assert torch.equal(a, e), f"{name}: the half entry points differ from the one-launch backward"


def test_sampled_rows_match_the_oracle(mta):
    # the last (batch, KV group) of BASELINE config 2's shape, the group the
    # slice-wise parity test does not sample, against the fp64 oracle
    b, t, hq, hkv, d = SHAPES[0]
    (q, k, v, do, cos, sin), (dq, dk, dv) = _run(mta, SHAPES[0], True, float("nan"))
    r = hq // hkv
    bi, g = b - 1, hkv - 1
    hs = slice(g * r, (g + 1) * r)
    f = lambda x: x.float().cpu().numpy()  # noqa: E731
    cs, sn = cos.cpu().numpy(), sin.cpu().numpy()
    edq, edk, edv = orc.rope_attention_backward(f(q[bi:bi + 1, hs]), f(k[bi:bi + 1, g:g + 1]), f(v[bi:bi + 1, g:g + 1]),
                                                f(do[bi:bi + 1, hs]), cs, sn, r)
    got = (f(dq[bi:bi + 1, hs]), f(dk[bi:bi + 1, g:g + 1]), f(dv[bi:bi + 1, g:g + 1]))
    for name, a, e in zip(("dq", "dk", "dv"), got, (edq, edk, edv)):
        err = rel(a, np.asarray(e))
        print(name, f"{err:.2e}")
        assert err <= TOL_GRAD_REL, name
