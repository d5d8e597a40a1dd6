"""Benchmark: causal GQA fwd+bwd on one MI355X, the reference's headline metric.

``python bench.py [--gpus 1] [--steps K] [--warmup W]`` prints ONE JSON line.

* step: one forward + backward of the fused-RoPE causal GQA op over one batch
  of BASELINE config 3 (B=4, T=4096, Hq=16, Hkv=4, D=64, bf16, RoPE theta 1e4,
  Q/K/V ~ N(0, 0.5^2), dO ~ N(0, 1)), inputs resident in HBM.
* value: TFLOP/s with the reference's FLOP convention extended to fwd+bwd,
  14 * B * Hq * D * T(T+1)/2 (scripts/benchmark_triton_attention.py:179-190
  gives the forward 4 * B * Hq * D * T(T+1)/2; backward adds 2.5x).
* roofline: the dominant kernel's (the one-launch backward's) algorithmic
  MFMA FLOPs per launch over its average duration in a second set of the
  headline's timed windows (the same steps right after them), from HIP
  events that the library attaches to each of its dispatches
  (mt_time_kernel_queue; the backward runs on the autograd engine's thread)
  on the launch stream; traffic is its HBM bytes per launch from the
  committed rocprofv3 counter summary.
* cpu_baseline: the reference's CPU attention path (torch SDPA, fp32, forward
  + autograd backward, model.py:228-235) on the host cores over a bounded
  sample of the same workload.
* secondary: BASELINE config 2 (T=1024) and config 4 (D=128) fwd+bwd TFLOP/s,
  the un-fused op, and
  train tokens/sec of the 8-layer decoder with the HIP
  attention in every layer against the same model on the reference's SDPA
  route (the "train tokens/sec" half of the metric).
* secondary.sdpa: ROCm PyTorch SDPA fwd+bwd (the reference's eager attention,
  model.py:228-235) on the C2-C4 inputs, with torch's own backend choice and
  each backend the trainer can force (trainer.py:977-1001), and the aten ops
  and GPU kernels that ran.  secondary.C5_train adds the attention-only route:
  the SDPA model with only its attention calls on the HIP op.
* secondary.C5_generate: KV-cached generation on the HIP kernels against the
  reference's per-token full recompute (model.py:134-147).
* ops: the decoder operators' HIP kernels (RMSNorm, SwiGLU gate, cross-entropy
  rows) at their config 5 shapes, in GB/s against the 8 TB/s HBM peak.
* mfma_ceiling: what this GPU sustains for back-to-back bf16 MFMA with random
  and with zero operands, and the shader clock it ran at (libmt_probe.so),
  measured right after the attention runs: under data-dependent MFMA load the
  board's power management lowers the clock well below the 2.4 GHz that the
  2516.6 TFLOP/s peak assumes.
"""

from __future__ import annotations

import argparse
import ctypes
import gc
import importlib
import json
import math
import os
import sys
import time

import torch

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

PEAK_BF16_TFLOPS = 2516.6  # MI355X dense bf16 MFMA: 256 CU x 4096 FLOP/clk x 2.4 GHz
METRIC = "causal GQA fwd+bwd TFLOP/s (% bf16 MFMA peak) at T=1k/4k; train tokens/sec"

# (B, T, Hq, Hkv, D)
C1 = (2, 256, 4, 2, 32)     # fp32, N(0, 1), no RoPE: the reference's CPU-plumbing config
C2 = (16, 1024, 8, 2, 64)
C3 = (4, 4096, 16, 4, 64)
C4 = (8, 2048, 32, 8, 128)

# algorithmic MFMA FLOPs per launch, in units of B * Hq * D * T(T+1)/2
# FLOPs per launch in units of B*Hq*D*T(T+1)/2.  "algorithmic" is the work the
# metric credits (forward 4, backward 10: the FlashAttention convention, 14 per
# fwd+bwd step); "executed" what the kernel actually issues: the backward
# computes S and dP twice, once for its dQ tasks and once for its dK/dV tasks.
KERNEL_FLOP_UNITS = {
    "attn_fwd_kernel": (4, 4),      # S = QK^T, O = PV
    # the backward (D <= 64): dQ tasks and dK/dV tasks in one launch
    "attn_bwd_kernel": (10, 14),
    # the same kernel launched with one kind of task only (a diagnostic: the
    # half-backward entry points); credited with what they execute
    "attn_bwd_kernel[dq]": (6, 6),   # S, dP recomputed; dQ = dS K
    "attn_bwd_kernel[dkv]": (8, 8),  # S, dP recomputed; dV = P^T dO, dK = dS^T Q
}


def pairs(t: int) -> int:
    return t * (t + 1) // 2


def fwd_bwd_flops(b, t, hq, d) -> float:
    return 14.0 * b * hq * d * pairs(t)


def make_inputs(cfg, device, seed=0):
    b, t, hq, hkv, d = cfg
    g = torch.Generator().manual_seed(seed)
    q = (torch.randn(b, hq, t, d, generator=g) * 0.5).to(torch.bfloat16)
    k = (torch.randn(b, hkv, t, d, generator=g) * 0.5).to(torch.bfloat16)
    v = (torch.randn(b, hkv, t, d, generator=g) * 0.5).to(torch.bfloat16)
    do = torch.randn(b, hq, t, d, generator=g).to(torch.bfloat16)
    return [x.to(device) for x in (q, k, v, do)]


def rope_tables(t, d, theta, device):
    """RotaryEmbedding buffers as model.py:279-284 builds them (fp32)."""
    pos = torch.arange(t, dtype=torch.float32)
    inv_freq = 1.0 / (theta ** (torch.arange(0, d, 2, dtype=torch.float32) / d))
    freqs = torch.outer(pos, inv_freq)
    return freqs.cos().to(device), freqs.sin().to(device)


REPEATS = 5           # timed windows per measurement; the median is reported
MIN_WARMUP = 25       # warm-up steps before the timed windows (the reference harness: 25)
PREHEAT_S = 0.5       # and at least this long of back-to-back steps


def time_op_steps(pkg, cfg, steps, warmup, rope=True, repeats=REPEATS, preheat_s=PREHEAT_S, kernel_events=False):
    """fwd+bwd steps through the public op, timed in steady state.

    `warmup` untimed steps, then one timed window of `steps` steps (the cold
    window: the clock right after warm-up), then more untimed steps until at
    least MIN_WARMUP steps and `preheat_s` seconds of back-to-back steps have
    run, then `repeats` timed windows of exactly `steps` steps each, every
    window bracketed by synchronisation and HIP events on the current stream.
    Returns ms per step: median, fastest and slowest window, the cold
    window, and the median window's wall-clock time per step.  kernel_events:
    then `repeats` more windows of the same steps with HIP events that the
    library attaches to each dispatch of the step's two main kernels (the
    forward and the backward launch; mt_time_kernel_queue, since the backward
    is launched from the autograd engine's thread), giving their average
    durations and those windows' median ms per step (the events add about
    2 % to a step, so the plain windows give `ms`)."""
    b, t, hq, hkv, d = cfg
    dev = torch.device("cuda:0")
    q, k, v, do = make_inputs(cfg, dev)
    q.requires_grad_(True)
    k.requires_grad_(True)
    v.requires_grad_(True)
    cos, sin = rope_tables(t, d, 10_000.0, dev)

    def step():
        if rope:
            out = pkg.rope_attention(q, k, v, cos, sin, repeats=hq // hkv)
        else:
            out = pkg.attention(q, k, v, repeats=hq // hkv)
        return torch.autograd.grad(out, (q, k, v), do)

    def window():
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        start.record()
        for _ in range(steps):
            step()
        end.record()
        torch.cuda.synchronize()
        return start.elapsed_time(end) / steps, (time.perf_counter() - t0) / steps * 1e3

    for _ in range(warmup):
        step()
    cold, _ = window()
    t0, n = time.perf_counter(), warmup + steps
    while n < MIN_WARMUP or time.perf_counter() - t0 < preheat_s:
        for _ in range(8):
            step()
        n += 8
        torch.cuda.synchronize()
    runs = sorted(window() for _ in range(repeats))
    med_ms, med_wall = runs[len(runs) // 2]
    res = {"ms": med_ms, "ms_min": runs[0][0], "ms_max": runs[-1][0], "ms_cold": cold, "wall_ms": med_wall,
           "repeats": repeats, "warmup_steps": n}
    if kernel_events:
        # the same windows again with events on each kernel dispatch (they add
        # about 2 % to a step, so `ms` comes from the plain windows above)
        lib = pkg._native.load()
        ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
              for _ in range(2 * steps * repeats)]
        for a, b_ in ev:  # materialise the events on this device
            a.record()
            b_.record()
        torch.cuda.synchronize()
        arr = ctypes.c_void_p * len(ev)
        pkg._native.check(lib.mt_time_kernel_queue(arr(*[a.cuda_event for a, _ in ev]),
                                                   arr(*[b_.cuda_event for _, b_ in ev]), len(ev)),
                          "mt_time_kernel_queue")
        inst = sorted(window() for _ in range(repeats))
        pkg._native.check(lib.mt_time_kernel_queue(None, None, 0), "mt_time_kernel_queue")
        res["ms_instrumented"] = inst[len(inst) // 2][0]
        res["fwd_kernel_ms"] = sum(a.elapsed_time(b_) for a, b_ in ev[0::2]) / (len(ev) // 2)
        res["bwd_kernel_ms"] = sum(a.elapsed_time(b_) for a, b_ in ev[1::2]) / (len(ev) // 2)
    return res


# The reference's own configs use other query-heads-per-KV-head ratios R:
# configs/default.yaml:33-34 (R = 1), configs/mac.yaml:33-34 (R = 3),
# configs/modal.yaml:33-34 (R = 7).  Measured at C3's B, T and D with the
# query-head count nearest 16 that R divides.
GROUP_SIZE_CASES = {"R1": (4, 4096, 16, 16, 64), "R2": (4, 4096, 16, 8, 64), "R3": (4, 4096, 12, 4, 64),
                    "R4": C3, "R7": (4, 4096, 14, 2, 64), "R8": (4, 4096, 16, 2, 64)}


def time_group_sizes(pkg, steps):
    """fwd+bwd TFLOP/s of the fused-RoPE op at each group size R (same FLOP
    convention; the FLOPs scale with Hq) and each one's ratio to R = 4, timed
    as the headline is (median of REPEATS windows after the preheat)."""
    out = {}
    for name, cfg in GROUP_SIZE_CASES.items():
        b, t, hq, hkv, d = cfg
        ms = time_op_steps(pkg, cfg, steps, 3, rope=True)["ms"]
        out[name] = {"Hq": hq, "Hkv": hkv, "ms": round(ms, 4), "tflops": round(fwd_bwd_flops(b, t, hq, d) / (ms * 1e-3) / 1e12, 1)}
    for name in out:
        out[name]["vs_R4"] = round(out[name]["tflops"] / out["R4"]["tflops"], 3)
    return out


def mfma_ceiling(iters=20000, repeats=3):
    """Sustained whole-GPU bf16 MFMA rate (random and zero operands) with the clock it ran at."""
    path = os.path.join(ROOT, "mega-trading_amd", "libmt_probe.so")
    if not os.path.exists(path):
        return None
    lib = ctypes.CDLL(path)
    fp = ctypes.POINTER(ctypes.c_float)
    lib.mt_probe_mfma.argtypes = [ctypes.c_int, ctypes.c_int, ctypes.c_void_p, fp, fp, fp]
    stream = torch.cuda.current_stream().cuda_stream
    torch.cuda.synchronize()

    def run(random_operands):
        ms, tf, mhz = ctypes.c_float(), ctypes.c_float(), ctypes.c_float()
        rc = lib.mt_probe_mfma(iters, random_operands, stream, ctypes.byref(ms), ctypes.byref(tf), ctypes.byref(mhz))
        if rc:
            raise RuntimeError(f"mt_probe_mfma failed with HIP error {rc}")
        return tf.value, mhz.value

    out = {}
    for name, rnd in (("random_operands", 1), ("zero_operands", 0)):
        run(rnd)  # warm-up
        res = sorted(run(rnd) for _ in range(repeats))
        tf, mhz = res[len(res) // 2]
        out[name] = {"tflops": round(tf, 1), "clock_mhz": round(mhz), "frac_of_peak": round(tf / PEAK_BF16_TFLOPS, 4)}
    return out


PEAK_HBM_GBPS = 8000.0  # MI355X HBM3E


def time_ops(pkg, iters=20):
    """The decoder operators' HIP kernels at their BASELINE config 5 shapes
    (rows = 32 x 1024 tokens): average time per launch (HIP events around
    `iters` back-to-back launches on the current stream) and algorithmic HBM
    bytes per launch over that time, against the 8 TB/s HBM peak."""
    native = pkg._native
    lib = native.load()
    dev = torch.device("cuda:0")
    sp = torch.cuda.current_stream(dev).cuda_stream
    rows, hid, inter, vocab = 32 * 1024, 512, 1408, 16384
    g = torch.Generator(device=dev).manual_seed(0)
    x = torch.randn(rows, hid, device=dev, generator=g)
    w = torch.ones(hid, device=dev)
    y, dx, dy = torch.empty_like(x), torch.empty_like(x), torch.randn(rows, hid, device=dev, generator=g)
    rstd = torch.empty(rows, device=dev)
    dw = torch.empty_like(w)
    ws_bytes = lib.mt_rms_norm_bwd_workspace_size(rows, hid)
    ws = torch.empty(ws_bytes, device=dev, dtype=torch.uint8)
    gate = torch.randn(rows, inter, device=dev, generator=g).to(torch.bfloat16)
    up, dout = torch.randn_like(gate), torch.randn_like(gate)
    out, dgate, dup = torch.empty_like(gate), torch.empty_like(gate), torch.empty_like(gate)
    logits = torch.randn(rows, vocab, device=dev, generator=g).to(torch.bfloat16)
    labels = torch.randint(0, vocab, (rows,), device=dev, generator=g)
    n_valid = torch.tensor(rows, device=dev, dtype=torch.int64)
    loss_rows = torch.empty(rows, device=dev)
    f32, bf16 = native.DTYPE_FP32, native.DTYPE_BF16
    mb = lambda n_elems, elem: n_elems * elem  # noqa: E731
    # stand-alone RoPE of one C5 layer's q [32, 8, 1024, 64] and k [32, 2, 1024, 64] in the
    # projection layout ([B, T, H, D] memory, the model's views), tables [1024, 32] fp32
    hq, hkv, hd, tt = 8, 2, 64, 1024
    rq = torch.randn(32, tt, hq, hd, device=dev, generator=g).to(torch.bfloat16).transpose(1, 2)
    rk = torch.randn(32, tt, hkv, hd, device=dev, generator=g).to(torch.bfloat16).transpose(1, 2)
    rqo, rko = torch.empty_like(rq), torch.empty_like(rk)
    rcos = torch.randn(tt, hd // 2, device=dev, generator=g)
    rsin = torch.randn(tt, hd // 2, device=dev, generator=g)
    rst = (ctypes.c_int64 * 16)(*rq.stride(), *rqo.stride(), *rk.stride(), *rko.stride())
    cases = {
        "rms_norm_fwd (fp32 32768x512)": (
            lambda: lib.mt_rms_norm_fwd(x.data_ptr(), hid, w.data_ptr(), y.data_ptr(), rstd.data_ptr(), rows, hid,
                                        1e-5, f32, f32, sp),
            2 * mb(rows * hid, 4) + mb(rows, 4)),
        "rms_norm_bwd (fp32 32768x512, + dW column sum)": (
            lambda: lib.mt_rms_norm_bwd(x.data_ptr(), w.data_ptr(), rstd.data_ptr(), dy.data_ptr(), dx.data_ptr(),
                                        dw.data_ptr(), ws.data_ptr(), ws_bytes, rows, hid, f32, f32, sp),
            3 * mb(rows * hid, 4) + mb(rows, 4)),
        "swiglu_fwd (bf16 32768x1408)": (
            lambda: lib.mt_swiglu_fwd(gate.data_ptr(), up.data_ptr(), out.data_ptr(), gate.numel(), bf16, sp),
            3 * mb(gate.numel(), 2)),
        "swiglu_bwd (bf16 32768x1408)": (
            lambda: lib.mt_swiglu_bwd(gate.data_ptr(), up.data_ptr(), dout.data_ptr(), dgate.data_ptr(),
                                      dup.data_ptr(), gate.numel(), bf16, sp),
            5 * mb(gate.numel(), 2)),
        "apply_rope (bf16 q 32x8x1024x64 + k 32x2x1024x64)": (
            lambda: lib.mt_apply_rope(rq.data_ptr(), rk.data_ptr(), rqo.data_ptr(), rko.data_ptr(), 32, hq, hkv, tt,
                                      hd, rst, rcos.data_ptr(), rsin.data_ptr(), hd // 2, tt, 0, bf16, sp),
            2 * mb(rq.numel() + rk.numel(), 2) + 2 * mb(rcos.numel(), 4)),
        "cross_entropy_rows (bf16 32768x16384, grad in place)": (
            lambda: lib.mt_cross_entropy_rows(logits.data_ptr(), vocab, labels.data_ptr(), rows, vocab,
                                              n_valid.data_ptr(), -100, loss_rows.data_ptr(), 1, bf16, sp),
            2 * mb(rows * vocab, 2) + mb(rows, 12)),
    }
    res = {}
    for name, (fn, nbytes) in cases.items():
        for _ in range(3):
            native.check(fn(), name)
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(iters):
            native.check(fn(), name)
        e1.record()
        torch.cuda.synchronize()
        us = e0.elapsed_time(e1) / iters * 1e3
        gbps = nbytes / (us * 1e-6) / 1e9
        res[name] = {"us": round(us, 1), "bytes": int(nbytes), "GBps": round(gbps, 1),
                     "frac_hbm_peak": round(gbps / PEAK_HBM_GBPS, 3)}
    return res


DECODE_SHAPE = (32, 8, 2, 64, 1024)  # C5 generation: rollouts, Hq, Hkv, D, cache capacity (block_size)


DECODE_CASES = ((1024, 544), (1024, 1024), (512, 288), (512, 512))  # (cache capacity, length)


def time_decode(pkg, cases=DECODE_CASES, iters=50):
    """One decode step's attention kernels at the config 5 generation shape
    (32 rollouts, Hq 8, Hkv 2, D 64, bf16 cache of `capacity` positions:
    1024 = the config's block_size, and 512 for a shorter window), through the
    C ABI with preallocated buffers, the length read from device memory as the
    recorded decode step does: the attention (mt_gqa_attn_decode_dev: the
    split + combine pair for a 1024-position cache, the fused one-launch
    kernel for at most 512) and the RoPE / cache-append kernel, each timed
    over `iters` back-to-back launches with HIP events.  Algorithmic bytes:
    the attention reads the group's q and L cached K and V rows once and
    writes O; the split + combine pair also writes and reads one fp32 partial
    (o, m, l) per head and 64-key split; the append reads the fp32 q / k / v
    projections and writes q_rot and one K and one V cache row."""
    native = pkg._native
    lib = native.load()
    dev = torch.device("cuda:0")
    sp = torch.cuda.current_stream(dev).cuda_stream
    b, hq, hkv, d, _ = DECODE_SHAPE
    scale = 1.0 / math.sqrt(d)
    res = {}

    def timed(fn, n):
        for _ in range(3):
            fn()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(n):
            fn()
        e1.record()
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) / n * 1e3

    for cap, L in cases:
        g = torch.Generator(device=dev).manual_seed(0)
        kc = (torch.randn(b, hkv, cap, d, device=dev, generator=g) * 0.5).to(torch.bfloat16)
        vc = (torch.randn(b, hkv, cap, d, device=dev, generator=g) * 0.5).to(torch.bfloat16)
        q = (torch.randn(b, hq, 1, d, device=dev, generator=g) * 0.5).to(torch.bfloat16)
        out = torch.empty_like(q)
        ws_bytes = lib.mt_gqa_attn_decode_workspace_size(b, hq, cap, d)
        ws = torch.empty(ws_bytes, device=dev, dtype=torch.uint8)
        st = native.strides_array(q, kc, vc, out)
        length = torch.full((1,), L, device=dev, dtype=torch.int32)
        # fp32 projections of the new token (generation runs the fp32 model), RoPE tables [cap, D/2]
        xq = torch.randn(b, hq, 1, d, device=dev, generator=g)
        xk = torch.randn(b, hkv, 1, d, device=dev, generator=g)
        xv = torch.randn(b, hkv, 1, d, device=dev, generator=g)
        cos, sin = rope_tables(cap, d, 10_000.0, dev)
        q_rot = torch.empty_like(q)
        ins = (ctypes.c_int64 * 6)(xq.stride(0), xq.stride(1), xk.stride(0), xk.stride(1), xv.stride(0), xv.stride(1))
        cst = (ctypes.c_int64 * 6)(*kc.stride()[:3], *vc.stride()[:3])
        fused = (cap + 63) // 64 <= 8  # the library's rule: at most 8 splits of 64 keys in one launch
        ns = (L + 63) // 64
        attn = lambda: native.check(lib.mt_gqa_attn_decode_dev(  # noqa: E731
            q.data_ptr(), kc.data_ptr(), vc.data_ptr(), out.data_ptr(), b, hq, hkv, cap, length.data_ptr(), d, st,
            scale, native.DTYPE_BF16, ws.data_ptr(), ws_bytes, sp), "mt_gqa_attn_decode_dev")
        append = lambda: native.check(lib.mt_decode_rope_append(  # noqa: E731
            xq.data_ptr(), xk.data_ptr(), xv.data_ptr(), ins, cos.data_ptr(), sin.data_ptr(), cap, L - 1, None,
            q_rot.data_ptr(), kc.data_ptr(), vc.data_ptr(), cst, cap, b, hq, hkv, d, native.DTYPE_FP32,
            native.DTYPE_BF16, sp), "mt_decode_rope_append")
        attn_bytes = 2 * b * hkv * L * d * 2 + 2 * b * hq * d * 2
        if not fused:
            attn_bytes += 2 * b * hq * ns * (d + 2) * 4
        us = timed(attn, iters)
        us_app = timed(append, iters)
        app_bytes = b * (hq + 2 * hkv) * d * 4 + b * (hq + 2 * hkv) * d * 2 + d * 4
        res[f"cap{cap}_L{L}"] = {
            "attention_kernels": "attn_decode_fused_kernel" if fused else "attn_decode_split_kernel + attn_decode_combine_kernel",
            "attention_us": round(us, 2), "attention_bytes": attn_bytes,
            "attention_GBps": round(attn_bytes / (us * 1e-6) / 1e9, 1),
            "rope_append_us": round(us_app, 2), "rope_append_bytes": app_bytes}
    res["shape"] = "B=32 Hq=8 Hkv=2 D=64 bf16 cache of `cap` positions, length from device memory"
    return res


def time_kernels(pkg, cfg, iters, fp32=False):
    """Average duration of each main kernel (HIP events the library records
    around it on its launch stream, one pair per launch) and of each whole
    stage: the forward stage adds the K-RoPE pass, the backward stage the
    delta prep pass (and the partial-sum combine pass when the dK/dV heads
    are split).  The backward kernel is also timed with only its dQ tasks
    and only its dK/dV tasks (the library's two half-backward entry points),
    as a diagnostic of how the two kinds share the launch.  fp32: BASELINE
    config 1's form -- fp32 N(0, 1) inputs without RoPE, on the fp32 kernels."""
    native = pkg._native
    lib = native.load()
    b, t, hq, hkv, d = cfg
    dev = torch.device("cuda:0")
    if fp32:
        g = torch.Generator().manual_seed(0)
        q, k, v, do = (torch.randn(*shape, generator=g).to(dev)
                       for shape in ((b, hq, t, d), (b, hkv, t, d), (b, hkv, t, d), (b, hq, t, d)))
        cos = sin = None
    else:
        q, k, v, do = make_inputs(cfg, dev)
        cos, sin = rope_tables(t, d, 10_000.0, dev)
    dtype_code = native.DTYPE_FP32 if fp32 else native.DTYPE_BF16
    ptr = lambda x: None if x is None else x.data_ptr()  # noqa: E731
    o = torch.empty_like(q)
    lse = torch.empty((b, hq, t), device=dev, dtype=torch.float32)
    q_rot, k_rot = torch.empty_like(q), torch.empty_like(k)
    dq, dk, dv = torch.empty_like(q), torch.empty_like(k), torch.empty_like(v)
    ws_bytes = lib.mt_gqa_attn_bwd_workspace_size_dtype(b, hq, hkv, t, d, dtype_code)
    ws = torch.empty(ws_bytes, device=dev, dtype=torch.uint8)
    s_fwd = native.strides_array(q, k, v, o)
    s_bwd = native.strides_array(q_rot, k_rot, v, o, do, dq, dk, dv)
    stream = torch.cuda.current_stream(dev)
    sp = stream.cuda_stream
    scale = 1.0 / math.sqrt(d)

    # with RoPE the backward takes the forward's rotated Q and K
    qb, kb = (q, k) if cos is None else (q_rot, k_rot)

    def fwd():
        native.check(lib.mt_gqa_attn_fwd(q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(), lse.data_ptr(),
                                         q_rot.data_ptr(), k_rot.data_ptr(),
                                         b, hq, hkv, t, d, s_fwd, scale, dtype_code, ptr(cos), ptr(sin), sp), "fwd")

    def bwd(fn):
        native.check(fn(qb.data_ptr(), kb.data_ptr(), v.data_ptr(), o.data_ptr(), lse.data_ptr(), do.data_ptr(),
                        dq.data_ptr(), dk.data_ptr(), dv.data_ptr(), ws.data_ptr(), ws_bytes,
                        b, hq, hkv, t, d, s_bwd, scale, dtype_code, ptr(cos), ptr(sin), sp), "bwd")

    stages = [("attn_fwd_kernel", fwd), ("attn_bwd_kernel", lambda: bwd(lib.mt_gqa_attn_bwd)),
              ("attn_bwd_kernel[dq]", lambda: bwd(lib.mt_gqa_attn_bwd_dq)),
              ("attn_bwd_kernel[dkv]", lambda: bwd(lib.mt_gqa_attn_bwd_dkv))]
    for _ in range(3):
        for _, fn in stages:
            fn()
    torch.cuda.synchronize()
    out = {}
    for name, fn in stages:
        # the main kernel alone: a HIP event pair per launch, recorded by the
        # library on the launch stream right around that kernel
        pairs_ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(iters)]
        for a, b_ in pairs_ev:  # materialise the events on this device
            a.record(stream)
            b_.record(stream)
        torch.cuda.synchronize()
        for a, b_ in pairs_ev:
            native.check(lib.mt_time_next_kernel(ctypes.c_void_p(a.cuda_event), ctypes.c_void_p(b_.cuda_event)),
                         "mt_time_next_kernel")
            fn()
        torch.cuda.synchronize()
        ms = sum(a.elapsed_time(b_) for a, b_ in pairs_ev) / iters
        # the whole stage (with its helper pass) launched `iters` times back to back
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        for _ in range(iters):
            fn()
        e1.record(stream)
        torch.cuda.synchronize()
        stage_ms = e0.elapsed_time(e1) / iters
        alg, exe = (u * b * hq * d * pairs(t) for u in KERNEL_FLOP_UNITS[name])
        out[name] = {"ms": ms, "tflops": alg / (ms * 1e-3) / 1e12, "algorithmic_flop": alg,
                     "executed_tflops": exe / (ms * 1e-3) / 1e12, "stage_ms": stage_ms}
    return out


TRAFFIC_FILE = os.path.join(ROOT, "profiles", "hbm_traffic_C3.txt")


def hbm_traffic(kernel):
    """HBM bytes per launch of `kernel` at C3 (FETCH_SIZE + WRITE_SIZE, each
    scaled by the copy-kernel calibration), from the committed rocprofv3
    counter summary; None when the summary has no line for it."""
    try:
        lines = open(TRAFFIC_FILE).read().splitlines()
    except OSError:
        return None
    for line in lines:
        fields = dict(f.split("=", 1) for f in line.split() if "=" in f)
        if fields.get("kernel") == kernel and "traffic_bytes" in fields:
            return int(fields["traffic_bytes"])
    return None


def lscpu_fields() -> dict:
    """lscpu's "key: value" lines (first occurrence of each key); {} when lscpu is unavailable."""
    import subprocess

    fields = {}
    try:
        out = subprocess.run(["lscpu"], capture_output=True, text=True, timeout=10).stdout
    except (OSError, subprocess.SubprocessError):
        return fields
    for line in out.splitlines():
        if ":" in line:
            key, val = line.split(":", 1)
            fields.setdefault(key.strip(), val.strip())
    return fields


def cpu_model_name(fields=None) -> str:
    """The host CPU's "Model name" line as lscpu prints it (/proc/cpuinfo's
    "model name" when lscpu is unavailable)."""
    fields = lscpu_fields() if fields is None else fields
    if "Model name" in fields:
        # a virtualised host may report only the product family: add lscpu's
        # family / model / stepping numbers, which identify the part
        ids = [f"{k.lower()} {fields[k]}" for k in ("CPU family", "Model", "Stepping") if k in fields]
        return fields["Model name"] + (f" ({', '.join(ids)})" if ids else "")
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return ""


def cpu_quota() -> int | None:
    """CPUs this process's cgroup may use (cgroup v2 cpu.max), None when unlimited or unknown."""
    try:
        quota, period = open("/sys/fs/cgroup/cpu.max").read().split()[:2]
        if quota != "max":
            return max(1, int(int(quota) // int(period)))
    except (OSError, ValueError):
        pass
    return None


def cpu_threads(fields):
    """Threads for the CPU baseline: the host's physical cores (lscpu sockets x
    cores per socket), capped by the CPUs this process may run on (its
    affinity mask and cgroup quota).  Returns (threads, description)."""
    try:
        physical = int(fields["Socket(s)"]) * int(fields["Core(s) per socket"])
    except (KeyError, ValueError):
        physical = os.cpu_count() or 1
    allowed = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else (os.cpu_count() or 1)
    quota = cpu_quota()
    threads = max(1, min(physical, allowed, quota or allowed))
    topo = ", ".join(f"{k}: {fields[k]}" for k in ("Socket(s)", "Core(s) per socket", "Thread(s) per core", "CPU(s)")
                     if k in fields)
    desc = (f"lscpu {topo}; physical cores {physical}; CPUs this process may use: affinity {allowed}, "
            f"cgroup quota {quota if quota else 'none'}; threads used {threads}")
    return threads, desc


def cpu_baseline(cfg):
    """Reference CPU attention (torch SDPA fp32 fwd + autograd bwd) on one batch
    element of the workload, 1 warm-up + 3 timed repeats, median, on the
    host's physical cores (those this process may use)."""
    from oracle.sdpa_cpu import sdpa_forward_backward

    b, t, hq, hkv, d = cfg
    fields = lscpu_fields()
    threads, topo = cpu_threads(fields)
    torch.set_num_threads(threads)
    sample = (1, t, hq, hkv, d)
    q, k, v, do = (x.float() for x in make_inputs(sample, "cpu"))
    times = []
    for rep in range(4):
        t0 = time.perf_counter()
        sdpa_forward_backward(q, k, v, do, repeats=hq // hkv)
        if rep:
            times.append(time.perf_counter() - t0)
    times.sort()
    med = times[len(times) // 2]
    model = cpu_model_name(fields)
    return {
        "value": fwd_bwd_flops(1, t, hq, d) / med / 1e12,
        "unit": "TFLOP/s",
        "cores": torch.get_num_threads(),
        "kind": "reference",
        "sample": f"torch SDPA fp32 fwd+bwd (reference eager path, model.py:228-235) on 1 of {b} batch elements "
                  f"of the workload (B=1,T={t},Hq={hq},Hkv={hkv},D={d}), median of 3 after 1 warm-up: "
                  f"{med * 1e3:.1f} ms; host '{model}', {topo}, os.cpu_count()={os.cpu_count()}",
    }


SDPA_BACKEND_OPS = {
    "aten::_scaled_dot_product_flash_attention": "flash",
    "aten::_scaled_dot_product_efficient_attention": "efficient",
    "aten::_scaled_dot_product_attention_math": "math",
    "aten::_scaled_dot_product_cudnn_attention": "cudnn",
}


def sdpa_kernels_used(fn):
    """Run ``fn`` once under torch.profiler and report which SDPA implementation
    ran: the aten SDPA entry points dispatched (their names fix the backend)
    and the GPU kernels whose names mark them as attention kernels."""
    from torch.autograd import DeviceType
    from torch.profiler import ProfilerActivity, profile

    torch.cuda.synchronize()
    ops, kernels = set(), set()
    try:
        with profile(activities=[ProfilerActivity.CPU, ProfilerActivity.CUDA]) as prof:
            fn()
            torch.cuda.synchronize()
        events = prof.events()
    except RuntimeError as exc:  # profiler unavailable: report that instead of guessing
        return {"backend": None, "aten_ops": [], "gpu_kernels": [], "error": str(exc)[:200]}
    for e in events:
        name = e.name
        if name.startswith(("aten::_scaled_dot_product", "aten::_flash_attention", "aten::_efficient_attention")):
            ops.add(name)
        elif e.device_type == DeviceType.CUDA and any(s in name.lower() for s in ("attn", "attention", "fmha", "flash")):
            kernels.add(name[:160])
    backends = sorted({SDPA_BACKEND_OPS[o] for o in ops if o in SDPA_BACKEND_OPS})
    return {"backend": "+".join(backends) if backends else None, "aten_ops": sorted(ops), "gpu_kernels": sorted(kernels)}


def time_sdpa_steps(cfg, steps, warmup, backend="auto"):
    """ROCm PyTorch SDPA fwd+bwd (the reference's eager attention, model.py:228-235)
    on the inputs of time_op_steps: Q and K rotated once beforehand as the
    reference's RotaryEmbedding does (bf16 tables, model.py:290-294), then
    ``F.scaled_dot_product_attention(is_causal=True, enable_gqa=...)`` forward
    plus autograd into (q, k, v), under the trainer's backend context.
    Returns (ms per step by HIP events, kernels used)."""
    import torch.nn.functional as F

    pkg = importlib.import_module("mega-trading_amd")
    wl = pkg.workload
    b, t, hq, hkv, d = cfg
    dev = torch.device("cuda:0")
    q, k, v, do = make_inputs(cfg, dev)
    cos, sin = rope_tables(t, d, 10_000.0, dev)
    c16, s16 = cos.to(q.dtype), sin.to(q.dtype)
    q = pkg.model.rotate(q, c16, s16).detach().requires_grad_(True)
    k = pkg.model.rotate(k, c16, s16).detach().requires_grad_(True)
    v = v.detach().requires_grad_(True)

    def step():
        out = F.scaled_dot_product_attention(q, k, v, is_causal=True, enable_gqa=hq != hkv)
        return torch.autograd.grad(out, (q, k, v), do)

    with wl.attention_kernel_context(backend, dev):
        for _ in range(warmup):
            step()
        torch.cuda.synchronize()
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        start.record()
        for _ in range(steps):
            step()
        end.record()
        torch.cuda.synchronize()
        used = sdpa_kernels_used(step)
    return start.elapsed_time(end) / steps, used


def sdpa_comparators(pkg, configs, steps):
    """ROCm SDPA fwd+bwd at each named config: torch's own choice ("auto", what
    the reference's eager route runs) and every backend the trainer can force
    that accepts the call, each with the kernels that actually ran, beside the
    HIP op's time on the same inputs."""
    out = {}
    for name, cfg in configs.items():
        b, t, hq, hkv, d = cfg
        flops = fwd_bwd_flops(b, t, hq, d)
        row = {}
        for backend in ("auto", "flash", "efficient", "math"):
            try:
                ms, used = time_sdpa_steps(cfg, max(3, steps), 2, backend)
            except RuntimeError as exc:
                row[backend] = {"error": str(exc).splitlines()[0][:160]}
                torch.cuda.synchronize()
                continue
            row[backend] = {"ms": round(ms, 4), "tflops": round(flops / (ms * 1e-3) / 1e12, 2), **used}
            torch.cuda.empty_cache()
        out[name] = row
    return out


def sdpa_backends_usable(d=64, repeats=4):
    """Which forced SDPA backends accept a causal GQA bf16 call of head dim d on this GPU."""
    from torch.nn.attention import SDPBackend, sdpa_kernel
    import torch.nn.functional as F

    q = torch.randn(1, 2 * repeats, 128, d, device="cuda", dtype=torch.bfloat16)
    k = torch.randn(1, 2, 128, d, device="cuda", dtype=torch.bfloat16)
    ok = []
    for name, be in (("flash", SDPBackend.FLASH_ATTENTION), ("efficient", SDPBackend.EFFICIENT_ATTENTION),
                     ("math", SDPBackend.MATH)):
        try:
            with sdpa_kernel(be):
                F.scaled_dot_product_attention(q, k, k, is_causal=True, enable_gqa=True)
            ok.append(name)
        except RuntimeError:
            pass
    torch.cuda.synchronize()
    return ok


def train_tokens_per_second(pkg, steps, warmup):
    """the 8-layer decoder train step on the same seeded
    weights and Zipf batch through four routes:
      attention_only -- the SDPA route unchanged (torch norms, SwiGLU,
                projections, logits + nn.CrossEntropyLoss as trainer.py:309,
                336-338, default GEMM selection) except that every attention
                call (RoPE + SDPA) is the fused-RoPE HIP op: the attention's
                own contribution, the north-star figure;
      triton -- the reference's own Triton routing with the HIP kernels in its
                place (attention + SwiGLU gate + fused loss head; norms stay
                torch, model.py:166,176);
      hip    -- every HIP operator of this package (attention with fused RoPE,
                packed SwiGLU gate, RMSNorm) and its projections (q/k/v and
                w1/w3 each one GEMM, split-K fp32 weight gradients, tuned GEMMs);
      sdpa   -- the reference's eager route (SDPA + torch ops): the baseline.
    sdpa_backend records which SDPA implementation the baseline's attention
    calls ran (from a profiled step).
    """
    wl = pkg.workload
    ids, labels = wl.zipf_batch(wl.C5_BATCH, wl.C5_SEQ, wl.C5_MODEL["vocab_size"])
    out = {}
    for name, route in (("hip", "hip"), ("triton", "triton"), ("attention_only", "attention_only"), ("sdpa", "auto")):
        model = wl.build_model(route, seed=0, device="cuda")
        step = wl.TrainStep(model, ids, labels)
        tps, ms, loss = step.tokens_per_second(steps, warmup)
        out[name] = {"tokens_per_s": round(tps, 1), "ms_per_step": round(ms, 3), "loss": round(loss, 4),
                     "loss_form": step.loss_kind}
        if name == "sdpa":
            out["sdpa_backend"] = sdpa_kernels_used(step)
        del step, model
        torch.cuda.empty_cache()
    out["speedup_attention_only"] = round(out["attention_only"]["tokens_per_s"] / out["sdpa"]["tokens_per_s"], 4)
    out["speedup"] = round(out["hip"]["tokens_per_s"] / out["sdpa"]["tokens_per_s"], 4)
    out["speedup_reference_routing"] = round(out["triton"]["tokens_per_s"] / out["sdpa"]["tokens_per_s"], 4)
    out["sdpa_backends_usable"] = sdpa_backends_usable()
    out["workload"] = ("8-layer decoder d_model 512, Hq 8 Hkv 2 D 64, SwiGLU 1408, vocab 16384, B=32 T=1024 Zipf(1.1) "
                       f"tokens, bf16 autocast + fused AdamW; {steps} timed steps after {warmup} warm-up")
    return out


def _calibration_copy() -> None:
    """One 256 MiB device-to-device copy: the reference dispatch that scales the
    FETCH_SIZE / WRITE_SIZE counters of a profiling run to bytes."""
    src = torch.empty(256 << 20, dtype=torch.uint8, device="cuda:0").fill_(1)
    dst = torch.empty_like(src)
    torch.cuda.synchronize()
    dst.copy_(src)
    torch.cuda.synchronize()


def generate_tokens_per_second(pkg, rollouts=32, prompt=512, new_tokens=64):
    """Generation (the reference's TradingModel.generate, model.py:134-147, used by
    eval and backtest): `rollouts` sequences from a `prompt`-token Zipf context,
    `new_tokens` sampled tokens each (top-k 16), fp32 weights without autocast as
    the reference's eval runs it.  hip = KV-cached decode on the HIP kernels;
    reference = the full-context recompute loop on the SDPA route."""
    wl = pkg.workload
    ids, _ = wl.zipf_batch(rollouts, prompt, wl.C5_MODEL["vocab_size"], seed=3)
    ids = ids.cuda()
    out = {}
    for name, backend in (("hip", "hip"), ("reference", "auto")):
        model = wl.build_model(backend, seed=0, device="cuda").eval()
        torch.manual_seed(0)
        # warm-up at the timed length: one-time work (first launches, the
        # recording of the decode step) and the clock ramp after the host-side
        # set-up stay out of the timed call, for both routes alike
        model.generate(ids, max_new_tokens=new_tokens)
        torch.cuda.synchronize()
        gc.collect()
        gc.freeze()  # as TrainStep.tokens_per_second: no full collection inside the timed call
        try:
            t0 = time.perf_counter()
            model.generate(ids, max_new_tokens=new_tokens)
            torch.cuda.synchronize()
            dt = time.perf_counter() - t0
        finally:
            gc.unfreeze()
        out[name] = {"tokens_per_s": round(rollouts * new_tokens / dt, 1), "ms_per_token": round(dt / new_tokens * 1e3, 3)}
        del model
        torch.cuda.empty_cache()
    out["speedup"] = round(out["hip"]["tokens_per_s"] / out["reference"]["tokens_per_s"], 3)
    out["workload"] = (f"C5 decoder, {rollouts} rollouts x {new_tokens} new tokens after a {prompt}-token prompt, "
                       "top-k 16 sampling, fp32 weights (no autocast)")
    return out


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=100)
    ap.add_argument("--warmup", type=int, default=25)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--no-train", action="store_true", help="skip the config 5 train-step tokens/sec leg")
    ap.add_argument("--ops-only", action="store_true",
                    help="profiling driver: run only the decoder operators' kernels at config 5 shapes, then a "
                         "256 MiB device copy (counter calibration), and print their timings")
    ap.add_argument("--kernels-only", action="store_true",
                    help="profiling driver: run only the attention kernels of one config (--config, default C3) "
                         "stage by stage, then a 256 MiB device copy (the reference kernel for HBM-traffic counter "
                         "calibration), and print their timings")
    ap.add_argument("--decode-only", action="store_true",
                    help="profiling driver: run only the decode step's attention kernels at the config 5 generation "
                         "shape, then a 256 MiB device copy (counter calibration), and print their timings")
    ap.add_argument("--config", choices=("C1", "C2", "C3", "C4"), default="C3",
                    help="BASELINE config that --kernels-only runs")
    args = ap.parse_args(argv)
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (the path is single-GPU; got --gpus {args.gpus})", file=sys.stderr)
        return 2
    if not torch.cuda.is_available():
        print("bench.py needs an MI355X GPU", file=sys.stderr)
        return 2
    pkg = importlib.import_module("mega-trading_amd")
    pkg._native.load()

    if args.ops_only:
        ops_res = time_ops(pkg)
        _calibration_copy()
        print(json.dumps({"ops": ops_res, "copy_bytes_each_way": 256 << 20}), flush=True)
        return 0

    if args.decode_only:
        dec = time_decode(pkg)
        _calibration_copy()
        print(json.dumps({"decode": dec, "copy_bytes_each_way": 256 << 20}), flush=True)
        return 0

    if args.kernels_only:
        cfgs = {"C1": C1, "C2": C2, "C3": C3, "C4": C4}
        kern = time_kernels(pkg, cfgs[args.config], args.steps, fp32=args.config == "C1")
        _calibration_copy()
        print(json.dumps({"kernels": kern, "copy_bytes_each_way": 256 << 20}), flush=True)
        return 0

    b, t, hq, hkv, d = C3
    head = time_op_steps(pkg, C3, args.steps, args.warmup, rope=True, kernel_events=True)
    ms_event = head["ms"]
    flops = fwd_bwd_flops(b, t, hq, d)
    value = flops / (ms_event * 1e-3) / 1e12
    tflops = lambda ms: round(flops / (ms * 1e-3) / 1e12, 2)  # noqa: E731

    # the dominant kernel: the one-launch backward; its duration is averaged
    # over the headline's instrumented windows (the same steps, timed right
    # after the plain windows, with events on each of its dispatches)
    kern = time_kernels(pkg, C3, max(10, args.steps // 2))
    dom = "attn_bwd_kernel"
    unit_flop = b * hq * d * pairs(t)
    dom_ms = head["bwd_kernel_ms"]
    achieved = KERNEL_FLOP_UNITS[dom][0] * unit_flop / (dom_ms * 1e-3) / 1e12

    ms_c2 = time_op_steps(pkg, C2, args.steps, args.warmup, rope=True)["ms"]
    group_sizes = time_group_sizes(pkg, args.steps)
    ms_c3_plain = time_op_steps(pkg, C3, args.steps, 3, rope=False)["ms"]
    ms_c4 = time_op_steps(pkg, C4, max(10, args.steps // 2), 3, rope=True)["ms"]
    ceiling = mfma_ceiling()
    ops_line = time_ops(pkg)
    decode_line = time_decode(pkg)

    line = {
        "metric": METRIC,
        "value": round(value, 2),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_event, 4),
        "timing": {
            "method": f"median of {head['repeats']} windows of {args.steps} steps (HIP events, current stream), "
                      f"after {args.warmup} warm-up steps, one cold window and a preheat to at least "
                      f"{MIN_WARMUP} steps and {PREHEAT_S} s of back-to-back steps ({head['warmup_steps']} run)",
            "ms_median": round(head["ms"], 4), "ms_fastest": round(head["ms_min"], 4),
            "ms_slowest": round(head["ms_max"], 4), "tflops_slowest": tflops(head["ms_max"]),
            "ms_cold_window": round(head["ms_cold"], 4), "tflops_cold_window": tflops(head["ms_cold"]),
            "fwd_kernel_ms_in_windows": round(head["fwd_kernel_ms"], 4),
            "bwd_kernel_ms_in_windows": round(head["bwd_kernel_ms"], 4),
            "kernel_windows": f"{head['repeats']} further windows of the same steps with HIP events on each "
                              f"forward and backward dispatch (median {head['ms_instrumented']:.4f} ms per step)",
        },
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {
            "workload": "BASELINE config 3: causal GQA fwd+bwd, fused RoPE (theta 1e4), B=4 T=4096 Hq=16 Hkv=4 D=64 bf16",
            "B": b, "T": t, "Hq": hq, "Hkv": hkv, "D": d,
        },
        "pct_bf16_peak": round(100.0 * value / PEAK_BF16_TFLOPS, 2),
        "roofline": {
            "bound": "mfma",
            "kernel": dom,
            "achieved": round(achieved, 2),
            "peak": PEAK_BF16_TFLOPS,
            "unit": "TFLOP/s",
            "frac": round(achieved / PEAK_BF16_TFLOPS, 4),
            "kernel_ms": round(dom_ms, 4),
            "executed_tflops": round(KERNEL_FLOP_UNITS[dom][1] * unit_flop / (dom_ms * 1e-3) / 1e12, 2),
            "traffic": hbm_traffic(dom),
        },
        "kernels": {n: {"ms": round(x["ms"], 4), "tflops": round(x["tflops"], 1),
                        "executed_tflops": round(x["executed_tflops"], 1), "stage_ms": round(x["stage_ms"], 4)}
                    for n, x in kern.items()},
        "mfma_ceiling": ceiling,
        "ops": ops_line,
        "decode": decode_line,
        "secondary": {
            "C2_fwd_bwd_tflops": round(fwd_bwd_flops(*C2[:1], C2[1], C2[2], C2[4]) / (ms_c2 * 1e-3) / 1e12, 2),
            "C2_ms_per_step": round(ms_c2, 4),
            "C3_unfused_rope_free_tflops": round(flops / (ms_c3_plain * 1e-3) / 1e12, 2),
            "C4_fwd_bwd_tflops": round(fwd_bwd_flops(C4[0], C4[1], C4[2], C4[4]) / (ms_c4 * 1e-3) / 1e12, 2),
            "C4_ms_per_step": round(ms_c4, 4),
            "wall_ms_per_step": round(head["wall_ms"], 4),
            "group_sizes": group_sizes,
        },
    }
    sdpa = sdpa_comparators(pkg, {"C2": C2, "C3": C3, "C4": C4}, steps=max(5, args.steps // 5))
    line["secondary"]["sdpa"] = sdpa
    for name in ("C2", "C3", "C4"):
        line["secondary"][f"sdpa_{name}_ms"] = sdpa[name]["auto"].get("ms")
        line["secondary"][f"sdpa_{name}_backend"] = sdpa[name]["auto"].get("backend")
    line["secondary"]["hip_C2_C3_C4_ms"] = [round(ms_c2, 4), round(ms_event, 4), round(ms_c4, 4)]
    if not args.no_train:
        line["secondary"]["C5_train"] = train_tokens_per_second(pkg, steps=20, warmup=5)
        line["secondary"]["C5_generate"] = generate_tokens_per_second(pkg)
    if not args.no_cpu:
        line["cpu_baseline"] = cpu_baseline(C3)
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    raise SystemExit(main())
