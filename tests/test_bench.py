"""CPU tests of bench.py's contract: the FLOP convention, the one-GPU rule,
and the committed counter summary it reads for roofline.traffic."""

from __future__ import annotations

import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)

import bench  # noqa: E402


def test_fwd_bwd_flops_match_the_published_convention():
    # 14 * B * Hq * D * T(T+1)/2 (scripts/benchmark_triton_attention.py:187-189 counts
    # the forward's 4 units; fwd+bwd = 3.5x that): C2 60.19 GFLOP, C3 481.15 GFLOP,
    # C4 962.54 GFLOP
    assert bench.fwd_bwd_flops(*bench.C2[:3], bench.C2[4]) == pytest.approx(60.19e9, rel=1e-4)
    assert bench.fwd_bwd_flops(*bench.C3[:3], bench.C3[4]) == pytest.approx(481.15e9, rel=1e-4)
    assert bench.fwd_bwd_flops(*bench.C4[:3], bench.C4[4]) == pytest.approx(962.54e9, rel=1e-4)


def test_kernel_units_credit_the_algorithmic_work():
    units = bench.KERNEL_FLOP_UNITS
    # forward 4 + backward 10 = the 14 units of a step; the backward executes 14
    # (S and dP once for its dQ tasks and once for its dK/dV tasks)
    assert units["attn_fwd_kernel"][0] + units["attn_bwd_kernel"][0] == 14
    assert units["attn_bwd_kernel"][1] == units["attn_bwd_kernel[dq]"][1] + units["attn_bwd_kernel[dkv]"][1]


def test_more_than_one_gpu_is_refused_with_a_message(capsys):
    assert bench.main(["--gpus", "2"]) == 2
    assert "one GPU" in capsys.readouterr().err


def test_roofline_traffic_comes_from_the_committed_summary():
    traffic = bench.hbm_traffic("attn_bwd_kernel")
    assert isinstance(traffic, int) and traffic > 136_000_000  # at least the algorithmic bytes
    assert bench.hbm_traffic("attn_fwd_kernel") > 118_000_000
    assert bench.hbm_traffic("no_such_kernel") is None


def test_cpu_model_name_is_reported():
    assert bench.cpu_model_name().strip()
