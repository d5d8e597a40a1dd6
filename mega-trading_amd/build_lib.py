"""Build libmt_attn.so (and the bench-only libmt_probe.so) in-tree for gfx950 with hipcc.

Run as ``python mega-trading_amd/build_lib.py`` or through
``__graft_entry__.build()``.  The libraries land next to this file so they
travel with the source tree (they are git-ignored, not installed anywhere).
libmt_probe.so holds a sustained-MFMA-rate probe that bench.py reports beside
the roofline; it is not part of the attention ABI.
"""

from __future__ import annotations

import os
import shutil
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
LIB_NAME = "libmt_attn.so"
LIB_PATH = os.path.join(HERE, LIB_NAME)
SOURCES = ["mt_attention.hip", "mt_ops.hip"]
PROBE_NAME = "libmt_probe.so"
PROBE_PATH = os.path.join(HERE, PROBE_NAME)
PROBE_SOURCES = ["mfma_probe.hip"]
HEADERS = ["mt_common.h", "attn_kernels.h", "lds_tile.h", "mt_abi.h", "ops_kernels.h"]
ARCH = "gfx950"


def hipcc() -> str:
    path = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not os.path.exists(path):
        raise RuntimeError("hipcc not found; the ROCm toolchain is required to build libmt_attn.so")
    return path


def compile_command(out: str = LIB_PATH, sources: list[str] | None = None) -> list[str]:
    return [
        hipcc(),
        f"--offload-arch={ARCH}",
        "-O3",
        "-std=c++17",
        "-fPIC",
        "-shared",
        # never let the compiler form packed-fp32 ALU ops (v_pk_{add,mul,fma}_f32)
        "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
        "-Wno-pass-failed",
        "-o", out,
        *[os.path.join(CSRC, s) for s in (SOURCES if sources is None else sources)],
    ]


def build(verbose: bool = False) -> str:
    """Compile both libraries (always; a stale build is never reused)."""
    _compile(PROBE_PATH, PROBE_SOURCES, verbose)
    return _compile(LIB_PATH, SOURCES, verbose)


def _compile(path: str, sources: list[str], verbose: bool) -> str:
    tmp = path + ".tmp"
    cmd = compile_command(tmp, sources)
    if verbose:
        print(" ".join(cmd), flush=True)
    proc = subprocess.run(cmd, capture_output=True, text=True)
    noise = "is not a recognized feature for this target"
    err = "\n".join(line for line in proc.stderr.splitlines() if noise not in line)
    if proc.returncode != 0:
        raise RuntimeError(f"hipcc failed ({proc.returncode}):\n{err}")
    if verbose and err.strip():
        print(err, file=sys.stderr)
    os.replace(tmp, path)
    return path


if __name__ == "__main__":
    print(build(verbose=True))
