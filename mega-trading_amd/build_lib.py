"""Build libmt_attn.so in-tree for gfx950 with hipcc.

Run as ``python mega-trading_amd/build_lib.py`` or through
``__graft_entry__.build()``.  The library lands next to this file so it
travels with the source tree (it is git-ignored, not installed anywhere).
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
SOURCES = ["mt_attention.hip"]
HEADERS = ["mt_common.h", "attn_kernels.h"]
ARCH = "gfx950"


def hipcc() -> str:
    path = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not os.path.exists(path):
        raise RuntimeError("hipcc not found; the ROCm toolchain is required to build libmt_attn.so")
    return path


def compile_command(out: str = LIB_PATH) -> list[str]:
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
        *[os.path.join(CSRC, s) for s in SOURCES],
    ]


def build(verbose: bool = False) -> str:
    """Compile the library (always; a stale build is never reused)."""
    tmp = LIB_PATH + ".tmp"
    cmd = compile_command(tmp)
    if verbose:
        print(" ".join(cmd), flush=True)
    proc = subprocess.run(cmd, capture_output=True, text=True)
    noise = "is not a recognized feature for this target"
    err = "\n".join(line for line in proc.stderr.splitlines() if noise not in line)
    if proc.returncode != 0:
        raise RuntimeError(f"hipcc failed ({proc.returncode}):\n{err}")
    if verbose and err.strip():
        print(err, file=sys.stderr)
    os.replace(tmp, LIB_PATH)
    return LIB_PATH


if __name__ == "__main__":
    print(build(verbose=True))
