"""Wait states in front of the LDS tile copies (CPU: compiles gfx950 assembly, runs nothing).

The tile copies (`global_load_lds_dword[x4]`) are issued from inline assembly
(`csrc/lds_tile.h`), which the compiler's hazard recognizer cannot look into,
so the blocks provide the wait states gfx950 needs themselves: one after the
scalar write of M0 the copy reads, and five between a vector instruction
writing an SGPR and a vector-memory instruction reading it (the scalar-base
copies read a scalar-copied base instead).  This test compiles the forward
and one-launch backward kernels to assembly with the library's flags and
checks every copy against both rules.
"""

from __future__ import annotations

import os
import re
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CSRC = os.path.join(ROOT, "mega-trading_amd", "csrc")

TU = """#include "attn_kernels.h"
template __global__ void mt::attn_fwd_kernel<mt::BF16, 64, true, true>(mt::AttnParams);
template __global__ void mt::attn_fwd_w8_kernel<mt::BF16, 64, true, true, 8, 128>(mt::AttnParams);
template __global__ void mt::attn_fwd_w8_kernel<mt::BF16, 128, true, true, 4, 64>(mt::AttnParams);
template __global__ void mt::attn_bwd_kernel<mt::BF16, 64, true, true, 128>(mt::AttnParams);
template __global__ void mt::attn_bwd_kernel<mt::BF16, 64, true, true, 64>(mt::AttnParams);
"""


def _hipcc():
    path = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    return path if os.path.exists(path) else None


def _instructions(asm: str) -> list[str]:
    out = []
    for line in asm.splitlines():
        line = line.split(";")[0].strip()
        if not line or line.startswith("."):
            continue
        out.append(line)
    return out


def _wait_states(between: list[str]) -> int:
    n = 0
    for ins in between:
        m = re.match(r"s_nop\s+(\d+)", ins)
        n += int(m.group(1)) + 1 if m else 1
    return n


def _writes(ins: str, regs: set[str]) -> bool:
    parts = ins.replace(",", " ").split()
    if len(parts) < 2 or parts[0].startswith(("s_cmp", "s_cbranch", "s_waitcnt", "s_nop", "global_", "ds_", "buffer_")):
        return False
    dst = parts[1]
    m = re.match(r"s\[(\d+):(\d+)\]", dst)
    written = {f"s{i}" for i in range(int(m.group(1)), int(m.group(2)) + 1)} if m else {dst}
    return bool(written & regs)


@pytest.fixture(scope="module")
def kernels_asm(tmp_path_factory):
    hipcc = _hipcc()
    if hipcc is None:
        pytest.skip("hipcc not available")
    d = tmp_path_factory.mktemp("asm")
    src = d / "tu.hip"
    src.write_text(TU)
    out = d / "tu.s"
    cmd = [hipcc, "--offload-arch=gfx950", "-O3", "-std=c++17", "--cuda-device-only", "-S",
           "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops", "-Wno-pass-failed",
           "-I", CSRC, str(src), "-o", str(out)]
    proc = subprocess.run(cmd, capture_output=True, text=True, timeout=900)
    assert proc.returncode == 0, proc.stderr[-2000:]
    return _instructions(out.read_text())


def test_every_lds_copy_has_its_wait_states(kernels_asm):
    ins = kernels_asm
    copies = [i for i, x in enumerate(ins) if x.startswith("global_load_lds")]
    assert len(copies) >= 20, "expected the kernels' LDS tile copies in the assembly"
    for i in copies:
        # M0, written by a scalar instruction, needs one wait state before the copy
        j = i - 1
        while j >= 0 and not ins[j].endswith(":") and not _writes(ins[j], {"m0"}):
            j -= 1
        assert j >= 0 and not ins[j].endswith(":"), f"no M0 write in the block before {ins[i]!r}"
        assert _wait_states(ins[j + 1:i]) >= 1, f"{ins[j]!r} -> {ins[i]!r} without a wait state"
        # a scalar base written by a vector instruction needs five
        m = re.match(r"global_load_lds_dword\S*\s+v\d+,\s*s\[(\d+):(\d+)\]", ins[i])
        if m:
            regs = {f"s{m.group(1)}", f"s{m.group(2)}"}
            j = i - 1
            while j >= 0 and i - j <= 8 and not ins[j].endswith(":") and not _writes(ins[j], regs):
                j -= 1
            if j >= 0 and i - j <= 8 and _writes(ins[j], regs) and ins[j].startswith("v_"):
                assert _wait_states(ins[j + 1:i]) >= 5, f"{ins[j]!r} -> {ins[i]!r}: fewer than 5 wait states"


def test_the_checks_catch_the_hazards():
    """The same checks on hand-written sequences: the unsafe forms fail them."""
    bad_m0 = ["s_add_i32 m0, s40, 0x4000", "global_load_lds_dwordx4 v[4:5], off"]
    assert _wait_states(bad_m0[1:1]) == 0
    ok_m0 = ["s_add_i32 m0, s40, 0x4000", "s_nop 0", "global_load_lds_dwordx4 v[4:5], off"]
    assert _wait_states(ok_m0[1:2]) == 1
    assert _writes("v_readfirstlane_b32 s10, v24", {"s10", "s11"})
    assert _writes("s_mov_b64 s[10:11], s[20:21]", {"s10", "s11"})
    assert not _writes("global_load_lds_dword v185, s[10:11]", {"s10", "s11"})
    assert _wait_states(["s_nop 4"]) == 5 and _wait_states(["v_mov_b32 v1, 0", "s_nop 2"]) == 4
