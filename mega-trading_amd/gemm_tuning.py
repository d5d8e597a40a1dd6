"""Pre-tuned hipBLASLt / rocBLAS solutions for this package's own GEMMs.

The decoder's library GEMMs (the grouped projections of ``projection.py``
and the loss head of ``ops.fused_linear_cross_entropy``) run at shapes that
hipBLASLt's default heuristic covers poorly on MI355X (e.g. the packed
(w1; w3) product of the C5 step: 138 us by default, 89 us with the best
solution).  PyTorch's TunableOp can replay a recorded choice per shape;
``tuned_gemms()`` turns that replay on around these calls only, with tuning
itself off, and restores the process-wide TunableOp state afterwards, so
GEMMs outside this package (and the baseline routes the benchmark compares
against) keep the default selection.

The recorded choices live in ``tuned/gemm_gfx950.csv``.  They were recorded
on an MI355X by running the "hip" route's C5 train step (two steps, bf16
autocast) and its eager cached decode (fp32, 32 rows, two tokens) with
``_state["tuning"] = True`` and ``torch.cuda.tunable.set_filename(<csv>)``,
so TunableOp tuned exactly the GEMMs opened inside ``tuned_gemms()`` and
wrote the file at process exit.  TunableOp checks
the file's validators (PyTorch, HIP, hipBLASLt and rocBLAS versions, GPU
architecture) and ignores a file that does not match, in which case the
default selection runs: the file only ever changes which library kernel
computes a product, never the product.  ``MT_GEMM_TUNING=0`` switches the
replay off; without a GPU the context does nothing.
"""

from __future__ import annotations

import contextlib
import os
import threading

import torch

__all__ = ["RESULTS_FILE", "tuned_gemms"]

RESULTS_FILE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "tuned", "gemm_gfx950.csv")

_lock = threading.Lock()
# loaded: None = not tried, True / False = results read or unusable;
# tuning: set by tune_gemms to record new solutions instead of replaying
_state = {"loaded": None, "tuning": False}


def _load() -> bool:
    with _lock:
        if _state["loaded"] is None:
            ok = False
            if (os.environ.get("MT_GEMM_TUNING", "1") != "0" and torch.version.hip and os.path.exists(RESULTS_FILE)
                    and torch.cuda.is_available()):
                try:
                    ok = bool(torch.cuda.tunable.read_file(RESULTS_FILE))
                except RuntimeError:
                    ok = False
            _state["loaded"] = ok
        return _state["loaded"]


@contextlib.contextmanager
def tuned_gemms():
    """Replay the recorded GEMM solutions inside the block (no tuning).

    The TunableOp switches are process-wide: a GEMM that another thread runs
    while a block is open may also replay a recorded solution, and one
    started as a block closes may not.  Either way only the choice of library
    kernel changes, never what is computed."""
    if not (_state["tuning"] or _load()):
        yield
        return
    tun = torch.cuda.tunable
    was_enabled, was_tuning = tun.is_enabled(), tun.tuning_is_enabled()
    tun.tuning_enable(_state["tuning"])
    tun.enable(True)
    try:
        yield
    finally:
        tun.enable(was_enabled)
        tun.tuning_enable(was_tuning)
