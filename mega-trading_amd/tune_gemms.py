"""Record the fastest library solution for every GEMM shape this package runs
in the BASELINE config 5 workloads, into ``tuned/gemm_gfx950.csv``.

Run on the target GPU from the repository root::

    python -m mega-trading_amd.tune_gemms [results.csv]

(the optional argument writes the results elsewhere, e.g. to copy them back
from a remote GPU host).  It runs the "hip" route's train step (bf16 autocast) and its eager cached
decode (fp32, as generate runs it) with PyTorch's TunableOp tuning switched
on inside ``gemm_tuning.tuned_gemms()`` only, so only this package's GEMMs
are tuned; TunableOp writes the results file when the process exits.
"""

from __future__ import annotations

import importlib
import os
import sys

import torch


def main() -> int:
    pkg = importlib.import_module("mega-trading_amd")
    gt = importlib.import_module("mega-trading_amd.gemm_tuning")
    wl = pkg.workload
    if not torch.cuda.is_available():
        print("tune_gemms needs a GPU", file=sys.stderr)
        return 1
    out = os.path.abspath(sys.argv[1]) if len(sys.argv) > 1 else gt.RESULTS_FILE
    os.makedirs(os.path.dirname(out), exist_ok=True)
    tun = torch.cuda.tunable
    tun.set_filename(out, False)
    tun.set_max_tuning_duration(30)
    tun.set_max_tuning_iterations(20)
    gt._state["tuning"] = True
    # the train step: projections (forward, dgrad) and the loss head at the C5 shape
    ids, labels = wl.zipf_batch(wl.C5_BATCH, wl.C5_SEQ, wl.C5_MODEL["vocab_size"])
    model = wl.build_model("hip", seed=0, device="cuda")
    step = wl.TrainStep(model, ids, labels)
    for i in range(2):
        print(f"train step {i}: loss {float(step()):.4f}", flush=True)
    # the cached decode (fp32, 32 rows): eager, so every shape is tuned outside graph capture
    model.eval()
    model.decode_graphs = False
    prompt, _ = wl.zipf_batch(32, 512, wl.C5_MODEL["vocab_size"], seed=3)
    model.generate(prompt.cuda(), max_new_tokens=2)
    torch.cuda.synchronize()
    print(f"tuned; results are written to {out} at exit", flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
