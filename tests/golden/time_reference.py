"""Calibrate the CPU baseline's stand-in: time the genuine reference
(bigptq.BRAGPTQ + binary.Binarization, imported from the reference tree)
and the test oracle (oracle/crb_oracle.py) on BASELINE configs[0] (768 x 768
fp32 layer, 16 x 512 tokens, crb, blocksize 128, hessian metric) on the same
cores, and record the ratio in tests/golden/reference_timing.json.

Run in the build container only (the reference does not exist on the GPU
box):  python tests/golden/time_reference.py /path/to/reference
``torch.cuda.synchronize`` is replaced by a no-op because bigptq.py:272
calls it unconditionally and this container has no GPU.  Only timings are
written.
"""
from __future__ import annotations

import contextlib
import io
import json
import os
import platform
import sys
import time

import torch

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.abspath(os.path.join(HERE, "..", ".."))
sys.path.insert(0, ROOT)

from crb_amd import synth  # noqa: E402
from oracle import crb_oracle as O  # noqa: E402


def cpu_model() -> str:
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return platform.processor() or platform.machine()


def main(ref_root: str, reps: int = 3):
    sys.path.insert(0, ref_root)
    torch.cuda.synchronize = lambda *a, **k: None
    import binary  # noqa: E402  (reference)
    import bigptq  # noqa: E402  (reference)
    threads = len(os.sched_getaffinity(0))
    torch.set_num_threads(threads)
    W, X = synth.cfg1(0)

    def run_reference():
        layer = torch.nn.Linear(768, 768, bias=False)
        layer.weight.data = W.clone()
        q = binary.Binarization(layer.weight, method="crb", groupsize=128)
        bq = bigptq.BRAGPTQ(layer, q, "hessian")
        for s in range(X.shape[0]):
            bq.add_batch(X[s:s + 1], None)
        with contextlib.redirect_stdout(io.StringIO()):
            return bq.fasterquant(blocksize=128, percdamp=0.01, partition=3,
                                  orders=(1, 1, 2))["error"]

    def run_oracle():
        H = torch.zeros(768, 768)
        n = 0
        for s in range(X.shape[0]):
            H, n = O.hessian_add_batch(H, n, X[s:s + 1])
        return O.fasterquant(W, H, method="crb")[2]

    res = {}
    for name, fn in (("reference", run_reference), ("oracle", run_oracle)):
        fn()                                        # warm-up
        ts = []
        for _ in range(reps):
            t0 = time.time()
            err = fn()
            ts.append(time.time() - t0)
        res[name] = {"s": min(ts), "all_s": ts, "error": err}
    out = {"config": "BASELINE configs[0]: 768x768 fp32, 16x512 tokens, crb, blocksize 128, "
                     "hessian metric, add_batch per sequence + fasterquant",
           "cpu": cpu_model(), "threads": threads, "torch": torch.__version__,
           "reference_s": res["reference"]["s"], "oracle_s": res["oracle"]["s"],
           "oracle_over_reference": res["oracle"]["s"] / res["reference"]["s"],
           "errors_equal": res["reference"]["error"] == res["oracle"]["error"],
           "runs": res}
    with open(os.path.join(HERE, "reference_timing.json"), "w") as f:
        json.dump(out, f, indent=1)
    print(json.dumps({k: v for k, v in out.items() if k != "runs"}))


if __name__ == "__main__":
    main(sys.argv[1] if len(sys.argv) > 1 else "/root/reference")
