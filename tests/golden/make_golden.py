"""Write golden input/output vectors by running the reference itself.

Run in the build container only (the reference does not exist on the GPU
box):  python tests/golden/make_golden.py /path/to/reference

What it pins (functions no closed form or library routine pins on its own):
  * structural_searching (utils/autosearch.py:28-83): the chosen salient
    count i*, the chosen split and every candidate error, on seeded blocks;
  * BRAGPTQ.add_batch + fasterquant (bigptq.py:37-291) end to end for crb,
    braq and crbog: the quantized weight and the returned error.
  * the three binarizers (binary.py:18-39, 577-687, 1544-1638) on seeded
    rows and masks, as a direct cross-check of the closed-form tests;
  * the technique flags of fasterquant off the default path on one small
    layer: RTN (disable_gptq, bigptq.py:149-162), partition=1 (one all-ones
    mask, bigptq.py:138-140), the magnitude metric (utils/structure.py:11-12),
    the crb_norefine / crb_symdamp / crb_symdamp_norefine methods
    (binary.py:2885-2890), and bf16 weights and activations.

Only inputs and outputs are written (tests/golden/*.npz, *.json); no
reference source is copied.  ``torch.cuda.synchronize`` is replaced by a
no-op because bigptq.py:272 calls it unconditionally and this container has
no GPU.
"""
from __future__ import annotations

import contextlib
import hashlib
import io
import json
import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.abspath(os.path.join(HERE, "..", "..")))

from crb_amd import synth  # noqa: E402


def sha(t: torch.Tensor) -> str:
    return hashlib.sha256(t.detach().contiguous().cpu().numpy().tobytes()).hexdigest()


def main(ref_root: str):
    sys.path.insert(0, ref_root)
    torch.cuda.synchronize = lambda *a, **k: None
    import binary  # noqa: E402  (reference)
    import bigptq  # noqa: E402  (reference)
    from utils.autosearch import structural_searching  # noqa: E402  (reference)

    torch.set_num_threads(8)
    meta = {"torch": torch.__version__, "numpy": np.__version__,
            "note": "reference pins numpy<2 (requirements.txt:34); vectors made with the numpy above"}
    arrays = {}
    summary = {"meta": meta, "search": [], "binarize": [], "fasterquant": []}

    # ---- binarizers on seeded rows / masks -----------------------------------
    for case, (R, nc, seed) in enumerate([(16, 128, 11), (33, 128, 12), (8, 40, 13)]):
        g = synth.gen(seed)
        x = torch.randn(R, nc, generator=g) * 0.02
        x[:, :5] *= 8
        m = torch.rand(R, nc, generator=g) < 0.6
        m[0] = False            # an empty row
        m[1] = True             # a full row
        m[2, :] = False
        m[2, 3] = True          # a single-element row
        x[3, :] = 0.013         # an all-equal row
        arrays[f"bin{case}_x"] = x.numpy()
        arrays[f"bin{case}_m"] = m.numpy()
        for order in (1, 2):
            outs = {
                "braq": binary.high_order_residual(x, m, order=order),
                "crb": binary.coupled_residual_binarization_stable_v7(x, m, order=order),
                "crb_norefine": binary.coupled_residual_binarization_stable_v7(
                    x, m, order=order, skip_refinement=True),
                "crb_symdamp": binary.coupled_residual_binarization_stable_v7(
                    x, m, order=order, symmetric_damp=True),
                "crb_symdamp_norefine": binary.coupled_residual_binarization_stable_v7(
                    x, m, order=order, symmetric_damp=True, skip_refinement=True),
                "crbog": binary.coupled_residual_binarization(x, m, order=order),
            }
            for k, v in outs.items():
                arrays[f"bin{case}_o{order}_{k}"] = v.numpy()
        summary["binarize"].append({"case": case, "R": R, "ncols": nc, "seed": seed})

    # ---- structural searching on seeded blocks -------------------------------
    search_cases = [
        # (R, seed, kind)
        (8, 21, "hessian"), (64, 22, "hessian"), (256, 23, "hessian"),
        (64, 24, "magnitude"), (512, 25, "hessian"),
    ]
    for case, (R, seed, kind) in enumerate(search_cases):
        g = synth.gen(seed)
        w = torch.randn(R, 128, generator=g) * 0.02
        w[:, torch.randperm(128, generator=g)[:6]] *= 6
        if kind == "hessian":
            d = torch.rand(128, generator=g) * 0.5 + 0.05
            T = w ** 2 / (d.reshape(1, -1)) ** 2
        else:
            T = w
        with contextlib.redirect_stdout(io.StringIO()):
            split, m3 = structural_searching(T, 50)
        arrays[f"search{case}_T"] = T.numpy()
        arrays[f"search{case}_m3"] = m3.numpy()
        summary["search"].append({
            "case": case, "R": R, "seed": seed, "kind": kind,
            "split": float(split), "split_hex": float(split).hex(),
            "n_salient_cols": int(m3[0].sum()),
        })

    # ---- fasterquant end to end ----------------------------------------------
    fq_cases = [
        # (name, R, C, nseq, seqlen, seed, methods)
        ("small_a", 64, 256, 4, 64, 31, ("crb", "braq", "crbog")),
        ("small_b", 96, 384, 3, 80, 32, ("crb", "braq")),
        ("cfg1", 768, 768, 16, 512, 0, ("crb", "braq")),
    ]
    for name, R, C, nseq, seqlen, seed, methods in fq_cases:
        if name == "cfg1":
            W, X = synth.cfg1(seed)
        else:
            W = synth.weight(R, C, seed, outlier_frac=0.02)
            X = synth.calibration(nseq, seqlen, C, seed + 1, kind="lognormal")
        ent = {"name": name, "R": R, "C": C, "nseq": nseq, "seqlen": seqlen,
               "seed": seed, "W_sha": sha(W), "X_sha": sha(X), "methods": {}}
        # inputs are regenerated from the seed by crb_amd.synth and checked
        # against W_sha / X_sha; outputs of the small cases are stored whole
        small = R * C <= 64 * 1024
        for method in methods:
            layer = torch.nn.Linear(C, R, bias=False)
            layer.weight.data = W.clone()
            q = binary.Binarization(layer.weight, method=method, groupsize=128)
            bq = bigptq.BRAGPTQ(layer, q, "hessian")
            for s in range(nseq):
                bq.add_batch(X[s:s + 1], None)
            Hsnap = bq.H.clone()
            with contextlib.redirect_stdout(io.StringIO()):
                info = bq.fasterquant(blocksize=128, percdamp=0.01, partition=3,
                                      orders=(1, 1, 2))
            Wq = layer.weight.data.clone()
            ent["methods"][method] = {"error": info["error"],
                                      "error_hex": float(info["error"]).hex(),
                                      "Wq_sha": sha(Wq), "H_sha": sha(Hsnap)}
            if small:
                arrays[f"fq_{name}_{method}_Wq"] = Wq.numpy()
        summary["fasterquant"].append(ent)

    # ---- technique flags off the default path, on one small layer ----------
    # (case, method, salient_metric, disable_gptq, partition, dtype)
    flag_cases = [
        ("rtn", "crb", "hessian", True, 3, "f32"),
        ("rtn", "braq", "hessian", True, 3, "f32"),
        ("part1", "crb", "hessian", False, 1, "f32"),
        ("part1", "braq", "hessian", False, 1, "f32"),
        ("part1", "crbog", "hessian", False, 1, "f32"),
        ("rtn_part1", "crb", "hessian", True, 1, "f32"),
        ("magnitude", "crb", "magnitude", False, 3, "f32"),
        ("magnitude", "braq", "magnitude", False, 3, "f32"),
        ("norefine", "crb_norefine", "hessian", False, 3, "f32"),
        ("symdamp", "crb_symdamp", "hessian", False, 3, "f32"),
        ("symdamp_norefine", "crb_symdamp_norefine", "hessian", False, 3, "f32"),
        ("bf16", "crb", "hessian", False, 3, "bf16"),
        ("bf16", "crbog", "hessian", False, 3, "bf16"),
    ]
    R, C, nseq, seqlen, seed = 64, 256, 4, 64, 41
    summary["flags"] = {"R": R, "C": C, "nseq": nseq, "seqlen": seqlen, "seed": seed,
                        "cases": []}
    for case, method, metric, rtn, part, dt in flag_cases:
        if dt == "bf16":
            # 1 % of the input columns x10, bf16 in and out
            W = synth.weight(R, C, seed, outlier_frac=0.01, outlier_scale=10.0,
                             dtype=torch.bfloat16)
            X = synth.calibration(nseq, seqlen, C, seed + 1, kind="lognormal",
                                  dtype=torch.bfloat16)
        else:
            W = synth.weight(R, C, seed, outlier_frac=0.02)
            X = synth.calibration(nseq, seqlen, C, seed + 1, kind="lognormal")
        layer = torch.nn.Linear(C, R, bias=False).to(W.dtype)
        layer.weight.data = W.clone()
        q = binary.Binarization(layer.weight, method=method, groupsize=128)
        bq = bigptq.BRAGPTQ(layer, q, metric, disable_gptq=rtn)
        for s in range(nseq):
            bq.add_batch(X[s:s + 1], None)
        with contextlib.redirect_stdout(io.StringIO()):
            info = bq.fasterquant(blocksize=128, percdamp=0.01, partition=part,
                                  orders=(1, 1, 2))
        Wq = layer.weight.data.clone().float()
        key = f"flag_{case}_{method}"
        arrays[key + "_Wq"] = Wq.numpy()
        summary["flags"]["cases"].append({
            "case": case, "method": method, "metric": metric, "disable_gptq": rtn,
            "partition": part, "dtype": dt, "key": key, "W_sha": sha(W.float()),
            "X_sha": sha(X.float()), "error": info["error"],
            "error_hex": float(info["error"]).hex()})

    np.savez_compressed(os.path.join(HERE, "golden_vectors.npz"), **arrays)
    with open(os.path.join(HERE, "golden_summary.json"), "w") as f:
        json.dump(summary, f, indent=1)
    print("wrote", len(arrays), "arrays")


if __name__ == "__main__":
    main(sys.argv[1] if len(sys.argv) > 1 else "/root/reference")
