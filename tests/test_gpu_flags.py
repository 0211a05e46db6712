"""Technique flags off the default path, on the GPU, against the reference's
own outputs and the CPU oracle.

* fasterquant through the drop-in BRAGPTQ with RTN (disable_gptq,
  bigptq.py:149-162), partition=1 (one all-ones mask, bigptq.py:138-140),
  the magnitude metric (utils/structure.py:11-12), the crb_norefine /
  crb_symdamp / crb_symdamp_norefine methods (binary.py:2885-2890) and a
  bf16 layer with 1 % outlier columns x10 (crb and crbog), each against the
  weights and error the reference wrote (tests/golden/make_golden.py);
* CRB with more sign-refinement rounds than the reference's one
  (refine_iters 2 and 5): the binarizer on rows of
  bf16 weights with 1 % outlier columns x10, and fasterquant of a small
  layer, against the oracle (the reference has no such parameter, so the
  oracle's loop over binary.py:1617-1630 is the statement checked).

Bars (north star): error within 1e-3 relative (exactly 0 for RTN, which
accumulates no loss), reconstruction error ||(W - Wq) X^T|| within 1e-3
relative, >= 99.99 % of weights within 1e-4 relative (bf16 layers: within
one bf16 ulp, 2^-8 relative, since the reference's value is itself rounded
to bf16).  Binarizer: per-element |diff| <= 1e-5 * max|x| on >= 99.9 % of
elements (an element on its group's mean may take the other sign).
"""
import numpy as np
import pytest
import torch

from crb_amd import synth
from oracle import crb_oracle as O

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def _flag_inputs(f, ent):
    R, C, nseq, seqlen, seed = f["R"], f["C"], f["nseq"], f["seqlen"], f["seed"]
    if ent["dtype"] == "bf16":
        W = synth.weight(R, C, seed, outlier_frac=0.01, outlier_scale=10.0,
                         dtype=torch.bfloat16)
        X = synth.calibration(nseq, seqlen, C, seed + 1, kind="lognormal",
                              dtype=torch.bfloat16)
    else:
        W = synth.weight(R, C, seed, outlier_frac=0.02)
        X = synth.calibration(nseq, seqlen, C, seed + 1, kind="lognormal")
    return W, X


def _run_bragptq(W, X, method, metric="hessian", disable_gptq=False, partition=3,
                 refine_iters=1):
    from crb_amd import BRAGPTQ, Binarization
    R, C = W.shape
    layer = torch.nn.Linear(C, R, bias=False).to(DEV).to(W.dtype)
    layer.weight.data = W.to(DEV).clone()
    q = Binarization(layer.weight, method=method, groupsize=128)
    q.refine_iters = refine_iters
    bq = BRAGPTQ(layer, q, metric, disable_gptq=disable_gptq)
    for s in range(X.shape[0]):
        bq.add_batch(X[s:s + 1].to(DEV), None)
    info = bq.fasterquant(blocksize=128, percdamp=0.01, partition=partition,
                          orders=(1, 1, 2))
    assert layer.weight.dtype == W.dtype
    return layer.weight.data.float().cpu(), info["error"]


def _compare(W, X, Wg, eg, Wr, er, bf16):
    Xf = X.reshape(-1, X.shape[-1]).double()
    W0 = W.double()
    rg = float(((W0 - Wg.double()) @ Xf.t()).norm())
    rr = float(((W0 - Wr.double()) @ Xf.t()).norm())
    tol = 2.0 ** -8 if bf16 else 1e-4
    close = (Wg - Wr).abs() <= tol * Wr.abs() + 1e-7
    return {
        "err_rel": abs(eg - er) / abs(er) if er else abs(eg),
        "recon_rel": abs(rg - rr) / rr,
        "agree": float(close.float().mean()),
        "identical": float((Wg == Wr).float().mean()),
    }


def _flag_cases():
    import json
    import os
    here = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden",
                        "golden_summary.json")
    with open(here) as fh:
        return json.load(fh)["flags"]["cases"]


@pytest.mark.parametrize("ent", _flag_cases(), ids=lambda e: e["key"])
def test_fasterquant_flags_match_reference(golden, ent):
    summary, A = golden
    print(f"flags {ent['key']}", flush=True)
    W, X = _flag_inputs(summary["flags"], ent)
    Wg, eg = _run_bragptq(W, X, ent["method"], ent["metric"], ent["disable_gptq"],
                          ent["partition"])
    Wr = torch.from_numpy(A[ent["key"] + "_Wq"])
    m = _compare(W.float(), X.float(), Wg, eg, Wr, ent["error"], ent["dtype"] == "bf16")
    print("  ", m, flush=True)
    if ent["disable_gptq"]:
        assert eg == 0.0 and ent["error"] == 0.0        # RTN accumulates no loss
    else:
        assert m["err_rel"] < 1e-3
    assert m["recon_rel"] < 1e-3
    assert m["agree"] >= 0.9999


def _cfg5_rows(R, nc, seed):
    """Rows of a bf16 weight with 1 % of its columns x10."""
    return synth.weight(R, nc, seed, outlier_frac=0.01, outlier_scale=10.0,
                        dtype=torch.bfloat16).float()


@pytest.mark.parametrize("method", ["crb", "crb_symdamp", "crbog", "braq"])
@pytest.mark.parametrize("refine_iters", [1, 2, 5])
def test_binarize_refine_iters_bf16_outliers_vs_oracle(method, refine_iters):
    from crb_amd import kernels
    print(f"binarize {method} refine {refine_iters} bf16 outlier rows", flush=True)
    g = torch.Generator().manual_seed(100 + refine_iters)
    for R, nc in [(256, 128), (37, 128), (64, 100), (16, 512)]:
        x = _cfg5_rows(R, nc, 7 * R + nc)
        m = torch.rand(R, nc, generator=g) < 0.6
        for order in (1, 2):
            want = O.binarize(method, x, m, order, refine_iters=refine_iters)
            got = kernels.binarize(x.to(DEV), m.to(DEV), order, method,
                                   refine_iters=refine_iters).cpu()
            tol = 1e-5 * float(x.abs().max())
            bad = (got - want).abs() > tol
            print(f"  {R}x{nc} order {order}: max|d| {float((got - want).abs().max()):.3g} "
                  f"bad {float(bad.float().mean()):.4%}", flush=True)
            assert float(bad.float().mean()) <= 1e-3 or int(bad.sum()) <= 1


@pytest.mark.parametrize("refine_iters", [2, 5])
@pytest.mark.parametrize("dtype", ["f32", "bf16"])
def test_fasterquant_refine_iters_vs_oracle(refine_iters, dtype):
    """crb with refine_iters > 1 through BRAGPTQ against the oracle on a
    64 x 256 layer (fp32, and bf16 with 1 % outlier columns x10)."""
    print(f"fasterquant crb refine {refine_iters} {dtype}", flush=True)
    ent = {"dtype": dtype}
    f = {"R": 64, "C": 256, "nseq": 4, "seqlen": 64, "seed": 51}
    W, X = _flag_inputs(f, ent)
    Wg, eg = _run_bragptq(W, X, "crb", refine_iters=refine_iters)
    H = torch.zeros(256, 256)
    n = 0
    for s in range(X.shape[0]):
        H, n = O.hessian_add_batch(H, n, X[s:s + 1])
    Wr, _, er, _, _ = O.fasterquant(W, H, method="crb", refine_iters=refine_iters)
    Wr = Wr.to(W.dtype).float()
    m = _compare(W.float(), X.float(), Wg, eg, Wr, er, dtype == "bf16")
    print("  ", m, flush=True)
    assert m["err_rel"] < 1e-3
    assert m["recon_rel"] < 1e-3
    assert m["agree"] >= 0.9999
