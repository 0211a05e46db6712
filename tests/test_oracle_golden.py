"""Pin the CPU oracle against vectors written by the reference itself
(tests/golden/make_golden.py).  Both run torch-CPU fp32, so agreement is
expected to be bit-exact."""
import hashlib

import numpy as np
import pytest
import torch

from crb_amd import synth
from oracle import crb_oracle as O


def _sha(t):
    return hashlib.sha256(t.contiguous().numpy().tobytes()).hexdigest()


BINS = {
    "braq": lambda x, m, o: O.hor(x, m, o),
    "crb": lambda x, m, o: O.crb_v7(x, m, o),
    "crb_norefine": lambda x, m, o: O.crb_v7(x, m, o, skip_refinement=True),
    "crb_symdamp": lambda x, m, o: O.crb_v7(x, m, o, symmetric_damp=True),
    "crbog": lambda x, m, o: O.crbog(x, m, o),
}


@pytest.mark.parametrize("method", sorted(BINS))
@pytest.mark.parametrize("order", [1, 2])
def test_binarizers_match_reference(golden, method, order):
    summary, A = golden
    for c in summary["binarize"]:
        i = c["case"]
        x = torch.from_numpy(A[f"bin{i}_x"])
        m = torch.from_numpy(A[f"bin{i}_m"])
        want = A[f"bin{i}_o{order}_{method}"]
        got = BINS[method](x, m, order).numpy()
        np.testing.assert_array_equal(got, want)


def test_structural_searching_matches_reference(golden):
    summary, A = golden
    for c in summary["search"]:
        i = c["case"]
        T = torch.from_numpy(A[f"search{i}_T"])
        tr = O.SearchTrace()
        split, m3 = O.structural_searching(T, 50, trace=tr)
        assert float(split).hex() == c["split_hex"], c
        np.testing.assert_array_equal(m3.numpy(), A[f"search{i}_m3"])
        assert tr.i_star == c["n_salient_cols"]


def _fq_inputs(ent):
    if ent["name"] == "cfg1":
        W, X = synth.cfg1(ent["seed"])
    else:
        W = synth.weight(ent["R"], ent["C"], ent["seed"], outlier_frac=0.02)
        X = synth.calibration(ent["nseq"], ent["seqlen"], ent["C"], ent["seed"] + 1,
                              kind="lognormal")
    assert _sha(W) == ent["W_sha"], "synthetic W changed (torch RNG?)"
    assert _sha(X) == ent["X_sha"], "synthetic X changed (torch RNG?)"
    return W, X


def _oracle_H(X, C):
    H = torch.zeros(C, C)
    n = 0
    for s in range(X.shape[0]):
        H, n = O.hessian_add_batch(H, n, X[s:s + 1])
    return H


@pytest.mark.parametrize("name", ["small_a", "small_b", "cfg1"])
def test_fasterquant_matches_reference(golden, name):
    summary, A = golden
    ent = next(e for e in summary["fasterquant"] if e["name"] == name)
    W, X = _fq_inputs(ent)
    H = _oracle_H(X, ent["C"])
    for method, res in ent["methods"].items():
        assert _sha(H) == res["H_sha"]
        Wq, losses, err, info, U = O.fasterquant(W, H, method=method)
        assert float(err).hex() == res["error_hex"], (method, err, res["error"])
        assert _sha(Wq) == res["Wq_sha"], method
        key = f"fq_{name}_{method}_Wq"
        if key in A.files:
            np.testing.assert_array_equal(Wq.numpy(), A[key])


def _flag_inputs(summary, ent):
    f = summary["flags"]
    R, C, nseq, seqlen, seed = f["R"], f["C"], f["nseq"], f["seqlen"], f["seed"]
    if ent["dtype"] == "bf16":
        W = synth.weight(R, C, seed, outlier_frac=0.01, outlier_scale=10.0,
                         dtype=torch.bfloat16)
        X = synth.calibration(nseq, seqlen, C, seed + 1, kind="lognormal",
                              dtype=torch.bfloat16)
    else:
        W = synth.weight(R, C, seed, outlier_frac=0.02)
        X = synth.calibration(nseq, seqlen, C, seed + 1, kind="lognormal")
    assert _sha(W.float()) == ent["W_sha"] and _sha(X.float()) == ent["X_sha"]
    return W, X


def test_binarizer_symdamp_norefine_matches_reference(golden):
    summary, A = golden
    for c in summary["binarize"]:
        i = c["case"]
        x = torch.from_numpy(A[f"bin{i}_x"])
        m = torch.from_numpy(A[f"bin{i}_m"])
        for order in (1, 2):
            got = O.binarize("crb_symdamp_norefine", x, m, order).numpy()
            np.testing.assert_array_equal(got, A[f"bin{i}_o{order}_crb_symdamp_norefine"])


def test_fasterquant_flags_match_reference(golden):
    """RTN (bigptq.py:149-162), partition=1 (bigptq.py:138-140), the
    magnitude metric (utils/structure.py:11-12), the norefine / symdamp
    methods (binary.py:2885-2890) and bf16 layers: the oracle's weights and
    error bit for bit against the reference's."""
    summary, A = golden
    for ent in summary["flags"]["cases"]:
        W, X = _flag_inputs(summary, ent)
        H = _oracle_H(X, W.shape[1])
        Wq, losses, err, info, U = O.fasterquant(
            W, H, method=ent["method"], partition=ent["partition"],
            salient_metric=ent["metric"], disable_gptq=ent["disable_gptq"])
        Wq = Wq.to(W.dtype).float()
        assert float(err).hex() == ent["error_hex"], ent["key"]
        np.testing.assert_array_equal(Wq.numpy(), A[ent["key"] + "_Wq"], err_msg=ent["key"])
