"""Per-row scale parity (the north star's "per-row scales within 1e-4
relative in fp32"): crbq_binarize_scales returns each row's scales as the
reference computes them, compared with the oracle's (pinned bit for bit
against reference-written outputs, tests/test_oracle_golden.py):

* CRB variants (binary.py:1544-1638): row mean (:1599), mean correction
  (:1633-1635), alpha1 / alpha2 after the last solve (:1582-1596,
  1615-1630); CRBOG order 2 (binary.py:653-682): mean, alpha1, alpha2;
  BRAQ (binary.py:18-39) and CRBOG order 1: (mu_k, alpha_k) per pass.
* Bars: on every row whose binarized values agree with the oracle's
  (every element within 1e-5 * max|x|, i.e. the same sign planes and
  groups), each scale within 1e-4 relative; alphas relative to themselves,
  the location scales (means and the mean correction) relative to the
  row's own magnitude max(|value|, alpha1 + alpha2), since a zero-mean
  row's mean is itself near 0; alphas are floored at 1 % of the row's
  |mean| + alphas, since a row whose masked values are all equal has
  alphas made of the rounding noise of its mean (golden case 0, row 3).
  At least 99.9 % of the rows agree (the others are rows where an element
  sits within an ulp of its group's mean and the fp32 sum order decides
  its sign).
* Inputs: the reference-written golden rows (3 row sets), the groups of a
  4096 x 128 block of an OPT-6.7B-shaped layer under its own salient /
  bell masks from the GPU search, and bf16 rows with 1 % x10 outlier
  columns for CRB with 2 and 5 sign-refinement rounds.
"""
import pytest
import torch

from crb_amd import synth
from oracle import crb_oracle as O

pytestmark = pytest.mark.gpu
DEV = "cuda:0"
METHODS = ["braq", "crb", "crb_norefine", "crb_symdamp", "crbog"]


def _oracle_scales(method, x, m, order, refine_iters=1):
    if method == "braq":
        return O.hor(x, m, order, return_scales=True)
    if method == "crbog":
        return O.crbog(x, m, order, return_scales=True)
    skip, sym = O.CRB_METHODS[method]
    out, s = O.crb_v7(x, m, order, skip_refinement=skip, symmetric_damp=sym,
                      refine_iters=refine_iters, return_scales=True)
    return out, torch.stack([s.mean, s.mu_corr, s.a1, s.a2], dim=1)


def _check(tag, method, x, m, order, refine_iters=1):
    from crb_amd import kernels
    want_o, want_s = _oracle_scales(method, x, m, order, refine_iters)
    got_o, got_s = kernels.binarize_scales(x.to(DEV), m.to(DEV), order, method,
                                           refine_iters=refine_iters)
    got_o, got_s = got_o.cpu(), got_s.cpu()
    # the elementwise output of the scales kernel is the product kernel's
    prod = kernels.binarize(x.to(DEV), m.to(DEV), order, method,
                            refine_iters=refine_iters).cpu()
    tol = 1e-5 * float(x.abs().max())
    assert float(((prod - got_o).abs() > tol).float().mean()) <= 1e-3
    rows_ok = ((got_o - want_o).abs() <= tol).all(dim=1)
    frac = float(rows_ok.float().mean())
    passes = method == "braq" or (method == "crbog" and order == 1)
    if passes:
        loc = list(range(0, want_s.shape[1], 2))
        alph = list(range(1, want_s.shape[1], 2))
        mag = want_s[:, alph].abs().sum(dim=1)
    else:
        loc, alph = [0, 1], [2, 3]
        mag = want_s[:, 2:4].abs().sum(dim=1)
    d = (got_s - want_s).abs()
    # a row whose masked values are (nearly) all equal has alphas made of
    # rounding noise of its mean: alphas are floored at 1 % of the row's
    # magnitude |mean| + alphas
    size = (want_s[:, loc].abs().sum(dim=1) + mag).clamp_min(1e-30)
    r_alpha = d[:, alph] / torch.maximum(want_s[:, alph].abs(), 1e-2 * size[:, None])
    den = torch.maximum(want_s[:, loc].abs(), mag[:, None]).clamp_min(1e-30)
    r_loc = d[:, loc] / den
    r = torch.cat([r_alpha, r_loc], dim=1)[rows_ok]
    worst = float(r.max()) if r.numel() else 0.0
    print(f"  {tag} {method} order {order} refine {refine_iters}: rows {x.shape[0]}, "
          f"agreeing {frac:.5f}, worst scale rel {worst:.2e}", flush=True)
    assert frac >= 0.999 or int((~rows_ok).sum()) <= 1, frac
    assert worst <= 1e-4, worst


@pytest.mark.parametrize("method", METHODS)
def test_scales_golden_rows(golden, method):
    summary, A = golden
    for c in summary["binarize"]:
        i = c["case"]
        x = torch.from_numpy(A[f"bin{i}_x"])
        m = torch.from_numpy(A[f"bin{i}_m"])
        for order in (1, 2):
            _check(f"golden case {i}", method, x, m, order)


@pytest.mark.parametrize("method", METHODS)
def test_scales_block_groups(method):
    """The three mask groups of one block (orders 1, 1, 2 as
    bigptq.py:235-249 binarizes them) of a 4096-row OPT-6.7B-shaped layer
    whose masks come from the GPU's salient / bell search."""
    from crb_amd import kernels
    print(f"scales on a 4096 x 128 block, {method}", flush=True)
    g = torch.Generator().manual_seed(41)
    W = (torch.randn(4096, 128, generator=g) * 0.02).half().float()
    X = torch.randn(2048, 128, generator=g) * torch.exp(torch.randn(128, generator=g))
    H = X.t() @ X / 1024
    U, _ = O.hinv_upper(H.clone(), torch.zeros(1, 128), 0.01)
    masks, _ = kernels.block_search(W.to(DEV), U.to(DEV), "hessian", 50)
    mk = masks.cpu()
    for j, order in enumerate((1, 1, 2)):
        _check(f"block mask {j + 1}", method, W, mk == j + 1, order)


@pytest.mark.parametrize("iters", [2, 5])
def test_scales_bf16_outlier_rows_refined(iters):
    print(f"scales bf16 outlier rows, refine {iters}", flush=True)
    W = synth.weight(2048, 128, 77, outlier_frac=0.01, outlier_scale=10.0,
                     dtype=torch.bfloat16).float()
    m = torch.rand(2048, 128, generator=torch.Generator().manual_seed(78)) < 0.8
    for order in (1, 2):
        _check("bf16 outliers", "crb", W, m, order, refine_iters=iters)
