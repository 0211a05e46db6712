"""CPU oracle for the CRB layer-wise binarization quantizer.

TEST INFRASTRUCTURE ONLY.  This module is the checker, never the product:
only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may import it.  The product path (``crb_amd``) never imports it
and fails loudly when its HIP library is missing.

It is a from-scratch, op-for-op restatement in torch-CPU fp32 (plus
``numpy.quantile``, the library routine the reference calls) of the hot path
of SDMuhsin/CRB.  Every function cites the reference file:line it follows
(paths relative to the reference repository root).  Elementwise ops are kept
as separate torch ops in the reference's order so per-element rounding
matches; only reduction order (torch CPU vs. the reference's CUDA run) can
differ.

Pinning status (what checks each function; see tests/test_oracle_*.py):
  hessian_add_batch      closed form (float64 brute force), incremental identity
  hinv_upper             torch.linalg / LAPACK identities, retry/fallback cases
  hor                    closed form per row (float64), tiny brute force,
                         reference-held identity src/verify_braq_equiv.py
  crb_v7                 2x2 normal-equation solve checked with numpy lstsq,
                         invariants (a1, a2 >= 0), golden vectors
  crbog                  float64 least-squares per row, golden vectors
  structural_searching   golden vectors written by importing the reference
                         in the build container (tests/golden/make_golden.py)
  fasterquant            golden vectors (ditto), closed-form Err/Loss checks
"""
from __future__ import annotations

import math
from dataclasses import dataclass, field

import numpy as np
import torch

__all__ = [
    "hor", "crb_v7", "crbog", "binarize", "gen_structural_mask",
    "structural_searching", "structural_guassian_distribution",
    "hessian_add_batch", "hinv_upper", "fasterquant", "BlockTrace",
    "PERCENTILES",
]

# torch.linspace(0.10, 0.90, 81) in float32 (utils/autosearch.py:65)
PERCENTILES = torch.linspace(0.10, 0.90, 81)

_NAN = float("nan")


def _zero_nan(t: torch.Tensor) -> torch.Tensor:
    return torch.where(torch.isnan(t), torch.zeros_like(t), t)


# --------------------------------------------------------------------------
# binarizers
# --------------------------------------------------------------------------
@torch.no_grad()
def hor(x: torch.Tensor, mask: torch.Tensor, order: int = 2,
        return_scales: bool = False):
    """BRAQ / BiLLM high-order residual binarization, binary.py:18-39.

    Each pass: residual on the mask (NaN elsewhere), nanmean -> mu (NaN -> 0),
    center, nanmean |.| -> alpha (NaN -> 0), add (sign*alpha + mu) * mask.
    torch.sign(NaN) is 0, so off-mask entries contribute exactly 0.
    ``return_scales`` also returns the per-row (mu_k, alpha_k) of every pass
    as an [R, 2 * order] tensor (the reference's mean_tensor_all /
    scale_tensor_all, binary.py:26-33).
    """
    acc = torch.zeros_like(x)
    base = x.clone() * mask
    nan = torch.tensor(_NAN, dtype=x.dtype)
    scales = []
    for _ in range(order):
        res = base - acc
        m = torch.where(mask, res, nan)
        mu = _zero_nan(torch.nanmean(m, dim=1))
        m -= mu[:, None]
        alpha = _zero_nan(torch.nanmean(torch.abs(m), dim=1))
        b = torch.sign(m)
        b *= alpha[:, None]
        b += mu[:, None]
        acc = acc + b * mask
        scales += [mu, alpha]
    if return_scales:
        return acc, torch.stack(scales, dim=1)
    return acc


@dataclass
class CrbRowScales:
    """Per-row scales of one crb_v7 call (order 2): mean, mu-correction,
    alpha1, alpha2, and the final sign planes B1, B2."""
    mean: torch.Tensor
    mu_corr: torch.Tensor
    a1: torch.Tensor
    a2: torch.Tensor
    b1: torch.Tensor
    b2: torch.Tensor


@torch.no_grad()
def crb_v7(x, mask, order=2, lam=1e-5, corr_damp=0.1, skip_refinement=False,
           symmetric_damp=False, refine_iters=1, return_scales=False):
    """CRB: coupled two-plane binarization with Tikhonov-regularised 2x2 scale
    solve, correlation damping and two-way sign refinement.
    binary.py:1544-1638 (``coupled_residual_binarization_stable_v7``).

    ``refine_iters`` repeats steps 5-6 (binary.py:1617-1630); the reference
    runs exactly one round (refine_iters=1).
    """
    mf = mask.float()
    d = mf.sum(dim=1)
    ds = torch.clamp(d, min=1.0)
    base = x.clone() * mask

    if order == 1:                                           # :1570-1576
        mean = (base * mf).sum(dim=1) / ds
        cen = (base - mean[:, None]) * mf
        b1 = torch.sign(cen) * mf
        a1 = (cen.abs() * mf).sum(dim=1) / ds
        out = (mean[:, None] + a1[:, None] * b1) * mf
        if return_scales:
            z = torch.zeros_like(mean)
            return out, CrbRowScales(mean, z, a1, z, b1, torch.zeros_like(b1))
        return out

    def solve(b1, b2, c1w, c2w):                             # :1582-1596
        c12 = (b1 * b2 * mf).sum(dim=1)
        if symmetric_damp:
            c12 = c12 * (1.0 - corr_damp)
        else:
            c12 = torch.where(c12 > 0, c12 * (1.0 - corr_damp), c12)
        A = d + lam
        den = A * A - c12 * c12
        ok = den.abs() > 1e-12
        sden = torch.where(ok, den, torch.ones_like(den))
        a1 = torch.clamp((A * c1w - c12 * c2w) / sden, min=0.0)
        a2 = torch.clamp((A * c2w - c12 * c1w) / sden, min=0.0)
        a1 = torch.where(ok, a1, torch.zeros_like(a1))
        a2 = torch.where(ok, a2, torch.zeros_like(a2))
        return a1, a2

    mean = (base * mf).sum(dim=1) / ds                       # step 1
    cen = (base - mean[:, None]) * mf
    b1 = torch.sign(cen) * mf                                # step 2
    a1_0 = (cen.abs() * mf).sum(dim=1) / ds
    r = (cen - a1_0[:, None] * b1) * mf                      # step 3
    r_mean = (r * mf).sum(dim=1) / ds
    b2 = torch.sign((r - r_mean[:, None]) * mf) * mf
    c1w = (cen * b1).sum(dim=1)                              # step 4
    c2w = (cen * b2).sum(dim=1)
    a1, a2 = solve(b1, b2, c1w, c2w)
    if not skip_refinement:
        for _ in range(refine_iters):
            t5 = (cen - a1[:, None] * b1) * mf               # step 5
            t5m = (t5 * mf).sum(dim=1) / ds
            b2 = torch.sign((t5 - t5m[:, None]) * mf) * mf
            c2w = (cen * b2).sum(dim=1)
            a1, a2 = solve(b1, b2, c1w, c2w)
            t6 = (cen - a2[:, None] * b2) * mf               # step 6
            t6m = (t6 * mf).sum(dim=1) / ds
            b1 = torch.sign((t6 - t6m[:, None]) * mf) * mf
            c1w = (cen * b1).sum(dim=1)
            a1, a2 = solve(b1, b2, c1w, c2w)
    approx = (a1[:, None] * b1 + a2[:, None] * b2) * mf      # step 7
    resid = (cen - approx) * mf
    mu_c = (resid * mf).sum(dim=1) / ds
    out = (mean[:, None] + mu_c[:, None] + a1[:, None] * b1 + a2[:, None] * b2) * mf
    if return_scales:
        return out, CrbRowScales(mean, mu_c, a1, a2, b1, b2)
    return out


@torch.no_grad()
def crbog(x, mask, order=2, return_scales=False):
    """CRBOG, binary.py:577-687 (``coupled_residual_binarization``).

    order 1 is the single BRAQ pass; order >= 2 is a per-row loop over rows
    with a float64 (Python float) 2x2 solve without damping or Tikhonov term.
    ``return_scales`` also returns per-row scales: order 1 as ``hor``; order
    >= 2 an [R, 4] tensor (row_mean, 0, alpha1, alpha2) with the alphas as
    the fp32 values the final approximation uses (:653-682).
    """
    if order == 1:                                           # :595-630
        return hor(x, mask, order=1, return_scales=return_scales)
    out = torch.zeros_like(x)
    sc = torch.zeros(x.shape[0], 4, dtype=x.dtype)
    base = x.clone() * mask
    for i in range(base.shape[0]):                           # :644-685
        rm = mask[i, :]
        if not torch.any(rm):
            continue
        v = base[i, rm]
        mean = v.mean()
        cen = v - mean
        b1 = torch.sign(cen)
        a1 = cen.abs().mean()
        r = cen - a1 * b1
        b2 = torch.sign(r)
        a2 = r.abs().mean()
        n = float(v.numel())
        c12 = torch.sum(b1 * b2).item()
        c1w = torch.sum(cen * b1).item()
        c2w = torch.sum(cen * b2).item()
        det = n * n - c12 * c12
        if abs(det) > 1e-12:
            a1 = max((c1w * n - c2w * c12) / det, 0.0)
            a2 = max((c2w * n - c1w * c12) / det, 0.0)
        out[i, rm] = mean + a1 * b1 + a2 * b2
        sc[i, 0], sc[i, 2], sc[i, 3] = mean, float(a1), float(a2)
    if return_scales:
        return out, sc
    return out


CRB_METHODS = {
    # method -> (skip_refinement, symmetric_damp); binary.py:2883-2890
    "crb": (False, False),
    "crb_norefine": (True, False),
    "crb_symdamp": (False, True),
    "crb_symdamp_norefine": (True, True),
}


def binarize(method, w, mask, order, lam=1e-5, corr_damp=0.1, refine_iters=1):
    """``Binarization.quantize`` dispatch for the in-scope methods,
    binary.py:2874-2890."""
    if method == "braq":
        return hor(w, mask, order=order)
    if method == "crbog":
        return crbog(w, mask, order=order)
    if method in CRB_METHODS:
        skip, sym = CRB_METHODS[method]
        return crb_v7(w, mask, order=order, lam=lam, corr_damp=corr_damp,
                      skip_refinement=skip, symmetric_damp=sym,
                      refine_iters=refine_iters)
    raise NotImplementedError(method)


# --------------------------------------------------------------------------
# salient-column search and bell-shaped split
# --------------------------------------------------------------------------
def gen_structural_mask(T, m3, split):
    """utils/mask.py:7-18 (``generate_structural_mask``)."""
    keep = ~m3
    g = torch.abs(T * keep)
    m2 = (g >= split) * keep
    m1 = (g < split) * keep
    return m1, m2


def _err(T, q):
    """utils/autosearch.py:8-10: fp32 mean squared error."""
    return torch.mean((T - q) ** 2)


@dataclass
class SearchTrace:
    colscore: torch.Tensor = None
    top: torch.Tensor = None
    errs_a: list = field(default_factory=list)
    i_star: int = 0
    pvals: torch.Tensor = None
    errs_c: list = field(default_factory=list)
    k_star: int = 0
    split: float = 0.0


@torch.no_grad()
def structural_searching(T, up_lim=30, trace: SearchTrace | None = None):
    """utils/autosearch.py:28-83.  Returns (split, mask3)."""
    R, nc = T.shape
    colscore = T.abs().sum(dim=0)                            # :37
    _, top = torch.topk(colscore, up_lim)                    # :42
    best0, i_star = float("inf"), max(1, up_lim // 3)        # :43
    errs_a = []
    for i in range(1, up_lim):                               # :44-55
        m3 = torch.zeros((R, nc), dtype=torch.bool)
        m3[:, top[:i]] = True
        g3 = hor(T, m3, order=2)
        g4 = hor(T, ~m3, order=2)
        e = _err(T, g4 + g3)
        errs_a.append(e.item())
        if e < best0:
            best0, i_star = e, i
    _, top2 = torch.topk(colscore, i_star)                   # :57-60
    m3 = torch.zeros((R, nc), dtype=torch.bool)
    m3[:, top2] = True
    g3 = hor(T, m3, order=2)
    flat = torch.abs(T * (~m3)).view(-1)                     # :62-68
    pv = torch.tensor(np.quantile(flat.numpy(), q=PERCENTILES.numpy(),
                                  axis=None, keepdims=False))
    k_star = len(pv) // 2                                    # :71
    split = pv[k_star]
    best = float("inf")
    errs_c = []
    for k in range(len(pv)):                                 # :72-80
        m1, m2 = gen_structural_mask(T, m3, pv[k])
        g1 = hor(T, m1, order=1)
        g2 = hor(T, m2, order=1)
        e = _err(T, g1 + g2 + g3)
        errs_c.append(e.item())
        if e < best:
            best, split, k_star = e, pv[k], k
    if trace is not None:
        trace.colscore, trace.top = colscore, top
        trace.errs_a, trace.i_star = errs_a, i_star
        trace.pvals, trace.errs_c = pv, errs_c
        trace.k_star, trace.split = k_star, float(split)
    return split, m3


@torch.no_grad()
def structural_guassian_distribution(tmp, H=None, metric="magnitude", up_lim=30,
                                     trace: SearchTrace | None = None):
    """utils/structure.py:8-20 (without the mask-fraction print)."""
    if metric == "hessian":
        T = tmp ** 2 / (torch.diag(H).reshape((1, -1))) ** 2
    elif metric == "magnitude":
        T = tmp
    else:
        raise NotImplementedError(metric)
    split, m3 = structural_searching(T, up_lim, trace=trace)
    m1, m2 = gen_structural_mask(T, m3, split)
    return m1, m2, m3


# --------------------------------------------------------------------------
# Hessian and inverse factor
# --------------------------------------------------------------------------
@torch.no_grad()
def hessian_add_batch(H: torch.Tensor, nsamples: int, inp: torch.Tensor):
    """bigptq.py:37-53 for an nn.Linear.  Returns (H, nsamples)."""
    if inp.dim() == 2:
        inp = inp.unsqueeze(0)
    b = inp.shape[0]
    if inp.dim() == 3:
        inp = inp.reshape((-1, inp.shape[-1]))
    inp = inp.t()
    H *= nsamples / (nsamples + b)
    nsamples += b
    inp = math.sqrt(2 / nsamples) * inp.float()
    H += inp.matmul(inp.t())
    return H, nsamples


@dataclass
class HinvInfo:
    retries: int = 0
    fallback: bool = False
    dead: torch.Tensor = None


@torch.no_grad()
def hinv_upper(H: torch.Tensor, W: torch.Tensor, percdamp=0.01):
    """bigptq.py:101-129: dead columns, damping, Cholesky with up to 10
    retries (+1e-3 mean diag each, 1e-6 if that is 0), diagonal fallback,
    cholesky_inverse, upper Cholesky of the inverse.

    Mutates H and W like the reference.  Returns (U, HinvInfo).
    """
    C = H.shape[0]
    dead = torch.diag(H) == 0
    H[dead, dead] = 1
    W[:, dead] = 0
    damp = percdamp * torch.mean(torch.diag(H))
    idx = torch.arange(C)
    H[idx, idx] += damp
    info = HinvInfo(dead=dead)
    for _ in range(10):
        try:
            L = torch.linalg.cholesky(H)
            break
        except torch._C._LinAlgError:
            info.retries += 1
            extra = 1e-3 * torch.mean(torch.diag(H))
            if extra == 0:
                extra = 1e-6
            H[idx, idx] += extra
    else:
        info.fallback = True
        L = torch.diag(torch.sqrt(torch.diag(H).clamp(min=1e-8)))
    Hi = torch.cholesky_inverse(L)
    U = torch.linalg.cholesky(Hi, upper=True)
    return U, info


# --------------------------------------------------------------------------
# fasterquant
# --------------------------------------------------------------------------
@dataclass
class BlockTrace:
    st: int
    search: SearchTrace
    masks: torch.Tensor          # uint8 [R, ncols]: 1 / 2 / 3 = mask1 / mask2 / mask3


@torch.no_grad()
def fasterquant(W0: torch.Tensor, H0: torch.Tensor, method="crb", blocksize=128,
                percdamp=0.01, partition=3, orders=(1, 1, 2),
                salient_metric="hessian", lam=1e-5, corr_damp=0.1,
                refine_iters=1, disable_gptq=False, up_lim=50,
                max_blocks=None, trace: list | None = None, U0=None):
    """``BRAGPTQ.fasterquant`` legacy partitioned path, bigptq.py:56-291.

    W0: [R, C] weight (any float dtype); H0: [C, C] fp32 Hessian.
    Returns (Wq fp32 [R, C] before the dtype cast, Losses fp32 [R],
    error float = torch.sum(Losses).item(), HinvInfo, U).
    ``max_blocks`` stops after that many column blocks (CPU baseline timing,
    parity of the first blocks of full-size layers); the unprocessed columns
    of Wq then hold the propagated, unquantized W.
    ``U0`` (optional, fp32 [C, C] upper) is an inverse factor computed
    elsewhere: the block loop (bigptq.py:131-264) then starts from it and
    H0 is not used (no dead-column handling, which belongs to the factor).
    """
    W = W0.clone().float()
    R, C = W.shape
    if U0 is None:
        H = H0.clone().float()
        U, hinfo = hinv_upper(H, W, percdamp)
    else:
        U, hinfo = U0.float(), HinvInfo()
    losses = torch.zeros(R)
    for bi, st in enumerate(range(0, C, blocksize)):
        if max_blocks is not None and bi >= max_blocks:
            break
        ed = min(st + blocksize, C)
        masks = torch.zeros((3, R, ed - st), dtype=torch.bool)
        st_trace = SearchTrace()
        if partition == 1:
            masks[0] = True
        else:
            m1, m2, m3 = structural_guassian_distribution(
                W[:, st:ed], U[st:ed, st:ed], salient_metric, up_lim,
                trace=st_trace)
            masks[0], masks[1], masks[2] = m1, m2, m3
        if disable_gptq:                                     # :149-162
            w = W[:, st:ed]
            parts = [binarize(method, w, masks[j], orders[j], lam, corr_damp,
                              refine_iters) for j in range(3)]
            q = torch.zeros_like(w)
            for j in range(3):
                q += parts[j][:] * masks[j, :]
            W[:, st:ed] = q
        else:                                                # :235-264
            W1 = W[:, st:ed].clone()
            Uq = U[st:ed, st:ed]
            parts = [binarize(method, W1, masks[j], orders[j], lam, corr_damp,
                              refine_iters) for j in range(3)]
            Q1 = torch.zeros_like(W1)
            Err1 = torch.zeros_like(W1)
            L1 = torch.zeros_like(W1)
            for i in range(ed - st):
                w = W1[:, i]
                dd = Uq[i, i]
                q = torch.zeros_like(w)
                for j in range(3):
                    q += parts[j][:, i] * masks[j, :, i]
                Q1[:, i] = q
                L1[:, i] = (w - q) ** 2 / dd ** 2
                Err1[:, i] = (w - q) / dd
            W[:, st:ed] = Q1
            losses += torch.sum(L1, 1) / 2
            W[:, ed:] -= Err1.matmul(U[st:ed, ed:])
        if trace is not None:
            mk = (masks[0].to(torch.uint8) * 1 + masks[1].to(torch.uint8) * 2
                  + masks[2].to(torch.uint8) * 3)
            trace.append(BlockTrace(st, st_trace, mk))
    return W, losses, torch.sum(losses).item(), hinfo, U
