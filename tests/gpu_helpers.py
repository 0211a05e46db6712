"""Helpers shared by the full-size GPU parity tests (not a test module).

* acts / hessian: seeded calibration activations (Student-t(4) channel
  scales, 128 x 2048 tokens) and their Hessian H = (2 / nseq) X^T X through
  the library's SYRK.
* u_checks: the exact identities of the factor and the block loop in
  float64 (hold to fp32 backward error whatever the conditioning).
* teacher_forced: the GPU block loop run one 128-column block at a time,
  each block's input recorded, and the CPU oracle's single block run from
  that same input (bigptq.py:131-264 for one block): elementwise parity of
  every checked block, so a near-tie resolved differently in one block does
  not carry into the next.
"""
from __future__ import annotations

import numpy as np
import torch

from crb_amd import synth
from oracle import crb_oracle as O

DEV = "cuda:0"
NTOK = 128 * 2048


def acts(C, seed, ntok=NTOK):
    s = synth.channel_scales(C, seed, kind="student_t4", device=DEV)
    g = torch.Generator(device=DEV)
    g.manual_seed(seed)
    x = torch.empty(ntok, C, dtype=torch.float16, device=DEV)
    for t0 in range(0, ntok, 8192):
        n = min(8192, ntok - t0)
        x[t0:t0 + n] = (torch.randn(n, C, generator=g, device=DEV) * s).half()
    return x


def hessian(X, nseq=128):
    from crb_amd import kernels
    C = X.shape[1]
    S = torch.zeros(C, C, device=DEV)
    kernels.hessian_accum(X, S)
    return kernels.hessian_finalize(S, 2.0 / nseq, S)


def u_checks(W0, Q, Hd, U, err):
    """Two identities in float64 from the fp32 U:
    * the factor: U^-1 U^-T against H_d (U is the upper Cholesky factor of
      H_d^-1), relative Frobenius error;
    * the block loop: the reference quantizes a 128-column block from its
      values at the block's start (no feedback inside the block,
      bigptq.py:235-262) and then updates the later blocks,
      W[:, ed:] -= Err1 U[st:ed, ed:] (:264), so W0 - Q = E U' with U' = U
      without the strictly upper entries inside each 128 x 128 diagonal
      block; E = (W0 - Q) U'^-1 and sum(E^2) / 2 is the accumulated loss.
    Returns (factor backward error, relative loss difference)."""
    U64 = U.double()
    C = U.shape[0]
    I = torch.eye(C, dtype=torch.float64, device=U.device)
    Ui = torch.linalg.solve_triangular(U64, I, upper=True)
    Ht = Ui @ Ui.t()
    back = float((Ht - Hd.double()).norm() / Hd.double().norm())
    del Ht, Ui
    idx = torch.arange(C, device=U.device)
    blk = idx // 128
    inner = (blk[:, None] == blk[None, :]) & (idx[:, None] != idx[None, :])
    U64.masked_fill_(inner, 0.0)
    del inner
    Upi = torch.linalg.solve_triangular(U64, I, upper=True)
    del I, U64
    D = (W0.float() - Q.float()).double()
    tot = 0.0
    for r0 in range(0, D.shape[0], 2048):
        E = D[r0:r0 + 2048] @ Upi
        tot += float((E * E).sum()) / 2
    return back, abs(tot - err) / err


def _oracle_q_from_masks(method, W1, mk, refine_iters, orders=(1, 1, 2)):
    """The oracle's quantized block for given mask codes (1/2/3):
    binary.py's binarizer per mask group, summed as bigptq.py:244-249."""
    q = torch.zeros_like(W1)
    for j in range(3):
        m = mk == j + 1
        part = O.binarize(method, W1, m, orders[j], refine_iters=refine_iters)
        q += part * m
    return q


def teacher_forced(name, W0, U, method="crb", refine_iters=1, check=None,
                   out_dtype=None, min_block_agree=0.9999):
    """GPU block loop one block at a time from the GPU's own state, each
    checked block compared with the oracle's single block from the same
    input.  Per checked block: the salient count i* and split k* equal the
    oracle's unless the oracle's own candidate errors tie within 1e-5
    (then the oracle's binarization is evaluated on the GPU's masks);
    >= min_block_agree of the weights within 1e-4 relative; with out_dtype
    (the layer's 16-bit dtype), >= min_block_agree of the cast weights
    within one ulp of the oracle's cast.  Returns a summary dict."""
    from crb_amd import _lib, kernels
    p = _lib.params(method, refine_iters=refine_iters)
    R, C = W0.shape
    nblk = (C + 127) // 128
    check = set(range(nblk)) if check is None else {b % nblk for b in check}
    W = W0.float().clone()
    lo = torch.zeros(R, device=DEV)
    worst, worst_b, n_close, n_tot, ties, ident = 1.0, -1, 0, 0, 0, 0
    for b in range(nblk):
        st, ed = b * 128, min(C, (b + 1) * 128)
        Win = W[:, st:ed].clone()
        Ub = U[st:ed, st:ed].contiguous()
        lo.zero_()
        masks, tr = kernels.fasterquant_blocks(W[:, st:ed], Ub, p, lo, want_masks=True,
                                               want_traces=True)
        if ed < C:
            err = (Win - W[:, st:ed]) / torch.diagonal(Ub)[None, :]
            kernels.sgemm(err, U[st:ed, ed:], W[:, ed:], alpha=-1.0, beta=1.0)
        if b % 16 == 15:
            print(f"    {name}: block {b + 1} of {nblk}", flush=True)
        if b not in check:
            continue
        trace = []
        Wr, Lr, _, _, _ = O.fasterquant(Win.cpu(), None, method=method, U0=Ub.cpu(),
                                        refine_iters=refine_iters, trace=trace)
        so, tg = trace[0].search, tr[0]
        tie = False
        if tg["i_star"] != so.i_star:
            ea = np.asarray(so.errs_a)
            assert abs(ea[tg["i_star"] - 1] - ea[so.i_star - 1]) <= 1e-5 * ea[so.i_star - 1], \
                (name, b, "i*", tg["i_star"], so.i_star)
            tie = True
        elif tg["k_star"] != so.k_star:
            ec = np.asarray(so.errs_c)
            assert abs(ec[tg["k_star"]] - ec[so.k_star]) <= 1e-5 * ec[so.k_star], \
                (name, b, "k*", tg["k_star"], so.k_star)
            tie = True
        else:
            assert torch.equal(masks.cpu(), trace[0].masks), (name, b, "masks")
        if tie:
            ties += 1
            Wr = _oracle_q_from_masks(method, Win.cpu(), masks.cpu(), refine_iters)
        Wg = W[:, st:ed].cpu()
        close = (Wg - Wr).abs() <= 1e-4 * Wr.abs() + 1e-7
        agree = float(close.float().mean())
        if out_dtype is not None:
            ig = Wg.to(out_dtype).view(torch.int16).int()
            ir = Wr.to(out_dtype).view(torch.int16).int()
            agree = min(agree, float(((ig - ir).abs() <= 1).float().mean()))
        ident += int(torch.equal(Wg, Wr))
        n_close += int(close.sum())
        n_tot += close.numel()
        if agree < worst or worst_b < 0:
            worst, worst_b = min(agree, worst), b
    res = dict(blocks=nblk, checked=len(check), worst=worst, worst_block=worst_b,
               overall=n_close / max(n_tot, 1), ties=ties, identical_blocks=ident)
    print(f"  {name} {R}x{C} {method}: {len(check)} of {nblk} blocks checked, "
          f"{ident} bit-identical, {ties} tie blocks, worst block {worst_b} agree {worst:.6f}, "
          f"overall {res['overall']:.7f}", flush=True)
    assert worst >= min_block_agree, (name, res)
    return res
