"""Drop-in ``Binarization`` for the crbq techniques (binary.py:2850-2890).

Same constructor and ``quantize(w, mask, order, groupi, col_weights)``
signature as the reference.  The in-scope methods (``braq``, ``crb``,
``crbog`` and the ``crb_norefine`` / ``crb_symdamp`` flags of CRB v7) run
the gfx950 per-row binarization kernel; every other reference method raises
NotImplementedError.
"""
from __future__ import annotations

import math

import torch
import torch.nn as nn

from . import kernels
from ._lib import METHODS


class Binarization(nn.Module):
    """binary.py:2850-2868.  ``refine_iters`` (default 1, the reference's
    single two-way refinement round, binary.py:1617-1630) is an extension
    for raising the number of CRB sign-refinement rounds."""

    def __init__(self, weight, method="2bit", groupsize=-1, corr_damp=0.1, lam=1e-5,
                 coupling=0.5, refine_iters=1):
        super().__init__()
        oc, ic = weight.shape
        if groupsize == -1:
            groupsize = ic
        self.groupsize = groupsize
        self.n_groups = math.ceil(ic / groupsize)
        self.method = method
        self.mean = 0
        self.kappa = 1.0
        self.order = 2
        self.corr_damp = corr_damp
        self.lam = lam
        self.coupling = coupling
        self.refine_iters = refine_iters

    @property
    def on_crbq_path(self) -> bool:
        return self.method in METHODS

    def quantize(self, w, mask, order=2, groupi=0, col_weights=None):
        """binary.py:2874-2890.  ``col_weights`` and ``groupi`` are ignored by
        these methods in the reference as well.

        The kernels compute in fp32.  ``BRAGPTQ.fasterquant`` always passes
        fp32 blocks (bigptq.py:60), so on that path the arithmetic is the
        reference's.  A direct caller passing fp16/bf16 ``w`` gets the fp32
        result rounded once to ``w``'s dtype, where the reference computes
        every step in the input dtype (each torch op rounding to fp16/bf16);
        the two agree to within that dtype's rounding of the scales, and a
        sign decision sitting within one such ulp of its group's mean may
        differ."""
        if not self.on_crbq_path:
            raise NotImplementedError(
                f"Binarization method {self.method!r} is outside the crbq hot path")
        out = kernels.binarize(w, mask, order, self.method, lam=self.lam,
                               corr_damp=self.corr_damp, refine_iters=self.refine_iters)
        return out.to(w.dtype) if w.dtype != torch.float32 else out
