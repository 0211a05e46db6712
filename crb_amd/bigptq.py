"""Drop-in ``BRAGPTQ`` (bigptq.py:18-298) on the gfx950 crbq kernels.

Same constructor, ``add_batch(inp, out, blocksize=1024)``,
``fasterquant(blocksize=128, percdamp=.01, partition=3, orders=(1,1,2),
global_scale=False) -> {"error": float}`` and ``free()`` contract, same
in-place write-back of ``layer.weight.data`` in the layer's dtype and the
same ``time``/``error`` prints.

Differences in mechanism, not in result:
  * add_batch accumulates the unscaled sum S = sum x x^T on MFMA (exact
    f16/bf16 products, fp32 accumulate) and applies the reference's
    running factor 2/nsamples once at fasterquant time.  ``self.H`` is a
    property that materialises the reference's H on demand.
  * U = chol(H^-1)^T comes from one reversed blocked factorization
    (2C^3/3 flops) instead of chol -> cholesky_inverse -> chol.
  * the 128-column block loop, its salient/bell search and the trailing
    rank-128 update run on the device with no host synchronisation.
"""
from __future__ import annotations

import time

import torch
import torch.nn as nn

from . import _lib, kernels

try:  # transformers is only needed for the Conv1D isinstance check
    from transformers import Conv1D as _Conv1D  # type: ignore
except Exception:  # pragma: no cover - optional dependency
    _Conv1D = ()

DEBUG = False


class BRAGPTQ:
    """bigptq.py:18-298."""

    def __init__(self, layer, braq_quantizer, salient_metric, disable_gptq=False):
        self.layer = layer
        self.dev = self.layer.weight.device
        W = layer.weight.data
        if isinstance(self.layer, nn.Conv2d):
            W = W.flatten(1)
        if _Conv1D and isinstance(self.layer, _Conv1D):
            W = W.t()
        self.rows = W.shape[0]
        self.columns = W.shape[1]
        # S = sum over calibration tokens of x x^T (upper triangle), fp32
        self._S = torch.zeros((self.columns, self.columns), device=self.dev)
        self.nsamples = 0
        self.braq_quantizer = braq_quantizer
        self.salient_metric = salient_metric  # "magnitude" or "hessian"
        self.disable_gptq = disable_gptq
        self.last = {}

    # -- bigptq.py:37-53 ----------------------------------------------------
    def add_batch(self, inp, out, blocksize=1024):
        if len(inp.shape) == 2:
            inp = inp.unsqueeze(0)
        tmp = inp.shape[0]
        if isinstance(self.layer, nn.Linear) or (_Conv1D and isinstance(self.layer, _Conv1D)):
            if len(inp.shape) == 3:
                inp = inp.reshape((-1, inp.shape[-1]))
        else:
            raise NotImplementedError("add_batch supports nn.Linear / Conv1D layers, as the "
                                      "reference's Hessian reshape does (bigptq.py:45-49)")
        if self._S is None:
            raise RuntimeError("add_batch after fasterquant/free")
        kernels.hessian_accum(inp, self._S)
        self.nsamples += tmp

    @property
    def H(self) -> torch.Tensor:
        """The reference's H = (2 / nsamples) * sum x x^T (bigptq.py:50-53)."""
        if self._S is None:
            raise AttributeError("H")
        scale = 2.0 / self.nsamples if self.nsamples else 0.0
        return kernels.hessian_finalize(self._S, scale)

    # -- bigptq.py:56-291 ---------------------------------------------------
    def fasterquant(self, blocksize=128, percdamp=0.01, partition=3, orders=(1, 1, 2),
                    global_scale=False):
        W = self.layer.weight.data.clone()
        if isinstance(self.layer, nn.Conv2d):
            W = W.flatten(1)
        if _Conv1D and isinstance(self.layer, _Conv1D):
            W = W.t()
        W = W.float().contiguous()
        tick = time.time()

        q = self.braq_quantizer
        method = getattr(q, "method", None)
        if method not in _lib.METHODS:
            raise NotImplementedError(f"method {method!r} is outside the crbq hot path")
        # bigptq.py:94-99: non-integer methods clear any stale global scale
        if hasattr(q, "global_scale"):
            q.global_scale = None
        if hasattr(q, "global_zero"):
            q.global_zero = None
        assert q.groupsize % blocksize == 0                            # bigptq.py:147

        if self._S is None:
            raise RuntimeError("fasterquant called twice or after free()")
        scale = 2.0 / self.nsamples if self.nsamples else 0.0
        H = kernels.hessian_finalize(self._S, scale, self._S)          # in place
        self._S = None                                                 # bigptq.py:101 del self.H
        U, retries, fallback = kernels.hinv_upper(H, W, percdamp)
        del H
        losses = torch.zeros(self.rows, device=self.dev)
        p = _lib.params(method, metric=self.salient_metric, blocksize=blocksize,
                        partition=partition, orders=orders,
                        up_lim=50, refine_iters=getattr(q, "refine_iters", 1),
                        disable_gptq=self.disable_gptq, lam=getattr(q, "lam", 1e-5),
                        corr_damp=getattr(q, "corr_damp", 0.1))
        kernels.fasterquant_blocks(W, U, p, losses)

        torch.cuda.synchronize()
        err = torch.sum(losses).item()
        print("time %.2f" % (time.time() - tick))
        print("error", err)
        self.last = {"retries": retries, "fallback": fallback, "time_s": time.time() - tick}

        if _Conv1D and isinstance(self.layer, _Conv1D):
            W = W.t()
        self.layer.weight.data = W.reshape(self.layer.weight.shape).to(
            self.layer.weight.data.dtype)
        del U
        return {"error": err}

    def free(self):
        self._S = None
        torch.cuda.empty_cache()
