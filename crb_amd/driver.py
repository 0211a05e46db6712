"""Per-decoder-layer quantization driver (the caller side of run.py:236-385).

run.py builds one BRAGPTQ per nn.Linear of a decoder layer, feeds every
sublayer's input through add_batch hooks, then calls fasterquant per
sublayer (run.py:326-374).  Sublayers that read the same activation
(q/k/v in OPT and Llama, gate/up in Llama) get identical Hessians and
therefore identical inverse factors U; this driver accumulates each
distinct input's Hessian once and factors it once, then runs every
sublayer's block loop.  The quantized weights are exactly what the
per-sublayer API computes.
"""
from __future__ import annotations

from dataclasses import dataclass, field

import torch

from . import _lib, kernels


@dataclass
class Sublayer:
    name: str
    weight: torch.Tensor        # [rows, cols] fp16/bf16/fp32, on the GPU (updated in place)
    group: str                  # name of the activation this sublayer reads


@dataclass
class PhaseTimes:
    hessian_ms: float = 0.0
    hinv_ms: float = 0.0
    blocks_ms: float = 0.0
    per_group: dict = field(default_factory=dict)


class LayerQuantizer:
    """Quantize the sublayers of one decoder layer with shared Hessians."""

    def __init__(self, sublayers, method="crb", metric="hessian", blocksize=128,
                 percdamp=0.01, partition=3, orders=(1, 1, 2), refine_iters=1,
                 lam=1e-5, corr_damp=0.1, disable_gptq=False):
        self.sublayers = list(sublayers)
        self.p = _lib.params(method, metric=metric, blocksize=blocksize, partition=partition,
                             orders=orders, up_lim=50, refine_iters=refine_iters,
                             disable_gptq=disable_gptq, lam=lam, corr_damp=corr_damp)
        self.percdamp = percdamp
        dev = self.sublayers[0].weight.device
        self.dev = dev
        self.S = {}
        self.nsamples = {}
        for s in self.sublayers:
            if s.group not in self.S:
                C = s.weight.shape[1]
                self.S[s.group] = torch.zeros((C, C), dtype=torch.float32, device=dev)
                self.nsamples[s.group] = 0
        self.errors = {}
        self.info = {}

    def add_batch(self, group: str, inp: torch.Tensor) -> None:
        """bigptq.py:37-53 for every sublayer reading `group`."""
        if inp.dim() == 2:
            inp = inp.unsqueeze(0)
        nseq = inp.shape[0]
        kernels.hessian_accum(inp.reshape(-1, inp.shape[-1]), self.S[group])
        self.nsamples[group] += nseq

    def quantize(self, events: PhaseTimes | None = None) -> dict:
        """fasterquant for every sublayer; returns {name: error}."""
        def ev():
            e = torch.cuda.Event(enable_timing=True)
            e.record()
            return e

        e0 = ev() if events is not None else None
        U = {}
        for g, S in self.S.items():
            n = self.nsamples[g]
            H = kernels.hessian_finalize(S, 2.0 / n if n else 0.0, S)
            U[g] = H  # placeholder, replaced below
        # dead-column handling needs W: q/k/v share H, and a dead column of H
        # zeroes the same input column of every sublayer reading it, so
        # factor once and clear dead columns per sublayer.
        dead = {}
        for g in list(U.keys()):
            H = U[g]
            dead[g] = torch.diag(H) == 0
            Ug, retries, fb = kernels.hinv_upper(H, None, self.percdamp)
            U[g] = Ug
            self.info[g] = {"retries": retries, "fallback": fb}
            self.S[g] = None
            del H
        e1 = ev() if events is not None else None
        errs = {}
        Ws = []
        for s in self.sublayers:
            W = s.weight.float().contiguous() if s.weight.dtype != torch.float32 else s.weight
            if bool(dead[s.group].any()):
                W[:, dead[s.group]] = 0
            losses = torch.zeros(W.shape[0], device=self.dev)
            kernels.fasterquant_blocks(W, U[s.group], self.p, losses)
            Ws.append((s, W, losses))
        for s, W, losses in Ws:
            if s.weight.dtype != torch.float32:
                s.weight.copy_(W.to(s.weight.dtype))
        e2 = ev() if events is not None else None
        for s, W, losses in Ws:
            errs[s.name] = losses
        if events is not None:
            torch.cuda.synchronize()
            events.hinv_ms += e0.elapsed_time(e1)
            events.blocks_ms += e1.elapsed_time(e2)
        self.errors = {k: float(v.sum()) for k, v in errs.items()}
        return self.errors
