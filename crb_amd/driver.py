"""Per-decoder-layer quantization driver (the caller side of run.py:236-385).

run.py builds one BRAGPTQ per nn.Linear of a decoder layer, feeds every
sublayer's input through add_batch hooks, then calls fasterquant per
sublayer (run.py:326-374).  Every sublayer's Hessian is captured before any
weight changes, so the sublayers are independent; sublayers that read the
same activation (q/k/v in OPT and Llama, gate/up in Llama) get identical
Hessians and therefore identical inverse factors U.  This driver
  * accumulates each distinct input's Hessian once,
  * factors the distinct Hessians concurrently on separate HIP streams,
  * runs the sublayers' block loops concurrently on those streams,
and writes every quantized weight back in its own dtype.  The result is
what the per-sublayer API computes for each sublayer.
"""
from __future__ import annotations

from dataclasses import dataclass, field

import torch

from . import _lib, kernels

NSTREAMS = 4   # one per hardware queue (GPU_MAX_HW_QUEUES defaults to 4)


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
                 lam=1e-5, corr_damp=0.1, disable_gptq=False, nstreams=NSTREAMS):
        self.sublayers = list(sublayers)
        self.p = _lib.params(method, metric=metric, blocksize=blocksize, partition=partition,
                             orders=orders, up_lim=50, refine_iters=refine_iters,
                             disable_gptq=disable_gptq, lam=lam, corr_damp=corr_damp)
        self.percdamp = percdamp
        self.dev = self.sublayers[0].weight.device
        self.nstreams = max(1, int(nstreams))
        self.S = {}
        self.nsamples = {}
        for s in self.sublayers:
            if s.group not in self.S:
                C = s.weight.shape[1]
                self.S[s.group] = torch.zeros((C, C), dtype=torch.float32, device=self.dev)
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
        main = torch.cuda.current_stream(self.dev)
        streams = [torch.cuda.Stream(device=self.dev) for _ in range(self.nstreams)]
        start = torch.cuda.Event()
        start.record(main)
        for st in streams:
            st.wait_event(start)

        def ev(stream):
            e = torch.cuda.Event(enable_timing=True)
            e.record(stream)
            return e

        e0 = ev(main) if events is not None else None
        # distinct Hessians -> U, concurrently
        groups = list(self.S.keys())
        jobs, dead = {}, {}
        for gi, g in enumerate(groups):
            st = streams[gi % len(streams)]
            with torch.cuda.stream(st):
                n = self.nsamples[g]
                H = kernels.hessian_finalize(self.S[g], 2.0 / n if n else 0.0, self.S[g])
                dead[g] = torch.diag(H) == 0
                jobs[g] = kernels.hinv_upper_async(H, None, self.percdamp)
        U, has_dead = {}, {}
        for g in groups:
            Ug, retries, fb = kernels.hinv_upper_finish(jobs[g])   # synchronises g's stream
            U[g] = Ug
            has_dead[g] = bool(dead[g].any())
            self.info[g] = {"retries": retries, "fallback": fb}
        if events is not None:
            e1 = torch.cuda.Event(enable_timing=True)
            e1.record(main)
            for st in streams:
                main.wait_stream(st)
            e1b = ev(main)
        # every U is ready (finish synchronised its stream); block loops
        work = []
        for si, s in enumerate(self.sublayers):
            st = streams[si % len(streams)]
            U[s.group].record_stream(st)
            dead[s.group].record_stream(st)
            with torch.cuda.stream(st):
                if events is not None:
                    st.wait_stream(main)
                W = s.weight.float().contiguous() if s.weight.dtype != torch.float32 else s.weight
                if has_dead[s.group]:
                    W[:, dead[s.group]] = 0                      # bigptq.py:105
                losses = torch.zeros(W.shape[0], device=self.dev)
                kernels.fasterquant_blocks(W, U[s.group], self.p, losses)
                if s.weight.dtype != torch.float32:
                    s.weight.copy_(W.to(s.weight.dtype))
                work.append((s, W, losses))
        for st in streams:
            main.wait_stream(st)
        e2 = ev(main) if events is not None else None
        for s, W, losses in work:
            W.record_stream(main)
            losses.record_stream(main)
        self.S = {g: None for g in groups}
        self.errors = {s.name: float(losses.sum()) for s, W, losses in work}
        if events is not None:
            torch.cuda.synchronize()
            events.hinv_ms += e0.elapsed_time(e1b)
            events.blocks_ms += e1b.elapsed_time(e2)
        return self.errors
