"""Per-decoder-layer quantization driver (the caller side of run.py:236-385).

run.py builds one BRAGPTQ per nn.Linear of a decoder layer, feeds every
sublayer's input through add_batch hooks, then calls fasterquant per
sublayer (run.py:326-374).  Every sublayer's Hessian is captured before any
weight changes, so the sublayers are independent; sublayers that read the
same activation (q/k/v in OPT and Llama, gate/up in Llama) get identical
Hessians and therefore identical inverse factors U.  This driver
  * accumulates each distinct input's Hessian once,
  * starts each distinct input's inverse factor on a stream of its own as
    soon as that input's Hessian is complete,
  * enqueues every sublayer's block loop right behind its factor (an event
    wait, no host synchronisation), the widest input's chain first and on
    a stream of its own since it is the longest,
  * runs the block loops of up to four sublayers of one weight shape
    (q/k/v/out, gate/up), each with its own input's factor, as one loop
    whose launches cover all of them (kernels.fasterquant_blocks_batched:
    the same results, a quarter of the launches for q/k/v/out),
  * checks the factorizations once at the end and, for an input whose
    Cholesky needed the reference's retries or fallback (bigptq.py:114-126),
    recomputes its sublayers with the final factor,
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
    quantize_ms: float = 0.0                     # inverse factors + block loops, overlapped
    hinv_ms: dict = field(default_factory=dict)  # per input: its inverse factor
    chain_ms: dict = field(default_factory=dict) # per input: factor + its sublayers' block loops


class LayerQuantizer:
    """Quantize the sublayers of one decoder layer with shared Hessians."""

    def __init__(self, sublayers, method="crb", metric="hessian", blocksize=128,
                 percdamp=0.01, partition=3, orders=(1, 1, 2), refine_iters=1,
                 lam=1e-5, corr_damp=0.1, disable_gptq=False, nstreams=NSTREAMS,
                 keep_masks=False, keep_factors=False, batch_sublayers=True):
        self.sublayers = list(sublayers)
        self.p = _lib.params(method, metric=metric, blocksize=blocksize, partition=partition,
                             orders=orders, up_lim=50, refine_iters=refine_iters,
                             disable_gptq=disable_gptq, lam=lam, corr_damp=corr_damp)
        self.percdamp = percdamp
        self.dev = self.sublayers[0].weight.device
        self.nstreams = max(1, int(nstreams))
        self.batch_sublayers = bool(batch_sublayers)
        self.keep_masks = bool(keep_masks)
        self.masks = {}            # keep_masks: name -> uint8 [R, C] mask codes 1/2/3
        # keep_factors (for checks): group -> (damped H, U), name -> (fp32
        # quantized weight before the cast to the layer dtype, per-row losses)
        self.keep_factors = bool(keep_factors)
        self.factors = {}
        self.quantized = {}
        self.S = {}
        self.nsamples = {}
        self.ready = {}
        self.syrk_ev = {}          # group -> (start, end) events around its Hessian updates
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
        self.nsamples[group] += nseq
        cur = torch.cuda.current_stream(self.dev)
        self._accum(group, inp, cur)
        ev = self.ready.get(group)
        if ev is None:
            ev = self.ready[group] = torch.cuda.Event()
        ev.record(cur)

    def add_batch_cm(self, group: str, xt: torch.Tensor, ntok: int, nseq: int) -> None:
        """add_batch for nseq sequences whose ntok tokens in total are
        already in a channel-major store (kernels.hessian_transpose), the
        same Hessian update as add_batch on those tokens."""
        self.nsamples[group] += nseq
        cur = torch.cuda.current_stream(self.dev)
        a = torch.cuda.Event(enable_timing=True)
        b = torch.cuda.Event(enable_timing=True)
        a.record(cur)
        kernels.hessian_accum_cm(xt, ntok, self.S[group].shape[0], self.S[group])
        b.record(cur)
        first = self.syrk_ev.get(group)
        self.syrk_ev[group] = (first[0] if first else a, b)
        ev = self.ready.get(group)
        if ev is None:
            ev = self.ready[group] = torch.cuda.Event()
        ev.record(cur)

    def _accum(self, group, inp, stream):
        """Hessian update of `group` on `stream`, bracketed by timing events."""
        a = torch.cuda.Event(enable_timing=True)
        b = torch.cuda.Event(enable_timing=True)
        a.record(stream)
        kernels.hessian_accum(inp.reshape(-1, inp.shape[-1]), self.S[group])
        b.record(stream)
        first = self.syrk_ev.get(group)
        self.syrk_ev[group] = (first[0] if first else a, b)

    def syrk_ms(self, group: str) -> float:
        """GPU time from the first to the last Hessian update of `group`
        (after the work has completed)."""
        a, b = self.syrk_ev[group]
        return a.elapsed_time(b)

    def _batches(self, groups):
        """The sublayers in the order their loops are enqueued (the widest
        input's first, larger weights first), and that order cut into
        batches: sublayers of one weight shape and dtype, whatever input
        they read, up to kernels.MAX_BATCH per batch, in order of first
        appearance (single sublayers when batching is off)."""
        order = sorted(self.sublayers, key=lambda s: (groups.index(s.group), -s.weight.numel()))
        if not self.batch_sublayers:
            return order, [[s] for s in order]
        buckets = {}
        for s in order:
            buckets.setdefault((tuple(s.weight.shape), s.weight.dtype), []).append(s)
        out = []
        for lst in buckets.values():
            for i in range(0, len(lst), kernels.MAX_BATCH):
                out.append(lst[i:i + kernels.MAX_BATCH])
        return order, out

    def _assign_streams(self, groups, batches):
        """The widest input gets stream 0 for its factor and the batches
        holding its sublayers; the other factors and batches share the
        remaining streams, balanced by weight count."""
        ns = self.nstreams
        gstream = {}
        for i, g in enumerate(groups):
            gstream[g] = 0 if i == 0 or ns == 1 else 1 + (i - 1) % (ns - 1)
        load = [0] * ns
        bstream = [0] * len(batches)
        for i in sorted(range(len(batches)), key=lambda i: -sum(s.weight.numel()
                                                               for s in batches[i])):
            b = batches[i]
            if ns == 1 or any(s.group == groups[0] for s in b):
                k = 0
            else:
                k = min(range(1, ns), key=lambda j: load[j])
            load[k] += sum(s.weight.numel() for s in b)
            bstream[i] = k
        return gstream, bstream

    def _blocks(self, batch, U, dead):
        """Block loops of one batch (U, dead: per input): {name: (W fp32,
        losses, masks)}."""
        Ws, ls = [], []
        for s in batch:
            W = s.weight.float() if s.weight.dtype != torch.float32 else s.weight.clone()
            W = W.contiguous()
            W.masked_fill_(dead[s.group][None, :], 0.0)                  # bigptq.py:105
            Ws.append(W)
            ls.append(torch.zeros(W.shape[0], device=self.dev))
        if len(batch) == 1:
            m, _ = kernels.fasterquant_blocks(Ws[0], U[batch[0].group], self.p, ls[0],
                                              want_masks=self.keep_masks)
            masks = [m]
        else:
            masks, _ = kernels.fasterquant_blocks_batched(Ws, [U[s.group] for s in batch],
                                                          self.p, ls, want_masks=self.keep_masks)
        return {s.name: (Ws[i], ls[i], masks[i]) for i, s in enumerate(batch)}

    def quantize(self, times: PhaseTimes | None = None) -> dict:
        """fasterquant for every sublayer; returns {name: error}."""
        main = torch.cuda.current_stream(self.dev)
        streams = [torch.cuda.Stream(device=self.dev) for _ in range(self.nstreams)]
        groups = sorted(self.S.keys(), key=lambda g: -self.S[g].shape[0])
        order, batches = self._batches(groups)
        gstream, bstream = self._assign_streams(groups, batches)
        t0 = torch.cuda.Event(enable_timing=True)
        t0.record(main)

        def timed(stream):
            e = torch.cuda.Event(enable_timing=times is not None)
            e.record(stream)
            return e

        jobs, dead, U, hdone, hstart = {}, {}, {}, {}, {}
        for g in groups:
            st = streams[gstream[g]]
            st.wait_event(self.ready[g] if g in self.ready else t0)
            with torch.cuda.stream(st):
                hstart[g] = timed(st)
                n = self.nsamples[g]
                H = kernels.hessian_finalize(self.S[g], 2.0 / n if n else 0.0, self.S[g])
                dead[g] = torch.diag(H) == 0
                jobs[g] = kernels.hinv_upper_async(H, None, self.percdamp)
                U[g] = jobs[g].U
                hdone[g] = timed(st)
        work, sdone = {}, {}
        # the widest input's sublayers first (their chain is the longest)
        for b, k in zip(batches, bstream):
            st = streams[k]
            for g in dict.fromkeys(s.group for s in b):
                st.wait_event(hdone[g])
                U[g].record_stream(st)
                dead[g].record_stream(st)
            with torch.cuda.stream(st):
                work.update(self._blocks(b, U, dead))
                e = timed(st)
            for s in b:
                sdone[s.name] = e
        torch.cuda.synchronize(self.dev)
        # the first attempt of every factorization has finished: read its
        # outcome; retries / fallback (rare) recompute U and its sublayers
        redo = set()
        for g in groups:
            Ug, retries, fb = kernels.hinv_upper_finish(jobs[g])
            self.info[g] = {"retries": retries, "fallback": fb}
            if retries or fb:
                redo.add(g)
                # the retries / fallback write U on the factor's stream and
                # return without waiting: the redo below runs on `main`
                main.wait_stream(jobs[g].stream)
        for b in batches:
            if any(s.group in redo for s in b):
                work.update(self._blocks(b, U, dead))
        if self.keep_factors:
            self.factors = {g: (jobs[g].H, U[g]) for g in groups}
            self.quantized = {s.name: (work[s.name][0], work[s.name][1]) for s in order}
        for s in order:
            W, losses, masks = work[s.name]
            if masks is not None:
                self.masks[s.name] = masks
            if s.weight.dtype != torch.float32:
                s.weight.copy_(W.to(s.weight.dtype))
            else:
                s.weight.copy_(W)
        self.S = {g: None for g in groups}
        self.errors = {s.name: float(work[s.name][1].sum()) for s in order}
        if times is not None:
            torch.cuda.synchronize(self.dev)
            times.quantize_ms += t0.elapsed_time(max(sdone.values(), key=lambda e: t0.elapsed_time(e)))
            for g in groups:
                times.hinv_ms[g] = hstart[g].elapsed_time(hdone[g])
                last = max((sdone[s.name] for s in order if s.group == g),
                           key=lambda e: t0.elapsed_time(e))
                times.chain_ms[g] = hstart[g].elapsed_time(last)
        return self.errors
