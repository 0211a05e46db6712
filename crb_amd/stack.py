"""Model-level quantization driver: the caller side of run.py:122-387
(``quant_sequential``, standard path).

For every decoder layer, in order:
  1. a forward pass over the calibration samples whose hooks feed every
     distinct sublayer input to a LayerQuantizer (run.py:341-353); q/k/v,
     and Llama's gate/up, read one activation and share one Hessian;
  2. fasterquant of every sublayer (run.py:355-374), through
     LayerQuantizer.quantize;
  3. a second forward pass with the quantized weights, whose outputs are the
     next layer's inputs (run.py:376-385).
The layer-0 inputs come from a Catcher that replaces layer 0 during model
forwards of the calibration samples (run.py:175-201).

Differences in mechanism, not in result:
  * all samples' activations stay in device memory, in two
    [nsamples, seqlen, hidden] buffers swapped after every layer, instead
    of moving layers and activations between host and device;
  * forwards run on chunks of ``chunk`` samples; chunk=1 with
    defer_hessian=False reproduces the reference's per-sample forwards and
    add_batch calls exactly;
  * sublayers that read one activation are found at run time: during the
    first chunk every hook keeps its input tensor alive, and inputs that are
    the same tensor object form one group;
  * with defer_hessian=True each group's inputs are copied into one
    [tokens, C] store and its Hessian is accumulated by one call over all
    tokens at quantization time (the per-call SYRK launches of many small
    chunks cost more than the copy);
  * with pack=True every quantized nn.Linear is replaced, after the layer's
    quantized forward, by a PackedLinear holding the same weights in 3
    bits each (crb_amd/packed.py);
  * the hooked pass only needs the sublayers' inputs, so after the first
    chunk it stops at the input of the last hooked sublayer to run (OPT's
    fc2, Llama's down_proj) instead of computing the layer output that
    run.py stores and then overwrites.
"""
from __future__ import annotations

import time
from dataclasses import dataclass, field

import torch
import torch.nn as nn

from . import kernels
from .driver import LayerQuantizer, PhaseTimes, Sublayer


def find_linears(module: nn.Module, name: str = "") -> dict:
    """modelutils.py:8-15 (find_layers) for nn.Linear, in module order."""
    if isinstance(module, nn.Linear):
        return {name: module}
    out = {}
    for n, child in module.named_children():
        out.update(find_linears(child, name + "." + n if name else n))
    return out


def decoder_layers(model: nn.Module) -> nn.ModuleList:
    """The decoder layer list of the families run.py:131-160 handles."""
    for path in ("model.decoder.layers", "model.layers", "gpt_neox.layers", "transformer.h"):
        obj = model
        try:
            for p in path.split("."):
                obj = getattr(obj, p)
        except AttributeError:
            continue
        if isinstance(obj, nn.ModuleList):
            return obj
    raise NotImplementedError(f"no decoder layer list found on {type(model).__name__}")


def _fit_batch(obj, b: int, b0: int):
    """Layer kwargs captured for a chunk of b0 samples, cut to b samples."""
    if torch.is_tensor(obj):
        return obj[:b] if obj.dim() > 0 and obj.shape[0] == b0 and b != b0 else obj
    if isinstance(obj, tuple):
        return tuple(_fit_batch(o, b, b0) for o in obj)
    if isinstance(obj, list):
        return [_fit_batch(o, b, b0) for o in obj]
    if isinstance(obj, dict):
        return {k: _fit_batch(v, b, b0) for k, v in obj.items()}
    return obj


def _first(out):
    return out[0] if isinstance(out, (tuple, list)) else out


class _Catch(Exception):
    pass


class _Clock:
    """Phase marks: HIP events on the current stream, or host time."""

    def __init__(self, cuda: bool):
        self.cuda = cuda
        self.marks = []
        self.mark()

    def mark(self):
        if self.cuda:
            e = torch.cuda.Event(enable_timing=True)
            e.record()
            self.marks.append(e)
        else:
            self.marks.append(time.perf_counter())

    def spans(self):
        if self.cuda:
            torch.cuda.synchronize()
            return [a.elapsed_time(b) for a, b in zip(self.marks, self.marks[1:])]
        return [(b - a) * 1e3 for a, b in zip(self.marks, self.marks[1:])]


@dataclass
class LayerStats:
    errors: dict
    groups: dict                      # group -> [sublayer names]
    capture_ms: float = 0.0           # hooked forwards (Hessian inputs)
    hessian_ms: float = 0.0           # deferred Hessian accumulation
    quantize_ms: float = 0.0          # inverse factors + block loops
    forward_ms: float = 0.0           # forward with the quantized weights
    packed_bytes: int = 0             # pack=True: bytes of the packed sublayers
    phase: PhaseTimes = field(default_factory=PhaseTimes)


class StackQuantizer:
    """Quantize the linear sublayers of a decoder stack in place."""

    def __init__(self, model, method="crb", salient_metric="hessian", blocksize=128,
                 percdamp=0.01, chunk=8, defer_hessian=True, name_filter=None,
                 pack=False, layer_quantizer=LayerQuantizer, **quant_kw):
        self.model = model
        self.layers = decoder_layers(model)
        self.method = method
        self.metric = salient_metric
        self.blocksize = blocksize
        self.percdamp = percdamp
        self.chunk = max(1, int(chunk))
        self.defer = bool(defer_hessian)
        self.name_filter = name_filter or (lambda i, name: True)
        self.layer_quantizer = layer_quantizer
        self.quant_kw = dict(quant_kw)
        self.pack = bool(pack)
        if self.pack:
            self.quant_kw["keep_masks"] = True
        self.kwargs = {}
        self.kw_batch = 0

    # -- run.py:175-201 ------------------------------------------------------
    @torch.no_grad()
    def capture(self, samples: torch.Tensor) -> torch.Tensor:
        """Layer-0 inputs [nsamples, seqlen, hidden] for token ids
        [nsamples, seqlen], and the layer kwargs of the first chunk."""
        layers = self.layers
        dev = samples.device
        n = samples.shape[0]
        store = {}

        class Catcher(nn.Module):
            def __init__(self, module):
                super().__init__()
                self.module = module

            def forward(self, inp, **kw):
                store["inp"] = inp
                store.setdefault("kw", kw)
                raise _Catch

        use_cache = getattr(self.model.config, "use_cache", None)
        if use_cache is not None:
            self.model.config.use_cache = False
        inps = None
        orig = layers[0]
        layers[0] = Catcher(orig)
        try:
            for j in range(0, n, self.chunk):
                try:
                    self.model(samples[j:j + self.chunk].to(dev))
                except _Catch:
                    pass
                x = store.pop("inp")
                if inps is None:
                    inps = torch.empty((n,) + tuple(x.shape[1:]), dtype=x.dtype, device=x.device)
                inps[j:j + x.shape[0]] = x
        finally:
            layers[0] = orig
            if use_cache is not None:
                self.model.config.use_cache = use_cache
        self.kwargs = store.get("kw", {})
        self.kwargs.pop("past_key_values", None)
        self.kwargs.pop("past_key_value", None)
        self.kwargs["use_cache"] = False
        self.kw_batch = min(self.chunk, n)
        return inps

    def _kw(self, b):
        return _fit_batch(self.kwargs, b, self.kw_batch)

    @torch.no_grad()
    def _forward(self, layer, inps, outs):
        n = inps.shape[0]
        for j in range(0, n, self.chunk):
            x = inps[j:j + self.chunk]
            y = _first(layer(x, **self._kw(x.shape[0])))
            if outs is not None:
                outs[j:j + x.shape[0]] = y

    # -- run.py:326-374 ------------------------------------------------------
    @torch.no_grad()
    def _capture_layer(self, i, layer, inps):
        """Hooked forwards of layer i.  Returns the LayerQuantizer, the
        groups and, with defer_hessian, the per-group token stores still to
        be handed to add_batch."""
        subset = {k: v for k, v in find_linears(layer).items() if self.name_filter(i, k)}
        n = inps.shape[0]
        seen, order = {}, []

        def probe(mod, args, name):
            seen[name] = args[0]
            order.append(name)

        hooks = [m.register_forward_pre_hook(lambda mod, args, name=k: probe(mod, args, name))
                 for k, m in subset.items()]
        try:
            x = inps[0:self.chunk]
            _first(layer(x, **self._kw(x.shape[0])))
        finally:
            for h in hooks:
                h.remove()
        # group sublayers by input tensor identity (all kept alive in `seen`)
        groups, rep = {}, {}
        for k in subset:
            t = seen[k]
            g = next((gname for gname, r in rep.items() if seen[r] is t), None)
            if g is None:
                g = k
                rep[g] = k
            groups.setdefault(g, []).append(k)
        sl = [Sublayer(k, subset[k].weight.data, g) for g, names in groups.items() for k in names]
        lq = self.layer_quantizer(sl, method=self.method, metric=self.metric,
                                  blocksize=self.blocksize, percdamp=self.percdamp,
                                  **self.quant_kw)
        stores = {}

        def feed(g, t, j, b):
            # b samples in this chunk; 2-D inputs (layers that flatten the
            # tokens before a linear) are [b * tokens, C]
            if t.dim() == 2:
                t = t.reshape(b, -1, t.shape[-1])
            if not self.defer:
                lq.add_batch(g, t)
                return
            st = stores.get(g)
            if st is None:
                per, C = t.shape[1], t.shape[2]
                if self._cm_ok(lq, t, n * per):
                    # channel-major store: the copy of each chunk into it is
                    # the Hessian's transpose (kernels.hessian_transpose)
                    buf = kernels.hessian_cm_store(n * per, C, t.dtype, t.device)
                    st = stores[g] = [buf, per, 0, True]
                else:
                    st = stores[g] = [torch.empty((n * per, C), dtype=t.dtype,
                                                  device=t.device), per, 0, False]
            per = st[1]
            if st[3]:
                kernels.hessian_transpose(t.reshape(-1, t.shape[-1]), st[0], j * per)
            else:
                st[0][j * per:(j + b) * per] = t.reshape(-1, t.shape[-1])
            st[2] += b

        b0 = min(self.chunk, n)
        for g in groups:
            feed(g, seen[rep[g]], 0, b0)
        del seen
        if n > self.chunk:
            # The layer's output is not needed here: the pass stops at the
            # input of the last hooked sublayer to run.
            cur = {}

            def stop(mod, args):
                raise _Catch

            hooks = [subset[rep[g]].register_forward_pre_hook(
                lambda mod, args, g=g: feed(g, args[0], cur["j"], cur["b"])) for g in groups]
            hooks.append(subset[order[-1]].register_forward_pre_hook(stop))
            try:
                for j in range(self.chunk, n, self.chunk):
                    x = inps[j:j + self.chunk]
                    cur["j"], cur["b"] = j, x.shape[0]
                    try:
                        layer(x, **self._kw(x.shape[0]))
                    except _Catch:
                        pass
            finally:
                for h in hooks:
                    h.remove()
        pending = [(g, (buf, per * nseq, nseq) if cm else buf.view(nseq, per, buf.shape[1]))
                   for g, (buf, per, nseq, cm) in stores.items()]
        return lq, groups, pending

    @staticmethod
    def _cm_ok(lq, t, ntok):
        """The deferred store can be the Hessian's channel-major operand:
        16-bit activations on the GPU, every chunk starting at a multiple of
        64 tokens (whole samples of a multiple of 64 tokens), and all tokens
        in one SYRK pass (at most 2^21 tokens and 8 GiB), so the update's
        sums are those of add_batch on the same tokens."""
        if not (t.is_cuda and t.dtype in (torch.float16, torch.bfloat16)):
            return False
        if not hasattr(lq, "add_batch_cm") or t.shape[1] % 64:
            return False
        rows = (t.shape[2] + 255) // 256 * 256
        ldt = (ntok + 63) // 64 * 64
        return ldt <= (1 << 21) and rows * ldt * 2 <= (1 << 33)

    @torch.no_grad()
    def quantize_layer(self, i: int, inps: torch.Tensor, outs: torch.Tensor | None) -> LayerStats:
        """Quantize layer i from its inputs; write the quantized layer's
        outputs to outs (if given)."""
        layer = self.layers[i]
        clock = _Clock(inps.is_cuda)
        if not any(self.name_filter(i, k) for k in find_linears(layer)):
            # nothing selected in this layer (run.py:332-336): its output only
            clock.mark()
            clock.mark()
            clock.mark()
            if outs is not None:
                self._forward(layer, inps, outs)
            clock.mark()
            stats = LayerStats(errors={}, groups={})
            stats.capture_ms, stats.hessian_ms, stats.quantize_ms, stats.forward_ms = \
                clock.spans()
            return stats
        lq, groups, pending = self._capture_layer(i, layer, inps)
        clock.mark()
        for g, x in pending:
            if isinstance(x, tuple):
                lq.add_batch_cm(g, *x)
            else:
                lq.add_batch(g, x)
        del pending
        clock.mark()
        stats = LayerStats(errors={}, groups=groups)
        stats.errors = lq.quantize(stats.phase if inps.is_cuda else None)
        clock.mark()
        if outs is not None:
            self._forward(layer, inps, outs)
        clock.mark()
        stats.capture_ms, stats.hessian_ms, stats.quantize_ms, stats.forward_ms = clock.spans()
        if self.pack:
            from .packed import PackedLinear, replace_linears
            subset = find_linears(layer)
            packed = {k: PackedLinear.from_linear(subset[k], lq.masks[k]) for k in lq.masks}
            replace_linears(layer, packed)
            stats.packed_bytes = sum(p.packed_bytes() for p in packed.values())
        return stats

    @torch.no_grad()
    def run(self, samples: torch.Tensor, layer_ids=None, verbose=False) -> list:
        """quant_sequential: capture, then every layer in order (run.py:236-385)."""
        inps = self.capture(samples)
        outs = torch.empty_like(inps)
        ids = list(range(len(self.layers))) if layer_ids is None else list(layer_ids)
        stats = []
        for i in ids:
            t0 = time.time()
            st = self.quantize_layer(i, inps, outs)
            stats.append(st)
            if verbose:
                print(f"layer {i}: capture {st.capture_ms:.1f} ms, Hessian "
                      f"{st.hessian_ms:.1f} ms, quantize {st.quantize_ms:.1f} ms, forward "
                      f"{st.forward_ms:.1f} ms "
                      f"({time.time() - t0:.2f} s)", flush=True)
            inps, outs = outs, inps
        return stats
