"""Perplexity of a causal LM over consecutive token windows, as the
reference evaluates its (fake-)quantized models: eval_ppl_utils.py
``opt_eval`` (:538-637), ``llama_eval`` (:36-134), ``qwen_eval`` /
``granite_eval`` (:136-340), ``pythia_eval`` (:342-439) and ``bloom_eval``
(:441-536).

The token stream is cut into nsamples = numel // seqlen windows.  Layer-0
inputs of every window come from a Catcher in place of layer 0; the windows
then run through the decoder layers one layer at a time; the family's final
norm and output head give the logits; each window contributes its mean
shifted cross entropy times seqlen, and the perplexity is
exp(sum / (nsamples * seqlen)) (the reference's weighting, which counts
seqlen tokens per window although seqlen - 1 are predicted).

Differences in mechanism, not in result: everything stays on the model's
device (the reference moves layers between host and device), and windows
run through a layer in chunks of ``chunk`` (chunk=1 is the reference's
per-window order).  Works on dense models and on models whose linears were
replaced by PackedLinear.
"""
from __future__ import annotations

import torch
import torch.nn as nn
import torch.nn.functional as F

from .stack import _Catch, _first, _fit_batch, decoder_layers


def _head(model: nn.Module):
    """(final modules applied in order, logit divisor) of the families the
    reference evaluates."""
    inner = getattr(model, "model", None)
    dec = getattr(inner, "decoder", None)
    if dec is not None and hasattr(dec, "final_layer_norm"):          # OPT (:620-625)
        mods = [dec.final_layer_norm]
        if getattr(dec, "project_out", None) is not None:
            mods.append(dec.project_out)
        return mods + [model.lm_head], 1.0
    if inner is not None and hasattr(inner, "norm"):                   # Llama/Qwen/Granite
        scale = float(getattr(model.config, "logits_scaling", 1.0) or 1.0)   # :311, :320
        return [m for m in (inner.norm, model.lm_head) if m is not None], scale
    if hasattr(model, "gpt_neox"):                                     # Pythia (:411-412)
        return [model.gpt_neox.final_layer_norm, model.embed_out], 1.0
    if hasattr(model, "transformer") and hasattr(model.transformer, "ln_f"):   # BLOOM
        return [model.transformer.ln_f, model.lm_head], 1.0
    raise NotImplementedError(f"no output head known for {type(model).__name__}")


@torch.no_grad()
def layer0_inputs(model: nn.Module, windows: torch.Tensor, chunk: int):
    """Layer-0 hidden states [nsamples, seqlen, hidden] of token windows
    [nsamples, seqlen] and the layer kwargs captured with the first chunk."""
    layers = decoder_layers(model)
    store = {}

    class Catcher(nn.Module):
        def __init__(self, module):
            super().__init__()
            self.module = module

        def forward(self, inp, **kw):
            store["inp"] = inp
            store.setdefault("kw", kw)
            raise _Catch

    n = windows.shape[0]
    use_cache = getattr(model.config, "use_cache", None)
    if use_cache is not None:
        model.config.use_cache = False
    inps = None
    orig = layers[0]
    layers[0] = Catcher(orig)
    try:
        for j in range(0, n, chunk):
            try:
                model(windows[j:j + chunk])
            except _Catch:
                pass
            x = store.pop("inp")
            if inps is None:
                inps = torch.empty((n,) + tuple(x.shape[1:]), dtype=x.dtype, device=x.device)
            inps[j:j + x.shape[0]] = x
    finally:
        layers[0] = orig
        if use_cache is not None:
            model.config.use_cache = use_cache
    kw = store.get("kw", {})
    kw.pop("past_key_values", None)
    kw.pop("past_key_value", None)
    kw["use_cache"] = False
    return inps, kw, min(chunk, n)


@torch.no_grad()
def eval_ppl(model: nn.Module, input_ids: torch.Tensor, seqlen: int, chunk: int = 8,
             return_nlls: bool = False):
    """Perplexity of ``model`` on the token stream ``input_ids`` ([1, T] as
    the reference's testenc.input_ids, or [T]) in windows of ``seqlen``."""
    if seqlen < 2:
        raise ValueError("seqlen must be at least 2")
    ids = input_ids.reshape(1, -1)
    nsamples = ids.numel() // seqlen
    if nsamples == 0:
        raise ValueError(f"{ids.numel()} tokens hold no window of {seqlen}")
    chunk = max(1, int(chunk))
    dev = next(model.parameters()).device
    windows = ids[:, :nsamples * seqlen].reshape(nsamples, seqlen).to(dev)
    inps, kw, kw_batch = layer0_inputs(model, windows, chunk)
    outs = torch.empty_like(inps)
    for layer in decoder_layers(model):
        for j in range(0, nsamples, chunk):
            x = inps[j:j + chunk]
            outs[j:j + x.shape[0]] = _first(layer(x, **_fit_batch(kw, x.shape[0], kw_batch)))
        inps, outs = outs, inps
    mods, scale = _head(model)
    nlls = []
    for j in range(0, nsamples, chunk):
        h = inps[j:j + chunk]
        for m in mods:
            h = m(h)
        logits = h / scale if scale != 1.0 else h
        for k in range(h.shape[0]):
            shift_logits = logits[k:k + 1, :-1, :].contiguous()
            shift_labels = windows[j + k:j + k + 1, 1:]
            loss = F.cross_entropy(shift_logits.view(-1, shift_logits.size(-1)),
                                   shift_labels.reshape(-1))
            nlls.append(loss.float() * seqlen)
    nll = torch.stack(nlls)
    ppl = float(torch.exp(nll.sum() / (nsamples * seqlen)))
    if return_nlls:
        return ppl, nll
    return ppl
