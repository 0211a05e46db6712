"""Host logic of the model-level driver (crb_amd/stack.py) on the CPU, with a
stub layer quantizer: Catcher capture, sublayer grouping by shared input,
chunked forwards with batch-sized kwargs, deferred vs. per-call Hessian
inputs, the quantized second forward and the layer-to-layer handoff.  The
expected result is a plain restatement of run.py:175-385 (per-sample
forwards and hooks)."""
import pytest
import torch
import torch.nn as nn

transformers = pytest.importorskip("transformers")


class StubLayerQuantizer:
    """Same interface as LayerQuantizer: accumulates sum x x^T per group in
    float64, then rounds every weight row to sign(w) * mean|w| * (1 + tr(H) % 3
    / 10) so the result depends on the Hessian it was given."""
    log = []

    def __init__(self, sublayers, **kw):
        self.sublayers = list(sublayers)
        self.S, self.n = {}, {}

    def add_batch(self, group, inp):
        if inp.dim() == 2:
            inp = inp.unsqueeze(0)
        x = inp.reshape(-1, inp.shape[-1]).double()
        self.S[group] = self.S.get(group, 0) + x.t() @ x
        self.n[group] = self.n.get(group, 0) + inp.shape[0]

    def quantize(self, times=None):
        errs = {}
        for s in self.sublayers:
            S = self.S[s.group]
            f = 1.0 + float(torch.trace(S)) % 3 / 10
            W = s.weight.double()
            Q = torch.sign(W) * W.abs().mean(1, keepdim=True) * f
            errs[s.name] = float(((W - Q) ** 2).sum())
            s.weight.copy_(Q.to(s.weight.dtype))
            StubLayerQuantizer.log.append((s.name, s.group, self.n[s.group], float(torch.trace(S))))
        return errs


def tiny_opt(seed=0):
    from transformers import OPTConfig, OPTForCausalLM
    torch.manual_seed(seed)
    cfg = OPTConfig(hidden_size=32, ffn_dim=64, num_attention_heads=4, num_hidden_layers=2,
                    max_position_embeddings=64, vocab_size=50, word_embed_proj_dim=32)
    return OPTForCausalLM(cfg).eval()


@torch.no_grad()
def reference_loop(model, samples):
    """run.py:175-385 with per-sample forwards and per-sublayer add_batch."""
    from crb_amd.driver import Sublayer
    from crb_amd.stack import decoder_layers, find_linears
    layers = decoder_layers(model)
    cache = {}

    class Catcher(nn.Module):
        def __init__(self, m):
            super().__init__()
            self.module = m

        def forward(self, inp, **kw):
            cache.setdefault("inps", []).append(inp)
            cache["kw"] = kw
            raise ValueError

    model.config.use_cache = False
    layers[0] = Catcher(layers[0])
    for j in range(samples.shape[0]):
        try:
            model(samples[j:j + 1])
        except ValueError:
            pass
    layers[0] = layers[0].module
    kw = {k: v for k, v in cache["kw"].items() if k not in ("past_key_values",)}
    kw["use_cache"] = False
    inps = torch.cat(cache["inps"])
    outs = torch.zeros_like(inps)
    errs = []
    for layer in layers:
        subset = find_linears(layer)
        q = {k: StubLayerQuantizer([Sublayer(k, subset[k].weight.data, k)]) for k in subset}
        hooks = [subset[k].register_forward_hook(
            lambda m, i, o, k=k: q[k].add_batch(k, i[0])) for k in subset]
        for j in range(inps.shape[0]):
            layer(inps[j:j + 1], **kw)
        for h in hooks:
            h.remove()
        e = {}
        for k in subset:
            e.update(q[k].quantize())
        errs.append(e)
        for j in range(inps.shape[0]):
            r = layer(inps[j:j + 1], **kw)
            outs[j:j + 1] = r[0] if isinstance(r, tuple) else r
        inps, outs = outs, inps
    return errs


@pytest.mark.parametrize("chunk,defer", [(1, False), (1, True), (3, False), (3, True), (8, True)])
def test_stack_matches_reference_loop(chunk, defer):
    from crb_amd.stack import StackQuantizer
    g = torch.Generator().manual_seed(1)
    samples = torch.randint(0, 50, (5, 16), generator=g)
    ref_model = tiny_opt()
    StubLayerQuantizer.log = []
    ref_errs = reference_loop(ref_model, samples)
    model = tiny_opt()
    StubLayerQuantizer.log = []
    sq = StackQuantizer(model, chunk=chunk, defer_hessian=defer,
                        layer_quantizer=StubLayerQuantizer)
    stats = sq.run(samples)
    got_errs = [st.errors for st in stats]
    assert stats[0].groups == {"self_attn.k_proj": ["self_attn.k_proj", "self_attn.v_proj",
                                                    "self_attn.q_proj"],
                               "self_attn.out_proj": ["self_attn.out_proj"],
                               "fc1": ["fc1"], "fc2": ["fc2"]}
    # every group saw all samples, once
    assert all(n == samples.shape[0] for (_, _, n, _) in StubLayerQuantizer.log)
    for a, b in zip(got_errs, ref_errs):
        assert a.keys() == b.keys()
        for k in a:
            assert a[k] == pytest.approx(b[k], rel=1e-5), k
    for (n1, p1), (n2, p2) in zip(model.named_parameters(), ref_model.named_parameters()):
        assert n1 == n2
        assert torch.allclose(p1, p2, rtol=1e-5, atol=1e-6), n1


def test_fit_batch_cuts_batch_dim_only():
    from crb_amd.stack import _fit_batch
    kw = {"position_ids": torch.arange(12).view(3, 4), "mask": torch.zeros(3, 1, 4, 4),
          "pe": (torch.ones(3, 4, 2), torch.ones(3, 4, 2)), "flag": True,
          "other": torch.zeros(4, 3)}
    out = _fit_batch(kw, 2, 3)
    assert out["position_ids"].shape == (2, 4) and out["mask"].shape == (2, 1, 4, 4)
    assert out["pe"][0].shape == (2, 4, 2) and out["flag"] is True
    assert out["other"].shape == (4, 3)
