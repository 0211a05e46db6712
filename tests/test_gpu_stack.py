"""The model-level driver (crb_amd/stack.py) against run.py's own loop
(run.py:175-385: per-sample forwards, one BRAGPTQ per nn.Linear fed by
forward hooks, fasterquant per sublayer, quantized second forward), both on
the GPU through the crbq kernels.

* chunk=1 with per-call Hessian updates makes the same calls in the same
  order, so weights and errors are bitwise equal.
* Batched forwards with one Hessian update per input over all tokens are
  compared with the same loop making one add_batch call per sublayer over
  all samples (the sum over tokens in the same order); the forwards of
  these models give bitwise-equal activations batched or per sample, so
  the results are again bitwise equal.  Per-sample vs. one-call Hessians
  differ by ~1e-7 relative (summation order), which flips 26 % of the
  binarized weights of the 512-channel fc2 of the OPT case (Hessian
  condition ~5e3): per-element parity needs the same summation order.
"""
import pytest
import torch
import torch.nn as nn

transformers = pytest.importorskip("transformers")
pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def tiny_model(kind, seed=0):
    torch.manual_seed(seed)
    if kind == "opt":
        from transformers import OPTConfig, OPTForCausalLM
        cfg = OPTConfig(hidden_size=128, ffn_dim=512, num_attention_heads=4,
                        num_hidden_layers=2, max_position_embeddings=256, vocab_size=200,
                        word_embed_proj_dim=128)
        return OPTForCausalLM(cfg).eval().to(DEV).half()
    from transformers import LlamaConfig, LlamaForCausalLM
    cfg = LlamaConfig(hidden_size=128, intermediate_size=384, num_attention_heads=4,
                      num_key_value_heads=2, num_hidden_layers=2, max_position_embeddings=256,
                      vocab_size=200)
    return LlamaForCausalLM(cfg).eval().to(DEV).to(torch.bfloat16)


@torch.no_grad()
def run_py_loop(model, samples, method="crb", per_call=True):
    """run.py:175-385, standard path, with the drop-in per-sublayer API.
    per_call=False hands each sublayer all samples' inputs in one add_batch."""
    from crb_amd import BRAGPTQ, Binarization
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
    kw = {k: v for k, v in cache["kw"].items() if k != "past_key_values"}
    kw["use_cache"] = False
    inps = torch.cat(cache["inps"])
    outs = torch.zeros_like(inps)
    errs = []
    for layer in layers:
        subset = find_linears(layer)
        gptq = {}
        for name in subset:
            q = Binarization(subset[name].weight, method=method, groupsize=128)
            gptq[name] = BRAGPTQ(subset[name], q, "hessian")
        got = {k: [] for k in subset}

        def hook(m, i, o, k):
            if per_call:
                gptq[k].add_batch(i[0].data, o.data)
            else:
                x = i[0].data
                got[k].append(x if x.dim() == 3 else x.unsqueeze(0))

        hooks = [subset[k].register_forward_hook(
            lambda m, i, o, k=k: hook(m, i, o, k)) for k in subset]
        for j in range(inps.shape[0]):
            layer(inps[j:j + 1], **kw)
        for h in hooks:
            h.remove()
        if not per_call:
            for k in subset:
                gptq[k].add_batch(torch.cat(got[k]), None)
        e = {}
        for name in subset:
            e[name] = gptq[name].fasterquant(percdamp=0.01, blocksize=128)["error"]
            gptq[name].free()
        errs.append(e)
        for j in range(inps.shape[0]):
            r = layer(inps[j:j + 1], **kw)
            outs[j:j + 1] = r[0] if isinstance(r, tuple) else r
        inps, outs = outs, inps
    return errs


def _samples(n=6, seq=96, seed=3):
    g = torch.Generator().manual_seed(seed)
    return torch.randint(0, 200, (n, seq), generator=g).to(DEV)


def test_stack_bitwise_equal_to_run_py_loop():
    print("stack opt chunk=1", flush=True)
    from crb_amd.stack import StackQuantizer
    samples = _samples()
    ref = tiny_model("opt")
    ref_errs = run_py_loop(ref, samples)
    model = tiny_model("opt")
    stats = StackQuantizer(model, chunk=1, defer_hessian=False).run(samples)
    assert stats[0].groups["self_attn.k_proj"] == ["self_attn.k_proj", "self_attn.v_proj",
                                                   "self_attn.q_proj"]
    for st, e in zip(stats, ref_errs):
        assert st.errors.keys() == e.keys()
        for k in e:
            assert abs(st.errors[k] - e[k]) <= 1e-6 * abs(e[k]), k
    for (n1, p1), (n2, p2) in zip(model.named_parameters(), ref.named_parameters()):
        assert torch.equal(p1, p2), n1


@pytest.mark.parametrize("kind,chunk", [("opt", 4), ("llama", 4), ("opt", 16)])
def test_stack_batched_equal_to_one_call_loop(kind, chunk):
    print(f"stack {kind} chunk={chunk} deferred", flush=True)
    from crb_amd.stack import StackQuantizer, find_linears
    samples = _samples(n=10, seq=240)
    ref = tiny_model(kind)
    ref_errs = run_py_loop(ref, samples, per_call=False)
    model = tiny_model(kind)
    stats = StackQuantizer(model, chunk=chunk, defer_hessian=True).run(samples)
    if kind == "llama":
        g = stats[0].groups
        assert g["self_attn.q_proj"] == ["self_attn.q_proj", "self_attn.k_proj",
                                         "self_attn.v_proj"]
        assert g["mlp.gate_proj"] == ["mlp.gate_proj", "mlp.up_proj"]
    bad = []
    for st, e in zip(stats, ref_errs):
        for k in e:
            d = abs(st.errors[k] - e[k]) / abs(e[k])
            print(f"  {k}: error rel diff {d:.2e}", flush=True)
            if d > 1e-6:
                bad.append((k, "error", d))
    layers_a = [find_linears(l) for l in model.model.decoder.layers] if kind == "opt" else \
        [find_linears(l) for l in model.model.layers]
    layers_b = [find_linears(l) for l in ref.model.decoder.layers] if kind == "opt" else \
        [find_linears(l) for l in ref.model.layers]
    for la, lb in zip(layers_a, layers_b):
        for k in la:
            wa, wb = la[k].weight.float(), lb[k].weight.float()
            same = (wa == wb).float().mean().item()
            rel = ((wa - wb).norm() / wb.norm()).item()
            print(f"  {k}: identical {same:.4f}, rel {rel:.2e}", flush=True)
            if same < 1.0:
                bad.append((k, same, rel))
    assert not bad, bad


def _opt(hidden, ffn, heads, seed=0):
    from transformers import OPTConfig, OPTForCausalLM
    torch.manual_seed(seed)
    cfg = OPTConfig(hidden_size=hidden, ffn_dim=ffn, num_attention_heads=heads,
                    num_hidden_layers=2, max_position_embeddings=512, vocab_size=200,
                    word_embed_proj_dim=hidden)
    return OPTForCausalLM(cfg).eval().to(DEV).half()


def test_stack_default_mode_vs_per_call_mode():
    """The stack driver's default mode (chunks of 8 samples, one Hessian
    call per input over all tokens) against per-sample forwards with
    per-call Hessian updates (run.py:341-374's order, which the first test
    shows bitwise equal to run.py's loop), layer by layer from the same
    layer inputs, on a case with tokens >> C (hidden 256, ffn 1024,
    64 x 256 = 16384 tokens).

    The two Hessians differ by fp32 summation order only (~1e-7 relative).
    Where no block's salient count or split sits on a near-tie of its
    candidate errors the two runs make the same choices and the losses
    agree to ~1e-7; where one does, the choice can resolve the other way
    and that sublayer's loss moves by up to a few percent (measured 3e-2
    on the ReLU-fed fc2), in either direction.  Bars: each layer's summed
    GPTQ loss (= (W0 - Q) H_d (W0 - Q)^T / 2, the reconstruction error in
    the damped-Hessian metric) within 1e-3 relative; each sublayer within
    5e-2; and most sublayers (>= 8 of 12) without any flipped choice
    (within 1e-5)."""
    print("stack default mode vs per-call mode", flush=True)
    from crb_amd.stack import StackQuantizer
    g = torch.Generator().manual_seed(9)
    samples = torch.randint(0, 200, (64, 256), generator=g).to(DEV)
    a = StackQuantizer(_opt(256, 1024, 4), chunk=8, defer_hessian=True)
    b = StackQuantizer(_opt(256, 1024, 4), chunk=1, defer_hessian=False)
    x = a.capture(samples)
    assert torch.equal(b.capture(samples), x)
    nxt = torch.empty_like(x)
    worst_layer, worst_sub, stable = 0.0, 0.0, 0
    for i in range(2):
        sa = a.quantize_layer(i, x, nxt)          # default mode; its outputs feed layer i+1
        sb = b.quantize_layer(i, x, None)         # per-call mode on the same inputs
        la, lb = sum(sa.errors.values()), sum(sb.errors.values())
        d = abs(la - lb) / lb
        worst_layer = max(worst_layer, d)
        print(f"  layer {i}: loss default {la:.6g} per-call {lb:.6g} rel {d:.2e}", flush=True)
        for k in sb.errors:
            ds = abs(sa.errors[k] - sb.errors[k]) / sb.errors[k]
            worst_sub = max(worst_sub, ds)
            stable += ds <= 1e-5
            print(f"    {k}: {sa.errors[k]:.6g} vs {sb.errors[k]:.6g} rel {ds:.2e}", flush=True)
        x, nxt = nxt, x
    assert worst_layer < 1e-3, worst_layer
    assert worst_sub < 5e-2, worst_sub
    assert stable >= 8, stable
