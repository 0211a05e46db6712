"""Perplexity evaluation (crb_amd/evaluate.py, eval_ppl_utils.py:36-637) on
tiny random-init OPT and Llama models on the CPU, against the quantity the
reference computes written out with whole-model forwards:
ppl = exp(sum_i CE(logits_i[:-1], ids_i[1:]) * seqlen / (n * seqlen)).
The layer-by-layer propagation with captured layer kwargs must give the
same logits as the model's own forward."""
import math

import pytest
import torch

transformers = pytest.importorskip("transformers")


def tiny(kind, seed=0):
    torch.manual_seed(seed)
    if kind == "opt":
        from transformers import OPTConfig, OPTForCausalLM
        cfg = OPTConfig(hidden_size=64, ffn_dim=128, num_attention_heads=4, num_hidden_layers=2,
                        max_position_embeddings=128, vocab_size=97, word_embed_proj_dim=64)
        return OPTForCausalLM(cfg).eval()
    from transformers import LlamaConfig, LlamaForCausalLM
    cfg = LlamaConfig(hidden_size=64, intermediate_size=160, num_attention_heads=4,
                      num_key_value_heads=2, num_hidden_layers=2, max_position_embeddings=128,
                      vocab_size=97)
    return LlamaForCausalLM(cfg).eval()


@torch.no_grad()
def direct_ppl(model, ids, seqlen):
    n = ids.numel() // seqlen
    tot = 0.0
    for i in range(n):
        w = ids[:, i * seqlen:(i + 1) * seqlen]
        logits = model(w).logits
        loss = torch.nn.functional.cross_entropy(logits[0, :-1].double(), w[0, 1:])
        tot += float(loss) * seqlen
    return math.exp(tot / (n * seqlen))


@pytest.mark.parametrize("kind", ["opt", "llama"])
@pytest.mark.parametrize("chunk", [1, 3])
def test_ppl_matches_whole_model_forward(kind, chunk):
    from crb_amd.evaluate import eval_ppl
    model = tiny(kind)
    g = torch.Generator().manual_seed(5)
    ids = torch.randint(0, 97, (1, 7 * 48 + 13), generator=g)    # 7 windows and a tail
    got, nll = eval_ppl(model, ids, 48, chunk=chunk, return_nlls=True)
    assert nll.shape == (7,)
    want = direct_ppl(model, ids, 48)
    assert abs(got - want) <= 1e-5 * want, (got, want)
    # a random model predicts random tokens at about the vocabulary size
    assert 20 < got < 500


def test_uniform_logits_give_vocab_size():
    """With the output head zeroed every logit is equal, so each window's
    mean loss is log(vocab); weighted by seqlen and divided by
    nsamples * seqlen that gives ppl = vocab, whatever the token order."""
    from crb_amd.evaluate import eval_ppl
    model = tiny("opt")
    ids = torch.arange(0, 96 * 4).remainder(8).reshape(1, -1)
    with torch.no_grad():
        model.lm_head.weight.zero_()
    base = eval_ppl(model, ids, 96)
    assert abs(base - 97.0) < 1e-3                       # uniform logits: ppl = vocab
    g = torch.Generator().manual_seed(1)
    shuffled = ids[:, torch.randperm(ids.numel(), generator=g)]
    assert abs(eval_ppl(model, shuffled, 96) - 97.0) < 1e-3


def test_window_errors():
    from crb_amd.evaluate import eval_ppl
    model = tiny("opt")
    with pytest.raises(ValueError):
        eval_ppl(model, torch.zeros(1, 10, dtype=torch.long), 48)
    with pytest.raises(ValueError):
        eval_ppl(model, torch.zeros(1, 10, dtype=torch.long), 1)
