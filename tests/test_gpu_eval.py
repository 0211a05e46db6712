"""Perplexity (crb_amd/evaluate.py) of tiny random-init models on the GPU
before and after quantization by the stack driver, and with the quantized
linears packed (PackedLinear): the packed model decodes to the same weights,
so its perplexity matches the unpacked quantized model's up to fp16 sums."""
import pytest
import torch

pytest.importorskip("transformers")
pytestmark = pytest.mark.gpu


def _ids(n_tokens, vocab=200, seed=11):
    g = torch.Generator().manual_seed(seed)
    return torch.randint(0, vocab, (1, n_tokens), generator=g)


def test_ppl_quantized_and_packed():
    print("eval ppl tiny opt", flush=True)
    from test_gpu_stack import _samples, tiny_model
    from crb_amd.evaluate import eval_ppl
    from crb_amd.stack import StackQuantizer
    ids = _ids(5 * 96 + 7).to("cuda:0")
    dense = tiny_model("opt")
    p_dense = eval_ppl(dense, ids, 96, chunk=2)
    assert eval_ppl(dense, ids, 96, chunk=1) == pytest.approx(p_dense, rel=2e-3)
    samples = _samples(n=6, seq=96)
    q = tiny_model("opt")
    StackQuantizer(q, chunk=3).run(samples)
    p_q = eval_ppl(q, ids, 96, chunk=2)
    pk = tiny_model("opt")
    StackQuantizer(pk, chunk=3, pack=True).run(samples)
    p_pk = eval_ppl(pk, ids, 96, chunk=2)
    print(f"ppl dense {p_dense:.3f} quantized {p_q:.3f} packed {p_pk:.3f}", flush=True)
    assert all(map(lambda v: v == v and 1.0 < v < 1e4, (p_dense, p_q, p_pk)))
    assert p_pk == pytest.approx(p_q, rel=1e-2)
    assert p_q != p_dense


def test_ppl_llama_bf16():
    print("eval ppl tiny llama", flush=True)
    from test_gpu_stack import tiny_model
    from crb_amd.evaluate import eval_ppl
    m = tiny_model("llama")
    ids = _ids(3 * 64).to("cuda:0")
    a = eval_ppl(m, ids, 64, chunk=3)
    b = eval_ppl(m, ids, 64, chunk=1)
    assert a == pytest.approx(b, rel=5e-3) and 1.0 < a < 1e4


@torch.no_grad()
def _direct_ppl(model, ids, seqlen):
    """eval_ppl_utils.py:538-637's quantity with whole-model forwards:
    exp(sum_i CE(logits_i[:-1], ids_i[1:]) * seqlen / (n * seqlen)), the
    cross entropy taken on the model-dtype logits as the reference does
    (:620-625, then loss.float())."""
    import math
    n = ids.numel() // seqlen
    tot = 0.0
    for i in range(n):
        w = ids[:, i * seqlen:(i + 1) * seqlen]
        logits = model(w).logits
        loss = torch.nn.functional.cross_entropy(logits[0, :-1], w[0, 1:])
        tot += float(loss.float()) * seqlen
    return math.exp(tot / (n * seqlen))


@pytest.mark.parametrize("kind", ["opt", "llama"])
def test_ppl_matches_whole_model_forward_after_quantization(kind):
    """Layer-by-layer evaluation (eval_ppl) of a model quantized by the stack
    driver, dense and packed, against the same model's own forward on whole
    windows.  With chunk=1 each window goes through the same modules with
    the same shapes, so the two agree to fp32 rounding of the loss sum
    (1e-5); with chunks of 3 the batched products may round differently in
    fp16/bf16 (2e-3)."""
    print(f"eval ppl vs whole-model forward, {kind}", flush=True)
    from test_gpu_stack import _samples, tiny_model
    from crb_amd.evaluate import eval_ppl
    from crb_amd.stack import StackQuantizer
    ids = _ids(5 * 96 + 7).to("cuda:0")
    samples = _samples(n=6, seq=96)
    for pack in (False, True):
        m = tiny_model(kind)
        StackQuantizer(m, chunk=3, pack=pack).run(samples)
        want = _direct_ppl(m, ids, 96)
        got1 = eval_ppl(m, ids, 96, chunk=1)
        got3 = eval_ppl(m, ids, 96, chunk=3)
        print(f"  pack={pack}: direct {want:.5f} chunk1 {got1:.5f} chunk3 {got3:.5f}",
              flush=True)
        assert abs(got1 - want) <= 1e-5 * want
        assert abs(got3 - want) <= 2e-3 * want
