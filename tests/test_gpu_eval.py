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
