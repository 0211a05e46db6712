"""The run.py-compatible command line (crb_amd/run.py) on the CPU: its
defaults are run.py's (run.py:764-873), the flags reach the quantizer as
run.py:326-374 passes them (Binarization(method, groupsize=blocksize,
corr_damp, lam), BRAGPTQ(salient_metric, disable_gptq),
fasterquant(percdamp, blocksize, partition)), and the layer filter is
run.py:332-336's.  A stub stands in for the GPU layer quantizer."""
import itertools

import pytest
import torch

transformers = pytest.importorskip("transformers")

from crb_amd import run as cli  # noqa: E402


def test_defaults_are_run_py_defaults():
    a = cli.build_parser().parse_args(["facebook/opt-6.7b", "synthetic", "crb"])
    assert (a.seed, a.nsamples, a.percdamp, a.blocksize, a.salient_metric, a.partition,
            a.disable_gptq, a.minlayer, a.maxlayer, a.quant_only, a.invert, a.corr_damp,
            a.lam, a.coupling) == (0, 128, 0.01, 128, "magnitude", 3, False, -1, 1000, "",
                                   False, 0.1, 1e-5, 0.5)
    assert cli.model_key("facebook/opt-6.7b") == "opt-6.7b"
    assert cli.model_key("meta-llama/Meta-Llama-3-8B") == "llama-3-8b"
    with pytest.raises(SystemExit):
        cli.build_parser().parse_args(["opt-6.7b", "synthetic", "xnor"])


def test_name_filter_is_run_py_condition():
    names = ["self_attn.q_proj", "self_attn.k_proj", "fc1", "fc2"]
    for mn, mx, q, inv in itertools.product([-1, 1], [1, 1000], ["", "fc", "q_proj"],
                                            [False, True]):
        a = cli.build_parser().parse_args(
            ["opt-125m", "synthetic", "braq", "--minlayer", str(mn), "--maxlayer", str(mx),
             "--quant_only", q] + (["--invert"] if inv else []))
        keep = cli.name_filter(a)
        for i in range(3):
            for n in names:
                skip = (not (mn <= i < mx and q in n)) == (not inv)     # run.py:332-336
                assert keep(i, n) == (not skip), (mn, mx, q, inv, i, n)


class Recorder:
    """LayerQuantizer stand-in that records its arguments and leaves the
    weights unchanged."""
    calls = []

    def __init__(self, sublayers, **kw):
        self.sublayers = list(sublayers)
        Recorder.calls.append(({s.name for s in self.sublayers}, kw))

    def add_batch(self, group, inp):
        pass

    def quantize(self, times=None):
        return {s.name: 0.0 for s in self.sublayers}


def test_flags_reach_the_quantizer():
    a = cli.build_parser().parse_args(
        ["tiny-opt", "synthetic", "crb_symdamp", "--blocksize", "64", "--salient_metric",
         "hessian", "--percdamp", "0.02", "--partition", "1", "--disable_gptq",
         "--corr_damp", "0.2", "--lam", "1e-4", "--refine_iters", "3", "--maxlayer", "1",
         "--quant_only", "fc", "--nsamples", "4", "--seqlen", "32", "--device", "cpu"])
    kw = cli.stack_kwargs(a)
    from crb_amd.stack import StackQuantizer
    model = cli.build_model("tiny-opt", None, torch.device("cpu"), 0).float()
    samples = cli.calibration(a, model.config.vocab_size, 32)
    assert samples.shape == (4, 32)
    Recorder.calls = []
    StackQuantizer(model, layer_quantizer=Recorder, **kw).run(samples)
    assert len(Recorder.calls) == 1                      # layer 0 only, fc1 and fc2
    names, got = Recorder.calls[0]
    assert names == {"fc1", "fc2"}
    assert got == dict(method="crb_symdamp", metric="hessian", blocksize=64, percdamp=0.02,
                       partition=1, orders=(1, 1, 2), refine_iters=3, lam=1e-4,
                       corr_damp=0.2, disable_gptq=True)
