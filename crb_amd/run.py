"""Command line of the reference's quantization script (run.py:756-944) over
the crbq stack driver.

    python -m crb_amd.run facebook/opt-6.7b synthetic crb --blocksize 128 \\
        --salient_metric hessian [--layers 2] [--nsamples 128] [--seqlen 2048]

The positional arguments and the flags of the hot path keep run.py's names,
defaults and meaning:
  model             run.py:766; here the architecture of a known model name
                    (MODELS below), built with random-init fp16 weights
                    ~ N(0, 0.02^2) (there is no network for checkpoints)
  dataset           run.py:769-773; "synthetic" = seeded uniform token ids;
                    wikitext2 / ptb / c4 need --token_file (a local .npy or
                    .pt of token ids), as the datasets cannot be downloaded
  low_quant_method  run.py:775-780, the methods on this path:
                    crb, crbog, braq, crb_norefine, crb_symdamp,
                    crb_symdamp_norefine
  --seed --nsamples --seqlen --percdamp --blocksize --salient_metric
  --partition --disable_gptq --minlayer --maxlayer --quant_only --invert
  --corr_damp --lam --coupling --device   (run.py:782-873)
Each decoder layer's nn.Linear sublayers are quantized as run.py:326-374
does it: Binarization(method, groupsize=blocksize, corr_damp, lam,
coupling), BRAGPTQ(salient_metric, disable_gptq), fasterquant(percdamp,
blocksize, partition), with the minlayer / maxlayer / quant_only / invert
filter of run.py:332-336.  Extensions: --refine_iters (CRB sign-refinement
rounds; the reference has one), --layers (decoder layers to build), --pack
(3-bit packed storage), --eval_tokens (perplexity on held-out synthetic
windows, eval_ppl_utils.py:538-637).
"""
from __future__ import annotations

import argparse
import json
import sys
import time

import torch

# model name -> (family, hidden, ffn, heads, kv_heads, layers, vocab, max_pos)
MODELS = {
    "opt-125m": ("opt", 768, 3072, 12, 12, 12, 50272, 2048),
    "opt-1.3b": ("opt", 2048, 8192, 32, 32, 24, 50272, 2048),
    "opt-6.7b": ("opt", 4096, 16384, 32, 32, 32, 50272, 2048),
    "opt-66b": ("opt", 9216, 36864, 72, 72, 64, 50272, 2048),
    "llama-3-8b": ("llama", 4096, 14336, 32, 8, 32, 128256, 8192),
    "tiny-opt": ("opt", 128, 512, 4, 4, 2, 200, 512),
    "tiny-llama": ("llama", 128, 384, 4, 2, 2, 200, 512),
}
METHODS = ["crb", "crbog", "braq", "crb_norefine", "crb_symdamp", "crb_symdamp_norefine"]
DATASETS = ["synthetic", "wikitext2", "ptb", "c4"]


def model_key(name: str) -> str:
    """facebook/opt-6.7b, opt-6.7b, meta-llama/Meta-Llama-3-8B ... -> MODELS key."""
    n = name.lower().split("/")[-1].replace("meta-llama-3", "llama-3")
    if n not in MODELS:
        raise SystemExit(f"unknown model {name!r}: known architectures {sorted(MODELS)}")
    return n


def build_parser() -> argparse.ArgumentParser:
    p = argparse.ArgumentParser(prog="python -m crb_amd.run",
                                description="CRB layer-wise binarization on the crbq kernels")
    p.add_argument("model", type=str)
    p.add_argument("dataset", type=str, choices=DATASETS)
    p.add_argument("low_quant_method", type=str, choices=METHODS)
    p.add_argument("--seed", type=int, default=0)
    p.add_argument("--nsamples", type=int, default=128)
    p.add_argument("--seqlen", type=int, default=None)
    p.add_argument("--percdamp", type=float, default=0.01)
    p.add_argument("--blocksize", type=int, default=128)
    p.add_argument("--salient_metric", type=str, default="magnitude",
                   choices=["magnitude", "hessian"])
    p.add_argument("--partition", type=int, default=3, choices=[1, 3])
    p.add_argument("--device", type=str, default="cuda:0")
    p.add_argument("--disable_gptq", action="store_true")
    p.add_argument("--minlayer", type=int, default=-1)
    p.add_argument("--maxlayer", type=int, default=1000)
    p.add_argument("--quant_only", type=str, default="")
    p.add_argument("--invert", action="store_true")
    p.add_argument("--corr_damp", type=float, default=0.1)
    p.add_argument("--lam", type=float, default=1e-5)
    p.add_argument("--coupling", type=float, default=0.5)
    # extensions
    p.add_argument("--refine_iters", type=int, default=1)
    p.add_argument("--layers", type=int, default=None)
    p.add_argument("--chunk", type=int, default=8)
    p.add_argument("--pack", action="store_true")
    p.add_argument("--token_file", type=str, default=None)
    p.add_argument("--eval_tokens", type=int, default=0)
    return p


def name_filter(args):
    """run.py:332-336: a sublayer is quantized iff
    (minlayer <= i < maxlayer and quant_only in name) != invert."""
    def keep(i: int, name: str) -> bool:
        sel = args.minlayer <= i < args.maxlayer and args.quant_only in name
        return sel != args.invert
    return keep


def stack_kwargs(args) -> dict:
    """StackQuantizer arguments for the run.py flags: the Binarization and
    BRAGPTQ arguments run.py:337-349 passes, and fasterquant's
    (percdamp, blocksize, partition) of run.py:364-370 (orders stay
    (1, 1, 2), fasterquant's default)."""
    return dict(method=args.low_quant_method, salient_metric=args.salient_metric,
                blocksize=args.blocksize, percdamp=args.percdamp, chunk=args.chunk,
                name_filter=name_filter(args), pack=args.pack,
                partition=args.partition, orders=(1, 1, 2), refine_iters=args.refine_iters,
                lam=args.lam, corr_damp=args.corr_damp, disable_gptq=args.disable_gptq)


def build_model(key: str, nlayers: int | None, device, seed: int):
    fam, h, f, heads, kv, layers, vocab, maxpos = MODELS[key]
    nl = layers if nlayers is None else int(nlayers)
    torch.manual_seed(seed)
    if fam == "opt":
        from transformers import OPTConfig, OPTForCausalLM
        cfg = OPTConfig(hidden_size=h, ffn_dim=f, num_attention_heads=heads,
                        num_hidden_layers=nl, max_position_embeddings=maxpos,
                        vocab_size=vocab, word_embed_proj_dim=h)
        cls, dtype = OPTForCausalLM, torch.float16
    else:
        from transformers import LlamaConfig, LlamaForCausalLM
        cfg = LlamaConfig(hidden_size=h, intermediate_size=f, num_attention_heads=heads,
                          num_key_value_heads=kv, num_hidden_layers=nl,
                          max_position_embeddings=maxpos, vocab_size=vocab)
        cls, dtype = LlamaForCausalLM, torch.bfloat16
    with torch.device(device):
        model = cls(cfg).to(dtype).eval()
    model.seqlen = maxpos if fam == "opt" else min(maxpos, 2048)
    return model


def calibration(args, vocab: int, seqlen: int) -> torch.Tensor:
    """[nsamples, seqlen] token ids: seeded uniform ids, or nsamples random
    windows of a local token file (datautils.py's sampling of the train
    split, without the download)."""
    g = torch.Generator().manual_seed(args.seed)
    if args.dataset == "synthetic":
        return torch.randint(0, vocab, (args.nsamples, seqlen), generator=g)
    if not args.token_file:
        raise SystemExit(f"dataset {args.dataset!r} cannot be downloaded here: pass "
                         "--token_file with its token ids, or use 'synthetic'")
    if args.token_file.endswith(".npy"):
        import numpy as np
        ids = torch.from_numpy(np.load(args.token_file, allow_pickle=False)).reshape(-1)
    else:
        ids = torch.load(args.token_file, weights_only=True).reshape(-1)
    if ids.numel() <= seqlen:
        raise SystemExit("token file shorter than one window")
    starts = torch.randint(0, ids.numel() - seqlen - 1, (args.nsamples,), generator=g)
    return torch.stack([ids[s:s + seqlen] for s in starts.tolist()]).long()


def main(argv=None) -> dict:
    args = build_parser().parse_args(argv)
    if args.blocksize < 1 or args.blocksize > 128:
        raise SystemExit("--blocksize must be in 1..128 on this path")
    from .stack import StackQuantizer
    key = model_key(args.model)
    dev = torch.device(args.device)
    model = build_model(key, args.layers, dev, args.seed)
    seqlen = args.seqlen or model.seqlen
    samples = calibration(args, model.config.vocab_size, seqlen).to(dev)
    tick = time.time()
    sq = StackQuantizer(model, **stack_kwargs(args))
    stats = sq.run(samples, verbose=True)
    torch.cuda.synchronize(dev)
    qtime = time.time() - tick
    print("quantization time:", qtime, "s")                       # run.py:1015
    out = {"model": args.model, "method": args.low_quant_method, "layers": len(stats),
           "quantization_time_s": qtime,
           "errors": [st.errors for st in stats]}
    if args.eval_tokens:
        from .evaluate import eval_ppl
        g = torch.Generator().manual_seed(args.seed + 1)
        ids = torch.randint(0, model.config.vocab_size, (1, args.eval_tokens), generator=g)
        out["ppl"] = eval_ppl(model, ids.to(dev), seqlen, chunk=args.chunk)
        print("ppl", out["ppl"])
    print(json.dumps({k: v for k, v in out.items() if k != "errors"}))
    return out


if __name__ == "__main__":
    main(sys.argv[1:])
