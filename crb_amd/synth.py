"""Seeded synthetic weights and calibration activations.

The reference quantizes pretrained checkpoints on wikitext2/ptb/c4
calibration (run.py:19-71, datautils.py:306-341), which need the network.
These generators produce inputs of the same shapes from fixed seeds, on the
CPU (bit-reproducible for a given torch version) or directly on a device.
"""
from __future__ import annotations

import torch

# Sublayer shapes (rows = out_features, cols = in_features), in the order
# find_layers() returns them for an OPT decoder layer (modelutils.py:8-15).
OPT_SHAPES = {
    "opt-125m": dict(hidden=768, ffn=3072),
    "opt-1.3b": dict(hidden=2048, ffn=8192),
    "opt-6.7b": dict(hidden=4096, ffn=16384),
    "opt-66b": dict(hidden=9216, ffn=36864),
}


def opt_sublayers(model: str):
    """[(name, rows, cols, input_group)] for one OPT decoder layer.
    input_group names the activation the sublayer's add_batch sees: q/k/v
    share one input, so their Hessians are identical."""
    s = OPT_SHAPES[model]
    h, f = s["hidden"], s["ffn"]
    return [
        ("self_attn.k_proj", h, h, "qkv"),
        ("self_attn.v_proj", h, h, "qkv"),
        ("self_attn.q_proj", h, h, "qkv"),
        ("self_attn.out_proj", h, h, "out"),
        ("fc1", f, h, "fc1"),
        ("fc2", h, f, "fc2"),
    ]


def llama3_8b_sublayers():
    h, kv, f = 4096, 1024, 14336
    return [
        ("self_attn.q_proj", h, h, "qkv"),
        ("self_attn.k_proj", kv, h, "qkv"),
        ("self_attn.v_proj", kv, h, "qkv"),
        ("self_attn.o_proj", h, h, "o"),
        ("mlp.gate_proj", f, h, "gateup"),
        ("mlp.up_proj", f, h, "gateup"),
        ("mlp.down_proj", h, f, "down"),
    ]


def gen(seed: int, device="cpu") -> torch.Generator:
    g = torch.Generator(device=device)
    g.manual_seed(seed)
    return g


def weight(rows, cols, seed, std=0.02, outlier_frac=0.0, outlier_scale=8.0,
           dtype=torch.float32, device="cpu"):
    """W ~ N(0, std^2); a seeded fraction of input columns scaled as outliers."""
    g = gen(seed, device)
    W = torch.randn(rows, cols, generator=g, device=device) * std
    n_out = int(round(outlier_frac * cols))
    if n_out:
        cols_idx = torch.randperm(cols, generator=g, device=device)[:n_out]
        W[:, cols_idx] *= outlier_scale
    return W.to(dtype)


def channel_scales(cols, seed, kind="lognormal", device="cpu"):
    g = gen(seed + 7919, device)
    if kind == "lognormal":
        return torch.exp(torch.randn(cols, generator=g, device=device))
    if kind == "student_t4":
        # |t_4| = |z| / sqrt(chi2_4 / 4)
        z = torch.randn(cols, generator=g, device=device)
        chi = (torch.randn(4, cols, generator=g, device=device) ** 2).sum(0)
        return (z / torch.sqrt(chi / 4.0)).abs() + 1e-3
    if kind == "unit":
        return torch.ones(cols, device=device)
    raise ValueError(kind)


def calibration(nseq, seqlen, cols, seed, kind="lognormal", dtype=torch.float32,
                device="cpu"):
    """X[nseq, seqlen, cols] = z * s_c with z ~ N(0,1) and per-channel s_c."""
    s = channel_scales(cols, seed, kind, device)
    g = gen(seed, device)
    X = torch.randn(nseq, seqlen, cols, generator=g, device=device) * s
    return X.to(dtype)


def cfg1(seed=0):
    """one 768x768 fp32 layer, 2% outlier columns x8,
    X = 16 seqs x 512 tokens x 768 with log-normal(0, 1) channel scales."""
    W = weight(768, 768, seed, outlier_frac=0.02, outlier_scale=8.0)
    X = calibration(16, 512, 768, seed + 1, kind="lognormal")
    return W, X
