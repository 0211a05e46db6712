"""BASELINE configs[2] on the GPU: the OPT-6.7B shapes the headline metric
is quoted on (hidden 4096, ffn 16384, 128 x 2048 calibration tokens).

1. One full decoder layer through the layer driver (LayerQuantizer, the path
   bench.py times): k/v/q/out_proj 4096 x 4096, fc1 16384 x 4096 and
   fc2 4096 x 16384, fp16 weights W ~ N(0, 0.02^2), seeded fp16 activations
   with Student-t(4) channel scales.
   * GPTQ identity per sublayer, sum_j e_j^2 / 2 = (W0 - Q) H_d (W0 - Q)^T / 2
     (H_d the damped Hessian, the left side the loss the block loop
     accumulates, bigptq.py:240-262), within 1e-3 relative: it holds where
     U, the upper Cholesky factor of H_d^-1, is near-diagonal inside each
     128-column block, as these near-diagonal Hessians give;
   * the exact forms: U^-1 U^-T = H_d to 1e-5 and W0 - Q = E U' to 1e-5
     (gpu_helpers.u_checks).
   * every quantized sublayer packs (shared salient columns, at most 2 / 4
     values per group apart from rare ties at a group mean) and unpacks
     bit-exactly.
   * elementwise parity on the first 4 column blocks of q_proj (4096 rows)
     and fc1 (16384 rows) against the CPU oracle (bigptq.py:131-264)
     started from the same U and W: >= 99.99 % of weights within 1e-4
     relative, and the salient count / split of every block identical to
     the oracle's unless the oracle's own candidate errors tie within 1e-5.
2. A two-layer OPT-6.7B-shaped model quantized by the stack driver
   (crb_amd/stack.py, default mode) from 128 x 2048 random token ids
   propagated through the layers (run.py:122-387), for every sublayer of
   both layers: U^-1 U^-T = H_d to 1e-5 (the factor's backward error) and
   W0 - Q = E U' with sum(E^2) / 2 = the accumulated loss to 1e-5 (the
   block loop's error feedback; U' defined in gpu_helpers.u_checks), both evaluated in
   float64.  The H_d-metric form above is printed but not asserted here:
   it assumes feedback inside each block too, which the reference's
   pre-quantize-then-read path (bigptq.py:235-262) does not do, so it only
   holds where the in-block entries of U are small (near-diagonal
   Hessians, as the synthetic activations of test 1 give); the real
   activations' Hessians are strongly correlated.
"""
import numpy as np
import pytest
import torch

from crb_amd import synth
from gpu_helpers import acts as _acts
from gpu_helpers import u_checks as _u_checks
from oracle import crb_oracle as O

pytestmark = pytest.mark.gpu
DEV = "cuda:0"
NTOK = 128 * 2048
NBLK = 4


def _identity(W0, Q, Hd, err):
    """(W0 - Q) H_d (W0 - Q)^T / 2 summed over rows, against the block loop's
    summed loss: relative difference.  The quadratic form is evaluated in
    float64: GPTQ pushes W0 - Q towards the small-eigenvalue directions of
    H_d, so an fp32 product would cancel most of its digits."""
    D = (W0 - Q).double()
    Hd64 = Hd.double()
    quad = 0.0
    for r0 in range(0, D.shape[0], 2048):
        d = D[r0:r0 + 2048]
        quad += float(((d @ Hd64) * d).sum()) / 2
    return abs(quad - err) / err


def _pack_check(name, Q, masks):
    from crb_amd import kernels
    Wq = Q.half().contiguous()
    codes, lut, sal, ex = kernels.pack(Wq, masks)
    n_ex = int(ex.idx.numel())
    back = kernels.unpack(codes, lut, sal, Q.shape[1], ex)
    assert torch.equal(back.view(torch.int16), Wq.view(torch.int16)), name
    assert n_ex * 10000 <= Wq.numel(), (name, n_ex)
    return n_ex


def _first_blocks(name, W0, Qd, H, p):
    """First NBLK blocks of one sublayer: the oracle's block loop started
    from the GPU's U and the same W, against the driver's output."""
    from crb_amd import kernels
    U, retries, fb = kernels.hinv_upper(H.clone(), None, 0.01)
    assert retries == 0 and not fb
    nc = NBLK * 128
    # the GPU's per-block choices: its block loop on the first NBLK blocks
    Wsub = W0[:, :nc].clone()
    lo = torch.zeros(W0.shape[0], device=DEV)
    _, tr = kernels.fasterquant_blocks(Wsub, U[:nc, :nc].contiguous(), p, lo, want_traces=True)
    same = bool(torch.equal(Wsub, Qd[:, :nc]))
    trace = []
    Wr, _, _, _, _ = O.fasterquant(W0.cpu(), None, method="crb", U0=U.cpu(), max_blocks=NBLK,
                                   trace=trace)
    Wr = Wr[:, :nc]
    Wg = Qd[:, :nc].cpu()
    close = (Wg - Wr).abs() <= 1e-4 * Wr.abs() + 1e-7
    agree = float(close.float().mean())
    print(f"  {name}: first {NBLK} blocks agree {agree:.6f}, identical "
          f"{float((Wg == Wr).float().mean()):.6f}, driver == block-loop sub-run: {same}",
          flush=True)
    for b, (t_o, t_g) in enumerate(zip(trace, tr)):
        so = t_o.search
        print(f"    block {b}: i* {t_g['i_star']} vs {so.i_star}, k* {t_g['k_star']} vs "
              f"{so.k_star}", flush=True)
        if t_g["i_star"] != so.i_star:
            ea = np.asarray(so.errs_a)
            assert abs(ea[t_g["i_star"] - 1] - ea[so.i_star - 1]) <= 1e-5 * ea[so.i_star - 1]
        elif t_g["k_star"] != so.k_star:
            ec = np.asarray(so.errs_c)
            assert abs(ec[t_g["k_star"]] - ec[so.k_star]) <= 1e-5 * ec[so.k_star]
    assert agree >= 0.9999, agree


def test_opt67b_layer_driver():
    from crb_amd import _lib
    from crb_amd.driver import LayerQuantizer, Sublayer
    print("OPT-6.7B layer through the layer driver", flush=True)
    subs = synth.opt_sublayers("opt-6.7b")
    W0 = {}
    for j, (name, r, c, grp) in enumerate(subs):
        g = torch.Generator(device=DEV).manual_seed(500 + j)
        W0[name] = (torch.randn(r, c, generator=g, device=DEV) * 0.02).half().float()
    sl = [Sublayer(name, W0[name].clone(), grp) for name, r, c, grp in subs]
    lq = LayerQuantizer(sl, method="crb", keep_masks=True, keep_factors=True)
    H = {}
    for j, grp in enumerate(("qkv", "out", "fc1", "fc2")):
        C = 16384 if grp == "fc2" else 4096
        x = _acts(C, 600 + j)
        lq.add_batch(grp, x.view(128, 2048, C))
        # an undamped copy of the Hessian for the first-block checks
        from crb_amd import kernels
        S = torch.zeros(C, C, device=DEV)
        kernels.hessian_accum(x, S)
        H[grp] = kernels.hessian_finalize(S, 2.0 / 128, S)
        del x
    errs = lq.quantize()
    torch.cuda.synchronize()
    for name, r, c, grp in subs:
        Hd, U = lq.factors[grp]
        Q, losses = lq.quantized[name]
        assert abs(float(losses.sum()) - errs[name]) <= 1e-6 * errs[name]
        rel = _identity(W0[name], Q, Hd, errs[name])
        back, loop = _u_checks(W0[name], Q, Hd, U, errs[name])
        n_ex = _pack_check(name, Q, lq.masks[name])
        print(f"  {name} {r}x{c}: error {errs[name]:.6g}, identity rel {rel:.2e}, "
              f"U backward {back:.2e}, loop rel {loop:.2e}, {n_ex} pack exceptions",
              flush=True)
        assert rel < 1e-3, (name, rel)
        assert back < 1e-5 and loop < 1e-5, (name, back, loop)
    p = _lib.params("crb")
    for name in ("self_attn.q_proj", "fc1"):
        grp = next(gg for n, _, _, gg in subs if n == name)
        _first_blocks(name, W0[name], lq.quantized[name][0], H[grp], p)


def test_opt67b_two_layer_stack():
    transformers = pytest.importorskip("transformers")
    from crb_amd.driver import LayerQuantizer
    from crb_amd.stack import StackQuantizer
    print("OPT-6.7B two-layer stack, 128 x 2048 token ids", flush=True)
    results = []

    class Checked(LayerQuantizer):
        def quantize(self, times=None):
            w0 = {s.name: s.weight.float() for s in self.sublayers}
            errs = super().quantize(times)
            for s in self.sublayers:
                Hd, U = self.factors[s.group]
                Q, _ = self.quantized[s.name]
                rel = _identity(w0[s.name], Q, Hd, errs[s.name])
                back, loop = _u_checks(w0[s.name], Q, Hd, U, errs[s.name])
                d = torch.diagonal(Hd).double()
                results.append((s.name, errs[s.name], back, loop))
                print(f"  {s.name}: error {errs[s.name]:.6g}, U backward {back:.2e}, loop "
                      f"rel {loop:.2e} (H_d identity rel {rel:.2e}, diag max/min "
                      f"{float(d.max() / d.min()):.3g})", flush=True)
            self.factors, self.quantized = {}, {}
            return errs

    torch.manual_seed(0)
    cfg = transformers.OPTConfig(hidden_size=4096, ffn_dim=16384, num_attention_heads=32,
                                 num_hidden_layers=2, max_position_embeddings=2048,
                                 vocab_size=50272, word_embed_proj_dim=4096)
    with torch.device(DEV):
        model = transformers.OPTForCausalLM(cfg).half().eval()
    g = torch.Generator().manual_seed(1)
    samples = torch.randint(0, cfg.vocab_size, (128, 2048), generator=g).to(DEV)
    stats = StackQuantizer(model, layer_quantizer=Checked, keep_factors=True).run(samples)
    assert len(stats) == 2 and len(results) == 12
    for name, err, back, loop in results:
        assert err > 0 and back < 1e-5 and loop < 1e-5, (name, err, back, loop)


def test_opt67b_stack_default_vs_per_call():
    """One OPT-6.7B-shaped decoder layer (hidden 4096, ffn 16384) from
    128 x 2048 random token ids, quantized by the stack driver's default mode
    (chunks of 8 samples, one Hessian call per input over all 262144 tokens)
    and by its per-call mode (one forward and one add_batch per sample:
    128 Hessian calls per input, run.py:341-374's order), from the same layer
    input, plus per-call mode with 2 samples per call (64 calls): a third,
    equally valid summation order that measures the noise floor.  The
    Hessians differ by fp32 summation order only (~1e-7 relative), but the
    random-init model's activations give strongly correlated Hessians on
    which such differences move near-tied block choices (salient count,
    split), so each sublayer's error moves by up to ~1e-2 in either
    direction between any two orders.  The layer's reconstruction error
    sum_s ||(W_s - Q_s) X_s^T||_F^2 over the calibration tokens
    ((nseq / 2) sum((D H) * D), H the undamped Hessian recovered from the
    damped one, H_d = H + 0.01 mean(diag H) I, the 1-sample per-call run's H
    for all three) is printed for all three orders.  Bars: the default
    mode's layer error no more than 1e-3 above the per-call mode's (it may
    be lower), and within 5e-3 of it both ways."""
    transformers = pytest.importorskip("transformers")
    from crb_amd.driver import LayerQuantizer
    from crb_amd.stack import StackQuantizer
    print("OPT-6.7B layer: stack default mode vs per-call mode", flush=True)
    rec = {}

    def recorder(tag):
        class Rec(LayerQuantizer):
            def quantize(self, times=None):
                w0 = {s.name: s.weight.float() for s in self.sublayers}
                errs = super().quantize(times)
                for s in self.sublayers:
                    Hd, _ = self.factors[s.group]
                    Q, _ = self.quantized[s.name]
                    rec[(tag, s.name)] = (w0[s.name], Q.clone(), Hd if tag == "per_call" else None,
                                          errs[s.name])
                self.factors, self.quantized = {}, {}
                return errs
        return Rec

    def model():
        torch.manual_seed(0)
        cfg = transformers.OPTConfig(hidden_size=4096, ffn_dim=16384, num_attention_heads=32,
                                     num_hidden_layers=1, max_position_embeddings=2048,
                                     vocab_size=50272, word_embed_proj_dim=4096)
        with torch.device(DEV):
            return transformers.OPTForCausalLM(cfg).half().eval()

    g = torch.Generator().manual_seed(1)
    samples = torch.randint(0, 50272, (128, 2048), generator=g).to(DEV)
    x = None
    for tag, chunk, defer in (("default", 8, True), ("per_call", 1, False),
                              ("per_call2", 2, False)):
        q = StackQuantizer(model(), chunk=chunk, defer_hessian=defer,
                           layer_quantizer=recorder(tag), keep_factors=True)
        xc = q.capture(samples)
        if x is None:
            x = xc
        else:
            assert torch.equal(xc, x)
        del xc
        q.quantize_layer(0, x, None)
        del q
        torch.cuda.empty_cache()
    del x
    tags = ("default", "per_call", "per_call2")
    names = [k for t, k in rec if t == "per_call"]
    tot = {t: 0.0 for t in tags}
    for k in names:
        w0, _, hd, _ = rec[("per_call", k)]
        hd64 = hd.double()
        lam = 0.01 * float(torch.diagonal(hd64).mean()) / 1.01
        h64 = hd64 - lam * torch.eye(hd.shape[0], dtype=torch.float64, device=DEV)
        r = {}
        for tag in tags:
            q, e = rec[(tag, k)][1], rec[(tag, k)][3]
            v = 0.0
            d = (w0 - q).double()
            for r0 in range(0, d.shape[0], 2048):
                dd = d[r0:r0 + 2048]
                v += float(((dd @ h64) * dd).sum()) * 128 / 2
            r[tag] = v
            tot[tag] += v
        print(f"  {k}: recon^2 default {r['default']:.6g} per-call {r['per_call']:.6g} "
              f"per-call(2) {r['per_call2']:.6g}; default vs per-call "
              f"{(r['default'] - r['per_call']) / r['per_call']:+.2e}, per-call(2) vs per-call "
              f"{(r['per_call2'] - r['per_call']) / r['per_call']:+.2e}", flush=True)
        del h64, hd64
    f = {t: tot[t] ** 0.5 for t in tags}
    d_def = (f["default"] - f["per_call"]) / f["per_call"]
    d_two = (f["per_call2"] - f["per_call"]) / f["per_call"]
    print(f"  layer ||(W - Q) X^T||_F default {f['default']:.6g} per-call {f['per_call']:.6g} "
          f"per-call(2) {f['per_call2']:.6g}: default vs per-call {d_def:+.2e}, per-call(2) vs "
          f"per-call {d_two:+.2e}", flush=True)
    assert d_def <= 1e-3, d_def
    assert abs(d_def) < 5e-3, d_def
