"""Size-independent properties at the BASELINE configs' full sizes
(configs[1] OPT-1.3B layer crb vs braq, configs[3] the whole OPT-66B layer
with fc2's 36864^2 Hessian, configs[4] Llama-3-8B layer in bf16 with 1 %
outlier columns, crb with 5 refinement rounds against crbog by per-layer
reconstruction error), where the CPU oracle is too slow to run:

* Hessian: 256 sampled entries against float64 dot products over all
  128 x 2048 tokens (relative to sqrt(H_ii H_jj)).
* The exact identities of the factor and the block loop, in float64
  (gpu_helpers.u_checks): U^-1 U^-T = H_d (H_d the damped Hessian, U the
  upper Cholesky factor of H_d^-1) to 1e-5, and W0 - Q = E U' with E the
  per-column errors (w - q) / U_jj and U' = U without the strictly upper
  entries of each 128 x 128 diagonal block (the reference quantizes a
  block from its values at the block's start, bigptq.py:235-264), so that
  sum(E^2) / 2 = the loss the loop accumulates (bigptq.py:240-262) to 1e-5.
  It holds whatever the quantizer and the conditioning, and ties the
  Hessian, the factor, the block loop and every trailing update together.
  The looser H_d-metric form (W0 - Q) H_d (W0 - Q)^T / 2 = loss, which
  assumes feedback inside each block as well, is printed for reference.
* Binarization structure: all rows share the salient columns (crbq_pack
  accepts the layer), the quantized values of each group fit the packed
  table apart from rare exceptions (an element equal to its group's mean
  binarizes to the mean itself), and the packed layer unpacks bit-exactly.
"""
import pytest
import torch

from crb_amd import synth
from gpu_helpers import u_checks

pytestmark = pytest.mark.gpu
DEV = "cuda:0"
NTOK = 128 * 2048


def _k():
    from crb_amd import kernels
    return kernels


def _acts(C, seed):
    """[NTOK, C] fp16 activations with Student-t(4) channel scales."""
    s = synth.channel_scales(C, seed, kind="student_t4", device=DEV)
    g = torch.Generator(device=DEV)
    g.manual_seed(seed)
    x = torch.empty(NTOK, C, dtype=torch.float16, device=DEV)
    for t0 in range(0, NTOK, 8192):
        x[t0:t0 + 8192] = (torch.randn(8192, C, generator=g, device=DEV) * s).half()
    return x


def _hessian(X, nseq=128):
    C = X.shape[1]
    S = torch.zeros(C, C, device=DEV)
    _k().hessian_accum(X, S)
    H = _k().hessian_finalize(S, 2.0 / nseq, S)
    # sampled entries against float64 sums over every token
    g = torch.Generator().manual_seed(C)
    i = torch.randint(0, C, (256,), generator=g).to(DEV)
    j = torch.randint(0, C, (256,), generator=g).to(DEV)
    want = torch.zeros(256, dtype=torch.float64, device=DEV)
    for t0 in range(0, X.shape[0], 32768):
        xa = X[t0:t0 + 32768, i].double()
        xb = X[t0:t0 + 32768, j].double()
        want += (xa * xb).sum(0)
    want *= 2.0 / nseq
    d = torch.diagonal(H).double()
    rel = (H[i, j].double() - want).abs() / torch.sqrt(d[i] * d[j])
    assert float(rel.max()) < 1e-5, float(rel.max())
    return H


def _quantize_check(name, W16, H, method, refine_iters=1, nseq=128, recon=None):
    """One sublayer through the factor and the block loop; checks the GPTQ
    identity and the binarization structure.  Returns the sublayer's GPTQ
    loss.  With recon (a dict), also adds the reconstruction error
    ||(W - Q) X^T||_F^2 over the calibration tokens to recon[method]: with
    H = (2 / nseq) X^T X (undamped), it is (nseq / 2) sum((D H) * D)."""
    Hd = H.clone()
    W = W16.float().contiguous()
    U, retries, fb = _k().hinv_upper(Hd, W, 0.01)          # Hd is now the damped H
    assert retries == 0 and not fb
    W0 = W.clone()
    L = torch.zeros(W.shape[0], device=DEV)
    from crb_amd import _lib
    p = _lib.params(method, refine_iters=refine_iters)
    masks, _ = _k().fasterquant_blocks(W, U, p, L, want_masks=True)
    D = W0 - W
    quad = ((D @ Hd) * D).sum(1) / 2
    tot = abs(float(quad.double().sum()) - float(L.double().sum())) / float(L.double().sum())
    back, loop = u_checks(W0, W, Hd, U, float(L.double().sum()))
    print(f"  {name} {method}: error {float(L.sum()):.5g}  U backward {back:.2e}, loop "
          f"identity rel {loop:.2e} (H_d-metric form rel {tot:.2e})", flush=True)
    assert back < 1e-5, back
    assert loop < 1e-5, loop
    if recon is not None:
        r2 = float((((D @ H) * D).sum(1)).double().sum()) * nseq / 2
        assert r2 > 0 and r2 == r2
        recon[method] = recon.get(method, 0.0) + r2
    Wq = W.to(W16.dtype).contiguous()
    codes, lut, sal, ex = _k().pack(Wq, masks)               # raises on a structure violation
    n_ex = int(ex.idx.numel())
    print(f"  {name} {method}: packed, {n_ex} exceptions", flush=True)
    assert n_ex * 10000 <= Wq.numel(), n_ex                 # rare: ties at a group mean
    back = _k().unpack(codes, lut, sal, W.shape[1], ex)
    assert torch.equal(back.view(torch.int16), Wq.view(torch.int16))
    return float(L.sum())


def test_cfg1_opt13b_layer_crb_and_braq():
    print("cfg1 OPT-1.3B layer", flush=True)
    subs = synth.opt_sublayers("opt-1.3b")
    groups = {}
    for j, (name, r, c, grp) in enumerate(subs):
        if grp not in groups:
            groups[grp] = _hessian(_acts(c, 100 + j))
    errs = {}
    for method in ("crb", "braq"):
        tot = 0.0
        for j, (name, r, c, grp) in enumerate(subs):
            W = (torch.randn(r, c, generator=torch.Generator(device=DEV).manual_seed(j),
                             device=DEV) * 0.02).half()
            tot += _quantize_check(name, W, groups[grp], method)
        errs[method] = tot
    print(f"  layer error crb {errs['crb']:.5g} braq {errs['braq']:.5g}", flush=True)


def test_cfg3_opt66b_layer_max_shape():
    """every sublayer of an OPT-66B-shaped layer, fc2's input
    giving the 36864^2 Hessian and fc1 a 36864-row block loop."""
    print("cfg3 OPT-66B layer (fc2 C = 36864, fc1 36864 rows)", flush=True)
    subs = synth.opt_sublayers("opt-66b")
    groups = {}
    for j, (name, r, c, grp) in enumerate(subs):
        if grp not in groups:
            X = _acts(c, 7 + j)
            groups[grp] = _hessian(X)
            del X
            torch.cuda.empty_cache()
    for j, (name, r, c, grp) in enumerate(subs):
        W = (torch.randn(r, c, generator=torch.Generator(device=DEV).manual_seed(3 + j),
                         device=DEV) * 0.02).half()
        _quantize_check(name, W, groups[grp], "crb")


def test_cfg4_llama3_8b_layer_bf16():
    print("cfg4 Llama-3-8B layer bf16", flush=True)
    subs = synth.llama3_8b_sublayers()
    groups = {}
    for j, (name, r, c, grp) in enumerate(subs):
        if grp not in groups:
            groups[grp] = _hessian(_acts(c, 200 + j))
    errs, recon = {}, {}
    for method, it in (("crb", 5), ("crbog", 1)):
        tot = 0.0
        for j, (name, r, c, grp) in enumerate(subs):
            W = synth.weight(r, c, 300 + j, outlier_frac=0.01, outlier_scale=10.0,
                             dtype=torch.bfloat16, device=DEV)
            tot += _quantize_check(name, W, groups[grp], method, refine_iters=it, recon=recon)
        errs[method] = tot
    print(f"  layer GPTQ loss crb(refine 5) {errs['crb']:.5g} crbog {errs['crbog']:.5g}",
          flush=True)
    print(f"  layer reconstruction error ||(W - Q) X^T||_F: crb(refine 5) "
          f"{recon['crb'] ** 0.5:.5g} crbog {recon['crbog'] ** 0.5:.5g} "
          f"(ratio {(recon['crb'] / recon['crbog']) ** 0.5:.4f})", flush=True)
