"""The per-layer driver (shared Hessians/factors across sublayers reading
the same input, concurrent streams) against the per-sublayer drop-in API
(BRAGPTQ per nn.Linear, as run.py:326-374 uses it): bit-identical weights
and errors, for OPT-style and Llama-style layers."""
import pytest
import torch

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def _layer(kind, seed=0):
    h, f = 256, 512
    if kind == "opt":
        subs = [("k_proj", h, h, "qkv"), ("v_proj", h, h, "qkv"), ("q_proj", h, h, "qkv"),
                ("out_proj", h, h, "out"), ("fc1", f, h, "fc1"), ("fc2", h, f, "fc2")]
        dtype = torch.float16
    else:
        kv = 128
        subs = [("q_proj", h, h, "qkv"), ("k_proj", kv, h, "qkv"), ("v_proj", kv, h, "qkv"),
                ("o_proj", h, h, "o"), ("gate_proj", f, h, "gu"), ("up_proj", f, h, "gu"),
                ("down_proj", h, f, "down")]
        dtype = torch.bfloat16
    g = torch.Generator().manual_seed(seed)
    Ws = {n: (torch.randn(r, c, generator=g) * 0.02).to(dtype) for n, r, c, _ in subs}
    cols = {grp: c for _, _, c, grp in subs}
    X = {grp: (torch.randn(4, 96, c, generator=g) * torch.exp(torch.randn(c, generator=g)))
         .to(dtype) for grp, c in cols.items()}
    return subs, Ws, X


@pytest.mark.parametrize("kind,method", [("opt", "crb"), ("llama", "crb"), ("opt", "braq")])
def test_driver_matches_per_sublayer_api(kind, method):
    print(f"driver {kind} {method}", flush=True)
    from crb_amd import BRAGPTQ, Binarization
    from crb_amd.driver import LayerQuantizer, Sublayer
    subs, Ws, X = _layer(kind)
    # per-sublayer API
    ref_w, ref_err = {}, {}
    for n, r, c, grp in subs:
        layer = torch.nn.Linear(c, r, bias=False).to(DEV).to(Ws[n].dtype)
        layer.weight.data = Ws[n].to(DEV).clone()
        q = Binarization(layer.weight, method=method, groupsize=128)
        bq = BRAGPTQ(layer, q, "hessian")
        for s in range(X[grp].shape[0]):
            bq.add_batch(X[grp][s:s + 1].to(DEV), None)
        ref_err[n] = bq.fasterquant()["error"]
        ref_w[n] = layer.weight.data.cpu()
    # driver
    sl = [Sublayer(n, Ws[n].to(DEV).clone(), grp) for n, r, c, grp in subs]
    lq = LayerQuantizer(sl, method=method)
    for grp, x in X.items():
        for s in range(x.shape[0]):          # same per-sequence calls as the API path
            lq.add_batch(grp, x[s:s + 1].to(DEV))
    errs = lq.quantize()
    for s in sl:
        assert torch.equal(s.weight.cpu(), ref_w[s.name]), s.name
        assert abs(errs[s.name] - ref_err[s.name]) <= 1e-6 * abs(ref_err[s.name]), s.name


@pytest.mark.parametrize("need", [3, "fallback"])
def test_driver_retry_and_fallback_match_per_sublayer_api(need):
    """A Hessian whose Cholesky needs the reference's extra damping rounds
    (bigptq.py:114-123) or its diagonal fallback (:124-126) for one input:
    the driver recomputes that input's sublayers with the final factor,
    which must give what the per-sublayer API gives."""
    print(f"driver retries {need}", flush=True)
    from crb_amd import BRAGPTQ, Binarization
    from crb_amd.driver import LayerQuantizer, Sublayer
    subs, Ws, X = _layer("opt")
    C = 256
    g = torch.Generator().manual_seed(11)
    if need == "fallback":
        Hbad = torch.eye(C) * 2.0
        Hbad[3, 3] = -1e9
    else:
        Q, _ = torch.linalg.qr(torch.randn(C, C, generator=g, dtype=torch.float64))
        ev = torch.rand(C, generator=g, dtype=torch.float64) + 0.5
        ev[0] = -(0.01 + (need - 0.5) * 1e-3) * float(ev.mean()) * 0.994
        Hbad = ((Q * ev) @ Q.t()).float()
    special = "qkv"
    ref_w, ref_err = {}, {}
    for n, r, c, grp in subs:
        layer = torch.nn.Linear(c, r, bias=False).to(DEV).to(Ws[n].dtype)
        layer.weight.data = Ws[n].to(DEV).clone()
        q = Binarization(layer.weight, method="crb", groupsize=128)
        bq = BRAGPTQ(layer, q, "hessian")
        if grp == special:
            bq._S = Hbad.to(DEV).clone()
            bq.nsamples = 2                     # H = (2 / 2) * S
        else:
            for s in range(X[grp].shape[0]):
                bq.add_batch(X[grp][s:s + 1].to(DEV), None)
        ref_err[n] = bq.fasterquant()["error"]
        if grp == special:
            info = bq.last
            assert info["fallback"] if need == "fallback" else info["retries"] == need, info
        ref_w[n] = layer.weight.data.cpu()
    sl = [Sublayer(n, Ws[n].to(DEV).clone(), grp) for n, r, c, grp in subs]
    lq = LayerQuantizer(sl, method="crb")
    for grp, x in X.items():
        if grp == special:
            lq.S[grp] = Hbad.to(DEV).clone()
            lq.nsamples[grp] = 2
            continue
        for s in range(x.shape[0]):
            lq.add_batch(grp, x[s:s + 1].to(DEV))
    errs = lq.quantize()
    assert lq.info[special]["fallback"] if need == "fallback" else \
        lq.info[special]["retries"] == need
    for s in sl:
        assert torch.equal(s.weight.cpu(), ref_w[s.name]), s.name
        assert abs(errs[s.name] - ref_err[s.name]) <= 1e-6 * abs(ref_err[s.name]), s.name
