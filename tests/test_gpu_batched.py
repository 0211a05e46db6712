"""crbq_fasterquant_batched (the block loop of up to four sublayers of one
shape, q/k/v/out or gate/up, each with its own or a shared inverse factor,
every launch covering all of them) against one crbq_fasterquant call per
sublayer: bitwise-equal weights, losses, masks and block traces for every
sublayer, across methods, both partitions, ragged shapes, row strides that
rule out the 16-byte path, and GPTQ off."""
import pytest
import torch

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def _factor(C, seed):
    from crb_amd import kernels
    g = torch.Generator(device=DEV).manual_seed(seed)
    X = torch.randn(4 * C, C, generator=g, device=DEV) * torch.exp(
        torch.randn(C, generator=g, device=DEV))
    H = (X.t() @ X) * (2.0 / 16)
    U, retries, fb = kernels.hinv_upper(H, None, 0.01)
    assert retries == 0 and not fb
    return U


def _weights(n, R, C, ldw, seed):
    g = torch.Generator(device=DEV).manual_seed(seed)
    base = torch.randn(n, R, ldw, generator=g, device=DEV) * 0.02
    for i in range(n):
        base[i, :, torch.randperm(C, generator=g, device=DEV)[:max(1, C // 50)]] *= 8
    return base


def _one_by_one(base, C, Us, p):
    from crb_amd import kernels
    out = []
    for i in range(base.shape[0]):
        W = base[i].clone()[:, :C]
        L = torch.zeros(W.shape[0], device=DEV)
        m, t = kernels.fasterquant_blocks(W, Us[i], p, L, want_masks=True, want_traces=True)
        out.append((W, L, m, t))
    return out


@pytest.mark.parametrize("method,partition,gptq", [
    ("crb", 3, True), ("braq", 3, True), ("crbog", 3, True), ("crb", 1, True),
    ("crb", 3, False)])
@pytest.mark.parametrize("n,R,C,ldw,seed", [
    (3, 4096, 1280, 1280, 1),      # q/k/v of a 1280-wide block
    (2, 1000, 384, 384, 2),        # gate/up
    (4, 333, 200, 203, 3),         # ragged last block, rows not 16-byte aligned
])
@pytest.mark.parametrize("factors", ["shared", "own"])
def test_batched_matches_one_call_per_sublayer(method, partition, gptq, n, R, C, ldw, seed,
                                               factors):
    from crb_amd import _lib, kernels
    print(f"batched n={n} {R}x{C} ldw={ldw} {method} p{partition} gptq={gptq} {factors}",
          flush=True)
    p = _lib.params(method, partition=partition, disable_gptq=not gptq)
    if factors == "shared":
        Us = [_factor(C, seed)] * n
    else:                              # q/k/v with one factor, out with another
        Us = [_factor(C, seed)] * (n - 1) + [_factor(C, seed + 100)]
    base = _weights(n, R, C, ldw, seed)
    ref = _one_by_one(base, C, Us, p)
    Wb = base.clone()
    Ws = [Wb[i][:, :C] for i in range(n)]
    Ls = [torch.zeros(R, device=DEV) for _ in range(n)]
    masks, traces = kernels.fasterquant_blocks_batched(Ws, Us[0] if factors == "shared" else Us,
                                                       p, Ls, want_masks=True, want_traces=True)
    torch.cuda.synchronize()
    for i in range(n):
        W, L, m, t = ref[i]
        assert torch.equal(Ws[i], W), i
        assert torch.equal(Ls[i], L), i
        assert torch.equal(masks[i], m), i
        assert traces[i] == t, i
        # columns beyond C of the padded rows are untouched
        assert torch.equal(Wb[i][:, C:], base[i][:, C:]), i


def test_batched_single_segment_and_argument_checks():
    from crb_amd import _lib, kernels
    print("batched nseg=1 and argument checks", flush=True)
    p = _lib.params("crb")
    R, C = 512, 256
    U = _factor(C, 5)
    base = _weights(1, R, C, C, 5)
    ref = _one_by_one(base, C, [U], p)
    W = base[0].clone()
    L = torch.zeros(R, device=DEV)
    masks, _ = kernels.fasterquant_blocks_batched([W], U, p, [L], want_masks=True)
    assert torch.equal(W, ref[0][0]) and torch.equal(L, ref[0][1])
    assert torch.equal(masks[0], ref[0][2])
    five = [base[0].clone() for _ in range(5)]
    with pytest.raises(_lib.CrbqError):
        kernels.fasterquant_blocks_batched(five, U, p, [torch.zeros(R, device=DEV)] * 5)
    with pytest.raises(_lib.CrbqError):
        kernels.fasterquant_blocks_batched([base[0].clone(), base[0][:, :C - 8].clone()], U, p,
                                           [torch.zeros(R, device=DEV)] * 2)
    with pytest.raises(_lib.CrbqError):              # factors of two sizes
        kernels.fasterquant_blocks_batched([base[0].clone(), base[0].clone()],
                                           [U, _factor(C + 8, 6)], p,
                                           [torch.zeros(R, device=DEV)] * 2)
    Wd = base[0].clone()                      # the same weight twice: rejected
    with pytest.raises(_lib.CrbqError):
        kernels.fasterquant_blocks_batched([Wd, Wd], U, p,
                                           [torch.zeros(R, device=DEV) for _ in range(2)])
    Ld = torch.zeros(R, device=DEV)           # the same loss vector twice: rejected
    with pytest.raises(_lib.CrbqError):
        kernels.fasterquant_blocks_batched([base[0].clone(), base[0].clone()], U, p, [Ld, Ld])
    lib = _lib.load()
    assert lib.crbq_fasterquant_batched_workspace_size(0, R, C, p) == 0
    assert lib.crbq_fasterquant_batched_workspace_size(5, R, C, p) == 0


@pytest.mark.parametrize("name,n,R,C,nfac,method,iters", [
    ("opt-6.7b q/k/v/out", 4, 4096, 4096, 2, "crb", 1),
    ("llama-3-8b q/o", 2, 4096, 4096, 2, "crb", 5),
    ("llama-3-8b k/v", 2, 1024, 4096, 1, "crbog", 1),
    ("llama-3-8b gate/up", 2, 14336, 4096, 1, "crb", 5),
])
def test_batched_full_size_layers(name, n, R, C, nfac, method, iters):
    """The sublayer groups the layer driver batches, at full model shapes:
    bitwise the weights and losses of one call per sublayer."""
    from crb_amd import _lib, kernels
    print(f"batched full size: {name} ({n} x {R} x {C}, {nfac} factors, {method})", flush=True)
    p = _lib.params(method, refine_iters=iters)
    facs = [_factor(C, 40 + f) for f in range(nfac)]
    Us = [facs[0]] * (n - nfac + 1) + facs[1:]
    base = _weights(n, R, C, C, 41)
    Wb = base.clone()
    Ws = [Wb[i] for i in range(n)]
    Ls = [torch.zeros(R, device=DEV) for _ in range(n)]
    kernels.fasterquant_blocks_batched(Ws, Us, p, Ls)
    for i in range(n):
        W = base[i].clone()
        L = torch.zeros(R, device=DEV)
        kernels.fasterquant_blocks(W, Us[i], p, L)
        assert torch.equal(Ws[i], W), i
        assert torch.equal(Ls[i], L), i
        del W


def test_batched_magnitude_metric_and_partial_traces():
    """Magnitude salient metric (utils/structure.py:11-12) through the
    batched loop, with block traces requested for some sublayers only (a
    NULL entry in the host array): bitwise the single-call results, and the
    traced sublayers' traces equal to their single-call traces."""
    import ctypes
    from crb_amd import _lib, kernels
    print("batched magnitude metric, partial traces", flush=True)
    p = _lib.params("crb", metric="magnitude")
    n, R, C = 3, 512, 384
    Us = [_factor(C, 51), _factor(C, 52), _factor(C, 51)]
    base = _weights(n, R, C, C, 53)
    ref = _one_by_one(base, C, Us, p)
    lib = _lib.ready(torch.device(DEV))
    nblk = (C + 127) // 128
    Ws = [base[i].clone() for i in range(n)]
    Ls = [torch.zeros(R, device=DEV) for _ in range(n)]
    trs = [torch.zeros(nblk * _lib.TRACE_BYTES, dtype=torch.uint8, device=DEV), None,
           torch.zeros(nblk * _lib.TRACE_BYTES, dtype=torch.uint8, device=DEV)]
    ws = torch.empty(lib.crbq_fasterquant_batched_workspace_size(n, R, C, ctypes.byref(p)),
                     dtype=torch.uint8, device=DEV)
    arr = ctypes.c_void_p * n
    _lib.check(lib.crbq_fasterquant_batched(
        n, arr(*[w.data_ptr() for w in Ws]), R, C, C, arr(*[u.data_ptr() for u in Us]), C,
        ctypes.byref(p), arr(*[l.data_ptr() for l in Ls]), None, 0,
        arr(*[t.data_ptr() if t is not None else None for t in trs]), ws.data_ptr(), ws.numel(),
        torch.cuda.current_stream().cuda_stream), "crbq_fasterquant_batched")
    torch.cuda.synchronize()
    for i in range(n):
        W, L, _, t = ref[i]
        assert torch.equal(Ws[i], W), i
        assert torch.equal(Ls[i], L), i
        if trs[i] is not None:
            assert kernels.decode_traces(trs[i], nblk) == t, i
