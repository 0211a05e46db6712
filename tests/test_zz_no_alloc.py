"""crbq_fasterquant_noalloc (the allocation-free entry point, scratch in a
static device array) against crbq_fasterquant with a caller workspace:
bitwise-equal weights, losses, masks and block traces, on two calls in a row
with the second one smaller (the scratch keeps the first call's contents),
no device memory allocated by the call, and problems beyond the static
scratch rejected before any device work."""
import pytest
import torch

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def _problem(R, C, seed):
    from crb_amd import kernels
    g = torch.Generator(device=DEV).manual_seed(seed)
    W = torch.randn(R, C, generator=g, device=DEV) * 0.02
    W[:, torch.randperm(C, generator=g, device=DEV)[:C // 50]] *= 8
    X = torch.randn(4 * C, C, generator=g, device=DEV) * torch.exp(
        torch.randn(C, generator=g, device=DEV))
    H = (X.t() @ X) * (2.0 / 16)
    U, retries, fb = kernels.hinv_upper(H, None, 0.01)
    assert retries == 0 and not fb
    return W, U


@pytest.mark.parametrize("method", ["crb", "braq"])
def test_noalloc_matches_workspace_entry_point(method):
    from crb_amd import _lib, kernels
    print(f"noalloc vs workspace entry point, {method}", flush=True)
    p = _lib.params(method)
    for R, C, seed in [(4096, 1280, 1), (1000, 384, 2)]:
        W, U = _problem(R, C, seed)
        nblk = (C + 127) // 128
        Wa, La = W.clone(), torch.zeros(R, device=DEV)
        ma, ta = kernels.fasterquant_blocks(Wa, U, p, La, want_masks=True, want_traces=True)
        Wb, Lb = W.clone(), torch.zeros(R, device=DEV)
        mb = torch.zeros(R, C, dtype=torch.uint8, device=DEV)
        tb = torch.zeros(nblk * _lib.TRACE_BYTES, dtype=torch.uint8, device=DEV)
        torch.cuda.synchronize()
        free0 = torch.cuda.mem_get_info()[0]
        kernels.fasterquant_blocks_noalloc(Wb, U, p, Lb, mb, tb)
        torch.cuda.synchronize()
        free1 = torch.cuda.mem_get_info()[0]
        print(f"  {R}x{C}: free device memory before/after {free0} / {free1}", flush=True)
        assert free1 == free0
        assert torch.equal(Wa, Wb)
        assert torch.equal(La, Lb)
        assert torch.equal(ma, mb)
        assert kernels.decode_traces(tb, nblk) == ta


def test_noalloc_rejects_problems_beyond_its_scratch():
    from crb_amd import _lib, kernels
    print("noalloc too large", flush=True)
    p = _lib.params("crb")
    R, C = 20000, 1024          # 20000 x 1024 fp32 errors alone exceed the 80 MiB
    assert _lib.load().crbq_fasterquant_workspace_size(R, C, p) > _lib.NOALLOC_SCRATCH_BYTES
    W = torch.zeros(R, C, device=DEV)
    U = torch.eye(C, device=DEV)
    L = torch.zeros(R, device=DEV)
    with pytest.raises(_lib.CrbqError, match="static scratch"):
        kernels.fasterquant_blocks_noalloc(W, U, p, L)
    assert torch.count_nonzero(W) == 0                    # nothing ran


def test_noalloc_replays_under_graph_capture():
    """Captured with torch.cuda.graph after one eager call on the device (the
    per-device set-up, the percentile table and the scratch address, is done
    on the first call and cannot be captured: a first call under capture
    returns CRBQ_ERR_CAPTURE), then replayed three times with eager work and
    synchronizations between the replays: every replay's weights, losses and
    masks bitwise equal to the eager call's.  The graph holds kernel nodes
    only (the library clears its counters with a kernel, not a memset)."""
    from crb_amd import _lib, kernels
    print("noalloc under graph capture", flush=True)
    p = _lib.params("crb")
    R, C = 2048, 640
    W0, U = _problem(R, C, 5)
    We, Le = W0.clone(), torch.zeros(R, device=DEV)
    me = torch.zeros(R, C, dtype=torch.uint8, device=DEV)
    kernels.fasterquant_blocks_noalloc(We, U, p, Le, me)      # eager: warm-up and reference
    Wg, Lg = W0.clone(), torch.zeros(R, device=DEV)
    mg = torch.zeros_like(me)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        kernels.fasterquant_blocks_noalloc(Wg, U, p, Lg, mg)
    torch.cuda.synchronize()
    for rep in range(3):
        Wg.copy_(W0)
        Lg.zero_()
        mg.zero_()
        a = torch.randn(1024, 1024, device=DEV)
        (a @ a).sum().item()                                  # eager work in between
        graph.replay()
        torch.cuda.synchronize()
        print(f"  replay {rep}: weights equal {torch.equal(Wg, We)}", flush=True)
        assert torch.equal(Wg, We)
        assert torch.equal(Lg, Le)
        assert torch.equal(mg, me)
