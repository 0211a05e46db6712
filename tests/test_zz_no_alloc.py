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
