"""GPU parity of the individual crbq kernels against the CPU oracle, the
reference-written golden vectors and float64 closed forms.

Tolerances (fp32 kernels vs. fp32 torch-CPU reductions, which differ only in
summation order):
  * GEMM / Hessian / U: relative Frobenius error <= 1e-5 (GEMM, Hessian),
    <= 1e-4 (U, through a factorization);
  * binarizers: per-element |diff| <= 1e-5 * max|x| on >= 99.9% of elements
    (ulp-level differences of a row mean can flip sign(x - mean) for an
    element sitting on the mean), and all per-row values match to 1e-4 rel;
  * search: split and salient count identical to the reference's, unless the
    reference's own candidate errors tie within 1e-6 relative.
"""
import numpy as np
import pytest
import torch

from oracle import crb_oracle as O

pytestmark = pytest.mark.gpu

DEV = "cuda:0"


def _k():
    from crb_amd import kernels
    return kernels


def rel(a, b):
    a = a.double().cpu()
    b = b.double().cpu()
    return float((a - b).norm() / max(b.norm(), 1e-300))


# ---------------------------------------------------------------------------
@pytest.mark.parametrize("ta,tb", [(False, False), (False, True), (True, False), (True, True)])
@pytest.mark.parametrize("M,N,K", [(1, 1, 1), (130, 70, 37), (256, 384, 128), (300, 129, 200)])
def test_sgemm(ta, tb, M, N, K):
    print(f"sgemm ta={ta} tb={tb} M={M} N={N} K={K}", flush=True)
    g = torch.Generator().manual_seed(M * 7 + N * 3 + K)
    A = torch.randn((K, M) if ta else (M, K), generator=g)
    B = torch.randn((N, K) if tb else (K, N), generator=g)
    C = torch.randn(M, N, generator=g)
    want = 0.5 * C.double() + (-1.25) * ((A.double().t() if ta else A.double())
                                         @ (B.double().t() if tb else B.double()))
    Cd = C.to(DEV)
    _k().sgemm(A.to(DEV), B.to(DEV), Cd, alpha=-1.25, beta=0.5, transa=ta, transb=tb)
    torch.cuda.synchronize()
    assert rel(Cd, want) < 1e-5


@pytest.mark.parametrize("tb", [False, True])
@pytest.mark.parametrize("M,N,K,pad", [(3000, 2900, 160, 0), (3000, 2900, 170, 0),
                                       (3072, 2816, 96, 12), (2816, 3072, 1024, 4),
                                       (2990, 3001, 77, 3)])
def test_sgemm_large_tiles(tb, M, N, K, pad):
    """Products with >= 512 tiles of 128 x 128 (the size from which the
    128 x 128 tiles are used; 552 / 528 / 552 tiles here): interior tiles
    whose chunks are all full run the hand-scheduled asm K loop, edge tiles
    (ragged M and N) and ragged K the compiled one; both B layouts, against
    float64, on row strides padded by `pad` floats."""
    print(f"sgemm large tb={tb} M={M} N={N} K={K} pad={pad}", flush=True)
    g = torch.Generator().manual_seed(M + N + K + pad)
    Af = torch.randn(M, K + pad, generator=g)
    Bf = torch.randn(N, K + pad, generator=g) if tb else torch.randn(K, N + pad, generator=g)
    C = torch.randn(M, N, generator=g)
    A, B = Af[:, :K], (Bf[:, :K] if tb else Bf[:, :N])
    want = 0.75 * C.double() + (-1.5) * (A.double() @ (B.double().t() if tb else B.double()))
    Cd = C.to(DEV)
    # slices of device tensors keep the padded row strides
    Ad = Af.to(DEV)[:, :K]
    Bd = Bf.to(DEV)[:, :K] if tb else Bf.to(DEV)[:, :N]
    _k().sgemm(Ad, Bd, Cd, alpha=-1.5, beta=0.75, transb=tb)
    torch.cuda.synchronize()
    assert rel(Cd, want) < 1e-6


def test_sgemm_trailing_update_shape():
    """W[:, ed:] -= Err @ U[st:ed, ed:] on strided views (bigptq.py:264)."""
    print("sgemm trailing", flush=True)
    g = torch.Generator().manual_seed(5)
    R, C, st, ed = 200, 520, 128, 256
    W = torch.randn(R, C, generator=g)
    U = torch.triu(torch.randn(C, C, generator=g))
    E = torch.randn(R, ed - st, generator=g)
    want = W.double().clone()
    want[:, ed:] -= E.double() @ U[st:ed, ed:].double()
    Wd, Ud, Ed = W.to(DEV), U.to(DEV), E.to(DEV)
    _k().sgemm(Ed, Ud[st:ed, ed:], Wd[:, ed:], alpha=-1.0, beta=1.0)
    torch.cuda.synchronize()
    assert rel(Wd, want) < 1e-6
    assert torch.equal(Wd[:, :ed].cpu(), W[:, :ed])


# ---------------------------------------------------------------------------
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16, torch.float32])
@pytest.mark.parametrize("T,C", [(300, 200), (64, 128), (1000, 384), (5, 8)])
def test_hessian_accum(dtype, T, C):
    print(f"hessian {dtype} T={T} C={C}", flush=True)
    g = torch.Generator().manual_seed(T + C)
    X = (torch.randn(T, C, generator=g) * torch.exp(torch.randn(C, generator=g))).to(dtype)
    S = torch.zeros(C, C, device=DEV)
    _k().hessian_accum(X.to(DEV), S)
    _k().hessian_accum(X[: T // 2].to(DEV), S)      # accumulates
    torch.cuda.synchronize()
    Xd = X.double()
    want = Xd.t() @ Xd + Xd[: T // 2].t() @ Xd[: T // 2]
    got = S.cpu().double()
    iu = torch.triu_indices(C, C)
    assert rel(got[iu[0], iu[1]], want[iu[0], iu[1]]) < 1e-5
    H = _k().hessian_finalize(S, 0.5)
    torch.cuda.synchronize()
    assert rel(H, 0.5 * want) < 1e-5
    assert torch.equal(H.cpu(), H.cpu().t())


@pytest.mark.parametrize("C,pad", [(1, 0), (63, 1), (64, 0), (130, 6), (300, 0)])
def test_hessian_finalize_tiles(C, pad):
    """H = scale * sym(upper(S)) in place and into another buffer, with
    padded row strides; the lower triangle of S is never read."""
    print(f"finalize C={C} pad={pad}", flush=True)
    g = torch.Generator().manual_seed(C)
    up = torch.randn(C, C, generator=g)
    junk = torch.full((C, C), float("nan"))
    S0 = torch.where(torch.ones(C, C, dtype=torch.bool).triu(), up, junk)
    want = 0.25 * (torch.triu(up) + torch.triu(up, 1).t())
    buf = torch.full((C, C + pad), float("nan"), device=DEV)
    S = buf[:, :C]
    S.copy_(S0.to(DEV))
    Hbuf = torch.full((C, C + pad + 3), float("nan"), device=DEV)
    H = Hbuf[:, :C]
    _k().hessian_finalize(S, 0.25, H)
    _k().hessian_finalize(S, 0.25, S)                  # in place
    torch.cuda.synchronize()
    assert torch.equal(H.cpu(), want)
    assert torch.equal(S.cpu(), want)
    assert torch.isnan(Hbuf[:, C:].cpu()).all()        # nothing written past C


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("T,C", [(8192, 520), (16384, 256)])
def test_hessian_accum_split_k(dtype, T, C):
    """Token ranges split across workgroups (few output tiles): partial
    sums go through the workspace and are added in split order."""
    print(f"hessian split {dtype} T={T} C={C}", flush=True)
    from crb_amd import _lib
    lib = _lib.load()
    assert lib.crbq_hessian_workspace_size(T, C) > 0      # the split path is taken
    g = torch.Generator().manual_seed(T + 7 * C)
    X = (torch.randn(T, C, generator=g) * torch.exp(torch.randn(C, generator=g))).to(dtype)
    S = torch.full((C, C), 0.5, device=DEV)
    _k().hessian_accum(X.to(DEV), S)
    torch.cuda.synchronize()
    Xd = X.double()
    want = Xd.t() @ Xd + 0.5
    got = S.cpu().double()
    iu = torch.triu_indices(C, C)
    assert rel(got[iu[0], iu[1]], want[iu[0], iu[1]]) < 1e-5
    # deterministic: a second run gives the same bits
    S2 = torch.full((C, C), 0.5, device=DEV)
    _k().hessian_accum(X.to(DEV), S2)
    torch.cuda.synchronize()
    assert torch.equal(torch.triu(S2).cpu(), torch.triu(S).cpu())


def _accum_raw(X, S, ws_bytes):
    """crbq_hessian_accum with a workspace of exactly ws_bytes (0: NULL)."""
    from crb_amd import _lib
    lib = _lib.ready(X.device)
    ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=X.device)
    _lib.check(lib.crbq_hessian_accum(X.data_ptr(), _lib.DTYPES[X.dtype], X.shape[0],
                                      X.stride(0), X.shape[1], S.data_ptr(), S.stride(0),
                                      ws.data_ptr() if ws_bytes else None, ws_bytes,
                                      _lib.stream_of(S)), "crbq_hessian_accum")


def _hess_want(X, S0):
    Xd = X.double()
    return Xd.t() @ Xd + S0


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("T,C,ldx", [(300, 200, 200), (1000, 384, 392), (77, 8, 13),
                                     (8192, 520, 520)])
def test_hessian_token_major_path(dtype, T, C, ldx):
    """The in-place SYRK taken when the workspace cannot hold the
    channel-major copy: NULL workspace, and a workspace sized for the split
    partials only."""
    print(f"hessian token-major {dtype} T={T} C={C} ldx={ldx}", flush=True)
    from crb_amd import _lib
    lib = _lib.load()
    g = torch.Generator().manual_seed(T + 3 * C)
    Xf = (torch.randn(T, ldx, generator=g) * torch.exp(torch.randn(ldx, generator=g))).to(dtype)
    X = Xf.to(DEV)[:, :C]
    want = _hess_want(Xf[:, :C], 0.25)
    iu = torch.triu_indices(C, C)
    xt_bytes = -(-C // 256) * 256 * (-(-T // 64) * 64) * 2     # the channel-major copy
    part = 4 * C * C * 4                       # room for 4 split partials
    nbs = (0, part) if part < xt_bytes else (0,)
    if T >= 8192:
        assert len(nbs) == 2 and lib.crbq_hessian_workspace_size(T, C) > xt_bytes
    for nb in nbs:
        S = torch.full((C, C), 0.25, device=DEV)
        _accum_raw(X, S, nb)
        torch.cuda.synchronize()
        got = S.cpu().double()
        assert rel(got[iu[0], iu[1]], want[iu[0], iu[1]]) < 1e-5, nb


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("T,C,ldx,pass_tok", [(5000, 200, 200, 1024), (3000, 520, 528, 700),
                                              (129, 64, 72, 64)])
def test_hessian_channel_major_passes(dtype, T, C, ldx, pass_tok, monkeypatch):
    """Inputs longer than one transposed pass run in several passes (the pass
    length is lowered through CRBQ_XT_PASS_TOKENS); ragged last pass, C not a
    multiple of the 256-channel tile, strided rows."""
    print(f"hessian passes {dtype} T={T} C={C} pass={pass_tok}", flush=True)
    from crb_amd import _lib
    lib = _lib.load()
    g = torch.Generator().manual_seed(T + 5 * C)
    Xf = (torch.randn(T, ldx, generator=g) * torch.exp(torch.randn(ldx, generator=g))).to(dtype)
    X = Xf.to(DEV)[:, :C]
    want = _hess_want(Xf[:, :C], 1.0)
    iu = torch.triu_indices(C, C)
    one = torch.ones(C, C, device=DEV)
    S1 = one.clone()
    _accum_raw(X, S1, lib.crbq_hessian_workspace_size(T, C))       # one pass
    monkeypatch.setenv("CRBQ_XT_PASS_TOKENS", str(pass_tok))
    nb = lib.crbq_hessian_workspace_size(T, C)
    S = one.clone()
    _accum_raw(X, S, nb)
    # passes = calls on consecutive token slices of the pass length
    S2 = one.clone()
    step = max(64, pass_tok // 64 * 64)
    for t0 in range(0, T, step):
        _accum_raw(X[t0:t0 + step], S2, nb)
    torch.cuda.synchronize()
    for got in (S1, S):
        got = got.cpu().double()
        assert rel(got[iu[0], iu[1]], want[iu[0], iu[1]]) < 1e-5
    assert torch.equal(torch.triu(S).cpu(), torch.triu(S2).cpu())


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("C,chunks", [(300, (128, 64, 192, 100)), (512, (2048, 2048)),
                                      (1000, (64,))])
def test_hessian_channel_major_store(dtype, C, chunks):
    """crbq_hessian_transpose chunk by chunk into a channel-major store, then
    crbq_hessian_accum_cm: bitwise the sums of crbq_hessian_accum on the same
    tokens (same operand layout, same token splits), and against float64;
    the last chunk may be ragged (its padding columns are zeroed)."""
    print(f"hessian channel-major store {dtype} C={C} chunks={chunks}", flush=True)
    g = torch.Generator().manual_seed(C + len(chunks))
    T = sum(chunks)
    X = (torch.randn(T, C, generator=g) * torch.exp(torch.randn(C, generator=g))).to(dtype)
    Xd = X.to(DEV)
    Xt = _k().hessian_cm_store(T, C, dtype, DEV)
    assert Xt.shape[0] % 256 == 0 and Xt.shape[1] % 64 == 0
    Xt.fill_(1.0)                       # every entry must be written (data or padding)
    t0 = 0
    for n in chunks:
        _k().hessian_transpose(Xd[t0:t0 + n], Xt, t0)
        t0 += n
    S1 = torch.zeros(C, C, device=DEV)
    _k().hessian_accum_cm(Xt, T, C, S1)
    S2 = torch.zeros(C, C, device=DEV)
    _k().hessian_accum(Xd, S2)
    torch.cuda.synchronize()
    assert torch.equal(torch.triu(S1), torch.triu(S2))
    want = X.double().t() @ X.double()
    assert rel(torch.triu(S1), torch.triu(want)) < 1e-5


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("T,C,ldx", [(77, 256, 256), (1000, 512, 520), (4109, 4096, 4096),
                                     (3000, 8192, 8200), (20000, 8192, 8192)])
def test_hessian_token_major_stages(dtype, T, C, ldx):
    """C a multiple of 256 with 16-byte aligned rows: the SYRK stages the
    token-major X as it is and reads its MFMA operands with LDS transpose
    reads.  Bitwise the sums of the channel-major path (crbq_hessian_transpose
    + crbq_hessian_accum_cm, same token splits) on the same tokens, and
    against float64: ragged token counts (rows past ntok read as zeros),
    strided rows, the launched grid, the persistent kernel (C = 8192) and
    several token splits; also with no workspace (one split, launched
    grid)."""
    print(f"hessian token-major stages {dtype} T={T} C={C} ldx={ldx}", flush=True)
    g = torch.Generator(device=DEV).manual_seed(T + C)
    Xf = (torch.randn(T, ldx, device=DEV, generator=g) *
          torch.exp(torch.randn(ldx, device=DEV, generator=g))).to(dtype)
    X = Xf[:, :C]
    S1 = torch.full((C, C), 0.5, device=DEV)
    _k().hessian_accum(X, S1)
    Xt = _k().hessian_cm_store(T, C, dtype, DEV)
    _k().hessian_transpose(X, Xt, 0)
    S2 = torch.full((C, C), 0.5, device=DEV)
    _k().hessian_accum_cm(Xt, T, C, S2)
    del Xt
    torch.cuda.synchronize()
    assert torch.equal(torch.triu(S1), torch.triu(S2))
    del S2
    Xd = X.double()
    want = torch.triu(Xd.t() @ Xd + 0.5)
    assert float((torch.triu(S1.double()) - want).norm() / want.norm()) < 1e-5
    del want, Xd
    if T <= 4109:
        S3 = torch.full((C, C), 0.5, device=DEV)
        _accum_raw(X, S3, 0)
        torch.cuda.synchronize()
        if T < 4096:
            # one token split either way: the same sums bit for bit
            assert torch.equal(torch.triu(S3), torch.triu(S1))
        Xd = X.double()
        want = torch.triu(Xd.t() @ Xd + 0.5)
        assert float((torch.triu(S3.double()) - want).norm() / want.norm()) < 1e-5


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("T,C,ldx", [(300, 512, 513), (5000, 256, 260)])
def test_hessian_token_major_unaligned(dtype, T, C, ldx):
    """C a multiple of 256 but rows that cannot be staged with 16-byte loads
    (odd or non-multiple-of-8 row stride): crbq_hessian_workspace_size then
    holds only the split partials, so the SYRK transposes in registers
    (k_syrk16p); against float64."""
    print(f"hessian token-major unaligned {dtype} T={T} C={C} ldx={ldx}", flush=True)
    from crb_amd import _lib
    lib = _lib.load()
    g = torch.Generator(device=DEV).manual_seed(T + 3 * C)
    Xf = (torch.randn(T, ldx, device=DEV, generator=g) *
          torch.exp(torch.randn(ldx, device=DEV, generator=g))).to(dtype)
    X = Xf[:, :C]
    nb = lib.crbq_hessian_workspace_size(T, C)
    assert nb < -(-T // 64) * 64 * C * 2          # no room for a channel-major copy
    S = torch.full((C, C), 0.25, device=DEV)
    _accum_raw(X, S, nb)
    torch.cuda.synchronize()
    Xd = X.double()
    want = torch.triu(Xd.t() @ Xd + 0.25)
    assert float((torch.triu(S.double()) - want).norm() / want.norm()) < 1e-5


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("T,C", [(2048, 8192), (1000, 8300), (16384, 8192)])
def test_hessian_persistent_paced(dtype, T, C):
    """From 8192 channels the SYRK runs as the persistent, XCD-paced kernel
    (items claimed per XCD, control words at the end of the workspace).
    Against float64 on the GPU; with one token split (T < 4096) bitwise
    equal to the launched grid (C = 8192: no workspace; C = 8300: a
    workspace without room for the control words) and, for C = 8300, to
    the in-place path (NULL workspace), which issue the same MFMAs per tile;
    with several splits, the same bits on a rerun."""
    print(f"hessian persistent {dtype} T={T} C={C}", flush=True)
    from crb_amd import _lib
    lib = _lib.load()
    g = torch.Generator(device=DEV).manual_seed(T + C)
    X = (torch.randn(T, C, device=DEV, generator=g) *
         torch.exp(torch.randn(C, device=DEV, generator=g))).to(dtype)
    full = lib.crbq_hessian_workspace_size(T, C)
    S = torch.full((C, C), 0.5, device=DEV)
    _accum_raw(X, S, full)
    Xd = X.double()
    want = torch.triu(Xd.t() @ Xd + 0.5)
    got = torch.triu(S.double())
    assert float((got - want).norm() / want.norm()) < 1e-5
    del want, got
    xt_bytes = -(-C // 256) * 256 * (-(-T // 64) * 64) * 2
    if T < 4096:
        if C % 256:
            assert full > xt_bytes              # room for the control words
        for nb in ((xt_bytes, 0) if C % 256 else (0,)):
            S2 = torch.full((C, C), 0.5, device=DEV)
            _accum_raw(X, S2, nb)
            torch.cuda.synchronize()
            assert torch.equal(torch.triu(S2), torch.triu(S)), nb
            del S2
    else:
        S2 = torch.full((C, C), 0.5, device=DEV)
        _accum_raw(X, S2, full)
        torch.cuda.synchronize()
        assert torch.equal(torch.triu(S2), torch.triu(S))


def test_hessian_matches_reference_add_batch():
    """Incremental rescale of bigptq.py:50-53 vs. one 2/n scaling."""
    print("hessian add_batch", flush=True)
    g = torch.Generator().manual_seed(3)
    X = torch.randn(6, 50, 96, generator=g).half()
    H = torch.zeros(96, 96)
    n = 0
    for s in range(6):
        H, n = O.hessian_add_batch(H, n, X[s:s + 1].float())
    S = torch.zeros(96, 96, device=DEV)
    for s in range(6):
        _k().hessian_accum(X[s].to(DEV), S)
    Hg = _k().hessian_finalize(S, 2.0 / 6)
    torch.cuda.synchronize()
    assert rel(Hg, H) < 1e-5


# ---------------------------------------------------------------------------
def _spd(C, seed, cond=1e3):
    g = torch.Generator().manual_seed(seed)
    Q, _ = torch.linalg.qr(torch.randn(C, C, generator=g, dtype=torch.float64))
    ev = torch.logspace(0, np.log10(cond), C, dtype=torch.float64)
    return (Q * ev) @ Q.t()


@pytest.mark.parametrize("C", [7, 128, 300, 512])
def test_hinv_upper_matches_oracle(C):
    print(f"hinv C={C}", flush=True)
    H = _spd(C, C).float()
    W = torch.randn(16, C)
    Uo, info = O.hinv_upper(H.clone(), W.clone(), 0.01)
    Hd, Wd = H.to(DEV), W.to(DEV)
    U, retries, fb = _k().hinv_upper(Hd, Wd, 0.01)
    torch.cuda.synchronize()
    assert retries == info.retries == 0 and not fb
    assert rel(U, Uo) < 1e-4
    assert torch.equal(torch.tril(U.cpu(), -1), torch.zeros(C, C))
    # invariant: U^T U (H + damp I) = I
    Hdamp = H.double() + 0.01 * torch.diag(H.double()).mean() * torch.eye(C, dtype=torch.float64)
    Ud = U.cpu().double()
    assert float((Ud.t() @ Ud @ Hdamp - torch.eye(C, dtype=torch.float64)).abs().max()) < 1e-3


@pytest.mark.parametrize("C", [1000, 2900])
def test_hinv_upper_ragged_levels(C):
    """Sizes whose recursion splits unevenly at several levels (node halves of
    different sizes, so the one-launch Schur update + Q product pairs grids of
    different shapes or falls back to two launches): U against the fp64
    Cholesky factor of the damped inverse (bigptq.py:111-129) and the
    U^T U (H + damp I) = I invariant."""
    print(f"hinv ragged C={C}", flush=True)
    H = _spd(C, C + 7).float()
    U, retries, fb = _k().hinv_upper(H.to(DEV), None, 0.01)
    torch.cuda.synchronize()
    assert retries == 0 and not fb
    Hdamp = H.double() + 0.01 * torch.diag(H.double()).mean() * torch.eye(C, dtype=torch.float64)
    Uref = torch.linalg.cholesky(torch.linalg.inv(Hdamp), upper=True)
    Uc = U.cpu()
    assert torch.equal(torch.tril(Uc, -1), torch.zeros(C, C))
    assert rel(Uc, Uref.float()) < 1e-4
    Ud = Uc.double()
    assert float((Ud.t() @ Ud @ Hdamp - torch.eye(C, dtype=torch.float64)).abs().max()) < 1e-3


@pytest.mark.parametrize("C", [8192, 8320])
def test_hinv_upper_large_vs_fp64(C):
    """Factors whose top-level products have >= 512 tiles of 128 x 128, so
    the triangular-K products (k ranges that skip zero halves) run on the
    asm K loop: U against the fp64 upper Cholesky factor of the damped
    inverse, and its backward error U^-1 U^-T = H_d, both in float64 on the
    GPU.  H = X^T X / T from 2C tokens with log-normal channel scales."""
    print(f"hinv large C={C}", flush=True)
    g = torch.Generator(device=DEV).manual_seed(C)
    s = torch.exp(0.5 * torch.randn(C, generator=g, device=DEV, dtype=torch.float64))
    X = torch.randn(2 * C, C, generator=g, device=DEV, dtype=torch.float64) * s
    H64 = (X.t() @ X) / (2 * C)
    del X
    U, retries, fb = _k().hinv_upper(H64.float(), None, 0.01)
    torch.cuda.synchronize()
    assert retries == 0 and not fb
    Hd = H64.float().double()
    Hd += 0.01 * torch.diag(Hd).mean() * torch.eye(C, dtype=torch.float64, device=DEV)
    Uref = torch.linalg.cholesky(torch.cholesky_inverse(torch.linalg.cholesky(Hd)), upper=True)
    assert torch.equal(torch.tril(U, -1), torch.zeros_like(U))
    r = float((U.double() - Uref).norm() / Uref.norm())
    I = torch.eye(C, dtype=torch.float64, device=DEV)
    Ui = torch.linalg.solve_triangular(U.double(), I, upper=True)
    back = float((Ui @ Ui.t() - Hd).norm() / Hd.norm())
    print(f"  U rel {r:.2e}, backward {back:.2e}", flush=True)
    assert r < 1e-4, r
    assert back < 1e-5, back


def test_hinv_dead_columns():
    print("hinv dead", flush=True)
    C = 160
    H = _spd(C, 4).float()
    H[:, 5] = 0
    H[5, :] = 0                                   # dead column (bigptq.py:103-105)
    W = torch.randn(8, C)
    Ho = H.clone()
    Uo, info = O.hinv_upper(Ho, W.clone(), 0.01)
    Hd, Wd = H.to(DEV), W.to(DEV)
    U, retries, fb = _k().hinv_upper(Hd, Wd, 0.01)
    torch.cuda.synchronize()
    assert retries == info.retries == 0 and not fb
    assert torch.all(Wd[:, 5].cpu() == 0) and torch.equal(Wd[:, 6:].cpu(), W[:, 6:])
    # dead diagonal set to 1, then damped like every other diagonal entry
    assert rel(torch.diag(Hd), torch.diag(Ho)) < 1e-6
    assert rel(U, Uo) < 1e-4


@pytest.mark.parametrize("need", [1, 3])
def test_hinv_retries(need):
    """An indefinite H whose smallest eigenvalue needs `need` extra damping
    rounds of 1e-3 * mean(diag) (bigptq.py:114-123) after the 1% damping."""
    print(f"hinv retries need={need}", flush=True)
    C = 160
    g = torch.Generator().manual_seed(11)
    Q, _ = torch.linalg.qr(torch.randn(C, C, generator=g, dtype=torch.float64))
    ev = torch.ones(C, dtype=torch.float64)
    ev[0] = -(0.01 + (need - 0.5) * 1e-3) * 0.994
    H = ((Q * ev) @ Q.t()).float()
    Uo, info = O.hinv_upper(H.clone(), torch.zeros(2, C), 0.01)
    U, retries, fb = _k().hinv_upper(H.to(DEV), None, 0.01)
    torch.cuda.synchronize()
    print("  retries gpu", retries, "oracle", info.retries)
    assert info.retries == need
    assert retries == info.retries and fb == info.fallback
    assert rel(U, Uo) < 1e-3


def test_hinv_fallback():
    print("hinv fallback", flush=True)
    C = 64
    H = torch.eye(C) * 2.0
    H[3, 3] = -1e9                                # no amount of damping rescues it
    Uo, info = O.hinv_upper(H.clone(), torch.zeros(2, C), 0.01)
    U, retries, fb = _k().hinv_upper(H.to(DEV), None, 0.01)
    torch.cuda.synchronize()
    assert info.fallback and fb and retries == 10
    assert rel(U, Uo) < 1e-6


# ---------------------------------------------------------------------------
BIN_METHODS = ["braq", "crb", "crb_norefine", "crb_symdamp", "crbog"]


@pytest.mark.parametrize("method", BIN_METHODS)
@pytest.mark.parametrize("order", [1, 2])
def test_binarize_matches_reference_golden(golden, method, order):
    print(f"binarize {method} order {order}", flush=True)
    summary, A = golden
    for c in summary["binarize"]:
        i = c["case"]
        x = torch.from_numpy(A[f"bin{i}_x"])
        m = torch.from_numpy(A[f"bin{i}_m"])
        want = torch.from_numpy(A[f"bin{i}_o{order}_{method}"])
        got = _k().binarize(x.to(DEV), m.to(DEV), order, method).cpu()
        tol = 1e-5 * float(x.abs().max())
        bad = ((got - want).abs() > tol)
        frac = float(bad.float().mean())
        print(f"  case {i}: max|d|={float((got - want).abs().max()):.3g} bad={frac:.4%}")
        assert frac <= 1e-3 or int(bad.sum()) <= 1


@pytest.mark.parametrize("method", BIN_METHODS)
def test_binarize_random_vs_oracle(method):
    print(f"binarize random {method}", flush=True)
    g = torch.Generator().manual_seed(17)
    for R, nc in [(64, 128), (40, 300), (9, 1024), (3, 1)]:
        x = torch.randn(R, nc, generator=g) * 0.02
        m = torch.rand(R, nc, generator=g) < 0.7
        for order in (1, 2):
            want = O.binarize(method, x, m, order)
            got = _k().binarize(x.to(DEV), m.to(DEV), order, method).cpu()
            tol = 1e-5 * float(x.abs().max())
            bad = (got - want).abs() > tol
            assert float(bad.float().mean()) <= 2e-3, (R, nc, order)


@pytest.mark.parametrize("method", BIN_METHODS)
def test_binarize_lane_groups_vs_oracle(method):
    """The 16- and 32-lane-per-row kernel (rows of <= 256 columns with
    16-byte aligned rows): full, ragged (100, 200 columns) and strided rows,
    row counts that leave part of the last workgroup empty."""
    print(f"binarize lane groups {method}", flush=True)
    g = torch.Generator().manual_seed(23)
    for R, nc, ld in [(33, 100, 100), (17, 200, 200), (5, 128, 128), (70, 256, 256),
                      (50, 128, 384), (9, 64, 64)]:
        big = torch.randn(R, ld, generator=g) * 0.02
        x = big[:, ld - nc:] if ld > nc else big       # 16-byte aligned column offset
        m = torch.rand(R, nc, generator=g) < 0.7
        for order in (1, 2):
            want = O.binarize(method, x, m, order)
            got = _k().binarize(big.to(DEV)[:, ld - nc:], m.to(DEV), order, method).cpu()
            tol = 1e-5 * float(x.abs().max())
            bad = (got - want).abs() > tol
            assert float(bad.float().mean()) <= 2e-3, (R, nc, ld, order)


# ---------------------------------------------------------------------------
def test_block_search_matches_reference_golden(golden):
    """structural_searching on the reference-written blocks: T is passed as W
    with the magnitude metric (T = W), which is exactly the reference's
    searching input (utils/autosearch.py:28)."""
    summary, A = golden
    for c in summary["search"]:
        i = c["case"]
        print(f"search case {i} R={c['R']}", flush=True)
        T = torch.from_numpy(A[f"search{i}_T"])
        tr = O.SearchTrace()
        split_o, m3_o = O.structural_searching(T, 50, trace=tr)
        Td = T.to(DEV)
        U = torch.eye(128, device=DEV)
        masks, gt = _k().block_search(Td, U, metric="magnitude", up_lim=50)
        torch.cuda.synchronize()
        # percentiles are exact (same T, same float32 index arithmetic)
        pv = np.asarray(gt["pvals"], dtype=np.float32)
        qo = np.quantile(np.abs((T * (~m3_o)).numpy()).ravel(),
                         O.PERCENTILES.numpy()).astype(np.float32)
        if gt["i_star"] == c["n_salient_cols"]:
            np.testing.assert_array_equal(pv, qo)
        ea = np.asarray(gt["errs_a"][1:50]) / T.numel()
        eo = np.asarray(tr.errs_a)
        print("  istar gpu", gt["i_star"], "ref", c["n_salient_cols"],
              "max rel errA diff", float(np.max(np.abs(ea - eo) / np.abs(eo))))
        assert np.max(np.abs(ea - eo) / np.abs(eo)) < 1e-4
        assert gt["i_star"] == c["n_salient_cols"]
        assert float(gt["split"]).hex() == c["split_hex"] or \
            abs(gt["split"] - c["split"]) <= 1e-6 * abs(c["split"])
        np.testing.assert_array_equal((masks.cpu() == 3).numpy(), A[f"search{i}_m3"])


@pytest.mark.parametrize("R,up_lim", [(64, 30), (37, 30), (1, 30), (300, 33), (130, 12),
                                     (37, 50), (1, 50), (300, 64), (1000, 50)])
def test_block_search_candidate_layouts_vs_oracle(R, up_lim):
    """Salient-count candidates in both packed layouts: two rows per
    wavefront (up_lim - 1 <= 32, structural_searching's default up_lim = 30)
    and (row, candidate) pairs over a workgroup (32 < up_lim - 1 <= 63,
    bigptq.py's up_lim = 50): per-candidate errors, i* and the salient
    columns against the oracle, with row counts that leave part of a
    wavefront or workgroup empty."""
    print(f"search two rows R={R} up_lim={up_lim}", flush=True)
    g = torch.Generator().manual_seed(R + up_lim)
    T = torch.randn(R, 128, generator=g) * torch.exp(torch.randn(128, generator=g))
    tr = O.SearchTrace()
    _, m3_o = O.structural_searching(T, up_lim, trace=tr)
    U = torch.eye(128, device=DEV)
    masks, gt = _k().block_search(T.to(DEV), U, metric="magnitude", up_lim=up_lim)
    torch.cuda.synchronize()
    ea = np.asarray(gt["errs_a"][1:up_lim]) / T.numel()
    eo = np.asarray(tr.errs_a)
    assert np.max(np.abs(ea - eo) / np.abs(eo)) < 1e-4
    assert gt["i_star"] == tr.i_star
    np.testing.assert_array_equal((masks.cpu() == 3).numpy(), m3_o.numpy())
