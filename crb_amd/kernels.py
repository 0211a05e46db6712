"""Torch-tensor wrappers of the crbq C ABI.

Each function takes CUDA (HIP) tensors, allocates what the call needs
through the PyTorch caching allocator (outputs and the workspace), runs on
torch's current stream and raises CrbqError on a non-zero status.
"""
from __future__ import annotations

import ctypes

from typing import NamedTuple

import torch

from . import _lib
from ._lib import CrbqBlockTrace, check, ptr, stream_of


def _dev_check(*ts):
    for t in ts:
        if t is not None and not t.is_cuda:
            raise _lib.CrbqError("crbq tensors must live on the GPU")


def _ws(nbytes: int, device) -> torch.Tensor:
    return torch.empty(max(int(nbytes), 1), dtype=torch.uint8, device=device)


def hessian_accum(X: torch.Tensor, S: torch.Tensor) -> None:
    """S[i, j] += sum_t X[t, i] X[t, j] (upper triangle i <= j), X [T, C]."""
    _dev_check(X, S)
    if X.dim() != 2 or X.stride(1) != 1:
        X = X.reshape(-1, X.shape[-1]).contiguous()
    if X.dtype not in _lib.DTYPES:
        X = X.float()
    T, C = X.shape
    lib = _lib.ready(X.device)
    nb = (lib.crbq_hessian_workspace_size(T, C)
          if S.stride(0) == C and X.dtype != torch.float32 else 0)
    ws = _ws(nb, X.device) if nb else None
    check(lib.crbq_hessian_accum(X.data_ptr(), _lib.DTYPES[X.dtype], T, X.stride(0), C,
                                 S.data_ptr(), S.stride(0), ptr(ws), nb, stream_of(S)),
          "crbq_hessian_accum")


def hessian_cm_store(ntok: int, C: int, dtype: torch.dtype, device) -> torch.Tensor:
    """An uninitialised channel-major activation store [rows, ldt] for
    hessian_transpose / hessian_accum_cm (crbq_hessian_cm_shape)."""
    rows, ldt = ctypes.c_int64(), ctypes.c_int64()
    check(_lib.load().crbq_hessian_cm_shape(int(ntok), int(C), ctypes.byref(rows),
                                            ctypes.byref(ldt)), "crbq_hessian_cm_shape")
    return torch.empty((rows.value, ldt.value), dtype=dtype, device=device)


def hessian_transpose(X: torch.Tensor, Xt: torch.Tensor, t0: int) -> None:
    """Write the token rows of X [T, C] (f16/bf16) into columns t0.. of the
    channel-major store Xt (t0 a multiple of 64)."""
    _dev_check(X, Xt)
    if X.dim() != 2 or X.stride(1) != 1:
        X = X.reshape(-1, X.shape[-1]).contiguous()
    if X.dtype not in (torch.float16, torch.bfloat16) or Xt.dtype != X.dtype:
        raise _lib.CrbqError("hessian_transpose takes 16-bit activations and a store of "
                             "the same dtype")
    if Xt.stride(1) != 1:
        raise _lib.CrbqError("hessian_transpose writes a row-major store")
    T, C = X.shape
    lib = _lib.ready(X.device)
    check(lib.crbq_hessian_transpose(X.data_ptr(), _lib.DTYPES[X.dtype], T, X.stride(0), C,
                                     Xt.data_ptr(), Xt.stride(0), int(t0), stream_of(Xt)),
          "crbq_hessian_transpose")


def hessian_accum_cm(Xt: torch.Tensor, ntok: int, C: int, S: torch.Tensor) -> None:
    """S += Xt[:C, :ntok] Xt[:C, :ntok]^T (upper triangle) from a store that
    hessian_transpose filled."""
    _dev_check(Xt, S)
    lib = _lib.ready(Xt.device)
    nb = lib.crbq_hessian_cm_workspace_size(int(ntok), int(C)) if S.stride(0) == C else 0
    ws = _ws(nb, Xt.device) if nb else None
    check(lib.crbq_hessian_accum_cm(Xt.data_ptr(), _lib.DTYPES[Xt.dtype], int(ntok),
                                    Xt.stride(0), int(C), S.data_ptr(), S.stride(0), ptr(ws),
                                    nb, stream_of(S)), "crbq_hessian_accum_cm")


def syrk_timing(on: bool) -> None:
    """Switch the per-launch SYRK timing of hessian_accum on or off."""
    check(_lib.load().crbq_syrk_timing(1 if on else 0), "crbq_syrk_timing")


def syrk_timing_collect(max_records: int = 4096):
    """[(C, ms)] of the SYRK launches recorded since the last collect
    (waits for them to finish)."""
    lib = _lib.load()
    ms = (ctypes.c_float * max_records)()
    cs = (ctypes.c_int64 * max_records)()
    n = ctypes.c_int32(0)
    check(lib.crbq_syrk_timing_collect(ms, cs, max_records, ctypes.byref(n)),
          "crbq_syrk_timing_collect")
    return [(int(cs[i]), float(ms[i])) for i in range(min(n.value, max_records))]


def hessian_finalize(S: torch.Tensor, scale: float, H: torch.Tensor | None = None) -> torch.Tensor:
    """H = scale * sym(S) from the upper triangle of S (H may be S)."""
    _dev_check(S)
    C = S.shape[0]
    if H is None:
        H = torch.empty_like(S)
    lib = _lib.ready(S.device)
    check(lib.crbq_hessian_finalize(S.data_ptr(), S.stride(0), C, float(scale), H.data_ptr(),
                                    H.stride(0), stream_of(S)), "crbq_hessian_finalize")
    return H


def hinv_upper(H: torch.Tensor, W: torch.Tensor | None, percdamp: float = 0.01):
    """bigptq.py:101-129.  Mutates H (and W's dead columns) like the
    reference.  Returns (U, retries, fallback)."""
    _dev_check(H, W)
    if H.stride(1) != 1 or (W is not None and W.stride(1) != 1):
        raise _lib.CrbqError("hinv_upper works in place on row-major H and W")
    C = H.shape[0]
    lib = _lib.ready(H.device)
    U = torch.empty((C, C), dtype=torch.float32, device=H.device)
    ws = _ws(lib.crbq_hinv_workspace_size(C), H.device)
    retries = ctypes.c_int32(0)
    fallback = ctypes.c_int32(0)
    R = W.shape[0] if W is not None else 0
    ldw = W.stride(0) if W is not None else 0
    check(lib.crbq_hinv_upper(H.data_ptr(), H.stride(0), C, ptr(W), R, ldw, float(percdamp),
                              U.data_ptr(), U.stride(0), ws.data_ptr(), ws.numel(),
                              ctypes.byref(retries), ctypes.byref(fallback), stream_of(H)),
          "crbq_hinv_upper")
    return U, int(retries.value), bool(fallback.value)


class HinvJob:
    """An inverse-factor computation enqueued with hinv_upper_async."""

    def __init__(self, H, U, ws, stream):
        self.H, self.U, self.ws, self.stream = H, U, ws, stream


def hinv_upper_async(H: torch.Tensor, W: torch.Tensor | None, percdamp: float = 0.01) -> HinvJob:
    """Enqueue bigptq.py:101-129 on the current stream without waiting."""
    _dev_check(H, W)
    if H.stride(1) != 1 or (W is not None and W.stride(1) != 1):
        raise _lib.CrbqError("hinv_upper works in place on row-major H and W")
    C = H.shape[0]
    lib = _lib.ready(H.device)
    U = torch.empty((C, C), dtype=torch.float32, device=H.device)
    ws = _ws(lib.crbq_hinv_workspace_size(C), H.device)
    R = W.shape[0] if W is not None else 0
    ldw = W.stride(0) if W is not None else 0
    st = stream_of(H)
    check(lib.crbq_hinv_upper_async(H.data_ptr(), H.stride(0), C, ptr(W), R, ldw,
                                    float(percdamp), U.data_ptr(), U.stride(0), ws.data_ptr(),
                                    ws.numel(), st), "crbq_hinv_upper_async")
    return HinvJob(H, U, ws, torch.cuda.current_stream(H.device))


def hinv_upper_finish(job: HinvJob):
    """Wait for the job's stream, retry/fallback if needed.  Returns
    (U, retries, fallback)."""
    lib = _lib.ready(job.H.device)
    retries = ctypes.c_int32(0)
    fallback = ctypes.c_int32(0)
    C = job.H.shape[0]
    check(lib.crbq_hinv_upper_finish(job.H.data_ptr(), job.H.stride(0), C, job.U.data_ptr(),
                                     job.U.stride(0), job.ws.data_ptr(), job.ws.numel(),
                                     ctypes.byref(retries), ctypes.byref(fallback),
                                     job.stream.cuda_stream), "crbq_hinv_upper_finish")
    return job.U, int(retries.value), bool(fallback.value)


def fasterquant_blocks(W: torch.Tensor, U: torch.Tensor, p: _lib.CrbqParams,
                       losses: torch.Tensor, want_masks: bool = False,
                       want_traces: bool = False):
    """Block loop of bigptq.py:131-264 on W (fp32, in place).
    Returns (masks uint8 [R, C] or None, traces list or None)."""
    _dev_check(W, U, losses)
    if W.dtype != torch.float32 or W.stride(1) != 1:
        raise _lib.CrbqError("fasterquant_blocks works in place on a row-major fp32 W")
    if U.stride(1) != 1:
        U = U.contiguous()
    R, C = W.shape
    lib = _lib.ready(W.device)
    ws = _ws(lib.crbq_fasterquant_workspace_size(R, C, ctypes.byref(p)), W.device)
    masks = torch.zeros((R, C), dtype=torch.uint8, device=W.device) if want_masks else None
    nblk = (C + p.blocksize - 1) // p.blocksize
    tr = torch.zeros(nblk * _lib.TRACE_BYTES, dtype=torch.uint8,
                     device=W.device) if want_traces else None
    check(lib.crbq_fasterquant(W.data_ptr(), R, C, W.stride(0), U.data_ptr(), U.stride(0),
                               ctypes.byref(p), losses.data_ptr(), ptr(masks),
                               masks.stride(0) if masks is not None else 0, ptr(tr),
                               ws.data_ptr(), ws.numel(), stream_of(W)),
          "crbq_fasterquant")
    traces = decode_traces(tr, nblk) if tr is not None else None
    return masks, traces


MAX_BATCH = 4   # sublayers per crbq_fasterquant_batched call


def fasterquant_blocks_batched(Ws, Us, p: _lib.CrbqParams, losses,
                               want_masks: bool = False, want_traces: bool = False):
    """fasterquant_blocks on up to MAX_BATCH weights of one shape and row
    stride, as one block loop.  Us is one factor for all of them or a list
    with one factor per weight (all of one size and row stride).  Every W
    is updated in place and every losses[i] accumulated exactly as
    fasterquant_blocks would for it alone.  Returns ([masks or None],
    [traces or None])."""
    n = len(Ws)
    if isinstance(Us, torch.Tensor):
        Us = [Us] * n
    if not 1 <= n <= MAX_BATCH or len(losses) != n or len(Us) != n:
        raise _lib.CrbqError(f"fasterquant_blocks_batched takes 1..{MAX_BATCH} weights and "
                             "as many factors and loss vectors")
    Us = [U if U.stride(1) == 1 else U.contiguous() for U in Us]
    _dev_check(*Us, *Ws, *losses)
    R, C = Ws[0].shape
    ldw, ldu = Ws[0].stride(0), Us[0].stride(0)
    for W in Ws:
        if W.dtype != torch.float32 or W.stride(1) != 1:
            raise _lib.CrbqError("fasterquant_blocks_batched works in place on row-major fp32 W")
        if tuple(W.shape) != (R, C) or W.stride(0) != ldw:
            raise _lib.CrbqError("fasterquant_blocks_batched needs weights of one shape and stride")
    for U in Us:
        if U.dtype != torch.float32 or tuple(U.shape) != (C, C) or U.stride(0) != ldu:
            raise _lib.CrbqError("fasterquant_blocks_batched needs fp32 C x C factors of one "
                                 "row stride")
    dev = Ws[0].device
    lib = _lib.ready(dev)
    ws = _ws(lib.crbq_fasterquant_batched_workspace_size(n, R, C, ctypes.byref(p)), dev)
    masks = [torch.zeros((R, C), dtype=torch.uint8, device=dev) if want_masks else None
             for _ in range(n)]
    nblk = (C + p.blocksize - 1) // p.blocksize
    trs = [torch.zeros(nblk * _lib.TRACE_BYTES, dtype=torch.uint8, device=dev)
           if want_traces else None for _ in range(n)]
    arr = ctypes.c_void_p * n
    check(lib.crbq_fasterquant_batched(
        n, arr(*[W.data_ptr() for W in Ws]), R, C, ldw, arr(*[U.data_ptr() for U in Us]), ldu,
        ctypes.byref(p), arr(*[x.data_ptr() for x in losses]), arr(*[ptr(m) for m in masks]),
        masks[0].stride(0) if want_masks else 0, arr(*[ptr(t) for t in trs]),
        ws.data_ptr(), ws.numel(), stream_of(Ws[0])), "crbq_fasterquant_batched")
    traces = [decode_traces(t, nblk) if t is not None else None for t in trs]
    return masks, traces


def fasterquant_blocks_noalloc(W: torch.Tensor, U: torch.Tensor, p: _lib.CrbqParams,
                               losses: torch.Tensor, masks: torch.Tensor | None = None,
                               traces: torch.Tensor | None = None) -> None:
    """fasterquant_blocks through crbq_fasterquant_noalloc: no workspace, and
    no allocation at all (the outputs, masks and the raw trace buffer are
    the caller's).  Raises CrbqError for problems beyond the library's
    static scratch."""
    _dev_check(W, U, losses, masks, traces)
    if W.dtype != torch.float32 or W.stride(1) != 1 or U.stride(1) != 1:
        raise _lib.CrbqError("fasterquant_blocks_noalloc works in place on row-major fp32 W, U")
    R, C = W.shape
    lib = _lib.ready(W.device)
    check(lib.crbq_fasterquant_noalloc(W.data_ptr(), R, C, W.stride(0), U.data_ptr(),
                                       U.stride(0), ctypes.byref(p), losses.data_ptr(),
                                       ptr(masks), masks.stride(0) if masks is not None else 0,
                                       ptr(traces), stream_of(W)),
          "crbq_fasterquant_noalloc")


def decode_traces(buf: torch.Tensor, n: int):
    raw = bytes(buf.cpu().numpy().tobytes())
    out = []
    for i in range(n):
        t = CrbqBlockTrace.from_buffer_copy(raw, i * _lib.TRACE_BYTES)
        out.append({
            "i_star": t.i_star, "k_star": t.k_star, "split": t.split,
            "pvals": list(t.pvals), "errs_a": list(t.errs_a), "errs_c": list(t.errs_c),
        })
    return out


def block_search(Wblk: torch.Tensor, Ublk: torch.Tensor, metric: str = "hessian",
                 up_lim: int = 50):
    """One block of utils/structure.py:8-20.  Wblk [R, ncols] (may be a
    column slice of W), Ublk [ncols, ncols] slice of U.
    Returns (mask codes uint8 [R, ncols]: 1/2/3, trace dict)."""
    _dev_check(Wblk, Ublk)
    if Wblk.stride(1) != 1:
        Wblk = Wblk.contiguous()
    if Ublk.stride(1) != 1:
        Ublk = Ublk.contiguous()
    R, nc = Wblk.shape
    lib = _lib.ready(Wblk.device)
    ws = _ws(lib.crbq_block_search_workspace_size(R, up_lim), Wblk.device)
    masks = torch.zeros((R, nc), dtype=torch.uint8, device=Wblk.device)
    tr = torch.zeros(_lib.TRACE_BYTES, dtype=torch.uint8, device=Wblk.device)
    check(lib.crbq_block_search(Wblk.data_ptr(), R, nc, Wblk.stride(0), Ublk.data_ptr(),
                                Ublk.stride(0), _lib.METRICS[metric], up_lim, masks.data_ptr(),
                                masks.stride(0), tr.data_ptr(), ws.data_ptr(), ws.numel(),
                                stream_of(Wblk)), "crbq_block_search")
    return masks, decode_traces(tr, 1)[0]


def binarize(x: torch.Tensor, mask: torch.Tensor, order: int, method: str, lam: float = 1e-5,
             corr_damp: float = 0.1, refine_iters: int = 1, out: torch.Tensor | None = None):
    """Binarization.quantize (binary.py:2874-2890) for the crbq methods."""
    _dev_check(x, mask)
    if method not in _lib.METHODS:
        raise NotImplementedError(method)
    xf = x if (x.dtype == torch.float32 and x.stride(-1) == 1) else x.float().contiguous()
    if xf.dim() != 2:
        raise _lib.CrbqError("binarize takes a [rows, cols] weight block")
    try:
        # the reference's elementwise ops broadcast the mask ([cols] or [1, cols])
        m = mask.expand_as(xf)
    except RuntimeError as e:
        raise _lib.CrbqError(f"binarize: mask of shape {tuple(mask.shape)} does not "
                             f"broadcast to {tuple(xf.shape)}") from e
    m = m.to(torch.uint8).contiguous()
    R, nc = xf.shape
    if out is None:
        out = torch.empty((R, nc), dtype=torch.float32, device=x.device)
    lib = _lib.ready(x.device)
    check(lib.crbq_binarize(xf.data_ptr(), R, nc, xf.stride(0), m.data_ptr(), m.stride(0),
                            int(order), _lib.METHODS[method], float(lam), float(corr_damp),
                            int(refine_iters), out.data_ptr(), out.stride(0), stream_of(xf)),
          "crbq_binarize")
    return out


def binarize_scales(x: torch.Tensor, mask: torch.Tensor, order: int, method: str,
                    lam: float = 1e-5, corr_damp: float = 0.1, refine_iters: int = 1):
    """Binarization.quantize with each row's scales (crbq_binarize_scales).
    Returns (out fp32 [R, cols], scales fp32 [R, n]): n = 4, (mean, mu
    correction, a1, a2), for the CRB variants and CRBOG at order >= 2;
    n = 2 * order, (mu_k, alpha_k) per pass, for BRAQ and CRBOG at order 1."""
    _dev_check(x, mask)
    if method not in _lib.METHODS:
        raise NotImplementedError(method)
    xf = x.float().contiguous()
    m = mask.expand_as(xf).to(torch.uint8).contiguous()
    R, nc = xf.shape
    passes = method == "braq" or (method == "crbog" and order == 1)
    nsc = 2 * order if passes else 4
    out = torch.empty((R, nc), dtype=torch.float32, device=x.device)
    sc = torch.zeros((R, nsc), dtype=torch.float32, device=x.device)
    lib = _lib.ready(x.device)
    check(lib.crbq_binarize_scales(xf.data_ptr(), R, nc, xf.stride(0), m.data_ptr(),
                                   m.stride(0), int(order), _lib.METHODS[method], float(lam),
                                   float(corr_damp), int(refine_iters), out.data_ptr(),
                                   out.stride(0), sc.data_ptr(), sc.stride(0), stream_of(xf)),
          "crbq_binarize_scales")
    return out, sc


def sgemm(A: torch.Tensor, B: torch.Tensor, C: torch.Tensor, alpha: float = 1.0,
          beta: float = 0.0, transa: bool = False, transb: bool = False) -> torch.Tensor:
    """C = beta*C + alpha*op(A) op(B) on fp32 MFMA (row-major operands)."""
    _dev_check(A, B, C)
    if C.stride(1) != 1:
        raise _lib.CrbqError("sgemm writes a row-major C")
    if A.stride(1) != 1:
        A = A.contiguous()
    if B.stride(1) != 1:
        B = B.contiguous()
    M, N = C.shape
    K = A.shape[0] if transa else A.shape[1]
    lib = _lib.ready(C.device)
    check(lib.crbq_sgemm(int(transa), int(transb), M, N, K, float(alpha), A.data_ptr(),
                         A.stride(0), B.data_ptr(), B.stride(0), float(beta), C.data_ptr(),
                         C.stride(0), stream_of(C)), "crbq_sgemm")
    return C


# -- packed low-bit storage ---------------------------------------------------
PACK_BLOCK = 128
PACK_ERRORS = {1: "more out-of-table values than the exception list holds (weights not "
                  "from the binarizer, or blocksize not a multiple of 128)",
               2: "salient columns differ between rows",
               4: "mask code outside 1..3"}


class PackedEx(NamedTuple):
    """Exceptions of a packed layer, sorted by flat index r * C + c."""
    idx: torch.Tensor      # int64 [n]
    val: torch.Tensor      # [n] in the weight dtype: the exact values
    delta: torch.Tensor    # fp32 [n]: value - the table entry their code decodes to


def _ex_args(ex, device, dtype):
    if ex is None or ex.idx.numel() == 0:
        return 0, 0, 0, 0
    _dev_check(ex.idx, ex.val, ex.delta)
    return ex.idx.data_ptr(), ex.val.data_ptr(), ex.delta.data_ptr(), int(ex.idx.numel())


def pack(Q: torch.Tensor, masks: torch.Tensor, ex_cap: int | None = None):
    """Packed form (codes, lut, sal, ex) of quantized fp16/bf16 weights
    Q [R, C] with their mask codes (uint8 1/2/3).  Raises CrbqError if Q
    does not have the per-block structure the format stores (beyond
    ex_cap exceptions, by default one per 8 row-blocks and at least 1024)."""
    _dev_check(Q, masks)
    if Q.dtype not in (torch.float16, torch.bfloat16) or Q.dim() != 2 or Q.stride(1) != 1:
        raise _lib.CrbqError("pack takes a row-major fp16/bf16 [R, C] weight")
    if masks.dtype != torch.uint8 or masks.shape != Q.shape or masks.stride(1) != 1:
        raise _lib.CrbqError("pack takes uint8 mask codes shaped like the weight")
    R, C = Q.shape
    nblk = (C + PACK_BLOCK - 1) // PACK_BLOCK
    cap = int(ex_cap) if ex_cap is not None else max(1024, R * nblk // 8)
    dev = Q.device
    codes = torch.empty((R, nblk * 32), dtype=torch.uint8, device=dev)
    lut = torch.empty((R, nblk, 8), dtype=Q.dtype, device=dev)
    sal = torch.empty((nblk, 16), dtype=torch.uint8, device=dev)
    ex_idx = torch.empty(max(cap, 1), dtype=torch.int64, device=dev)
    ex_val = torch.empty(max(cap, 1), dtype=Q.dtype, device=dev)
    ex_delta = torch.empty(max(cap, 1), dtype=torch.float32, device=dev)
    counters = torch.empty(2, dtype=torch.int32, device=dev)     # status, ex_count
    lib = _lib.ready(dev)
    check(lib.crbq_pack(Q.data_ptr(), _lib.DTYPES[Q.dtype], R, C, Q.stride(0),
                        masks.data_ptr(), masks.stride(0), codes.data_ptr(), codes.stride(0),
                        lut.data_ptr(), sal.data_ptr(), ex_idx.data_ptr(), ex_val.data_ptr(),
                        ex_delta.data_ptr(), cap, counters[1:].data_ptr(),
                        counters[:1].data_ptr(), stream_of(Q)),
          "crbq_pack")
    st, n = (int(v) for v in counters.tolist())
    if st:
        why = "; ".join(v for k, v in PACK_ERRORS.items() if st & k)
        raise _lib.CrbqError(f"crbq_pack: {why}")
    order = torch.argsort(ex_idx[:n])
    ex = PackedEx(ex_idx[:n][order].contiguous(), ex_val[:n][order].contiguous(),
                  ex_delta[:n][order].contiguous())
    return codes, lut, sal, ex


def unpack(codes: torch.Tensor, lut: torch.Tensor, sal: torch.Tensor, C: int,
           ex: PackedEx | None = None) -> torch.Tensor:
    """The weights [R, C] (lut's dtype) a packed layer encodes."""
    _dev_check(codes, lut, sal)
    R = codes.shape[0]
    Q = torch.empty((R, C), dtype=lut.dtype, device=codes.device)
    lib = _lib.ready(codes.device)
    ei, ev, _, n = _ex_args(ex, codes.device, lut.dtype)
    check(lib.crbq_unpack(codes.data_ptr(), codes.stride(0), lut.data_ptr(), sal.data_ptr(),
                          ei, ev, n, _lib.DTYPES[lut.dtype], R, C, Q.data_ptr(), Q.stride(0),
                          stream_of(Q)), "crbq_unpack")
    return Q


def _packed_x(x, lut, C, what):
    if x.dim() == 1:
        x = x.unsqueeze(0)
    if x.dtype != lut.dtype:
        x = x.to(lut.dtype)
    if x.shape[0] < 1 or x.shape[1] != C:
        raise _lib.CrbqError(f"{what} takes [T, C] activations of the weight's width")
    if x.stride(1) != 1 or x.stride(0) % 8 or x.data_ptr() % 16:
        # a fresh allocation: contiguous() would hand back a contiguous view
        # at a misaligned storage offset unchanged
        x = x.clone(memory_format=torch.contiguous_format)
        if C % 8:
            xp = torch.zeros((x.shape[0], (C + 7) // 8 * 8), dtype=x.dtype, device=x.device)
            xp[:, :C] = x
            x = xp
    return x


def gemv_packed(codes: torch.Tensor, lut: torch.Tensor, sal: torch.Tensor, C: int,
                x: torch.Tensor, ex: PackedEx | None = None) -> torch.Tensor:
    """y [nvec, R] (fp32) = x [nvec, C] @ W^T for the packed W, nvec <= 16."""
    _dev_check(codes, lut, sal, x)
    x = _packed_x(x, lut, C, "gemv_packed")
    nvec = x.shape[0]
    if nvec > 16:
        raise _lib.CrbqError("gemv_packed takes 1..16 vectors")
    R = codes.shape[0]
    y = torch.empty((nvec, R), dtype=torch.float32, device=x.device)
    lib = _lib.ready(x.device)
    ei, _, ed, n = _ex_args(ex, x.device, lut.dtype)
    check(lib.crbq_gemv_packed(codes.data_ptr(), codes.stride(0), lut.data_ptr(),
                               sal.data_ptr(), ei, ed, n, _lib.DTYPES[lut.dtype], R, C,
                               x.data_ptr(), x.stride(0), nvec, y.data_ptr(), y.stride(0),
                               stream_of(y)),
          "crbq_gemv_packed")
    return y


def gemm_packed(codes: torch.Tensor, lut: torch.Tensor, sal: torch.Tensor, C: int,
                x: torch.Tensor, ex: PackedEx | None = None) -> torch.Tensor:
    """Y [T, R] (fp32) = x [T, C] @ W^T for the packed W, any T >= 1."""
    _dev_check(codes, lut, sal, x)
    x = _packed_x(x, lut, C, "gemm_packed")
    T = x.shape[0]
    R = codes.shape[0]
    y = torch.empty((T, R), dtype=torch.float32, device=x.device)
    lib = _lib.ready(x.device)
    nws = int(lib.crbq_gemm_packed_workspace_size(R, C, T))
    ws = torch.empty(max(nws, 1), dtype=torch.uint8, device=x.device)
    ei, _, ed, n = _ex_args(ex, x.device, lut.dtype)
    check(lib.crbq_gemm_packed(codes.data_ptr(), codes.stride(0), lut.data_ptr(),
                               sal.data_ptr(), ei, ed, n, _lib.DTYPES[lut.dtype], R, C,
                               x.data_ptr(), x.stride(0), T, y.data_ptr(), y.stride(0),
                               ws.data_ptr(), nws, stream_of(y)),
          "crbq_gemm_packed")
    return y
