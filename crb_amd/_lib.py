"""ctypes binding of the crbq C ABI (include/crbq.h).

The library is built in-tree as crb_amd/libcrbq.so (``python -m
crb_amd.build``).  There is no fallback: if the library is missing or the
current device is not a gfx950, every entry point raises.
"""
from __future__ import annotations

import ctypes
import os
import threading

import torch

LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "libcrbq.so")

# enum crbq_dtype
DTYPES = {torch.float32: 0, torch.float16: 1, torch.bfloat16: 2}
# enum crbq_method (binary.py:2875-2890)
METHODS = {
    "braq": 0,
    "crb": 1,
    "crbog": 2,
    "crb_norefine": 3,
    "crb_symdamp": 4,
    "crb_symdamp_norefine": 5,
}
METRICS = {"magnitude": 0, "hessian": 1}

c_i64 = ctypes.c_int64
c_i32 = ctypes.c_int32
c_vp = ctypes.c_void_p
c_size = ctypes.c_size_t


class CrbqParams(ctypes.Structure):
    _fields_ = [
        ("method", c_i32), ("metric", c_i32), ("blocksize", c_i32),
        ("partition", c_i32), ("orders", c_i32 * 3), ("up_lim", c_i32),
        ("refine_iters", c_i32), ("disable_gptq", c_i32),
        ("lam", ctypes.c_float), ("corr_damp", ctypes.c_float),
    ]


class CrbqBlockTrace(ctypes.Structure):
    _fields_ = [
        ("i_star", c_i32), ("k_star", c_i32), ("split", ctypes.c_float),
        ("pvals", ctypes.c_float * 81),
        ("errs_a", ctypes.c_double * 64),
        ("errs_c", ctypes.c_double * 81),
    ]


TRACE_BYTES = ctypes.sizeof(CrbqBlockTrace)
NOALLOC_SCRATCH_BYTES = 80 << 20      # CRBQ_NOALLOC_SCRATCH_BYTES (include/crbq.h)
ERR_TOO_LARGE = -5                    # CRBQ_ERR_TOO_LARGE
ERR_CAPTURE = -6                      # CRBQ_ERR_CAPTURE

_SIGS = {
    "crbq_version": (c_i32, []),
    "crbq_status_string": (ctypes.c_char_p, [c_i32]),
    "crbq_device_ok": (c_i32, []),
    "crbq_set_percentiles": (c_i32, [c_vp]),
    "crbq_hessian_workspace_size": (c_size, [c_i64, c_i64]),
    "crbq_hessian_accum": (c_i32, [c_vp, c_i32, c_i64, c_i64, c_i64, c_vp, c_i64, c_vp, c_size,
                                   c_vp]),
    "crbq_hessian_cm_shape": (c_i32, [c_i64, c_i64, ctypes.POINTER(c_i64),
                                      ctypes.POINTER(c_i64)]),
    "crbq_hessian_transpose": (c_i32, [c_vp, c_i32, c_i64, c_i64, c_i64, c_vp, c_i64, c_i64,
                                       c_vp]),
    "crbq_hessian_cm_workspace_size": (c_size, [c_i64, c_i64]),
    "crbq_hessian_accum_cm": (c_i32, [c_vp, c_i32, c_i64, c_i64, c_i64, c_vp, c_i64, c_vp,
                                      c_size, c_vp]),
    "crbq_syrk_timing": (c_i32, [c_i32]),
    "crbq_syrk_timing_collect": (c_i32, [c_vp, c_vp, c_i32, ctypes.POINTER(c_i32)]),
    "crbq_hessian_finalize": (c_i32, [c_vp, c_i64, c_i64, ctypes.c_float, c_vp, c_i64, c_vp]),
    "crbq_hinv_workspace_size": (c_size, [c_i64]),
    "crbq_hinv_upper": (c_i32, [c_vp, c_i64, c_i64, c_vp, c_i64, c_i64, ctypes.c_float, c_vp,
                                c_i64, c_vp, c_size, ctypes.POINTER(c_i32),
                                ctypes.POINTER(c_i32), c_vp]),
    "crbq_hinv_upper_async": (c_i32, [c_vp, c_i64, c_i64, c_vp, c_i64, c_i64, ctypes.c_float,
                                      c_vp, c_i64, c_vp, c_size, c_vp]),
    "crbq_hinv_upper_finish": (c_i32, [c_vp, c_i64, c_i64, c_vp, c_i64, c_vp, c_size,
                                       ctypes.POINTER(c_i32), ctypes.POINTER(c_i32), c_vp]),
    "crbq_fasterquant_workspace_size": (c_size, [c_i64, c_i64, ctypes.POINTER(CrbqParams)]),
    "crbq_fasterquant": (c_i32, [c_vp, c_i64, c_i64, c_i64, c_vp, c_i64,
                                 ctypes.POINTER(CrbqParams), c_vp, c_vp, c_i64, c_vp, c_vp,
                                 c_size, c_vp]),
    "crbq_fasterquant_batched_workspace_size": (c_size, [c_i32, c_i64, c_i64,
                                                         ctypes.POINTER(CrbqParams)]),
    "crbq_fasterquant_batched": (c_i32, [c_i32, ctypes.POINTER(c_vp), c_i64, c_i64, c_i64,
                                         ctypes.POINTER(c_vp), c_i64, ctypes.POINTER(CrbqParams),
                                         ctypes.POINTER(c_vp), ctypes.POINTER(c_vp), c_i64,
                                         ctypes.POINTER(c_vp), c_vp, c_size, c_vp]),
    "crbq_fasterquant_noalloc": (c_i32, [c_vp, c_i64, c_i64, c_i64, c_vp, c_i64,
                                         ctypes.POINTER(CrbqParams), c_vp, c_vp, c_i64, c_vp,
                                         c_vp]),
    "crbq_block_search_workspace_size": (c_size, [c_i64, c_i32]),
    "crbq_block_search": (c_i32, [c_vp, c_i64, c_i32, c_i64, c_vp, c_i64, c_i32, c_i32, c_vp,
                                  c_i64, c_vp, c_vp, c_size, c_vp]),
    "crbq_binarize": (c_i32, [c_vp, c_i64, c_i32, c_i64, c_vp, c_i64, c_i32, c_i32,
                              ctypes.c_float, ctypes.c_float, c_i32, c_vp, c_i64, c_vp]),
    "crbq_binarize_scales": (c_i32, [c_vp, c_i64, c_i32, c_i64, c_vp, c_i64, c_i32, c_i32,
                                     ctypes.c_float, ctypes.c_float, c_i32, c_vp, c_i64, c_vp,
                                     c_i64, c_vp]),
    "crbq_sgemm": (c_i32, [c_i32, c_i32, c_i64, c_i64, c_i64, ctypes.c_float, c_vp, c_i64,
                           c_vp, c_i64, ctypes.c_float, c_vp, c_i64, c_vp]),
    "crbq_pack": (c_i32, [c_vp, c_i32, c_i64, c_i64, c_i64, c_vp, c_i64, c_vp, c_i64, c_vp,
                          c_vp, c_vp, c_vp, c_vp, c_i32, c_vp, c_vp, c_vp]),
    "crbq_unpack": (c_i32, [c_vp, c_i64, c_vp, c_vp, c_vp, c_vp, c_i64, c_i32, c_i64, c_i64,
                            c_vp, c_i64, c_vp]),
    "crbq_gemv_packed": (c_i32, [c_vp, c_i64, c_vp, c_vp, c_vp, c_vp, c_i64, c_i32, c_i64,
                                 c_i64, c_vp, c_i64, c_i32, c_vp, c_i64, c_vp]),
    "crbq_gemm_packed_workspace_size": (c_size, [c_i64, c_i64, c_i64]),
    "crbq_gemm_packed": (c_i32, [c_vp, c_i64, c_vp, c_vp, c_vp, c_vp, c_i64, c_i32, c_i64,
                                 c_i64, c_vp, c_i64, c_i64, c_vp, c_i64, c_vp, c_size, c_vp]),
}

_lock = threading.Lock()
_lib = None
_ready_devices: set = set()


class CrbqError(RuntimeError):
    pass


def load() -> ctypes.CDLL:
    """Load libcrbq.so (no GPU needed) and set the ctypes signatures."""
    global _lib
    with _lock:
        if _lib is None:
            if not os.path.exists(LIB_PATH):
                raise CrbqError(
                    f"{LIB_PATH} is missing: build it with `python -m crb_amd.build` "
                    "(there is no CPU fallback)")
            lib = ctypes.CDLL(LIB_PATH)
            for name, (res, args) in _SIGS.items():
                fn = getattr(lib, name)
                fn.restype = res
                fn.argtypes = args
            _lib = lib
    return _lib


def check(status: int, what: str) -> None:
    if status != 0:
        msg = load().crbq_status_string(status).decode()
        raise CrbqError(f"{what} failed: status {status} ({msg})")


def percentiles_cpu() -> torch.Tensor:
    """torch.linspace(0.10, 0.90, 81) on the CPU, as utils/autosearch.py:65."""
    return torch.linspace(0.10, 0.90, 81)


def ready(device: torch.device | None = None) -> ctypes.CDLL:
    """Library handle, after checking the device is a gfx950 and uploading
    the percentile table (once per device)."""
    lib = load()
    if not torch.cuda.is_available():
        raise CrbqError("no HIP device: the crbq path runs only on an MI355X (gfx950)")
    dev = torch.cuda.current_device() if device is None else (
        device.index if device.index is not None else torch.cuda.current_device())
    if dev not in _ready_devices:
        with torch.cuda.device(dev):
            check(lib.crbq_device_ok(), "crbq_device_ok (device is not gfx950)")
            q = percentiles_cpu().contiguous()
            check(lib.crbq_set_percentiles(q.data_ptr()), "crbq_set_percentiles")
        _ready_devices.add(dev)
    return lib


def stream_of(t: torch.Tensor) -> int:
    return torch.cuda.current_stream(t.device).cuda_stream


def ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


def params(method: str, metric: str = "hessian", blocksize: int = 128, partition: int = 3,
           orders=(1, 1, 2), up_lim: int = 50, refine_iters: int = 1,
           disable_gptq: bool = False, lam: float = 1e-5, corr_damp: float = 0.1) -> CrbqParams:
    if method not in METHODS:
        raise NotImplementedError(f"method {method!r} is not on the crbq path "
                                  f"(supported: {sorted(METHODS)})")
    if metric not in METRICS:
        raise NotImplementedError(metric)
    p = CrbqParams()
    p.method = METHODS[method]
    p.metric = METRICS[metric]
    p.blocksize = int(blocksize)
    p.partition = int(partition)
    for i in range(3):
        p.orders[i] = int(orders[i])
    p.up_lim = int(up_lim)
    p.refine_iters = int(refine_iters)
    p.disable_gptq = int(bool(disable_gptq))
    p.lam = float(lam)
    p.corr_damp = float(corr_damp)
    return p
