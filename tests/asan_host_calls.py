"""Host-side calls of the C ABI for the AddressSanitizer build (run by
tests/test_capi_asan.py in a process that preloads the ASan runtime; no GPU
is needed).  Every entry point gets the queries and argument sets its
validation handles: sizes and enums out of range, NULL pointers, pointer
arrays of exactly nseg entries (read on the host), and plausible fake device
pointers where validation must pass, after which the call stops at its first
HIP call (no device here) before touching device memory.  Exit status 0 when
every call returned; ASan aborts the process on a host memory error."""
import ctypes
import sys

sys.path.insert(0, sys.argv[2])
from crb_amd import _lib  # noqa: E402

_lib.LIB_PATH = sys.argv[1]
lib = _lib.load()
if lib.crbq_device_ok() == 0:
    # a gfx950 is visible: the calls below that pass validation would
    # launch kernels on the fake pointers, so none of them is made
    print("a device is visible: host calls not made", flush=True)
    sys.exit(3)
P = ctypes.c_void_p
FAKE = [P(0x7f0000100000 + (i << 24)) for i in range(16)]   # never dereferenced


def ok_err(st):
    assert st != 0, "an invalid call returned success"


lib.crbq_version()
for s in range(-8, 3):
    lib.crbq_status_string(s)
lib.crbq_device_ok()

# workspace queries across sizes
for T in (0, 1, 64, 4096, 262144, 1 << 22):
    for C in (1, 255, 256, 4096, 16384, 36864):
        lib.crbq_hessian_workspace_size(T, C)
p = _lib.params("crb")
for R in (1, 100, 4096, 16384):
    for C in (1, 128, 1000, 16384):
        lib.crbq_fasterquant_workspace_size(R, C, ctypes.byref(p))
        for n in range(0, 6):
            lib.crbq_fasterquant_batched_workspace_size(n, R, C, ctypes.byref(p))
for C in (1, 129, 4096, 16384):
    lib.crbq_hinv_workspace_size(C)
for T in (1, 17, 64, 256, 2048):
    lib.crbq_gemm_packed_workspace_size(4096, 16384, T)

# invalid parameters of the block loop
bad = []
for field, val in (("blocksize", 0), ("blocksize", 129), ("partition", 2), ("method", 9),
                   ("metric", 7), ("up_lim", 1), ("up_lim", 65), ("refine_iters", -1),
                   ("refine_iters", 65)):
    q = _lib.params("crb")
    setattr(q, field, val)
    bad.append(q)
q = _lib.params("crb")
q.orders[1] = 0
bad.append(q)
for q in bad:
    ok_err(lib.crbq_fasterquant(FAKE[0], 4096, 4096, 4096, FAKE[1], 4096, ctypes.byref(q),
                                FAKE[2], None, 0, None, FAKE[3], 1 << 30, None))
ok_err(lib.crbq_fasterquant(None, 4096, 4096, 4096, FAKE[1], 4096, ctypes.byref(p), FAKE[2],
                            None, 0, None, FAKE[3], 1 << 30, None))
ok_err(lib.crbq_fasterquant(FAKE[0], 4096, 4096, 100, FAKE[1], 4096, ctypes.byref(p), FAKE[2],
                            None, 0, None, FAKE[3], 1 << 30, None))
ok_err(lib.crbq_fasterquant(FAKE[0], 4096, 4096, 4096, FAKE[1], 4096, None, FAKE[2],
                            None, 0, None, FAKE[3], 1 << 30, None))
ok_err(lib.crbq_fasterquant(FAKE[0], 4096, 4096, 4096, FAKE[1], 4096, ctypes.byref(p), FAKE[2],
                            None, 0, None, None, 0, None))              # no workspace
ok_err(lib.crbq_fasterquant_noalloc(FAKE[0], 200000, 4096, 4096, FAKE[1], 4096,
                                    ctypes.byref(p), FAKE[2], None, 0, None, None))

# the batched loop: host arrays of exactly nseg pointers
def arr(ptrs):
    return (P * len(ptrs))(*ptrs)


for n in (1, 2, 3, 4):
    W, U, L = FAKE[0:n], FAKE[4:4 + n], FAKE[8:8 + n]
    ws = lib.crbq_fasterquant_batched_workspace_size(n, 4096, 4096, ctypes.byref(p))
    # validation passes; the first HIP call fails without a device
    ok_err(lib.crbq_fasterquant_batched(n, arr(W), 4096, 4096, 4096, arr(U), 4096,
                                        ctypes.byref(p), arr(L), arr([None] * n), 0,
                                        arr([None] * n), FAKE[12], ws, None))
    ok_err(lib.crbq_fasterquant_batched(n, arr(W), 4096, 4096, 4096, arr(U), 4096,
                                        ctypes.byref(p), arr(L), arr(FAKE[12:12 + n]), 4096,
                                        arr(FAKE[8:8 + n]), FAKE[13], ws, None))
    if n > 1:   # the same weight or loss buffer twice
        ok_err(lib.crbq_fasterquant_batched(n, arr([W[0]] * n), 4096, 4096, 4096, arr(U), 4096,
                                            ctypes.byref(p), arr(L), None, 0, None, FAKE[12],
                                            ws, None))
        ok_err(lib.crbq_fasterquant_batched(n, arr(W), 4096, 4096, 4096, arr(U), 4096,
                                            ctypes.byref(p), arr([L[0]] * n), None, 0, None,
                                            FAKE[12], ws, None))
        mixed = [FAKE[12]] + [None] * (n - 1)               # masks for some sublayers only
        ok_err(lib.crbq_fasterquant_batched(n, arr(W), 4096, 4096, 4096, arr(U), 4096,
                                            ctypes.byref(p), arr(L), arr(mixed), 4096, None,
                                            FAKE[13], ws, None))
    ok_err(lib.crbq_fasterquant_batched(n, arr(W), 4096, 4096, 4096, arr(U), 4096,
                                        ctypes.byref(p), arr(L), None, 0, None, FAKE[12], 16,
                                        None))                            # workspace too small
for n in (0, 5, -1):
    ok_err(lib.crbq_fasterquant_batched(n, arr(FAKE[0:4]), 4096, 4096, 4096, arr(FAKE[4:8]),
                                        4096, ctypes.byref(p), arr(FAKE[8:12]), None, 0, None,
                                        FAKE[12], 1 << 30, None))
ok_err(lib.crbq_fasterquant_batched(2, None, 4096, 4096, 4096, arr(FAKE[4:6]), 4096,
                                    ctypes.byref(p), arr(FAKE[8:10]), None, 0, None, FAKE[12],
                                    1 << 30, None))

# block search, binarize, Hessian, factor, packed storage
ok_err(lib.crbq_block_search(None, 4096, 128, 4096, FAKE[1], 4096, 1, 50, None, 0, None,
                             FAKE[2], 1 << 30, None))
ok_err(lib.crbq_block_search(FAKE[0], 4096, 129, 4096, FAKE[1], 4096, 1, 50, None, 0, None,
                             FAKE[2], 1 << 30, None))
ok_err(lib.crbq_block_search(FAKE[0], 4096, 40, 4096, FAKE[1], 4096, 1, 50, None, 0, None,
                             FAKE[2], 1 << 30, None))
ok_err(lib.crbq_binarize(None, 16, 128, 128, FAKE[1], 128, 2, 1, 1e-5, 0.1, 1, FAKE[2], 128,
                         None))
ok_err(lib.crbq_binarize(FAKE[0], 16, 2048, 2048, FAKE[1], 2048, 2, 1, 1e-5, 0.1, 1, FAKE[2],
                         2048, None))
ok_err(lib.crbq_hessian_accum(None, 1, 64, 256, 256, FAKE[1], 256, None, 0, None))
ok_err(lib.crbq_hessian_accum(FAKE[0], 7, 64, 256, 256, FAKE[1], 256, None, 0, None))
ok_err(lib.crbq_hessian_accum(FAKE[0], 1, 64, 100, 256, FAKE[1], 256, None, 0, None))
ok_err(lib.crbq_hessian_finalize(None, 256, 256, 1.0, FAKE[1], 256, None))
ok_err(lib.crbq_gemv_packed(None, 4096, FAKE[1], FAKE[2], None, None, 0, 1, 4096, 16384,
                            FAKE[3], 16384, 1, FAKE[4], 4096, None))
ok_err(lib.crbq_gemv_packed(FAKE[0], 4096, FAKE[1], FAKE[2], None, None, 0, 1, 4096, 16384,
                            FAKE[3], 16384, 17, FAKE[4], 4096, None))
ok_err(lib.crbq_gemm_packed(FAKE[0], 4096, FAKE[1], FAKE[2], None, None, 0, 1, 4096, 16384,
                            FAKE[3], 16384, 256, FAKE[4], 4096, None, 0, None))
print("host calls done", flush=True)
