"""The C ABI boundary on the CPU: libcrbq.so loads without a GPU, exports
every function include/crbq.h declares, the ctypes binding covers them all
with the declared arity, and the struct layouts seen from C (gcc on the
header) and from ctypes agree.  No compute call is made here."""
import ctypes
import os
import re
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "crbq.h")


def header_functions():
    txt = open(HEADER).read()
    txt = re.sub(r"/\*.*?\*/", "", txt, flags=re.S)
    out = {}
    for m in re.finditer(r"\b(?:int|size_t|const char\*)\s+(crbq_\w+)\s*\(([^)]*)\)\s*;", txt):
        args = [a for a in m.group(2).split(",") if a.strip() and a.strip() != "void"]
        out[m.group(1)] = len(args)
    return out


def test_header_parses():
    fns = header_functions()
    assert len(fns) >= 15
    assert "crbq_fasterquant" in fns and "crbq_hessian_accum" in fns


def test_library_exports_every_declared_symbol():
    from crb_amd import _lib
    lib = _lib.load()
    for name in header_functions():
        assert hasattr(lib, name), name


def test_ctypes_binding_matches_header_arity():
    from crb_amd import _lib
    fns = header_functions()
    assert set(_lib._SIGS) == set(fns)
    for name, nargs in fns.items():
        assert len(_lib._SIGS[name][1]) == nargs, name


def test_status_strings_without_gpu():
    from crb_amd import _lib
    lib = _lib.load()
    assert lib.crbq_version() >= 100
    for st in (0, -1, -2, -3, -4, -5, -6):
        assert lib.crbq_status_string(st) != b"unknown status"
    # a NULL argument is rejected before any device work
    assert lib.crbq_sgemm(0, 0, 1, 1, 1, 1.0, None, 1, None, 1, 0.0, None, 1, None) == -1


def test_syrk_timing_switch_without_gpu():
    """The timing switch and an empty collect make no device call."""
    from crb_amd import kernels
    kernels.syrk_timing(True)
    kernels.syrk_timing(False)
    assert kernels.syrk_timing_collect() == []
    from crb_amd import _lib
    n = ctypes.c_int32(7)
    assert _lib.load().crbq_syrk_timing_collect(None, None, 0, ctypes.byref(n)) == 0
    assert n.value == 0
    assert _lib.load().crbq_syrk_timing_collect(None, None, 4, ctypes.byref(n)) == -1


PROBE = r"""
#include <stdio.h>
#include <stddef.h>
#include "crbq.h"
int main(void) {
  printf("%zu %zu %zu %zu %zu %zu %zu %zu\n", sizeof(crbq_params), offsetof(crbq_params, orders),
         offsetof(crbq_params, lam), offsetof(crbq_params, corr_damp), sizeof(crbq_block_trace),
         offsetof(crbq_block_trace, pvals), offsetof(crbq_block_trace, errs_a),
         offsetof(crbq_block_trace, errs_c));
  return 0;
}
"""


def test_struct_layout_matches_c(tmp_path):
    from crb_amd import _lib
    src = tmp_path / "probe.c"
    exe = tmp_path / "probe"
    src.write_text(PROBE)
    r = subprocess.run(["gcc", "-std=c99", "-I", os.path.join(ROOT, "include"), str(src), "-o",
                        str(exe)], capture_output=True, text=True)
    if r.returncode != 0:
        pytest.skip("gcc unavailable: " + r.stderr[:200])
    vals = [int(v) for v in subprocess.run([str(exe)], capture_output=True, text=True,
                                           check=True).stdout.split()]
    P, T = _lib.CrbqParams, _lib.CrbqBlockTrace
    want = [ctypes.sizeof(P), P.orders.offset, P.lam.offset, P.corr_damp.offset, ctypes.sizeof(T),
            T.pvals.offset, T.errs_a.offset, T.errs_c.offset]
    assert vals == want


def test_product_path_has_no_oracle_dependency():
    """The package never imports the test-only oracle."""
    pkg = os.path.join(ROOT, "crb_amd")
    for dirpath, _, files in os.walk(pkg):
        for f in files:
            if f.endswith(".py"):
                txt = open(os.path.join(dirpath, f)).read()
                assert "oracle" not in re.findall(r"^\s*(?:from|import)\s+(\w+)", txt, flags=re.M), f
