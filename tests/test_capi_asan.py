"""The C ABI's host side under AddressSanitizer: the library rebuilt with
ASan on its host code (crb_amd.build.build_host_asan; the gfx950 code is the
same) and tests/asan_host_calls.py run against it in a process that preloads
the ASan runtime.  Host-only: it needs no GPU and is skipped where one is
visible (its calls use fake device pointers that pass validation)."""
import os
import shutil
import subprocess
import sys

import pytest
import torch

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def test_c_abi_host_side_under_asan(tmp_path):
    if torch.cuda.device_count() > 0:
        pytest.skip("host-only check with fake device pointers; a GPU is visible")
    from crb_amd.build import HIPCC, asan_runtime, build_host_asan
    rt = asan_runtime()
    if rt is None or shutil.which(HIPCC) is None and not os.path.exists(HIPCC):
        pytest.skip("no hipcc or no ASan runtime in the toolchain")
    lib = build_host_asan(str(tmp_path))
    pre = os.environ.get("LD_PRELOAD", "")
    env = dict(os.environ, LD_PRELOAD=rt + (":" + pre if pre else ""),
               ASAN_OPTIONS="detect_leaks=0:abort_on_error=1")
    r = subprocess.run([sys.executable, os.path.join(ROOT, "tests", "asan_host_calls.py"), lib,
                        ROOT], env=env, capture_output=True, text=True, timeout=600)
    assert r.returncode == 0, (r.stdout[-2000:], r.stderr[-6000:])
    assert "AddressSanitizer" not in r.stderr, r.stderr[-6000:]
    assert "host calls done" in r.stdout
