"""The blas.h drop-in (libphonon2_gemm.so) in each mode, one child process per mode because the mode is latched
once per process (blas.c:1049-1053)."""
import os
import subprocess
import sys

import pytest

pytestmark = pytest.mark.gpu

CHILD = os.path.join(os.path.dirname(__file__), "dropin_child.py")


@pytest.mark.parametrize("env", [{}, {"P2_GEMM": "int8"}, {"P2_GEMM": "exact"}, {"P2_GEMM": "int8", "P2_EXACT": "1"},
                                 {"P2_GEMM": "exact", "P2H_EXACT_CHAIN": "1"}, {"P2_GPU_WEIGHT_CACHE": "0"}])
def test_dropin_mode(env):
    e = dict(os.environ)
    for k in ("P2_GEMM", "P2_EXACT", "P2H_EXACT_CHAIN", "P2_GPU_WEIGHT_CACHE"):
        e.pop(k, None)
    e.update(env)
    print(f"drop-in child with {env}", flush=True)
    r = subprocess.run([sys.executable, CHILD], env=e, capture_output=True, text=True, timeout=300)
    assert r.returncode == 0, r.stdout + r.stderr
