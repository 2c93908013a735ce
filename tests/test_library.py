"""CPU checks of the built libraries: every function include/*.h declares is exported by its library, the libraries
load without a GPU, and the device library reports a missing device as an error instead of falling back."""
import ctypes as C
import os
import re

import pytest

import p2gemm as P

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADERS = {
    "p2hip.h": P.HIP_SO,
    "p2_blas.h": P.BLAS_SO,
    "p2gen.h": P.GEN_SO,
}


def _declared(header):
    text = open(os.path.join(ROOT, "include", header)).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    names = set(re.findall(r"\b(p2[a-z0-9_]*)\s*\(", text))
    return sorted(n for n in names if not n.isupper())


@pytest.mark.parametrize("header", sorted(HEADERS))
def test_header_symbols_exported(header):
    lib = C.CDLL(HEADERS[header])
    names = _declared(header)
    assert names, header
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, f"{os.path.basename(HEADERS[header])} lacks {missing}"


def test_blas_drop_in_exports_the_reference_api():
    """The reference's blas.h (blas.h:25-79) declares exactly these functions."""
    ref_api = ["p2_sgemm", "p2_sgemm_st", "p2_fv_pack_codes", "p2_sgemm_q8b", "p2_sgemm_fvb", "p2_gemm_mode",
               "p2_gemm_exact", "p2_quant_prepare", "p2_quant_row", "p2_sgemm_fvb_q8a", "p2_sgemm_q8b_q8a"]
    lib = C.CDLL(P.BLAS_SO)
    assert all(hasattr(lib, n) for n in ref_api)


def test_no_device_is_an_error_not_a_fallback():
    if os.path.exists("/dev/kfd"):
        pytest.skip("a GPU is present")
    rc = P.hip().p2h_init()
    assert rc == -2, rc
    assert "device" in P.last_error()


def test_q_tile_layout_matches_the_documented_index():
    """The tiled activation layout p2h_quant_rows documents: byte (m, k) at
    ((m/16)·(ldq/64) + k/64)·1024 + ((k%64)/16·16 + m%16)·16 + k%16; pads are zero; q_untile inverts q_tile."""
    import numpy as np
    rng = np.random.default_rng(5)
    for M, K, ldq in [(1, 4, 128), (17, 130, 256), (40, 256, 384)]:
        q = rng.integers(-127, 128, (M, K), dtype=np.int8)
        t = P.q_tile(q, ldq)
        Mp = (M + 15) // 16 * 16
        assert t.size == Mp * ldq
        expect = np.zeros(Mp * ldq, np.int8)
        for m in range(M):
            for k in range(K):
                idx = ((m // 16) * (ldq // 64) + k // 64) * 1024 + ((k % 64) // 16 * 16 + m % 16) * 16 + k % 16
                expect[idx] = q[m, k]
        assert np.array_equal(t, expect)
        back = P.q_untile(t, M, ldq)
        assert np.array_equal(back[:M, :K], q) and not back[M:].any() and not back[:, K:].any()
