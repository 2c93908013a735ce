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


def test_layer_norm_entries_reject_overlapping_rows():
    """p2h_layer_norm_rows and p2h_layer_norm2_quant_rows check their arguments before touching a device: Y may be X
    itself with the same pitch, but rows of Y that overlap other rows of X are refused (a wave's stores would land
    in rows another wave has not read), as is in place with another pitch. The pointers are never dereferenced."""
    if os.path.exists("/dev/kfd"):
        pytest.skip("fake device pointers: run where no GPU can be reached")
    lib = P.hip()
    vp = C.c_void_p
    base = 0x7f0000000000   # a fake device address: every call here must fail in its argument checks
    M, D = 8, 1024
    X = base
    g1, b1, g2, b2, Q, S = (base + 0x1000000 * k for k in range(1, 7))

    def ln2(Y, ldx, ldy, ldq=1024):
        return lib.p2h_layer_norm2_quant_rows(M, D, vp(X), ldx, vp(g1), vp(b1), vp(Y), ldy, vp(g2), vp(b2), vp(Q),
                                              ldq, vp(S), None)

    def ln(Y, ldx, ldy):
        return lib.p2h_layer_norm_rows(M, D, vp(X), ldx, vp(g1), vp(b1), vp(Y), ldy, None)

    for call in (ln2, ln):
        name = "p2h_layer_norm2_quant_rows" if call is ln2 else "p2h_layer_norm_rows"
        rc = call(X + 4 * D * 3, D, D)          # Y starts at row 3 of X: overlaps rows 3..7
        assert rc == -1 and "overlap" in P.last_error() and name in P.last_error(), (rc, P.last_error())
        rc = call(X - 4 * D * 2, D, D)          # Y ends inside X's first rows
        assert rc == -1 and "overlap" in P.last_error(), (rc, P.last_error())
        rc = call(X, D, D + 16)                 # in place with another pitch
        assert rc == -1 and "in place" in P.last_error(), (rc, P.last_error())
    # the rows right after X do not overlap: the call passes those checks and stops at the next one (an invalid ldq)
    rc = ln2(X + 4 * D * M, D, D, ldq=1000)
    assert rc == -1 and "ldq" in P.last_error(), (rc, P.last_error())
