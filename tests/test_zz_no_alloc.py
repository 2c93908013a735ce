"""p2h_fvb_gemm_noalloc, the entry point that allocates nothing (its workspace is the library's device scratch
array), against p2h_fvb_gemm with a workspace of its own: the same kernels, so the outputs must be equal bit for bit,
in every mode, on two calls in a row (the second with a smaller input, so it runs on what the first left in the
array). Called through the C ABI of libp2hip.so."""
import ctypes as C

import numpy as np
import pytest

import p2gemm as P

pytestmark = pytest.mark.gpu

SEED = 20261201
P2H_E_WORKSPACE = -4


@pytest.fixture(scope="module")
def lib():
    assert P.init().startswith("gfx950")
    L = P.hip()
    vp, i, f = C.c_void_p, C.c_int, C.c_float
    L.p2h_fvb_gemm_noalloc.argtypes = [i, i, i, i, f, vp, i, vp, f, vp, i, vp]
    L.p2h_fvb_gemm_noalloc.restype = i
    L.p2h_noalloc_scratch_bytes.argtypes = []
    L.p2h_noalloc_scratch_bytes.restype = C.c_size_t
    return L


def _case(M, K, N, tid):
    signs, flags, lo, hi = P.gen_fv_weight(SEED, tid, K, N)
    w = P.FvWeight(signs, flags, lo, hi, K, N)
    A = P.gen_activations(SEED, tid + 1, M, K)
    C0 = P.gen_activations(SEED, tid + 2, M, N)
    return w, P.to_device(A), C0


@pytest.mark.parametrize("mode", ["int8w", "int8", "exact"])
def test_noalloc_matches_workspace_entry(lib, mode):
    stream = P.Stream()
    m = P.MODES[mode]
    # the second call is smaller than the first: it must not depend on what the first left in the scratch array
    for M, K, N, alpha, beta, tid in ((375, 4096, 1024, 0.5, 1.0, 11), (38, 1024, 1024, 1.0, 0.0, 21)):
        print(f"noalloc {mode} M={M} K={K} N={N}", flush=True)
        w, dA, C0 = _case(M, K, N, tid)
        ws = P.Workspace(P.workspace_bytes(mode, M, N, K))
        assert P.workspace_bytes(mode, M, N, K) <= lib.p2h_noalloc_scratch_bytes()
        d_ref, d_got = P.to_device(C0), P.to_device(C0)
        P.fvb_gemm_dev(mode, M, N, K, alpha, dA.ptr, K, w, beta, d_ref.ptr, N, ws.ptr, ws.nbytes, stream.ptr)
        rc = lib.p2h_fvb_gemm_noalloc(m, M, N, K, alpha, dA.ptr, K, w.ptr, beta, d_got.ptr, N, stream.ptr)
        assert rc == 0, P.last_error()
        stream.sync()
        ref = d_ref.download((M, N), np.float32)
        got = d_got.download((M, N), np.float32)
        assert np.array_equal(got.view(np.uint32), ref.view(np.uint32)), f"{mode} {M}x{K}x{N}"


def test_noalloc_refuses_what_the_array_cannot_hold(lib):
    """A shape whose workspace exceeds the scratch array is refused on the host, before any launch; so is a NULL
    stream."""
    M, K, N = 20000, 4096, 1024
    assert P.workspace_bytes("int8w", M, N, K) > lib.p2h_noalloc_scratch_bytes()
    w, _, _ = _case(16, K, N, 31)
    stream = P.Stream()
    rc = lib.p2h_fvb_gemm_noalloc(P.INT8W, M, N, K, 1.0, None, K, w.ptr, 0.0, None, N, stream.ptr)
    assert rc == P2H_E_WORKSPACE and "scratch" in P.last_error()
    rc = lib.p2h_fvb_gemm_noalloc(P.INT8W, 16, N, K, 1.0, None, K, w.ptr, 0.0, None, N, None)
    assert rc != 0 and "stream" in P.last_error()
