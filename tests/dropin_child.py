"""Child process for tests/test_gpu_dropin.py: drives libphonon2_gemm.so – the reference's blas.h API – through
ctypes exactly as the reference's callers do (tensor_ops.c:30-63), in the mode P2_GEMM / P2_EXACT select, and
checks every result against the oracle. Exits 0 when all checks pass; prints what failed otherwise.

    P2_GEMM=int8w python tests/dropin_child.py
"""
import ctypes as C
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, HERE)
sys.path.insert(0, os.path.join(os.path.dirname(HERE), "phonon-2-c_amd"))

import _oracle as O  # noqa: E402
import p2gemm as P  # noqa: E402


class FiveValueB(C.Structure):
    _fields_ = [("signs", C.c_void_p), ("flags", C.c_void_p), ("lo", C.c_void_p), ("hi", C.c_void_p),
                ("codes", C.c_void_p)]


class QuantA(C.Structure):
    _fields_ = [("q", C.c_void_p), ("scales", C.c_void_p), ("M", C.c_int), ("K", C.c_int)]


def main():
    L = C.CDLL(P.BLAS_SO)
    vp, i, f = C.c_void_p, C.c_int, C.c_float
    L.p2_sgemm_fvb.argtypes = [i, i, i, f, vp, i, C.POINTER(FiveValueB), f, vp, i]
    L.p2_sgemm_fvb_q8a.argtypes = [i, i, i, f, C.POINTER(QuantA), C.POINTER(FiveValueB), f, vp, i]
    L.p2_quant_prepare.argtypes = [C.POINTER(QuantA), i, i]
    L.p2_quant_prepare.restype = i
    L.p2_quant_row.argtypes = [C.POINTER(QuantA), i, vp]
    L.p2_fv_pack_codes.argtypes = [C.POINTER(FiveValueB), i, i]
    L.p2_fv_pack_codes.restype = vp
    L.p2_gemm_mode.restype = C.c_char_p
    L.p2_gemm_exact.restype = i
    L.p2_sgemm_q8b.argtypes = [i, i, i, f, vp, i, vp, vp, i, f, vp, i]
    L.p2_sgemm_q8b_q8a.argtypes = [i, i, i, f, C.POINTER(QuantA), vp, vp, i, f, vp, i]
    L.p2_sgemm.argtypes = [i, i, i, i, i, f, vp, i, vp, i, f, vp, i]
    libc = C.CDLL("libc.so.6")
    libc.free.argtypes = [vp]

    mode_env = O.mode_from_env(os.environ.get("P2_GEMM"), os.environ.get("P2_EXACT"))
    mode_name = {O.INT8: "int8", O.EXACT: "exact", O.INT8W: "int8w"}[mode_env]
    failures = []

    def expect(cond, what):
        if not cond:
            failures.append(what)

    expect(L.p2_gemm_exact() == (mode_env == O.EXACT), "p2_gemm_exact")
    # blas.c:1060-1064
    names = {O.INT8: "int8 dot products, exact weights", O.INT8W: "int8 dot products, int8 weights",
             O.EXACT: "fp32 expansion (exact)"}
    expect(L.p2_gemm_mode().decode() == names[mode_env], "p2_gemm_mode string")

    chain = os.environ.get("P2H_EXACT_CHAIN", "0") not in ("", "0")

    def same(out, ref, K):
        """Bit-exact, except the five-value exact route (exact mode, or K % 4 != 0 in any mode, blas.c:1490-1493) on
        the matrix cores: within 1e-4 of the reference's."""
        if (mode_env == O.EXACT or K % 4 != 0) and not chain:
            rms = np.sqrt(np.mean(ref.astype(np.float64) ** 2, axis=1, keepdims=True))
            return bool(np.all(np.abs(out.astype(np.float64) - ref) <= 1e-4 * np.maximum(np.abs(ref), rms)))
        return np.array_equal(out.view(np.uint32), ref.view(np.uint32))

    seed = 7
    for (M, K, N, alpha, beta) in [(375, 1024, 1024, 1.0, 0.0), (38, 4096, 1024, 0.5, 1.0), (38, 1024, 1024, 1.0, 0.3),
                                   (5, 100, 48, 1.0, 0.0), (13, 6, 16, 1.0, 1.0)]:
        signs, flags, lo, hi = P.gen_fv_weight(seed, K * 7 + N, K, N)
        A = P.gen_activations(seed, M + K, M, K)
        C0 = P.gen_activations(seed, M + N, M, N)
        b = FiveValueB(signs.ctypes.data, flags.ctypes.data, lo.ctypes.data, hi.ctypes.data, None)
        out = C0.copy()
        L.p2_sgemm_fvb(M, N, K, alpha, A.ctypes.data, K, C.byref(b), beta, out.ctypes.data, N)
        ref = O.sgemm_fvb(mode_env, A, signs, flags, lo, hi, N, alpha=alpha, beta=beta, C0=C0)
        expect(same(out, ref, K), f"p2_sgemm_fvb {M}x{K}x{N}")
        # second call on the same weight: served from the device cache
        out2 = C0.copy()
        L.p2_sgemm_fvb(M, N, K, alpha, A.ctypes.data, K, C.byref(b), beta, out2.ctypes.data, N)
        expect(same(out2, ref, K), f"p2_sgemm_fvb cached {M}x{K}x{N}")

        qa = QuantA()
        rc = L.p2_quant_prepare(C.byref(qa), M, K)
        expect(rc == (-1 if (mode_env == O.EXACT or K % 4) else 0), f"p2_quant_prepare rc {rc}")
        if rc == 0:
            for m in range(M):
                L.p2_quant_row(C.byref(qa), m, A[m].ctypes.data)
            out3 = C0.copy()
            L.p2_sgemm_fvb_q8a(M, N, K, alpha, C.byref(qa), C.byref(b), beta, out3.ctypes.data, N)
            expect(np.array_equal(out3.view(np.uint32), ref.view(np.uint32)), f"p2_sgemm_fvb_q8a {M}x{K}x{N}")

    # strided A and C (lda > K, ldc > N)
    M, K, N = 9, 256, 32
    signs, flags, lo, hi = P.gen_fv_weight(seed, 99, K, N)
    A = P.gen_activations(seed, 98, M, K + 3)
    C0 = P.gen_activations(seed, 97, M, N + 5)
    b = FiveValueB(signs.ctypes.data, flags.ctypes.data, lo.ctypes.data, hi.ctypes.data, None)
    out = C0.copy()
    L.p2_sgemm_fvb(M, N, K, 1.5, A.ctypes.data, K + 3, C.byref(b), 1.0, out.ctypes.data, N + 5)
    ref = O.sgemm_fvb(mode_env, A, signs, flags, lo, hi, N, alpha=1.5, beta=1.0, C0=C0, K=K)
    expect(same(out, ref, K), "p2_sgemm_fvb strided")

    # the pre-packed codes
    K, N = 64, 32
    signs, flags, lo, hi = P.gen_fv_weight(seed, 55, K, N)
    b = FiveValueB(signs.ctypes.data, flags.ctypes.data, lo.ctypes.data, hi.ctypes.data, None)
    ptr = L.p2_fv_pack_codes(C.byref(b), K, N)
    expect(bool(ptr), "p2_fv_pack_codes returned NULL")
    if ptr:
        got = np.ctypeslib.as_array(C.cast(ptr, C.POINTER(C.c_int8)), shape=(K * N,)).copy()
        libc.free(ptr)
        expect(np.array_equal(got, O.fv_pack_codes(signs, flags, lo, hi, K, N)), "p2_fv_pack_codes")
    expect(not L.p2_fv_pack_codes(C.byref(b), 62, N), "p2_fv_pack_codes K % 4")

    # int8 tables
    M, K, N = 40, 1024, 64
    B8, sc = P.gen_i8_weight(seed, 61, K, N)
    A = P.gen_activations(seed, 62, M, K)
    out = np.zeros((M, N), np.float32)
    L.p2_sgemm_q8b(M, N, K, 1.0, A.ctypes.data, K, B8.ctypes.data, sc.ctypes.data, N, 0.0, out.ctypes.data, N)
    ref = O.sgemm_q8b(mode_env, A, B8, sc, N)
    expect(np.array_equal(out.view(np.uint32), ref.view(np.uint32)), "p2_sgemm_q8b")

    # fp32 GEMM (not a five-value path: within fp32 tolerance)
    rng = np.random.default_rng(3)
    A = rng.standard_normal((33, 70)).astype(np.float32)
    B = rng.standard_normal((70, 40)).astype(np.float32)
    out = np.ones((33, 40), np.float32)
    L.p2_sgemm(111, 111, 33, 40, 70, 1.0, A.ctypes.data, 70, B.ctypes.data, 40, 1.0, out.ctypes.data, 40)
    expect(np.allclose(out, A.astype(np.float64) @ B + 1.0, rtol=1e-4, atol=1e-4), "p2_sgemm")

    # K == 0 (blas.c:1436, 1488-1496): the int8 routes pre-scale C for beta outside {0, 1} and run no K block, so C
    # keeps its values otherwise (beta 0 included); the exact route scales C by beta (0 stores zeros)
    M, N = 7, 32
    z8, lo0, hi0 = np.zeros(16, np.uint8), np.full(N, 0.01, np.float32), np.full(N, 0.03, np.float32)
    b0 = FiveValueB(z8.ctypes.data, z8.ctypes.data, lo0.ctypes.data, hi0.ctypes.data, None)
    C0 = P.gen_activations(seed, 71, M, N)
    A0 = np.zeros((M, 4), np.float32)
    for beta in (0.0, 1.0, 0.5):
        out = C0.copy()
        L.p2_sgemm_fvb(M, N, 0, 1.0, A0.ctypes.data, 4, C.byref(b0), beta, out.ctypes.data, N)
        if mode_env == O.EXACT:
            want = (C0 * np.float32(beta)).astype(np.float32) if beta != 0.0 else np.zeros_like(C0)
        else:
            want = C0 if beta in (0.0, 1.0) else (C0 * np.float32(beta)).astype(np.float32)
        expect(np.array_equal(out.view(np.uint32), want.view(np.uint32)), f"p2_sgemm_fvb K=0 beta={beta}")

    # many threads on shared weights while the cache is cleared under them (phonon2.h:277-280: concurrent
    # transcriptions share one engine's weights): every result must still equal the oracle's
    import threading
    L.p2_gpu_weight_cache_clear.argtypes = []
    L.p2_gpu_weight_cache_clear.restype = None
    shared = []
    for t in range(3):
        M, K, N = (64, 1024, 256) if t < 2 else (16, 4096, 128)
        signs, flags, lo, hi = P.gen_fv_weight(seed, 300 + t, K, N)
        A = P.gen_activations(seed, 310 + t, M, K)
        ref = O.sgemm_fvb(mode_env, A, signs, flags, lo, hi, N)
        shared.append((M, K, N, signs, flags, lo, hi, A, ref,
                       FiveValueB(signs.ctypes.data, flags.ctypes.data, lo.ctypes.data, hi.ctypes.data, None)))
    bad = []
    stop = threading.Event()

    def worker(tid):
        for it in range(12):
            M, K, N, signs, flags, lo, hi, A, ref, fb = shared[(tid + it) % len(shared)]
            out = np.zeros((M, N), np.float32)
            if it % 2 == 0 or mode_env == O.EXACT:
                L.p2_sgemm_fvb(M, N, K, 1.0, A.ctypes.data, K, C.byref(fb), 0.0, out.ctypes.data, N)
            else:
                qa = QuantA()
                if L.p2_quant_prepare(C.byref(qa), M, K) != 0:
                    bad.append(f"thread {tid} prepare")
                    continue
                for m in range(M):
                    L.p2_quant_row(C.byref(qa), m, A[m].ctypes.data)
                L.p2_sgemm_fvb_q8a(M, N, K, 1.0, C.byref(qa), C.byref(fb), 0.0, out.ctypes.data, N)
            if not same(out, ref, K):
                bad.append(f"thread {tid} call {it}")

    def clearer():
        while not stop.is_set():
            L.p2_gpu_weight_cache_clear()
            stop.wait(0.002)

    cl = threading.Thread(target=clearer)
    cl.start()
    ths = [threading.Thread(target=worker, args=(t,)) for t in range(8)]
    for th in ths:
        th.start()
    for th in ths:
        th.join()
    stop.set()
    cl.join()
    expect(not bad, "concurrent calls: " + ", ".join(bad[:5]))

    if failures:
        print(f"mode {mode_name}: FAILED: " + "; ".join(failures))
        return 1
    print(f"mode {mode_name}: all drop-in checks passed")
    return 0


if __name__ == "__main__":
    sys.exit(main())
