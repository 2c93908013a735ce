"""Write the golden vectors of the reference's exact five-value GEMM (and its int8-table GEMM).

Runs the reference's own p2_sgemm_fvb / p2_sgemm_q8b, built from its C sources by `make -C oracle ref`
(oracle/_ref/libp2ref.so; on x86 the exact fp32 AVX2 route, blas.c:1043-1045), on small seeded inputs, and stores
inputs and outputs in tests/golden/ref_exact_gemm.npz with a SHA-256 of every array in ref_exact_gemm.sha256.json.

    python tests/golden/make_golden.py

The int8 / int8w routes cannot run here (blas.c:1021-1023: AArch64 with the dot-product extension only), so no
golden vectors exist for them; their oracle functions are pinned by the invariants in tests/test_oracle_int8.py.
"""
import hashlib
import json
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(HERE))
os.environ.setdefault("P2_THREADS", "4")
os.environ["P2_GEMM"] = "exact"

import _oracle as O  # noqa: E402


def fp16(x):
    return np.asarray(x, np.float32).astype(np.float16).astype(np.float32)


def fv_inputs(rng, K, N, code3=False, nonfp16=False):
    u = rng.random((K, N))
    sign = np.where(u < 0.4, 0, np.where(rng.random((K, N)) < 0.5, -1, 1)).astype(np.int8)
    is_hi = ((sign != 0) & (rng.random((K, N)) < 1 / 3)).astype(np.uint8)
    lo = rng.uniform(0.005, 0.02, N)
    hi = lo * rng.uniform(2, 4, N)
    if nonfp16:
        lo, hi = lo.astype(np.float32), hi.astype(np.float32)
    else:
        lo, hi = fp16(lo), fp16(hi)
    signs, flags = O.pack_planes(sign, is_hi)
    if code3:   # plant the never-written 2-bit code 3 (blas.h:40) at a few places
        idx = rng.choice(signs.size, size=max(4, signs.size // 16), replace=False)
        for i in idx:
            signs.reshape(-1)[i] |= np.uint8(3 << (2 * int(rng.integers(0, 4))))
    return signs, flags, lo.astype(np.float32), hi.astype(np.float32)


CASES = [
    # name, M, K, N, alpha, beta, lda_pad, ldc_pad, options
    ("fvb_m37_k1024_n64", 37, 1024, 64, 1.0, 0.0, 0, 0, {}),
    ("fvb_m5_k100_n32_beta1", 5, 100, 32, 0.5, 1.0, 0, 0, {}),
    ("fvb_m9_k300_n48_strided", 9, 300, 48, -1.25, 0.3, 3, 5, {}),
    ("fvb_m3_k64_n16_alpha0", 3, 64, 16, 0.0, 0.5, 0, 0, {}),
    ("fvb_m7_k256_n32_nonfp16", 7, 256, 32, 1.0, 0.0, 0, 0, {"nonfp16": True}),
    ("fvb_m6_k64_n32_code3", 6, 64, 32, 1.0, 0.0, 0, 0, {"code3": True}),
    ("fvb_m2_k4096_n16", 2, 4096, 16, 0.75, 1.0, 0, 0, {}),
    ("fvb_m1_k513_n16", 1, 513, 16, 1.0, 0.0, 0, 0, {}),
]

Q8B_CASES = [
    ("q8b_m11_k96_n32", 11, 96, 32, 0.75, 0.0),
    ("q8b_m4_k1030_n48_beta", 4, 1030, 48, 1.0, 1.0),
]


def main():
    if not O.ref_available():
        sys.exit("oracle/_ref/libp2ref.so missing: run `make -C oracle ref` where the reference tree is present")
    mode = O.ref().p2_gemm_mode().decode()
    assert "exact" in mode, mode
    out = {}
    rng = np.random.default_rng(20261201)
    for name, M, K, N, alpha, beta, lpad, cpad, opt in CASES:
        A = rng.standard_normal((M, K + lpad)).astype(np.float32)
        A[rng.random(A.shape) < 0.001] *= 20
        signs, flags, lo, hi = fv_inputs(rng, K, N, **opt)
        C0 = rng.standard_normal((M, N + cpad)).astype(np.float32)
        C = O.ref_sgemm_fvb(A, signs, flags, lo, hi, N, alpha, beta, C0, K=K)
        for k, v in dict(A=A, signs=signs, flags=flags, lo=lo, hi=hi, C0=C0, C=C,
                         dims=np.array([M, K, N], np.int32), ab=np.array([alpha, beta], np.float32)).items():
            out[f"{name}/{k}"] = v
    for name, M, K, N, alpha, beta in Q8B_CASES:
        A = rng.standard_normal((M, K)).astype(np.float32)
        B = rng.integers(-127, 128, (K, N)).astype(np.int8)
        scales = fp16(rng.uniform(0.0005, 0.002, N))
        C0 = rng.standard_normal((M, N)).astype(np.float32)
        C = O.ref_sgemm_q8b(A, B, scales, N, alpha, beta, C0)
        for k, v in dict(A=A, B=B, scales=scales, C0=C0, C=C, dims=np.array([M, K, N], np.int32),
                         ab=np.array([alpha, beta], np.float32)).items():
            out[f"{name}/{k}"] = v
    path = os.path.join(HERE, "ref_exact_gemm.npz")
    np.savez_compressed(path, **out)
    sums = {k: hashlib.sha256(np.ascontiguousarray(v).tobytes()).hexdigest() for k, v in sorted(out.items())}
    with open(os.path.join(HERE, "ref_exact_gemm.sha256.json"), "w") as f:
        json.dump({"source": "reference p2_sgemm_fvb / p2_sgemm_q8b, exact mode, " + mode, "arrays": sums}, f,
                  indent=1)
    print(f"wrote {path}: {len(out)} arrays, {os.path.getsize(path)} bytes")


if __name__ == "__main__":
    main()
