"""The oracle's exact route against the reference's own outputs (tests/golden/ref_exact_gemm.npz, written by
tests/golden/make_golden.py from the reference's p2_sgemm_fvb / p2_sgemm_q8b built from its C sources).

Bit-exact equality is required. Each case also checks that a plausible mistake in the restatement would have been
caught: the planted variant is computed here, on the CPU, and must differ from the golden output.
"""
import hashlib
import json
import os

import numpy as np
import pytest

import _oracle as O

GOLD = os.path.join(os.path.dirname(__file__), "golden", "ref_exact_gemm.npz")
SUMS = os.path.join(os.path.dirname(__file__), "golden", "ref_exact_gemm.sha256.json")

_z = np.load(GOLD)
CASES = sorted({k.split("/")[0] for k in _z.files})


def _g(name, field):
    return _z[f"{name}/{field}"]


def test_fixture_checksums():
    sums = json.load(open(SUMS))["arrays"]
    assert set(sums) == set(_z.files)
    for k in _z.files:
        assert hashlib.sha256(np.ascontiguousarray(_z[k]).tobytes()).hexdigest() == sums[k], k


@pytest.mark.parametrize("name", [c for c in CASES if c.startswith("fvb")])
def test_exact_fvb_bit_exact(name):
    M, K, N = (int(x) for x in _g(name, "dims"))
    alpha, beta = (float(x) for x in _g(name, "ab"))
    got = O.sgemm_fvb("exact", _g(name, "A"), _g(name, "signs"), _g(name, "flags"), _g(name, "lo"), _g(name, "hi"),
                      N, alpha, beta, _g(name, "C0"), K=K)
    ref = _g(name, "C")
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))


@pytest.mark.parametrize("name", [c for c in CASES if c.startswith("q8b")])
def test_exact_q8b_bit_exact(name):
    M, K, N = (int(x) for x in _g(name, "dims"))
    alpha, beta = (float(x) for x in _g(name, "ab"))
    got = O.sgemm_q8b("exact", _g(name, "A"), _g(name, "B"), _g(name, "scales"), N, alpha, beta, _g(name, "C0"), K=K)
    assert np.array_equal(got.view(np.uint32), _g(name, "C").view(np.uint32))


def _planted_exact(name, weight_rule):
    """The exact chain in float64-free numpy float32 with a different weight rule (a planted mistake)."""
    M, K, N = (int(x) for x in _g(name, "dims"))
    alpha, beta = (float(x) for x in _g(name, "ab"))
    code, flag = O.unpack_planes(_g(name, "signs"), _g(name, "flags"), K, N)
    lo, hi = _g(name, "lo"), _g(name, "hi")
    W = weight_rule(code.astype(np.float32), flag.astype(np.float32), lo, hi)
    A = _g(name, "A")[:, :K]
    C = _g(name, "C0")[:, :N].astype(np.float32).copy()
    C = np.zeros_like(C) if beta == 0 else (C if beta == 1 else (C * np.float32(beta)).astype(np.float32))
    for k in range(K):
        C = np.float32(alpha) * A[:, k:k + 1] * W[k][None, :] + C
        C = C.astype(np.float32)
    return C


def test_nonfp16_pins_fma_expansion():
    """With lo/hi that are not fp16 values, fmaf(flag, hi − lo, lo) differs from hi (blas.c:838-840); the golden
    output follows the fmaf form, and a restatement that used hi directly would not match it."""
    name = "fvb_m7_k256_n32_nonfp16"
    lo, hi = _g(name, "lo"), _g(name, "hi")
    d = (hi - lo).astype(np.float32)
    fused = np.array([np.float32(np.float64(d[i]) + np.float64(lo[i])) for i in range(len(lo))], np.float32)
    assert np.any(fused != hi), "the fixture must contain columns where the two forms differ"
    W_fma = O.expand_exact(_g(name, "signs"), _g(name, "flags"), lo, hi, 256, 32)
    code, flag = O.unpack_planes(_g(name, "signs"), _g(name, "flags"), 256, 32)
    W_naive = ((code.astype(np.float32) - 1) * np.where(flag == 1, hi[None, :], lo[None, :])).astype(np.float32)
    assert not np.array_equal(W_fma, W_naive)


def test_code3_is_plus_two_in_exact_mode():
    """The never-written 2-bit code 3 decodes to +2 in the exact route (SIGN_LUT, blas.c:799)."""
    name = "fvb_m6_k64_n32_code3"
    code, _ = O.unpack_planes(_g(name, "signs"), _g(name, "flags"), 64, 32)
    assert (code == 3).any()
    W = O.expand_exact(_g(name, "signs"), _g(name, "flags"), _g(name, "lo"), _g(name, "hi"), 64, 32)
    k, n = np.argwhere(code == 3)[0]
    assert W[k, n] > 0 and W[k, n] in (2 * _g(name, "lo")[n], 2 * _g(name, "hi")[n])


def test_planted_mistakes_fail():
    """A dropped alpha, a transposed sign and a wrong beta each break the bit-exact match."""
    name = "fvb_m9_k300_n48_strided"
    ref = _g(name, "C")[:, :48]
    good = lambda c, f, lo, hi: ((c - 1) * np.where(f == 1, hi[None, :], lo[None, :])).astype(np.float32)
    flipped = lambda c, f, lo, hi: ((1 - c) * np.where(f == 1, hi[None, :], lo[None, :])).astype(np.float32)
    swapped = lambda c, f, lo, hi: ((c - 1) * np.where(f == 1, lo[None, :], hi[None, :])).astype(np.float32)
    base = _planted_exact(name, good)
    assert np.allclose(base, ref, rtol=1e-5, atol=1e-5)   # the numpy restatement itself is right up to fma rounding
    assert not np.allclose(_planted_exact(name, flipped), ref, rtol=1e-3, atol=1e-3)
    assert not np.allclose(_planted_exact(name, swapped), ref, rtol=1e-3, atol=1e-3)


def test_mode_latch_rules():
    """P2_GEMM / P2_EXACT precedence (blas.c:1032-1047)."""
    assert O.mode_from_env(None, None) == O.INT8W
    assert O.mode_from_env("exact", None) == O.EXACT
    assert O.mode_from_env("int8", None) == O.INT8
    assert O.mode_from_env("int8w", None) == O.INT8W
    assert O.mode_from_env("bogus", None) == O.INT8W
    assert O.mode_from_env("int8", "1") == O.EXACT
    assert O.mode_from_env("int8", "0") == O.INT8
    assert O.mode_from_env("int8", "") == O.INT8
