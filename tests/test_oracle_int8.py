"""Pins for the oracle's int8 / int8w routes, which the reference cannot run on this host (blas.c:1021-1023).

Each check is something other than the restated formula: invariants the arithmetic must satisfy, exact integer
identities computed another way (int64 numpy), float64 evaluations, and constructed rows whose answer is known.
"""
import numpy as np
import pytest

import _oracle as O


def _rng(seed=5):
    return np.random.default_rng(seed)


def _fv(rng, K, N, p_zero=0.4, code3=False):
    u = rng.random((K, N))
    sign = np.where(u < p_zero, 0, np.where(rng.random((K, N)) < 0.5, -1, 1)).astype(np.int8)
    is_hi = ((sign != 0) & (rng.random((K, N)) < 1 / 3)).astype(np.uint8)
    lo = rng.uniform(0.005, 0.02, N).astype(np.float16).astype(np.float32)
    hi = (lo * rng.uniform(2, 4, N)).astype(np.float16).astype(np.float32)
    signs, flags = O.pack_planes(sign, is_hi)
    if code3:
        flat = signs.reshape(-1)
        for i in rng.choice(flat.size, size=max(2, flat.size // 10), replace=False):
            flat[i] |= np.uint8(3 << (2 * int(rng.integers(0, 4))))
    return signs, flags, lo, hi, sign, is_hi


def _np_decode(signs, flags, K, N):
    """An independent decoder: numpy bit operations on the planes (blas.h:40-41)."""
    s = signs.reshape(K, N // 4)
    code = np.stack([(s >> (2 * j)) & 3 for j in range(4)], axis=-1).reshape(K, N)
    flag = np.unpackbits(flags.reshape(K, N // 8), axis=1, bitorder="little")
    return code.astype(np.int16), flag.astype(np.int16)


# ── planes ──────────────────────────────────────────────────────────────────────────────────────────────────────

def test_pack_unpack_round_trip_and_numpy_decoder():
    rng = _rng()
    signs, flags, lo, hi, sign, is_hi = _fv(rng, 24, 48)
    code, flag = O.unpack_planes(signs, flags, 24, 48)
    assert np.array_equal(code.astype(np.int16) - 1, sign)
    assert np.array_equal(flag, is_hi)
    c2, f2 = _np_decode(signs, flags, 24, 48)
    assert np.array_equal(c2, code) and np.array_equal(f2, flag)


def test_pack_brute_force_tiny():
    """Every single-weight plane of a 1×16 weight packs to the bit the layout names."""
    for n in range(16):
        for s in (-1, 0, 1):
            for h in (0, 1):
                sign = np.zeros((1, 16), np.int8)
                is_hi = np.zeros((1, 16), np.uint8)
                sign[0, n], is_hi[0, n] = s, h
                signs, flags = O.pack_planes(sign, is_hi)
                expect_s = np.full(4, 0x55, np.uint8)
                expect_s[n // 4] = (0x55 & ~(3 << (2 * (n % 4)))) | ((s + 1) << (2 * (n % 4)))
                assert np.array_equal(signs.reshape(-1), expect_s)
                expect_f = np.zeros(2, np.uint8)
                expect_f[n // 8] = h << (n % 8)
                assert np.array_equal(flags.reshape(-1), expect_f)


# ── quantisation ────────────────────────────────────────────────────────────────────────────────────────────────

def test_quant_invariants():
    rng = _rng(1)
    A = rng.standard_normal((64, 1024)).astype(np.float32)
    A[rng.random(A.shape) < 0.001] *= 20
    q, sc = O.quant_rows(A)
    assert q.min() >= -127 and q.max() <= 127
    amax = np.abs(A).max(axis=1)
    assert np.allclose(sc, amax / 127, rtol=1e-6)
    err = np.abs(q.astype(np.float64) * sc[:, None] - A)
    assert (err <= sc[:, None] * (0.5 + 1e-5)).all()
    rows = np.arange(64)
    assert (np.abs(q[rows, np.abs(A).argmax(axis=1)]) == 127).all()


def test_quant_zero_row_and_power_of_two_scaling():
    rng = _rng(2)
    A = rng.standard_normal((3, 256)).astype(np.float32)
    A[1] = 0
    q, sc = O.quant_rows(A)
    assert sc[1] == 1.0 and (q[1] == 0).all()
    for j in (-3, 5):
        q2, sc2 = O.quant_rows(A * np.float32(2.0 ** j))
        assert np.array_equal(q2, q)
        assert sc2[0] == sc[0] * np.float32(2.0 ** j) and sc2[2] == sc[2] * np.float32(2.0 ** j)


def test_quant_ties_to_even():
    row = np.zeros(32, np.float32)
    row[0] = 127.0   # amax 127 → scale 1, inv 1
    row[1:7] = [2.5, 3.5, -2.5, -3.5, 0.5, -0.5]
    q, sc = O.quant_rows(row[None, :])
    assert sc[0] == 1.0
    assert list(q[0, 1:7]) == [2, 4, -2, -4, 0, 0]


def test_quant_tail_divides():
    """The K % 16 tail rounds x / scale (blas.c:1140) while the body rounds x · (1/scale): find a value where the
    two differ and check each position follows its own rule."""
    found = None
    for amax in np.arange(50, 150, 0.37, dtype=np.float32):
        scale = np.float32(amax / np.float32(127))
        inv = np.float32(np.float32(1) / scale)
        for n in range(127):   # x within a few ulps of a rounding boundary (n + 1/2)·scale
            x = np.float32((n + 0.5) * np.float64(scale))
            for _ in range(8):
                b, t = np.rint(np.float32(x * inv)), np.rint(np.float32(x / scale))
                if b != t:
                    found = (np.float32(amax), scale, x, b, t)
                    break
                x = np.nextafter(x, np.float32(np.inf))
            if found:
                break
        if found:
            break
    assert found is not None
    amax, scale, x, body, tail = found
    row = np.zeros(20, np.float32)   # K = 20: positions 16..19 are the tail
    row[0] = amax
    row[3] = x
    row[17] = x
    q, sc = O.quant_rows(row[None, :])
    assert sc[0] == scale
    assert q[0, 3] == body and q[0, 17] == tail


# ── codes ───────────────────────────────────────────────────────────────────────────────────────────────────────

def test_clo_rules():
    lo = np.array([0.01, 0.02, 0.01, 0.03, 0.01, 0.0], np.float32)
    hi = np.array([0.01, 0.04, 0.04, 0.01, -1.0, 0.02], np.float32)
    clo = O.clo(lo, hi)
    assert clo[0] == 127          # lo == hi
    assert clo[1] == 64           # 127 / 2 = 63.5 rounds to even
    assert clo[2] == 32           # 31.75
    assert clo[3] == 127          # lo > hi clamps
    assert clo[4] == 0            # hi <= 0
    assert clo[5] == 0
    rng = _rng(3)
    lo = rng.uniform(0.005, 0.02, 4096).astype(np.float16).astype(np.float32)
    hi = (lo * rng.uniform(2, 4, 4096)).astype(np.float16).astype(np.float32)
    clo = O.clo(lo, hi).astype(np.float64)
    assert clo.min() >= 31 and clo.max() <= 64
    assert (np.abs(clo * hi / 127 - lo) <= hi / 254 * (1 + 1e-6)).all()


def test_codes_values_and_wrap():
    rng = _rng(4)
    K, N = 32, 64
    signs, flags, lo, hi, _, _ = _fv(rng, K, N, code3=True)
    codes = O.codes_i8w(signs, flags, lo, hi, K, N).astype(np.int16)
    code, flag = _np_decode(signs, flags, K, N)
    clo = O.clo(lo, hi).astype(np.int16)[None, :].repeat(K, 0)
    expect = np.select(
        [code == 1, (code == 0) & (flag == 1), (code == 2) & (flag == 1), code == 0, code == 2,
         (code == 3) & (flag == 1)],
        [0, -127, 127, -clo, clo, -2],
        default=((2 * clo + 128) % 256) - 128)
    assert (code == 3).any()
    assert np.array_equal(codes, expect)


def test_pack_codes_layout_is_a_permutation():
    rng = _rng(6)
    K, N = 16, 48
    signs, flags, lo, hi, _, _ = _fv(rng, K, N)
    flat = O.codes_i8w(signs, flags, lo, hi, K, N)
    packed = O.fv_pack_codes(signs, flags, lo, hi, K, N)
    p, kq, j, i = np.meshgrid(np.arange(N // 16), np.arange(K // 4), np.arange(16), np.arange(4), indexing="ij")
    expect = flat[4 * kq + i, 16 * p + j]
    assert np.array_equal(packed.reshape(N // 16, K // 4, 16, 4), expect)


def test_two_planes():
    rng = _rng(7)
    signs, flags, lo, hi, sign, is_hi = _fv(rng, 16, 32)
    S, T = O.planes_i8(signs, flags, 16, 32)
    assert np.array_equal(S, sign)
    assert np.array_equal(T, sign * is_hi.astype(np.int8))


# ── accumulators and epilogue ───────────────────────────────────────────────────────────────────────────────────

def test_acc_matches_int64_matmul():
    rng = _rng(8)
    q = rng.integers(-127, 128, (9, 300)).astype(np.int8)
    B = rng.integers(-127, 128, (300, 32)).astype(np.int8)
    acc = O.acc_i32(q, B)
    assert np.array_equal(acc.astype(np.int64), q.astype(np.int64) @ B.astype(np.int64))
    part = O.acc_i32(q, B, 100, 250)
    assert np.array_equal(part.astype(np.int64), q[:, 100:250].astype(np.int64) @ B[100:250].astype(np.int64))


@pytest.mark.parametrize("mode", ["int8w", "int8"])
@pytest.mark.parametrize("K", [1024, 2052])
def test_gemm_i8_float64_evaluation(mode, K):
    rng = _rng(9)
    M, N = 5, 32
    signs, flags, lo, hi, sign, is_hi = _fv(rng, K, N)
    A = rng.standard_normal((M, K)).astype(np.float32)
    q, sc = O.quant_rows(A)
    alpha = 0.75
    C = O.gemm_i8_run(mode, q, sc, signs, flags, lo, hi, N, alpha=alpha)
    qd = q.astype(np.float64)
    if mode == "int8w":
        codes = O.codes_i8w(signs, flags, lo, hi, K, N).astype(np.float64)
        ref = (qd @ codes) * (hi.astype(np.float64) / 127)[None, :]
    else:
        S = sign.astype(np.float64)
        T = (sign * is_hi).astype(np.float64)
        ref = (qd @ S) * lo[None, :] + (qd @ T) * (hi - lo).astype(np.float64)[None, :]
    ref = ref * (sc.astype(np.float64) * alpha)[:, None]
    assert np.allclose(C, ref, rtol=1e-5, atol=1e-6 * np.abs(ref).max())


def test_gemm_i8_beta_accumulates():
    rng = _rng(10)
    K, N, M = 64, 16, 3
    signs, flags, lo, hi, _, _ = _fv(rng, K, N)
    q = rng.integers(-127, 128, (M, K)).astype(np.int8)
    sc = rng.uniform(0.01, 0.1, M).astype(np.float32)
    C0 = rng.standard_normal((M, N)).astype(np.float32)
    stored = O.gemm_i8_run("int8w", q, sc, signs, flags, lo, hi, N)
    acc = O.gemm_i8_run("int8w", q, sc, signs, flags, lo, hi, N, C0=C0, beta_zero=False)
    assert np.allclose(acc, C0 + stored, rtol=1e-6, atol=1e-6)


def test_int8w_close_to_exact():
    """Quantisation error bound: per product ≤ (scale/2)·|w| from A and ≤ |a|·hi/254 from lo's grid."""
    rng = _rng(11)
    M, K, N = 8, 512, 32
    signs, flags, lo, hi, _, _ = _fv(rng, K, N)
    A = rng.standard_normal((M, K)).astype(np.float32)
    ex = O.sgemm_fvb("exact", A, signs, flags, lo, hi, N)
    i8w = O.sgemm_fvb("int8w", A, signs, flags, lo, hi, N)
    i8 = O.sgemm_fvb("int8", A, signs, flags, lo, hi, N)
    W = np.abs(O.expand_exact(signs, flags, lo, hi, K, N)).astype(np.float64)
    _, sc = O.quant_rows(A)
    bound_a = (sc[:, None] / 2) * W.sum(axis=0)[None, :]
    bound_w = np.abs(A).astype(np.float64) @ np.broadcast_to(hi / 254, (K, N))
    assert (np.abs(i8 - ex) <= bound_a + 1e-5).all()
    assert (np.abs(i8w - ex) <= bound_a + bound_w + 1e-5).all()
    assert not np.array_equal(i8w, ex)


def test_alpha_zero_and_k_not_multiple_of_4():
    rng = _rng(12)
    signs, flags, lo, hi, _, _ = _fv(rng, 6, 16)
    A = rng.standard_normal((2, 6)).astype(np.float32)
    C0 = rng.standard_normal((2, 16)).astype(np.float32)
    out = O.sgemm_fvb("int8w", A, signs, flags, lo, hi, 16, alpha=0.0, beta=0.5, C0=C0)
    assert np.array_equal(out, (C0 * np.float32(0.5)).astype(np.float32))
    # K = 6 is not a multiple of 4: the int8 modes take the exact route (blas.c:1490)
    a = O.sgemm_fvb("int8w", A, signs, flags, lo, hi, 16)
    b = O.sgemm_fvb("exact", A, signs, flags, lo, hi, 16)
    assert np.array_equal(a, b)


# ── the int8-table route (p2_sgemm_q8b, blas.c:1448-1460) ──────────────────────────────────────────────────────

def _q8b_table(rng, K, N, ldb):
    """An int8 table [K, ldb] whose first N columns are the weight codes; the columns beyond N hold values that
    must never be read (a stride mistake picks them up)."""
    B = rng.integers(-127, 128, (K, ldb)).astype(np.int8)
    B[:, N:] = 127
    scales = rng.uniform(0.001, 0.01, N).astype(np.float32)
    return B, scales


def _q8b_run(M, N, K, alpha, q, sc, B, scales, beta_zero=True, C0=None):
    C = np.zeros((M, N), np.float32) if C0 is None else np.ascontiguousarray(C0, np.float32).copy()
    O.lib().p2o_gemm_q8b_run(M, N, K, alpha, np.ascontiguousarray(q, np.int8), np.ascontiguousarray(sc, np.float32),
                             np.ascontiguousarray(B, np.int8), B.shape[1], np.ascontiguousarray(scales, np.float32),
                             1 if beta_zero else 0, C, N)
    return C


@pytest.mark.parametrize("K,ldb", [(1024, 48), (2052, 40), (100, 32)])
def test_q8b_run_float64_evaluation_strided_table(K, ldb):
    """p2o_gemm_q8b_run against an int64 product folded in float64: C = alpha·a_scale[m]·scales[n]·Σ_k q·B, over a
    table whose row stride ldb exceeds N (K > 1024 spans two of the per-1024-row blocks; K = 100 is one partial)."""
    rng = _rng(40 + K)
    M, N = 7, 32
    B, scales = _q8b_table(rng, K, N, ldb)
    A = rng.standard_normal((M, K)).astype(np.float32)
    q, sc = O.quant_rows(A)
    alpha = 0.625
    C = _q8b_run(M, N, K, alpha, q, sc, B, scales)
    acc = q.astype(np.int64) @ B[:, :N].astype(np.int64)
    ref = acc.astype(np.float64) * scales.astype(np.float64)[None, :] * (sc.astype(np.float64) * alpha)[:, None]
    assert np.allclose(C, ref, rtol=1e-5, atol=1e-6 * np.abs(ref).max())
    # the same product against a table packed to exactly N columns
    assert np.array_equal(C, _q8b_run(M, N, K, alpha, q, sc, np.ascontiguousarray(B[:, :N]), scales))
    # and beta = 1 adds onto C, block by block
    C0 = rng.standard_normal((M, N)).astype(np.float32)
    acc_c = _q8b_run(M, N, K, alpha, q, sc, B, scales, beta_zero=False, C0=C0)
    assert np.allclose(acc_c, C0 + ref, rtol=1e-5, atol=1e-5)


@pytest.mark.parametrize("mode", ["int8w", "int8", "exact"])
def test_sgemm_q8b_float64_evaluation(mode):
    """p2o_sgemm_q8b (the public entry) with a strided table: the int8 modes quantise A and run the table route
    (float64 of the quantised product); exact expands B·scales and runs the fp32 chain (float64 of A·W)."""
    rng = _rng(50)
    M, K, N, ldb = 6, 1536, 24, 40
    B, scales = _q8b_table(rng, K, N, ldb)
    A = rng.standard_normal((M, K)).astype(np.float32)
    alpha = 1.5
    C = O.sgemm_q8b(mode, A, B, scales, N, alpha=alpha)
    if mode == "exact":
        W = B[:, :N].astype(np.float32) * scales[None, :]
        ref = alpha * (A.astype(np.float64) @ W.astype(np.float64))
        assert np.allclose(C, ref, rtol=1e-5, atol=1e-5 * np.abs(ref).max())
    else:
        q, sc = O.quant_rows(A)
        acc = (q.astype(np.int64) @ B[:, :N].astype(np.int64)).astype(np.float64)
        ref = acc * scales.astype(np.float64)[None, :] * (sc.astype(np.float64) * alpha)[:, None]
        assert np.allclose(C, ref, rtol=1e-5, atol=1e-6 * np.abs(ref).max())
        # quantisation error bound against the fp32 product: ≤ (scale/2)·Σ|w| per output
        W = np.abs(B[:, :N].astype(np.float64) * scales[None, :])
        exact = alpha * (A.astype(np.float64) @ (B[:, :N].astype(np.float64) * scales[None, :]))
        assert (np.abs(C - exact) <= alpha * (sc[:, None] / 2) * W.sum(axis=0)[None, :] + 1e-5).all()
    # beta = 0.5 scales C first
    C0 = rng.standard_normal((M, N)).astype(np.float32)
    Cb = O.sgemm_q8b(mode, A, B, scales, N, alpha=alpha, beta=0.5, C0=C0)
    assert np.allclose(Cb, C + np.float32(0.5) * C0, rtol=1e-5, atol=1e-5)
