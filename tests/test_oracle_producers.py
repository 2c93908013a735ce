"""Pins for the oracle's row producers: LayerNorm, SiLU, the head concatenation and the channel-major transpose, each
quantised as the linear that reads it (tensor_ops.c:204-268, 329-350, 437-511; encoder.c:449-463, 554-568).

The checks are float64 evaluations of the same functions, constructed rows whose answer is known in closed form,
the identity "producer then quantise" = "quantise the produced rows" against the already pinned quantiser, and,
where the reference's own tensor_ops.c builds here, agreement with it within the tolerance its x86 build's
approximate reciprocals leave (1/sqrtf as vrsqrtss plus a Newton step, 1/(1+e) as vrcpps plus a Newton step).
"""
import numpy as np
import pytest

import _oracle as O


def _rng(seed=11):
    return np.random.default_rng(seed)


def _ln64(X, g, b):
    X = X.astype(np.float64)
    mu = X.mean(axis=1, keepdims=True)
    var = ((X - mu) ** 2).mean(axis=1, keepdims=True)
    return (X - mu) / np.sqrt(var + 1e-5) * g.astype(np.float64) + b.astype(np.float64)


def _silu64(X):
    X = X.astype(np.float64)
    return X / (1.0 + np.exp(-X))


# ── LayerNorm ───────────────────────────────────────────────────────────────────────────────────────────────────

@pytest.mark.parametrize("D", [1024, 1027, 8, 5])
def test_layer_norm_against_float64(D):
    rng = _rng(D)
    X = (rng.standard_normal((16, D)) * 1.7 + 0.3).astype(np.float32)
    g = rng.uniform(0.5, 1.5, D).astype(np.float32)
    b = rng.uniform(-0.2, 0.2, D).astype(np.float32)
    got = O.layer_norm_rows(X, g, b)
    ref = _ln64(X, g, b)
    err = np.abs(got - ref).max(axis=1) / np.sqrt((ref ** 2).mean(axis=1))
    assert err.max() < 2e-6, err.max()


def test_layer_norm_constant_row_gives_beta():
    """x − mean is exactly 0 for a constant row of a representable value: the output is beta exactly."""
    D = 1024
    X = np.full((2, D), 0.5, np.float32)
    g = _rng().uniform(0.5, 1.5, D).astype(np.float32)
    b = _rng(2).uniform(-1, 1, D).astype(np.float32)
    assert np.array_equal(O.layer_norm_rows(X, g, b), np.stack([b, b]))


def test_layer_norm_epsilon_closed_form():
    """Alternating ±a: mean 0 and variance a² exactly, so y = ±a / sqrt(a² + 1e-5) in closed form; a = 1e-3 makes the
    epsilon a tenfold term, so a dropped or misplaced epsilon fails."""
    D, a = 1024, np.float32(1e-3)
    X = np.tile(np.array([a, -a], np.float32), D // 2)[None, :]
    one, zero = np.ones(D, np.float32), np.zeros(D, np.float32)
    got = O.layer_norm_rows(X, one, zero)[0]
    expect = np.float64(a) / np.sqrt(np.float64(a) ** 2 + 1e-5)
    assert np.allclose(got[0::2], expect, rtol=2e-7) and np.allclose(got[1::2], -expect, rtol=2e-7)


# ── SiLU ────────────────────────────────────────────────────────────────────────────────────────────────────────

def test_silu_against_float64():
    """The degree-5 exponential is within 3e-6 relative of e^x; a dropped Horner term costs 4e-5 and fails."""
    rng = _rng(3)
    X = (rng.standard_normal((8, 1024)) * 4).astype(np.float32)
    got = O.swish_rows(X).astype(np.float64)
    ref = _silu64(X)
    assert (np.abs(got - ref) <= 4e-6 * np.abs(ref) + 1e-30).all()


def test_silu_tail_against_float64():
    """Rows whose length is not a multiple of eight: the last len % 8 values take p2_sigmoid's expf route."""
    rng = _rng(13)
    X = (rng.standard_normal((4, 1027)) * 4).astype(np.float32)
    got = O.swish_rows(X).astype(np.float64)
    ref = _silu64(X)
    assert (np.abs(got - ref) <= 4e-6 * np.abs(ref) + 1e-30).all()
    tail = np.abs(got[:, 1024:] - ref[:, 1024:]) <= 2e-7 * np.abs(ref[:, 1024:]) + 1e-30   # libm expf: < 1 ulp
    assert tail.all()


def test_silu_special_values():
    X = np.array([[0.0, 100.0, 87.0, 30.0, -100.0, -87.5, -1e-30, 1e-30]], np.float32)
    got = O.swish_rows(X)[0]
    assert got[0] == 0.0
    assert got[1] == 100.0 and got[2] == 87.0 and got[3] == 30.0  # 1 + e^-x rounds to 1
    assert -1e-30 < got[4] <= 0.0 and -1e-30 < got[5] <= 0.0    # the clamp keeps e^87 finite: x · (≈1e-38)
    assert got[6] == np.float32(-5e-31) and got[7] == np.float32(5e-31)


# ── producer = quantise(produced rows) ────────────────────────────────────────────────────────────────────────────

def test_ln_quant_rows_is_quantised_layer_norm():
    rng = _rng(4)
    M, D, ldx = 20, 1024, 1030
    X = (rng.standard_normal((M, ldx)) + 0.1).astype(np.float32)
    g = rng.uniform(0.5, 1.5, D).astype(np.float32)
    b = rng.uniform(-0.2, 0.2, D).astype(np.float32)
    q, sc = O.ln_quant_rows(X, g, b, D=D)
    q2, sc2 = O.quant_rows(O.layer_norm_rows(np.ascontiguousarray(X[:, :D]), g, b))
    assert np.array_equal(q, q2) and np.array_equal(sc, sc2)


def test_silu_quant_rows_is_quantised_silu():
    rng = _rng(5)
    X = (rng.standard_normal((20, 4100)) * 3).astype(np.float32)
    q, sc = O.silu_quant_rows(X, K=4096)
    q2, sc2 = O.quant_rows(O.swish_rows(np.ascontiguousarray(X[:, :4096])))
    assert np.array_equal(q, q2) and np.array_equal(sc, sc2)


def test_concat_heads_and_channel_major_are_transposes():
    rng = _rng(6)
    H, T, Dh = 8, 37, 128
    A = rng.standard_normal((H, T, Dh)).astype(np.float32)
    q, sc = O.concat_heads_quant_rows(A)
    q2, sc2 = O.quant_rows(np.ascontiguousarray(A.transpose(1, 0, 2).reshape(T, H * Dh)))
    assert np.array_equal(q, q2) and np.array_equal(sc, sc2)
    W = rng.standard_normal((1024, T)).astype(np.float32)
    q, sc = O.channel_major_quant_rows(W)
    q2, sc2 = O.quant_rows(np.ascontiguousarray(W.T))
    assert np.array_equal(q, q2) and np.array_equal(sc, sc2)


# ── the reference's own build ─────────────────────────────────────────────────────────────────────────────────────

needs_ref = pytest.mark.skipif(not O.ref_available(), reason="reference library not built (make -C oracle ref)")


@needs_ref
def test_layer_norm_against_reference_build():
    rng = _rng(7)
    for D in (1024, 640):
        X = (rng.standard_normal((64, D)) * 2 + 0.5).astype(np.float32)
        g = rng.uniform(0.5, 1.5, D).astype(np.float32)
        b = rng.uniform(-0.2, 0.2, D).astype(np.float32)
        got, ref = O.layer_norm_rows(X, g, b), O.ref_layer_norm_rows(X, g, b)
        err = np.abs(got - ref).max(axis=1) / np.sqrt((ref.astype(np.float64) ** 2).mean(axis=1))
        assert err.max() < 1e-6, err.max()


@needs_ref
def test_silu_against_reference_build():
    rng = _rng(8)
    X = (rng.standard_normal((64, 4096)) * 4).astype(np.float32)
    got, ref = O.swish_rows(X), O.ref_swish_rows(X)
    ulp = np.abs(got.view(np.int32).astype(np.int64) - ref.view(np.int32).astype(np.int64))
    assert ulp.max() <= 4, ulp.max()


@needs_ref
def test_quantised_producers_against_reference_build():
    """Quantising rows that differ in the last bits moves a code by at most one, and rarely."""
    rng = _rng(9)
    M, D = 64, 1024
    X = (rng.standard_normal((M, D)) + 0.2).astype(np.float32)
    g = rng.uniform(0.5, 1.5, D).astype(np.float32)
    b = rng.uniform(-0.2, 0.2, D).astype(np.float32)
    q, sc = O.ln_quant_rows(X, g, b)
    qr, scr = O.quant_rows(O.ref_layer_norm_rows(X, g, b))
    dq = np.abs(q.astype(np.int32) - qr)
    assert dq.max() <= 1 and (dq != 0).sum() <= M * D // 1000
    assert np.allclose(sc, scr, rtol=1e-6, atol=0)
    H = (rng.standard_normal((M, 4096)) * 3).astype(np.float32)
    q, sc = O.silu_quant_rows(H)
    qr, scr = O.quant_rows(O.ref_swish_rows(H))
    dq = np.abs(q.astype(np.int32) - qr)
    assert dq.max() <= 1 and (dq != 0).sum() <= M * 4096 // 1000
    assert np.allclose(sc, scr, rtol=1e-6, atol=0)
