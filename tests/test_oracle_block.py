"""Pins for the oracle's restatement of the conformer block between its linears (encoder.c:252-613), against the
reference's own functions built from its sources (oracle/_ref/libp2refblock.so: ref_block.c over encoder.c, with
tensor_ops.c), and against closed forms.

Index moves (the head gather, the positional transpose, the head concatenation, the channel-major transpose) and the
residual fmadd are restated here in numpy and must equal the reference bit for bit. The softmax, GLU and SiLU
restatements (each operation rounded once, the reference's order of additions) may differ from the reference's x86
-ffast-math build, which divides through approximate reciprocals refined by one Newton step, in the last bits only:
they are held to 8 ulp of each value, and a constructed mistake (a relative shift off by one, a dropped clamp)
fails the same comparison by orders of magnitude.
"""
import numpy as np
import pytest

import _oracle as O

pytestmark = pytest.mark.skipif(not O.refblock_available(), reason="reference block library not built")

H, Dh, D = 8, 128, 1024


def _rng(seed):
    return np.random.default_rng(seed)


def _ulps(a, b):
    """|a − b| in units of the last place of b (float32)."""
    a, b = np.asarray(a, np.float32), np.asarray(b, np.float32)
    spacing = np.spacing(np.abs(b)).astype(np.float64)
    return np.abs(a.astype(np.float64) - b.astype(np.float64)) / np.maximum(spacing, np.finfo(np.float32).tiny)


def _p(a):
    return np.ascontiguousarray(a).ctypes.data


@pytest.mark.parametrize("T", [375, 17])
def test_gather_heads_and_transposes_are_index_moves(T):
    rng = _rng(T)
    qkv = rng.standard_normal((T, 3 * D)).astype(np.float32)
    bu, bv = (rng.standard_normal(D) * 0.1).astype(np.float32), (rng.standard_normal(D) * 0.1).astype(np.float32)
    out = [np.zeros(H * T * Dh, np.float32) for _ in range(4)]
    O.refblock().refblock_gather_heads(_p(qkv), _p(bu), _p(bv), *[_p(o) for o in out], T)
    q, k, v = (qkv[:, i * D:(i + 1) * D].reshape(T, H, Dh) for i in range(3))
    assert np.array_equal(out[0].reshape(H, T, Dh), (q + bu.reshape(H, Dh)).transpose(1, 0, 2))
    assert np.array_equal(out[1].reshape(H, T, Dh), (q + bv.reshape(H, Dh)).transpose(1, 0, 2))
    assert np.array_equal(out[2].reshape(H, Dh, T), k.transpose(1, 2, 0))
    assert np.array_equal(out[3].reshape(H, T, Dh), v.transpose(1, 0, 2))
    L = 2 * T - 1
    P = rng.standard_normal((L, D)).astype(np.float32)
    Pt = np.zeros(H * Dh * L, np.float32)
    O.refblock().refblock_transpose_pos(_p(P), _p(Pt), L)
    assert np.array_equal(Pt.reshape(H, Dh, L), P.reshape(L, H, Dh).transpose(1, 2, 0))
    attn_h = rng.standard_normal((H, T, Dh)).astype(np.float32)
    rows = np.zeros((T, D), np.float32)
    O.refblock().refblock_concat_heads(_p(attn_h), _p(rows), T)
    assert np.array_equal(rows, attn_h.transpose(1, 0, 2).reshape(T, D))
    dw = rng.standard_normal((D, T)).astype(np.float32)
    O.refblock().refblock_cm_to_rows(_p(dw), _p(rows), T)
    assert np.array_equal(rows, dw.T)


def test_add_residual_is_one_fma_per_element():
    rng = _rng(3)
    T = 33
    x = rng.standard_normal((T, D)).astype(np.float32)
    y = rng.standard_normal((T, D)).astype(np.float32)
    got = x.copy()
    O.refblock().refblock_add_residual(_p(got), _p(y), T, 0.5)
    ref = (y.astype(np.float64) * 0.5 + x.astype(np.float64)).astype(np.float32)   # exact product, one rounding
    assert np.array_equal(got, ref)


@pytest.mark.parametrize("T", [375, 376, 9, 5])
def test_combine_softmax_against_the_reference(T):
    """T = 375 has a tail of 7 (expf), T = 376 none, T < 8 only a tail."""
    rng = _rng(100 + T)
    L = 2 * T - 1
    ac = (rng.standard_normal((H * T, T)) * 3).astype(np.float32)
    bd = (rng.standard_normal((H * T, L)) * 3).astype(np.float32)
    ref = ac.copy()
    O.refblock().refblock_combine_softmax(_p(ref), _p(bd), T)
    got = O.combine_softmax(ac, bd)
    assert _ulps(got, ref).max() <= 8
    np.testing.assert_allclose(got.sum(axis=1), 1.0, rtol=2e-6)
    # float64 closed form of the shift and the softmax
    r = np.arange(H * T)
    idx = (T - 1 - (r % T))[:, None] + np.arange(T)[None, :]
    z = (ac.astype(np.float64) + np.take_along_axis(bd.astype(np.float64), idx, axis=1)) * float(O.SCORE_SCALE)
    e = np.exp(z - z.max(axis=1, keepdims=True))
    np.testing.assert_allclose(got, e / e.sum(axis=1, keepdims=True), rtol=1e-5, atol=1e-12)
    # a shift one position off is far outside that tolerance
    idx_bad = np.minimum(idx + 1, L - 1)
    z_bad = (ac.astype(np.float64) + np.take_along_axis(bd.astype(np.float64), idx_bad, axis=1)) * float(O.SCORE_SCALE)
    e_bad = np.exp(z_bad - z_bad.max(axis=1, keepdims=True))
    assert np.abs(got - e_bad / e_bad.sum(axis=1, keepdims=True)).max() > 1e-3


def test_softmax_of_a_constant_row_is_uniform():
    T = 40
    ac = np.full((H * T, T), 2.5, np.float32)
    bd = np.zeros((H * T, 2 * T - 1), np.float32)
    got = O.combine_softmax(ac, bd)
    assert np.array_equal(got, np.full_like(got, np.float32(1.0) / np.float32(40.0)))


@pytest.mark.parametrize("T", [375, 6])
def test_glu_against_the_reference(T):
    rng = _rng(200 + T)
    pw1 = (rng.standard_normal((T, 2 * D)) * 2).astype(np.float32)
    pw1[0, D:D + 4] = [-100.0, 100.0, -87.5, 88.0]   # the clamp at 87 and its neighbourhood
    ref = np.zeros((D, T), np.float32)
    O.refblock().refblock_glu(_p(pw1), _p(ref), T)
    got = O.glu_channel_major(pw1)
    assert _ulps(got, ref).max() <= 8
    a, g = pw1[:, :D].astype(np.float64), pw1[:, D:].astype(np.float64)
    np.testing.assert_allclose(got, (a / (1.0 + np.exp(np.minimum(-g, 87.0)))).T, rtol=1e-6, atol=1e-30)


def _scalar_edge_columns(T, K=9):
    """Outputs the reference computes in scalar code (tensor_ops.c:564-571, 599-614): t < pad, the interior
    remainder after its eight-wide groups, and t >= T − pad."""
    pad = (K - 1) // 2
    lo, hi = pad, max(T - pad, pad)
    body_end = lo + (hi - lo) // 8 * 8
    cols = np.zeros(T, bool)
    cols[:min(pad, T)] = True
    cols[body_end:] = True
    return cols


@pytest.mark.parametrize("T", [375, 5, 9, 12, 64])
def test_depthwise_conv_silu_against_the_reference(T):
    """The convolution equals the reference's bit for bit on the outputs its eight-wide fmadd body computes; on its
    scalar edges, which an -ffast-math build may reassociate, within 4 eps of the sum of the terms' magnitudes.
    SiLU then agrees with the reference's p2_swish within 8 ulp."""
    rng = _rng(300 + T)
    x = rng.standard_normal((D, T)).astype(np.float32)
    w = (rng.standard_normal((D, 9)) * 0.3).astype(np.float32)
    b = (rng.standard_normal(D) * 0.1).astype(np.float32)
    ref = np.zeros((D, T), np.float32)
    R = O.refblock()
    R.p2_depthwise_conv1d(_p(x), _p(w), _p(b), _p(ref), D, T, 9)
    conv = O.dwconv(x, w, b)
    edge = _scalar_edge_columns(T)
    assert np.array_equal(conv[:, ~edge], ref[:, ~edge])
    xp = np.pad(x.astype(np.float64), ((0, 0), (4, 4)))
    mag = np.abs(b[:, None]).astype(np.float64) + sum(np.abs(xp[:, k:k + T] * w[:, k:k + 1]) for k in range(9))
    c64 = b[:, None].astype(np.float64) + sum(xp[:, k:k + T] * w[:, k:k + 1] for k in range(9))
    eps = float(np.finfo(np.float32).eps)
    assert np.all(np.abs(conv.astype(np.float64) - ref) <= 4 * eps * mag)
    assert np.all(np.abs(conv.astype(np.float64) - c64) <= 9 * eps * mag)
    # a tap off by one position is far outside that bound
    c_bad = b[:, None].astype(np.float64) + sum(xp[:, k + 1:k + 1 + T] * w[:, k:k + 1] for k in range(8))
    assert np.abs(conv - c_bad).max() > 0.1
    # SiLU: the oracle's on the reference's convolution against the reference's own p2_swish
    got = O.dwconv_silu(x, w, b)
    assert np.array_equal(got.reshape(-1), _silu_oracle(conv.reshape(-1)))
    ref_silu = ref.copy()
    R.p2_swish(_p(ref_silu), D * T)
    ours = _silu_oracle(ref.reshape(-1)).reshape(D, T)
    assert _ulps(ours, ref_silu).max() <= 8
    np.testing.assert_allclose(ours, ref.astype(np.float64) / (1.0 + np.exp(-ref.astype(np.float64))), rtol=1e-5,
                               atol=1e-30)


def _silu_oracle(v):
    v = np.ascontiguousarray(v, np.float32).copy()
    O.lib().p2o_swish_row(v, v.size)
    return v


def test_reference_block_with_the_oracle_exact_gemms_is_the_reference_block(tmp_path):
    """The reference's conformer_block on its own blas.c (x86: the exact route) and on the oracle's drop-in in exact
    mode give the same bits: the harness binds the block's GEMMs where it says, and the oracle's exact five-value
    GEMM is the reference's. In int8w mode the same block differs from the exact one by the quantisation (about
    1 %), neither 0 nor a blow-up."""
    import os
    import subprocess
    import sys
    child = os.path.join(os.path.dirname(os.path.abspath(__file__)), "refblock_child.py")
    outs = {}
    for mode, gemms in (("exact", "reference"), ("exact", "oracle"), ("int8w", "oracle")):
        out = tmp_path / f"{mode}_{gemms}.npy"
        env = dict(os.environ, P2_GEMM=mode)
        env.pop("P2_EXACT", None)
        r = subprocess.run([sys.executable, child, "7", "64", str(out), gemms], env=env, capture_output=True,
                           text=True, timeout=300)
        assert r.returncode == 0, r.stdout + r.stderr
        outs[mode, gemms] = np.load(out)
    ref = outs["exact", "reference"]
    assert np.isfinite(ref).all() and 0.5 < ref.std() < 2.0
    assert np.array_equal(ref.view(np.uint32), outs["exact", "oracle"].view(np.uint32))
    rel = np.linalg.norm(outs["int8w", "oracle"] - ref) / np.linalg.norm(ref)
    assert 1e-3 < rel < 5e-2
