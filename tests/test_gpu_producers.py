"""The four producers on the GPU (p2h_layer_norm_quant_rows, p2h_silu_quant_rows, p2h_concat_heads_quant_rows,
p2h_channel_major_quant_rows, through the C ABI) against the oracle: codes, pads and scales bit-exact.

The oracle's LayerNorm and SiLU round every operation as the reference's source writes it; the GPU kernels do the
same, so the comparison is bit for bit. Shapes: the encoder's own (T = 375 frames of a 30 s window, D = 1024,
FF = 4096, 8 heads of 128; and T = 6000), plus ragged ones that take the element-wise load routes and the tails.
"""
import numpy as np
import pytest

import _oracle as O
import p2gemm as P

pytestmark = pytest.mark.gpu

SEED = 20261201


@pytest.fixture(scope="module", autouse=True)
def device():
    name = P.init()
    assert name.startswith("gfx950"), name
    return name


def _same(got, ref, M, K):
    """got: (untiled q [roundup(M, 16), ldq], scales); ref: (q [M, K], scales) from the oracle."""
    q, s = got
    qr, sr = ref
    assert np.array_equal(q[:M, :K], qr), f"{int((q[:M, :K] != qr).sum())} codes differ"
    assert not q[:M, K:].any() and not q[M:].any(), "pads not zero"
    assert np.array_equal(s.view(np.uint32), sr.view(np.uint32)), "scales differ"


def _rows(rng, M, ld, scale=1.0, shift=0.0):
    return (rng.standard_normal((M, ld)) * scale + shift).astype(np.float32)


@pytest.mark.parametrize("M,D,ldx", [(375, 1024, 1024), (6000, 1024, 1024), (37, 1027, 1030), (19, 640, 644),
                                     (5, 5, 5), (1, 4096, 4096), (16, 2048, 2050)])
def test_layer_norm_quant_rows(M, D, ldx):
    print(f"layer_norm_quant_rows M={M} D={D} ldx={ldx}", flush=True)
    rng = np.random.default_rng(SEED + M + D)
    X = _rows(rng, M, ldx, 1.7, 0.3)
    X[0, :D] = 0.5   # a constant row: x − mean is 0, the output is beta
    g = rng.uniform(0.5, 1.5, D).astype(np.float32)
    b = rng.uniform(-0.2, 0.2, D).astype(np.float32)
    _same(P.layer_norm_quant_rows(X, g, b, D=D), O.ln_quant_rows(X, g, b, D=D), M, D)


@pytest.mark.parametrize("M,K,ldh", [(375, 4096, 4096), (6000, 4096, 4096), (37, 1000, 1003), (3, 8, 8),
                                     (17, 2048, 2048), (21, 2056, 2059)])
def test_silu_quant_rows(M, K, ldh):
    print(f"silu_quant_rows M={M} K={K} ldh={ldh}", flush=True)
    rng = np.random.default_rng(SEED + 3 * M + K)
    H = _rows(rng, M, ldh, 4.0)
    H[0, :8] = [0.0, 100.0, -100.0, 87.0, -87.5, 30.0, -1e-30, 1e-30]
    _same(P.silu_quant_rows(H, K=K), O.silu_quant_rows(H, K=K), M, K)


@pytest.mark.parametrize("H,T,Dh", [(8, 375, 128), (8, 6000, 128), (3, 20, 20), (8, 1, 128), (2, 33, 48),
                                     (16, 50, 128), (3, 20, 400), (5, 9, 250)])
def test_concat_heads_quant_rows(H, T, Dh):
    print(f"concat_heads_quant_rows H={H} T={T} Dh={Dh}", flush=True)
    rng = np.random.default_rng(SEED + H * T + Dh)
    A = rng.standard_normal((H, T, Dh)).astype(np.float32)
    _same(P.concat_heads_quant_rows(A), O.concat_heads_quant_rows(A), T, H * Dh)


@pytest.mark.parametrize("D,T", [(1024, 375), (1024, 6000), (100, 7), (1, 3), (1500, 37), (4096, 20)])
def test_channel_major_quant_rows(D, T):
    print(f"channel_major_quant_rows D={D} T={T}", flush=True)
    rng = np.random.default_rng(SEED + D + T)
    W = rng.standard_normal((D, T)).astype(np.float32)
    _same(P.channel_major_quant_rows(W), O.channel_major_quant_rows(W), T, D)


@pytest.mark.parametrize("M,K,lda", [(375, 4096, 4096), (37, 1028, 1028), (19, 2052, 2055), (5, 8192, 8192),
                                     (3, 16384, 16388), (2, 20000, 20000)])
def test_quant_rows_long_rows(M, K, lda):
    """p2h_quant_rows on rows longer than 1024 (the row in registers up to ldq = 4096, read twice beyond)."""
    print(f"quant_rows M={M} K={K} lda={lda}", flush=True)
    rng = np.random.default_rng(SEED + M + K)
    A = _rows(rng, M, lda, 2.0)
    q, s = P.quant_rows(A, K=K)
    qr, sr = O.quant_rows(np.ascontiguousarray(A[:, :K]))
    _same((q, s), (qr, sr), M, K)


def test_silu_reciprocal_is_the_ieee_quotient_everywhere():
    """The SiLU producer's 1/(1 + e^-x) (hardware reciprocal + one Newton step) equals the correctly rounded quotient
    for every float of [1, 2^126), the whole range 1 + e^-x takes after the clamp at ±87."""
    bad, first, checked = P.recip_selftest()
    assert checked == 0x7E800000 - 0x3F800000
    assert bad == 0, f"{bad} differ, first 0x{first:08x}"


def test_zero_rows_is_a_no_op():
    q, s = P.silu_quant_rows(np.zeros((0, 64), np.float32))
    assert q.shape[0] == 0 and s.size == 0


def test_argument_errors():
    with pytest.raises(P.P2Error):
        P.silu_quant_rows(np.zeros((4, 12), np.float32))        # K % 8 != 0
    with pytest.raises(P.P2Error):
        P.silu_quant_rows(np.zeros((4, 4104), np.float32))      # longer than P2H_PROD_KMAX
    with pytest.raises(P.P2Error):
        P.layer_norm_quant_rows(np.zeros((4, 8), np.float32), np.ones(8, np.float32), np.zeros(8, np.float32), D=0)


def test_producer_feeds_the_gemm():
    """SiLU rows quantised on the device, then the five-value GEMM on those rows, equal the oracle's chain."""
    M, K, N = 64, 4096, 256
    rng = np.random.default_rng(SEED)
    Hh = _rows(rng, M, K, 3.0)
    signs, flags, lo, hi = P.gen_fv_weight(SEED, 7, K, N)
    w = P.FvWeight(signs, flags, lo, hi, K, N)
    dH = P.to_device(Hh)
    ldq = P.q_ld(K)
    dQ = P.DeviceBuffer(P.q_bytes(M, K))
    dS = P.DeviceBuffer(M * 4)
    dC = P.DeviceBuffer(M * N * 4)
    P.silu_quant_rows_dev(M, K, dH.ptr, K, dQ.ptr, ldq, dS.ptr)
    P.fvb_gemm_q8a_dev("int8w", M, N, K, 1.0, dQ.ptr, ldq, dS.ptr, w, 0.0, dC.ptr, N)
    got = dC.download((M, N), np.float32)
    q, s = O.silu_quant_rows(Hh)
    ref = O.gemm_i8_run("int8w", q, s, signs, flags, lo, hi, N)
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))


def _fvw(K, N, tid):
    signs, flags, lo, hi = P.gen_fv_weight(SEED, tid, K, N)
    return (signs, flags, lo, hi), P.FvWeight(signs, flags, lo, hi, K, N)


@pytest.mark.parametrize("mode", ["int8w", "int8"])
def test_feed_forward_module_on_device(mode):
    """encoder.c:340-348 with every step on the device: x += ½ · W2 · SiLU(W1 · LN(x)), the LayerNorm and the SiLU
    quantised as produced and the residual added in the second GEMM's epilogue (alpha 0.5, beta 1). Bit-exact
    against the oracle's chain of the same steps."""
    T, D, FF = 375, 1024, 4096
    print(f"feed_forward {mode} T={T} D={D} FF={FF}", flush=True)
    rng = np.random.default_rng(SEED + 17)
    x = _rows(rng, T, D, 1.0)
    g = rng.uniform(0.5, 1.5, D).astype(np.float32)
    b = rng.uniform(-0.2, 0.2, D).astype(np.float32)
    (s1, f1, l1, h1), w1 = _fvw(D, FF, 21)
    (s2, f2, l2, h2), w2 = _fvw(FF, D, 22)

    dx, dg, db = P.to_device(x), P.to_device(g), P.to_device(b)
    ldq1, ldq2 = P.q_ld(D), P.q_ld(FF)
    dQ1, dS1 = P.DeviceBuffer(P.q_bytes(T, D)), P.DeviceBuffer(T * 4)
    dH = P.DeviceBuffer(T * FF * 4)
    dQ2, dS2 = P.DeviceBuffer(P.q_bytes(T, FF)), P.DeviceBuffer(T * 4)
    P.layer_norm_quant_rows_dev(T, D, dx.ptr, D, dg.ptr, db.ptr, dQ1.ptr, ldq1, dS1.ptr)
    P.fvb_gemm_q8a_dev(mode, T, FF, D, 1.0, dQ1.ptr, ldq1, dS1.ptr, w1, 0.0, dH.ptr, FF)
    P.silu_quant_rows_dev(T, FF, dH.ptr, FF, dQ2.ptr, ldq2, dS2.ptr)
    P.fvb_gemm_q8a_dev(mode, T, D, FF, 0.5, dQ2.ptr, ldq2, dS2.ptr, w2, 1.0, dx.ptr, D)
    got = dx.download((T, D), np.float32)

    q1, sc1 = O.ln_quant_rows(x, g, b)
    h = O.gemm_i8_run(mode, q1, sc1, s1, f1, l1, h1, FF)
    q2, sc2 = O.silu_quant_rows(h)
    ref = O.gemm_i8_run(mode, q2, sc2, s2, f2, l2, h2, D, alpha=0.5, C0=x, beta_zero=False)
    neq = got.view(np.uint32) != ref.view(np.uint32)
    assert not neq.any(), f"{int(neq.sum())} of {neq.size} differ"


def test_attention_and_conv_outputs_on_device():
    """The two other residual linears: x += concat(heads) · W_o (encoder.c:525-527) and x += rows(dw) · W_pw2
    (encoder.c:600-604), each producer feeding the GEMM with alpha 1, beta 1."""
    T, D, H, Dh = 375, 1024, 8, 128
    print(f"attention/conv outputs T={T} D={D}", flush=True)
    rng = np.random.default_rng(SEED + 23)
    x = _rows(rng, T, D, 1.0)
    attn_h = rng.standard_normal((H, T, Dh)).astype(np.float32)
    dw = rng.standard_normal((D, T)).astype(np.float32)
    (so, fo, lo_, ho), wo = _fvw(D, D, 31)
    (sp, fp, lp, hp), wp = _fvw(D, D, 32)

    dx, dA, dW = P.to_device(x), P.to_device(attn_h), P.to_device(dw)
    ldq = P.q_ld(D)
    dQ, dS = P.DeviceBuffer(P.q_bytes(T, D)), P.DeviceBuffer(T * 4)
    P.concat_heads_quant_rows_dev(H, T, Dh, dA.ptr, dQ.ptr, ldq, dS.ptr)
    P.fvb_gemm_q8a_dev("int8w", T, D, D, 1.0, dQ.ptr, ldq, dS.ptr, wo, 1.0, dx.ptr, D)
    P.channel_major_quant_rows_dev(D, T, dW.ptr, dQ.ptr, ldq, dS.ptr)
    P.fvb_gemm_q8a_dev("int8w", T, D, D, 1.0, dQ.ptr, ldq, dS.ptr, wp, 1.0, dx.ptr, D)
    got = dx.download((T, D), np.float32)

    q, sc = O.concat_heads_quant_rows(attn_h)
    ref = O.gemm_i8_run("int8w", q, sc, so, fo, lo_, ho, D, alpha=1.0, C0=x, beta_zero=False)
    q, sc = O.channel_major_quant_rows(dw)
    ref = O.gemm_i8_run("int8w", q, sc, sp, fp, lp, hp, D, alpha=1.0, C0=ref, beta_zero=False)
    neq = got.view(np.uint32) != ref.view(np.uint32)
    assert not neq.any(), f"{int(neq.sum())} of {neq.size} differ"
