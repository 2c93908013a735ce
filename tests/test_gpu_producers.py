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
                                     (17, 2048, 2048)])
def test_silu_quant_rows(M, K, ldh):
    print(f"silu_quant_rows M={M} K={K} ldh={ldh}", flush=True)
    rng = np.random.default_rng(SEED + 3 * M + K)
    H = _rows(rng, M, ldh, 4.0)
    H[0, :8] = [0.0, 100.0, -100.0, 87.0, -87.5, 30.0, -1e-30, 1e-30]
    _same(P.silu_quant_rows(H, K=K), O.silu_quant_rows(H, K=K), M, K)


@pytest.mark.parametrize("H,T,Dh", [(8, 375, 128), (8, 6000, 128), (3, 20, 20), (8, 1, 128), (2, 33, 48)])
def test_concat_heads_quant_rows(H, T, Dh):
    print(f"concat_heads_quant_rows H={H} T={T} Dh={Dh}", flush=True)
    rng = np.random.default_rng(SEED + H * T + Dh)
    A = rng.standard_normal((H, T, Dh)).astype(np.float32)
    _same(P.concat_heads_quant_rows(A), O.concat_heads_quant_rows(A), T, H * Dh)


@pytest.mark.parametrize("D,T", [(1024, 375), (1024, 6000), (100, 7), (1, 3)])
def test_channel_major_quant_rows(D, T):
    print(f"channel_major_quant_rows D={D} T={T}", flush=True)
    rng = np.random.default_rng(SEED + D + T)
    W = rng.standard_normal((D, T)).astype(np.float32)
    _same(P.channel_major_quant_rows(W), O.channel_major_quant_rows(W), T, D)


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
