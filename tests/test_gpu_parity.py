"""Parity of the HIP path (libp2hip.so, through its C ABI) with the oracle, on the GPU.

Bars: int32 accumulators, quantised activations and codes bit-exact; exact mode within 1e-4 on the matrix cores and
bit-exact on the fmaf-chain route (P2H_EXACT_CHAIN=1); int8 / int8w fp32
outputs within 1e-5 relative (|gpu − ref| <= 1e-5 · max(|ref|, rms of the reference row)) – and, because the
kernel folds its int32 sums per 1024-row K block with the reference's own fp32 operations, also bit-exact.
Full-size shapes compare a sample of rows: the GEMM is row-independent, so rows of C depend only on the same rows
of A.
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


def _weight(K, N, tid, code3=False):
    signs, flags, lo, hi = P.gen_fv_weight(SEED, tid, K, N)
    if code3:
        rng = np.random.default_rng(tid)
        flat = signs.reshape(-1)
        for i in rng.choice(flat.size, size=max(2, flat.size // 50), replace=False):
            flat[i] |= np.uint8(3 << (2 * int(rng.integers(0, 4))))
    return signs, flags, lo, hi


def _assert_fp32(got, ref, bit_exact=True):
    rms = np.sqrt(np.mean(ref.astype(np.float64) ** 2, axis=1, keepdims=True))
    tol = 1e-5 * np.maximum(np.abs(ref), rms)
    bad = np.abs(got.astype(np.float64) - ref) > tol
    assert not bad.any(), f"{bad.sum()} of {bad.size} outside 1e-5 relative; first at {np.argwhere(bad)[0]}"
    if bit_exact:
        neq = got.view(np.uint32) != ref.view(np.uint32)
        assert not neq.any(), f"{neq.sum()} of {neq.size} not bit-exact; first at {np.argwhere(neq)[0]}"


def _assert_exact(got, ref):
    """The exact-mode bar: within 1e-4 of the reference's exact route, elementwise relative to max(|ref|, row rms)."""
    rms = np.sqrt(np.mean(ref.astype(np.float64) ** 2, axis=1, keepdims=True))
    tol = 1e-4 * np.maximum(np.abs(ref), rms)
    bad = np.abs(got.astype(np.float64) - ref) > tol
    assert not bad.any(), f"{bad.sum()} of {bad.size} outside 1e-4 relative; first at {np.argwhere(bad)[0]}"


def _check(mode, got, ref, chain=None):
    """int8 modes: bit-exact fp32 (and within 1e-5). exact: the matrix-core route within 1e-4; `chain`, the same
    call with P2H_EXACT_CHAIN=1, bit-exact (the reference's per-output fmaf chain)."""
    if mode != "exact":
        _assert_fp32(got, ref)
        return
    _assert_exact(got, ref)
    if chain is not None:
        _assert_fp32(chain, ref)


def _chain(monkeypatch, fn):
    monkeypatch.setenv("P2H_EXACT_CHAIN", "1")
    try:
        return fn()
    finally:
        monkeypatch.delenv("P2H_EXACT_CHAIN")


def _bits_equal(a, b):
    return np.array_equal(np.ascontiguousarray(a).view(np.uint32), np.ascontiguousarray(b).view(np.uint32))


# ── activation quantisation ─────────────────────────────────────────────────────────────────────────────────────

@pytest.mark.parametrize("rpw", ["0", "1", "4", "-4"])
@pytest.mark.parametrize("M,K", [(64, 1024), (7, 20), (300, 4096), (5, 4), (129, 1028), (38, 4096), (193, 5000),
                                 (17, 8188)])
def test_quant_rows_bit_exact(monkeypatch, rpw, M, K):
    """Every row configuration of the quantiser (P2H_QUANT_RPW: 0 the planner's, 1 or 4 rows per workgroup, −4 four
    waves per row), with the padding rows and columns zeroed."""
    monkeypatch.setenv("P2H_QUANT_RPW", rpw)
    A = P.gen_activations(SEED, 100 + K, M, K)
    if M > 3:
        A[2] = 0.0   # a zero row: scale 1, q 0
    q_gpu, s_gpu = P.quant_rows(A)
    q_ref, s_ref = O.quant_rows(A)
    assert _bits_equal(s_gpu, s_ref)
    assert np.array_equal(q_gpu[:M, :K], q_ref)
    assert (q_gpu[:M, K:] == 0).all(), "padding columns must be zero"
    assert (q_gpu[M:] == 0).all(), "padding rows must be zero"


def test_quant_rows_strided_unaligned():
    A = P.gen_activations(SEED, 7, 9, 303)
    q_gpu, s_gpu = P.quant_rows(A, K=300)   # lda 303: rows are not 16-byte aligned
    q_ref, s_ref = O.quant_rows(A, K=300)
    assert _bits_equal(s_gpu, s_ref) and np.array_equal(q_gpu[:9, :300], q_ref)


# ── int32 accumulators ──────────────────────────────────────────────────────────────────────────────────────────

ACC_SHAPES = [(1, 64, 16), (37, 1024, 64), (130, 1100, 272), (200, 4096, 144), (375, 1024, 1024)]


@pytest.mark.parametrize("mode", ["int8w", "int8"])
@pytest.mark.parametrize("M,K,N", ACC_SHAPES)
def test_acc_i32_bit_exact(mode, M, K, N):
    signs, flags, lo, hi = _weight(K, N, 200 + N, code3=(K == 1100))
    A = P.gen_activations(SEED, 300 + M, M, K)
    q, _ = O.quant_rows(A)
    w = P.FvWeight(signs, flags, lo, hi, K, N)
    got = P.fvb_acc_i32(mode, q, w)
    if mode == "int8w":
        ref = O.acc_i32(q, O.codes_i8w(signs, flags, lo, hi, K, N))
        assert np.array_equal(got, ref)
    else:
        S, T = O.planes_i8(signs, flags, K, N)
        assert np.array_equal(got[0], O.acc_i32(q, S))
        assert np.array_equal(got[1], O.acc_i32(q, T))


# ── the whole GEMM on fp32 activations ──────────────────────────────────────────────────────────────────────────

GEMM_CASES = [
    # M, K, N, alpha, beta
    (1, 64, 16, 1.0, 0.0),
    (37, 1024, 64, 1.0, 0.0),
    (38, 1024, 4096, 1.0, 0.0),
    (38, 4096, 1024, 0.5, 1.0),
    (130, 1028, 272, -1.5, 0.3),
    (375, 1024, 1024, 1.0, 0.0),
    (9, 100, 32, 1.0, 1.0),
    (200, 2052, 144, 0.7, 0.0),
]


@pytest.mark.parametrize("mode", ["int8w", "int8", "exact"])
@pytest.mark.parametrize("M,K,N,alpha,beta", GEMM_CASES)
def test_fvb_gemm_parity(monkeypatch, mode, M, K, N, alpha, beta):
    signs, flags, lo, hi = _weight(K, N, 400 + K + N)
    A = P.gen_activations(SEED, 500 + M, M, K)
    C0 = P.gen_activations(SEED, 600 + N, M, N)
    w = P.FvWeight(signs, flags, lo, hi, K, N)
    run = lambda: P.fvb_gemm(mode, A, w, alpha=alpha, beta=beta, C0=C0)
    ref = O.sgemm_fvb(mode, A, signs, flags, lo, hi, N, alpha=alpha, beta=beta, C0=C0)
    _check(mode, run(), ref, _chain(monkeypatch, run) if mode == "exact" else None)


def test_fvb_gemm_strides_and_alpha_zero(monkeypatch):
    K, N, M = 256, 48, 11
    signs, flags, lo, hi = _weight(K, N, 11)
    w = P.FvWeight(signs, flags, lo, hi, K, N)
    A = P.gen_activations(SEED, 12, M, K + 5)
    C0 = P.gen_activations(SEED, 13, M, N + 3)
    for mode in ("int8w", "int8", "exact"):
        run = lambda: P.fvb_gemm(mode, A, w, alpha=1.25, beta=1.0, C0=C0, K=K)
        ref = O.sgemm_fvb(mode, A, signs, flags, lo, hi, N, alpha=1.25, beta=1.0, C0=C0, K=K)
        _check(mode, run(), ref, _chain(monkeypatch, run) if mode == "exact" else None)
        got0 = P.fvb_gemm(mode, A, w, alpha=0.0, beta=0.5, C0=C0, K=K)
        ref0 = O.sgemm_fvb(mode, A, signs, flags, lo, hi, N, alpha=0.0, beta=0.5, C0=C0, K=K)
        assert _bits_equal(got0, ref0)


def test_fvb_gemm_q8a_matches_fp32_entry():
    K, N, M = 1024, 4096, 375
    signs, flags, lo, hi = _weight(K, N, 21)
    w = P.FvWeight(signs, flags, lo, hi, K, N)
    A = P.gen_activations(SEED, 22, M, K)
    q, sc = O.quant_rows(A)
    got = P.fvb_gemm_q8a("int8w", q, sc, w)
    ref = O.gemm_i8_run("int8w", q, sc, signs, flags, lo, hi, N)
    _assert_fp32(got, ref)


def test_code3_int8w_and_exact(monkeypatch):
    K, N, M = 128, 64, 20
    signs, flags, lo, hi = _weight(K, N, 31, code3=True)
    w = P.FvWeight(signs, flags, lo, hi, K, N)
    A = P.gen_activations(SEED, 32, M, K)
    for mode in ("int8w", "int8", "exact"):
        run = lambda: P.fvb_gemm(mode, A, w)
        _check(mode, run(), O.sgemm_fvb(mode, A, signs, flags, lo, hi, N),
               _chain(monkeypatch, run) if mode == "exact" else None)


@pytest.mark.parametrize("name", sorted({k.split("/")[0] for k in np.load(
    __import__("os").path.join(__import__("os").path.dirname(__file__), "golden", "ref_exact_gemm.npz")).files
    if k.startswith("fvb")}))
def test_exact_against_reference_golden(monkeypatch, name):
    """The reference binary's own exact outputs: the matrix-core route within 1e-4, the fmaf-chain route bit for bit."""
    import os
    z = np.load(os.path.join(os.path.dirname(__file__), "golden", "ref_exact_gemm.npz"))
    g = lambda f: z[f"{name}/{f}"]
    M, K, N = (int(x) for x in g("dims"))
    alpha, beta = (float(x) for x in g("ab"))
    w = P.FvWeight(g("signs"), g("flags"), g("lo"), g("hi"), K, N)
    run = lambda: P.fvb_gemm("exact", g("A"), w, alpha=alpha, beta=beta, C0=g("C0"), K=K)
    _assert_exact(run(), g("C"))
    assert _bits_equal(_chain(monkeypatch, run), g("C"))


# ── codes, int8 tables, fp32 GEMM ───────────────────────────────────────────────────────────────────────────────

@pytest.mark.parametrize("K,N", [(64, 16), (1024, 1024), (4096, 1024)])
def test_pack_codes_bit_exact(K, N):
    signs, flags, lo, hi = _weight(K, N, 41, code3=(K == 64))
    w = P.FvWeight(signs, flags, lo, hi, K, N)
    assert np.array_equal(P.fv_pack_codes(w), O.fv_pack_codes(signs, flags, lo, hi, K, N))


@pytest.mark.parametrize("K,N", [(100, 48), (1024, 1024), (1024, 4096), (4096, 1024)])
def test_weight_records_only(monkeypatch, K, N):
    """A device weight keeps its 4-bit records, lo, hi and clo, not the planes: at most 0.51 byte per weight at the
    encoder's shapes. Every route works from the records: the int8w and int8 GEMMs, the fmaf-chain exact route (bit
    for bit the oracle's exact GEMM, which reads the planes), and the reference's packed codes (bit for bit the
    oracle's p2_fv_pack_codes); a weight made from device planes (p2h_fv_weight_wrap) gives the same bits as one
    uploaded from the host. K = 100 leaves rows 100..127 of the last unit as padding; code 3 is planted."""
    signs, flags, lo, hi = _weight(K, N, 47 + K, code3=True)
    up = P.FvWeight(signs, flags, lo, hi, K, N)
    dev = [P.to_device(np.ascontiguousarray(x)) for x in (signs, flags, lo, hi)]
    wr = P.FvWeight.wrap(*(d.ptr for d in dev), K, N, keep=dev)
    if K >= 1024:
        assert up.device_bytes() <= 0.51 * K * N, up.device_bytes() / (K * N)
    A = P.gen_activations(SEED, 48 + K, 37, K)
    for mode in ("int8w", "int8"):
        got = P.fvb_gemm(mode, A, up)
        _assert_fp32(got, O.sgemm_fvb(mode, A, signs, flags, lo, hi, N))
        assert _bits_equal(got, P.fvb_gemm(mode, A, wr))
    ref = O.sgemm_fvb("exact", A, signs, flags, lo, hi, N)
    for w in (up, wr):
        assert _bits_equal(_chain(monkeypatch, lambda: P.fvb_gemm("exact", A, w)), ref)
        _assert_exact(P.fvb_gemm("exact", A, w), ref)
    if K % 4 == 0:
        packed = O.fv_pack_codes(signs, flags, lo, hi, K, N)
        assert np.array_equal(P.fv_pack_codes(up), packed) and np.array_equal(P.fv_pack_codes(wr), packed)


@pytest.mark.parametrize("mode", ["int8w", "exact"])
@pytest.mark.parametrize("M,K,N,beta", [(11, 96, 32, 0.0), (375, 4096, 1024, 1.0), (3, 1030, 48, 0.0),
                                        (375, 1024, 640, 0.0), (200, 2100, 48, 1.0)])
def test_q8b_parity(mode, M, K, N, beta):
    """The int8-table GEMM (p2_sgemm_q8b) against the oracle, with the workspace that lets it split K: the encoder's
    subsampling output (4096 -> 1024, split at the 1024-row blocks) and projector (1024 -> 640, 32 x 64 tiles) at
    T = 375, a ragged K beyond two blocks, and small shapes."""
    B, sc = P.gen_i8_weight(SEED, 51, K, N)
    A = P.gen_activations(SEED, 52, M, K)
    C0 = P.gen_activations(SEED, 53, M, N)
    got = P.q8b_gemm(mode, A, B, sc, alpha=0.75, beta=beta, C0=C0)
    ref = O.sgemm_q8b(mode, A, B, sc, N, alpha=0.75, beta=beta, C0=C0)
    _assert_fp32(got, ref)


@pytest.mark.parametrize("M,K,N,beta", [(375, 4096, 1024, 0.0), (375, 4096, 1024, 1.0), (200, 2100, 48, 0.5),
                                        (1024, 3072, 512, 1.0)])
def test_q8b_split_same_bits(M, K, N, beta):
    """p2h_q8b_gemm splits K at the 1024-row blocks when its workspace has room (p2h_q8b_workspace_bytes) and runs
    unsplit with only the quantised rows' room: the same bits either way."""
    B, sc = P.gen_i8_weight(SEED, 54, K, N)
    A = P.gen_activations(SEED, 55, M, K)
    C0 = P.gen_activations(SEED, 56, M, N)
    full = P.q8b_workspace_bytes("int8w", M, N, K)
    rows_only = P.q_bytes(M, K) + 4 * M + 512
    assert full > rows_only, "the shape must be one that splits"
    split = P.q8b_gemm("int8w", A, B, sc, alpha=-0.5, beta=beta, C0=C0)
    unsplit = P.q8b_gemm("int8w", A, B, sc, alpha=-0.5, beta=beta, C0=C0, ws_bytes=rows_only)
    assert _bits_equal(split, unsplit)


@pytest.mark.parametrize("tA,tB", [(False, False), (False, True), (True, False), (True, True)])
def test_sgemm_fp32(tA, tB):
    rng = np.random.default_rng(61)
    M, K, N = 45, 77, 50
    A = rng.standard_normal((K, M) if tA else (M, K)).astype(np.float32)
    B = rng.standard_normal((N, K) if tB else (K, N)).astype(np.float32)
    C0 = rng.standard_normal((M, N)).astype(np.float32)
    got = P.sgemm(A, B, tA, tB, alpha=0.5, beta=0.25, C0=C0)
    ref = 0.5 * ((A.T if tA else A).astype(np.float64) @ (B.T if tB else B).astype(np.float64)) + 0.25 * C0
    assert np.allclose(got, ref, rtol=1e-4, atol=1e-4)


@pytest.mark.parametrize("H,T,Dh", [(16, 375, 64), (4, 37, 64), (2, 129, 40)])
def test_sgemm_batched_attention_shapes(H, T, Dh):
    """The per-head products of relative-position attention (encoder.c:505-519): Q_u·K_t [T, T], Q_v·P_t [T, 2T−1]
    and scores·V [T, Dh], every head in one launch, against float64."""
    rng = np.random.default_rng(H * T)
    L = 2 * T - 1
    Qu = rng.standard_normal((H, T, Dh)).astype(np.float32)
    Kt = rng.standard_normal((H, Dh, T)).astype(np.float32)
    Pt = rng.standard_normal((H, Dh, L)).astype(np.float32)
    S = rng.random((H, T, T)).astype(np.float32)
    V = rng.standard_normal((H, T, Dh)).astype(np.float32)
    for A, B in ((Qu, Kt), (Qu, Pt), (S, V)):
        got = P.sgemm_batched(A, B)
        _assert_exact(got.reshape(-1, got.shape[2]),
                      np.matmul(A.astype(np.float64), B.astype(np.float64)).reshape(-1, got.shape[2]))


@pytest.mark.parametrize("tA,tB", [(False, True), (True, False)])
def test_sgemm_batched_transposed_beta(tA, tB):
    rng = np.random.default_rng(7)
    b, M, K, N = 3, 70, 33, 90
    A = rng.standard_normal((b, K, M) if tA else (b, M, K)).astype(np.float32)
    B = rng.standard_normal((b, N, K) if tB else (b, K, N)).astype(np.float32)
    C0 = rng.standard_normal((b, M, N)).astype(np.float32)
    got = P.sgemm_batched(A, B, tA, tB, alpha=-0.5, beta=1.0, C0=C0)
    opA = np.swapaxes(A, 1, 2) if tA else A
    opB = np.swapaxes(B, 1, 2) if tB else B
    ref = -0.5 * np.matmul(opA.astype(np.float64), opB.astype(np.float64)) + C0
    _assert_exact(got.reshape(-1, N), ref.reshape(-1, N))


@pytest.mark.parametrize("tA,tB", [(False, False), (False, True), (True, False), (True, True)])
@pytest.mark.parametrize("shape", [(2, 96, 200, 128), (3, 45, 77, 50), (1, 64, 33, 100), (2, 130, 259, 66)])
@pytest.mark.parametrize("loads", ["chosen", "element"])
def test_sgemm_batched_every_load_route(monkeypatch, tA, tB, shape, loads):
    """Every operand orientation with 16-byte loads (rows aligned, lengths multiples of 4), buffer loads (the rest) and
    the element loads kept for operands of 2 GiB or more (forced by P2H_SGEMM_ANY); K spans several 32-row stages,
    so the register ring wraps; against float64."""
    if loads == "element":
        monkeypatch.setenv("P2H_SGEMM_ANY", "1")
    b, M, K, N = shape
    rng = np.random.default_rng(M * K + N)
    A = rng.standard_normal((b, K, M) if tA else (b, M, K)).astype(np.float32)
    B = rng.standard_normal((b, N, K) if tB else (b, K, N)).astype(np.float32)
    C0 = rng.standard_normal((b, M, N)).astype(np.float32)
    got = P.sgemm_batched(A, B, tA, tB, alpha=0.75, beta=0.5, C0=C0)
    opA = np.swapaxes(A, 1, 2) if tA else A
    opB = np.swapaxes(B, 1, 2) if tB else B
    ref = 0.75 * np.matmul(opA.astype(np.float64), opB.astype(np.float64)) + 0.5 * C0.astype(np.float64)
    _assert_exact(got.reshape(-1, N), ref.reshape(-1, N))


# ── reading the next weight's records ahead ───────────────────────────────────────────────────────────────────────

@pytest.mark.parametrize("mode", ["int8w", "int8"])
@pytest.mark.parametrize("M,K,N,Kn,Nn,beta", [(375, 1024, 4096, 4096, 1024, 0.0), (375, 4096, 1024, 1024, 3072, 1.0),
                                              (38, 1024, 1024, 4096, 1024, 0.5), (2000, 1024, 1024, 1024, 4096, 0.0),
                                              (200, 1024, 272, 0, 0, 0.0)])
def test_q8a_next_matches_q8a(mode, M, K, N, Kn, Nn, beta):
    """p2h_fvb_gemm_q8a_next gives p2h_fvb_gemm_q8a's outputs bit for bit: with a next weight of another shape, with
    none (Kn = 0), at 2000 rows (the large-M kernel, which reads nothing ahead), and twice in a row (the second
    call's first loads find the records the first read ahead)."""
    A = P.gen_activations(SEED, 1800 + M, M, K)
    q, sc = O.quant_rows(A)
    w = P.FvWeight(*_weight(K, N, 1810), K, N)
    nxt = P.FvWeight(*_weight(Kn, Nn, 1811), Kn, Nn) if Kn else None
    C0 = P.gen_activations(SEED, 1820 + N, M, N)
    ldq = P.q_ld(K)
    dQ, dS = P.to_device(P.q_tile(q, ldq)), P.to_device(sc)
    ws = P.Workspace(P.q8a_workspace_bytes(mode, M, N, K))
    single = P.fvb_gemm_q8a(mode, q, sc, w, alpha=0.8, beta=beta, C0=C0)
    for rep in range(2):
        dC = P.to_device(C0)
        P.fvb_gemm_q8a_next_dev(mode, M, N, K, 0.8, dQ.ptr, ldq, dS.ptr, w, beta, dC.ptr, N, ws.ptr, ws.nbytes, nxt)
        assert _bits_equal(dC.download((M, N), np.float32), single), f"call {rep}"


# ── the feed-forward's SiLU in the up-projection's epilogue ───────────────────────────────────────────────────────

@pytest.mark.parametrize("mode", ["int8w", "int8"])
@pytest.mark.parametrize("M,K,N", [(375, 1024, 4096), (38, 1024, 4096), (375, 4096, 272), (2000, 1024, 1024)])
def test_q8a_silu_matches_gemm_then_silu(mode, M, K, N):
    """p2h_fvb_gemm_q8a_silu equals p2h_fvb_gemm_q8a followed by p2h_silu bit for bit: the small-M tiles apply
    silu_p2 as they store C; at 2000 rows (the large-M kernel) the library runs the SiLU kernel after the GEMM."""
    A = P.gen_activations(SEED, 1900 + M, M, K)
    q, sc = O.quant_rows(A)
    w = P.FvWeight(*_weight(K, N, 1910 + N), K, N)
    got = P.fvb_gemm_q8a_silu(mode, q, sc, w, alpha=0.7)
    ref = P.silu(P.fvb_gemm_q8a(mode, q, sc, w, alpha=0.7))
    assert np.isfinite(got).all()
    assert _bits_equal(got, ref)


# ── several weights against the same quantised rows in one launch ─────────────────────────────────────────────────

@pytest.mark.parametrize("mode", ["int8w", "int8"])
@pytest.mark.parametrize("M,K,N,groups,beta", [(749, 1024, 1024, 24, 0.0), (375, 1024, 4096, 3, 1.0),
                                               (38, 4096, 1024, 5, 0.5), (2000, 1024, 256, 2, 0.0),
                                               (600, 1024, 272, 20, 0.5), (375, 4096, 1024, 3, 0.0),
                                               (375, 4096, 1024, 2, 1.0)])
def test_grouped_q8a(mode, M, K, N, groups, beta):
    """Each group's output equals its own p2h_fvb_gemm_q8a call bit for bit (2000 rows: the per-weight path; int8w at
    749 × 24 · 1024 and 600 × 20 · 272: the large-M kernel's tiles, ragged in both dimensions for the latter; int8w at
    375 × 4096 → 1024: the eight-wave 32 × 64 small-M tile, whose grid has half as many column tiles as 32 × 32)."""
    A = P.gen_activations(SEED, 1500 + M, M, K)
    q, sc = O.quant_rows(A)
    ws = [P.FvWeight(*_weight(K, N, 1600 + i), K, N) for i in range(groups)]
    C0 = P.gen_activations(SEED, 1700 + N, M, N)
    ldq = P.q_ld(K)
    dQ, dS = P.to_device(P.q_tile(q, ldq)), P.to_device(sc)
    outs = [P.to_device(C0) for _ in range(groups)]
    P.fvb_gemm_q8a_grouped_dev(mode, M, N, K, 0.8, dQ.ptr, ldq, dS.ptr, ws, beta, [o.ptr for o in outs], N)
    for i, (w, o) in enumerate(zip(ws, outs)):
        got = o.download((M, N), np.float32)
        single = P.fvb_gemm_q8a(mode, q, sc, w, alpha=0.8, beta=beta, C0=C0)
        assert _bits_equal(got, single), f"group {i}"
    signs, flags, lo, hi = _weight(K, N, 1600 + groups - 1)
    rows = np.arange(min(M, 64))
    if beta == 0.0:
        ref = O.gemm_i8_run(mode, q[rows], sc[rows], signs, flags, lo, hi, N, alpha=0.8)
    else:   # beta outside {0, 1} pre-scales C in fp32 (blas.c:1436), then the product accumulates
        C0s = C0[rows] if beta == 1.0 else (C0[rows] * np.float32(beta)).astype(np.float32)
        ref = O.gemm_i8_run(mode, q[rows], sc[rows], signs, flags, lo, hi, N, alpha=0.8, C0=C0s, beta_zero=False)
    _assert_fp32(outs[-1].download((M, N), np.float32)[rows], ref)


# ── full-size shapes, sampled rows ──────────────────────────────────────────────────────────────────────────────

@pytest.mark.parametrize("M,K,N", [(6000, 1024, 4096), (6000, 4096, 1024), (749, 1024, 1024), (375, 1024, 3072)])
def test_full_size_sampled_rows(M, K, N):
    signs, flags, lo, hi = _weight(K, N, 700 + K + N)
    w = P.FvWeight(signs, flags, lo, hi, K, N)
    A = P.gen_activations(SEED, 800 + M, M, K)
    got = P.fvb_gemm("int8w", A, w)
    rows = np.unique(np.concatenate([[0, M - 1], np.random.default_rng(M).choice(M, 48, replace=False)]))
    ref = O.sgemm_fvb("int8w", A[rows], signs, flags, lo, hi, N)
    _assert_fp32(got[rows], ref)
    # a size-independent property over every row: rows scaled by 2^j give outputs scaled by exactly 2^j
    got2 = P.fvb_gemm("int8w", A * np.float32(4.0), w)
    assert _bits_equal(got2, (got * np.float32(4.0)).astype(np.float32))


def _i8w_fold_all_rows(q, sc, signs, flags, lo, hi, K, N, alpha):
    """int8w outputs for one 1024-row block, all rows: exact int32 sums (float64 products of the oracle's codes and
    the quantised rows, exact below 2^53) folded as the reference folds them, in float32 operations:
    f = (float)acc · (hi · (1/127)), C = f · (a_scale · alpha) (blas.c:1316-1328, 1355-1366)."""
    codes = O.codes_i8w(signs, flags, lo, hi, K, N)
    acc = (q.astype(np.float64) @ codes.astype(np.float64)).astype(np.float32)
    c1 = np.asarray(hi, np.float32) * (np.float32(1.0) / np.float32(127.0))
    asc = np.asarray(sc, np.float32) * np.float32(alpha)
    return (acc * c1[None, :]) * asc[:, None]


@pytest.mark.parametrize("M,K,N", [(8000, 1024, 1040), (4099, 900, 2064), (1100, 1024, 4096)])
def test_large_m_every_output(M, K, N):
    """The large-M kernel over whole matrices: every output bit-exact against the fold of exact int32 sums, itself
    checked against the oracle on sampled rows; ragged M and N (partial row and column tiles), K below 1024 (a
    zero-padded unit); C wider than N (ldc = N + 16) and filled with NaN beforehand: beta 0 never reads C, every
    output is written and nothing past column N is; two calls in a row give the same bits."""
    signs, flags, lo, hi = _weight(K, N, 960 + K + N)
    w = P.FvWeight(signs, flags, lo, hi, K, N)
    A = P.gen_activations(SEED, 961 + M, M, K)
    q, sc = O.quant_rows(A)
    ref = _i8w_fold_all_rows(q, sc, signs, flags, lo, hi, K, N, 0.7)
    rows = np.unique(np.concatenate([[0, M - 1], np.random.default_rng(M).choice(M, 24, replace=False)]))
    assert _bits_equal(ref[rows], O.gemm_i8_run("int8w", q[rows], sc[rows], signs, flags, lo, hi, N, alpha=0.7))
    C0 = np.full((M, N + 16), np.nan, np.float32)
    for _ in range(2):   # twice: nothing carries over between calls
        got = P.fvb_gemm_q8a("int8w", q, sc, w, alpha=0.7, C0=C0)
        _assert_fp32(got[:, :N], ref)
        assert np.isnan(got[:, N:]).all()


@pytest.mark.parametrize("M,K,N", [(1100, 1024, 4096), (4099, 900, 2064), (375, 1024, 4096), (38, 4096, 1024)])
def test_device_scope_stores_same_bits(monkeypatch, M, K, N):
    """C stored at device scope (buffer stores over the tile's rows) and plainly: the same bits, on the large-M and
    small-M tiles, into a C wider than N (ldc = N + 8) that beta = 1 accumulates into; nothing past column N is
    written."""
    signs, flags, lo, hi = _weight(K, N, 970 + M)
    w = P.FvWeight(signs, flags, lo, hi, K, N)
    A = P.gen_activations(SEED, 971 + M, M, K)
    q, sc = O.quant_rows(A)
    C0 = P.gen_activations(SEED, 972 + M, M, N + 8)
    C0[:, N:] = np.nan
    print(f"device-scope stores M={M} K={K} N={N} plan={P.plan('int8w', M, N, K)}", flush=True)
    got = {}
    for flag in ("0", "1"):
        monkeypatch.setenv("P2H_DEVICE_SCOPE_STORES", flag)
        got[flag] = P.fvb_gemm_q8a("int8w", q, sc, w, alpha=0.5, beta=1.0, C0=C0)
        assert np.isnan(got[flag][:, N:]).all()
    assert _bits_equal(got["0"], got["1"])
    rows = np.unique(np.concatenate([[0, M - 1], np.random.default_rng(M).choice(M, min(M, 16), replace=False)]))
    ref = O.gemm_i8_run("int8w", q[rows], sc[rows], signs, flags, lo, hi, N, alpha=0.5, C0=C0[rows, :N],
                        beta_zero=False)
    _assert_fp32(got["1"][rows, :N], ref)


@pytest.mark.parametrize("M,K,N,plan", [(6000, 1024, 4096, "96x256"), (3000, 1024, 4096, "96x256"),
                                         (6000, 1024, 2048, "96x256"), (4099, 1024, 4096, "96x256"),
                                         (6000, 1024, 1024, "96x128"), (3000, 1024, 1024, "96x128"),
                                         (1500, 1024, 4096, "96x128"), (2000, 1024, 3072, "96x128"),
                                         (6000, 4096, 1024, "96x128")])
def test_large_m_plans(M, K, N, plan):
    """The large-M tile: 96 × 256 for K <= 1024 while its tiles outnumber the CUs, else 96 × 128 (twice the
    workgroups, so that no CU is left with one); 96 × 128 with the fold in registers for K > 1024. Where the plan is
    96 × 128 at K <= 1024, sampled rows are checked against the oracle."""
    assert P.plan("int8w", M, N, K).startswith(f"tile {plan},")
    if plan == "96x128" and K <= 1024 and M * N <= 3000 * 1024:
        signs, flags, lo, hi = _weight(K, N, 990 + M)
        w = P.FvWeight(signs, flags, lo, hi, K, N)
        A = P.gen_activations(SEED, 991 + M, M, K)
        q, sc = O.quant_rows(A)
        got = P.fvb_gemm_q8a("int8w", q, sc, w, alpha=1.25)
        rows = np.unique(np.concatenate([[0, M - 1], np.random.default_rng(M).choice(M, 12, replace=False)]))
        _assert_fp32(got[rows], O.gemm_i8_run("int8w", q[rows], sc[rows], signs, flags, lo, hi, N, alpha=1.25))


@pytest.mark.parametrize("M,K,N,tile", [(1100, 1024, 4096, None), (4099, 900, 2064, None), (6000, 4096, 1024, None),
                                         (375, 4096, 1024, "8"), (130, 1028, 272, "9"), (200, 2048, 512, "8"),
                                         (1100, 640, 512, None), (2000, 384, 1040, "8"),
                                         (1500, 1024, 1024, "8-odd-ldc")])
def test_records_in_registers_same_bits(monkeypatch, M, K, N, tile):
    """The large-M tiles with each wave's weight records loaded into registers (gemm_fv_rb) and through the LDS ring
    (gemm_fv): the same bits, K below, at and above one 1024-row fold block, odd numbers of 128-row stages (K = 640,
    384, 1028), ragged M and N, beta 1 into a C wider than N (ldc = N + 4); checked against the oracle on sampled
    rows."""
    pad = 4
    if tile is not None and tile.endswith("-odd-ldc"):   # ldc = N + 3: rows not 16-byte aligned, element stores
        tile, pad = tile[:-8], 3
    if tile is not None:
        monkeypatch.setenv("P2H_TILE", tile)
    plan = P.plan("int8w", M, N, K)
    assert plan.startswith("tile 96x"), plan
    signs, flags, lo, hi = _weight(K, N, 980 + M)
    w = P.FvWeight(signs, flags, lo, hi, K, N)
    A = P.gen_activations(SEED, 981 + M, M, K)
    q, sc = O.quant_rows(A)
    C0 = P.gen_activations(SEED, 982 + M, M, N + pad)
    print(f"records in registers M={M} K={K} N={N} ldc={N + pad} plan={plan}", flush=True)
    got = {}
    for flag in ("0", "1"):
        monkeypatch.setenv("P2H_RECORDS_IN_REGISTERS", flag)
        got[flag] = P.fvb_gemm_q8a("int8w", q, sc, w, alpha=-0.75, beta=1.0, C0=C0)
    assert _bits_equal(got["0"], got["1"])
    assert _bits_equal(got["1"][:, N:], C0[:, N:])
    rows = np.unique(np.concatenate([[0, M - 1], np.random.default_rng(M).choice(M, min(M, 12), replace=False)]))
    ref = O.gemm_i8_run("int8w", q[rows], sc[rows], signs, flags, lo, hi, N, alpha=-0.75, C0=C0[rows, :N],
                        beta_zero=False)
    _assert_fp32(got["1"][rows, :N], ref)


@pytest.mark.parametrize("M,K,N", [(375, 4096, 1024), (375, 1024, 1024), (749, 1024, 1024), (375, 1024, 4096),
                                   (38, 4096, 1024), (256, 2048, 512)])
def test_xcd_grid_same_bits(monkeypatch, M, K, N):
    """The small-M tiles' XCD grid (P2H_XCD_ROWS: the default -4 takes four rows of XCDs where N < 4·M; 0, 2 and 4
    everywhere the tiles divide) is a permutation of the tiles: the same bits as the plain order, beta 1."""
    signs, flags, lo, hi = _weight(K, N, 970 + M)
    w = P.FvWeight(signs, flags, lo, hi, K, N)
    A = P.gen_activations(SEED, 971 + M, M, K)
    q, sc = O.quant_rows(A)
    C0 = P.gen_activations(SEED, 972 + M, M, N)
    got = {}
    for flag in ("0", "-4", "4", "2"):
        monkeypatch.setenv("P2H_XCD_ROWS", flag)
        got[flag] = P.fvb_gemm_q8a("int8w", q, sc, w, alpha=0.5, beta=1.0, C0=C0)
    for flag in ("-4", "4", "2"):
        assert _bits_equal(got["0"], got[flag]), flag
    rows = np.unique(np.concatenate([[0, M - 1], np.random.default_rng(M).choice(M, min(M, 8), replace=False)]))
    ref = O.gemm_i8_run("int8w", q[rows], sc[rows], signs, flags, lo, hi, N, alpha=0.5, C0=C0[rows], beta_zero=False)
    _assert_fp32(got["-4"][rows], ref)


@pytest.mark.parametrize("M,K,N", [(6000, 1024, 4096), (6000, 4096, 1024)])
def test_exact_full_size_sampled_rows(monkeypatch, M, K, N):
    """The exact route at the batched long-audio shapes (16 windows stacked, 12k+ workgroups on the fp32 matrix
    cores): sampled rows (first and last included) within 1e-4 of the oracle's exact route, the fmaf-chain route
    (P2H_EXACT_CHAIN=1) bit-exact on the same rows, and over every row the power-of-two property (rows scaled by 4
    give outputs scaled by exactly 4: every product and partial sum scales exactly)."""
    signs, flags, lo, hi = _weight(K, N, 740 + K + N)
    w = P.FvWeight(signs, flags, lo, hi, K, N)
    A = P.gen_activations(SEED, 840 + K, M, K)
    got = P.fvb_gemm("exact", A, w)
    rows = np.unique(np.concatenate([[0, M - 1], np.random.default_rng(M + K).choice(M, 40, replace=False)]))
    ref = O.sgemm_fvb("exact", A[rows], signs, flags, lo, hi, N)
    _assert_exact(got[rows], ref)
    chain = _chain(monkeypatch, lambda: P.fvb_gemm("exact", A, w))
    _assert_fp32(chain[rows], ref)
    got4 = P.fvb_gemm("exact", A * np.float32(4.0), w)
    assert _bits_equal(got4, (got * np.float32(4.0)).astype(np.float32))


@pytest.mark.parametrize("M,K,N", [(375, 4096, 1024), (38, 1024, 4096), (130, 1024, 208), (9, 4096, 64)])
def test_exact_tiles_same_bits(monkeypatch, M, K, N):
    """Every output of the exact route's matrix-core kernel is summed in the same order whatever the tile (each MFMA
    step covers the same four K rows, and the waves' K segments meet in wave order), so all five tiles give the same
    bits; the planner's choice among them is a matter of speed only."""
    signs, flags, lo, hi = _weight(K, N, 940 + M + N)
    w = P.FvWeight(signs, flags, lo, hi, K, N)
    A = P.gen_activations(SEED, 941 + M, M, K)
    C0 = np.random.default_rng(M).standard_normal((M, N)).astype(np.float32)
    base = P.fvb_gemm("exact", A, w, alpha=0.7, beta=1.0, C0=C0)
    for tile in (32, 64, 1616, 1632, 1664):
        monkeypatch.setenv("P2H_XF_TILE", str(tile))
        assert _bits_equal(P.fvb_gemm("exact", A, w, alpha=0.7, beta=1.0, C0=C0), base), f"tile {tile}"


@pytest.mark.parametrize("M,K,N,lda,ldc,tile", [
    (375, 1024, 4096, 1024, 4096, 0), (375, 4096, 1024, 4096, 1024, 0), (375, 1024, 1024, 1028, 1030, 0),
    (749, 1024, 1024, 1024, 1024, 64), (37, 256, 64, 260, 64, 32), (1, 128, 48, 128, 50, 0), (130, 384, 208, 388, 211, 64),
    (38, 4096, 1024, 4096, 1024, 1616), (75, 1024, 208, 1028, 211, 1632), (130, 384, 208, 388, 211, 1664)])
def test_exact_staged_rows_match_register_path(monkeypatch, M, K, N, lda, ldc, tile):
    """gemm_xf's two ways of bringing the fp32 rows to the matrix cores (staged through LDS by direct loads where
    K % 128 == 0 and the rows allow 16-byte loads; into registers otherwise, P2H_XF_STAGED=0) run the same MFMAs in
    the same order: the outputs are equal bit for bit, with beta = 0, 1 and 0.3, strided A and C, a last row tile cut
    short, and every tile (32 rows of 32 or 64 columns, 16 rows of 16, 32 or 64); and within 1e-4 of the oracle's
    exact route."""
    print(f"exact staged M={M} K={K} N={N} lda={lda} ldc={ldc} tile={tile}", flush=True)
    signs, flags, lo, hi = _weight(K, N, 930 + K + N)
    w = P.FvWeight(signs, flags, lo, hi, K, N)
    A = np.full((M, lda), np.nan, np.float32)   # columns past K are never read
    A[:, :K] = P.gen_activations(SEED, 950 + M, M, K)
    if tile:
        monkeypatch.setenv("P2H_XF_TILE", str(tile))
    C0 = np.random.default_rng(M + N).standard_normal((M, ldc)).astype(np.float32)
    for alpha, beta in [(1.0, 0.0), (0.5, 1.0), (-1.5, 0.3)]:
        got = P.fvb_gemm("exact", A, w, alpha=alpha, beta=beta, C0=C0)
        monkeypatch.setenv("P2H_XF_STAGED", "0")
        try:
            reg = P.fvb_gemm("exact", A, w, alpha=alpha, beta=beta, C0=C0)
        finally:
            monkeypatch.delenv("P2H_XF_STAGED")
        assert _bits_equal(got, reg), f"alpha={alpha} beta={beta}: staged and register paths differ"
        assert _bits_equal(got[:, N:], C0[:, N:])
    rows = np.unique(np.concatenate([[0, M - 1], np.random.default_rng(K).choice(M, min(M, 24), replace=False)]))
    ref = O.sgemm_fvb("exact", A[rows, :K], signs, flags, lo, hi, N, alpha=-1.5, beta=0.3, C0=C0[rows, :N])
    _assert_exact(got[rows, :N], ref)


# ── every tile configuration and K split (the planner's choices forced through its tuning variables) ─────────────

_TILE_CASES = {}


@pytest.mark.parametrize("tile", [0, 1, 2, 3, 4, 8, 9, 10, 11, 12, 13, 14, 15, 16, 17])
@pytest.mark.parametrize("split_rows", [-1, 0, 256, 512, 1024])
@pytest.mark.parametrize("M,K,N", [(375, 4096, 1024), (130, 1028, 272), (38, 1024, 4096), (300, 2048, 512)])
def test_tiles_and_splits_int8w(monkeypatch, tile, split_rows, M, K, N):
    monkeypatch.setenv("P2H_TILE", str(tile))
    monkeypatch.setenv("P2H_SPLIT_ROWS", str(split_rows))
    key = (M, K, N)
    if key not in _TILE_CASES:
        signs, flags, lo, hi = _weight(K, N, 900 + K + N)
        A = P.gen_activations(SEED, 901 + M, M, K)
        q, sc = O.quant_rows(A)
        C0 = P.gen_activations(SEED, 902 + N, M, N)
        ref = O.gemm_i8_run("int8w", q, sc, signs, flags, lo, hi, N, alpha=0.75, C0=C0, beta_zero=False)
        _TILE_CASES[key] = (P.FvWeight(signs, flags, lo, hi, K, N), q, sc, C0, ref)
    w, q, sc, C0, ref = _TILE_CASES[key]
    for rep in range(2):   # twice: a call must not depend on what the previous one left in its workspace
        got = P.fvb_gemm_q8a("int8w", q, sc, w, alpha=0.75, beta=1.0, C0=C0)
        _assert_fp32(got, ref)


@pytest.mark.parametrize("M,K,N,plan", [(9, 4096, 1024, "16x16"), (38, 4096, 1024, "16x16"), (100, 4096, 1024, "16x32"),
                                         (160, 4096, 1024, "32x32"), (250, 4096, 1024, "32x32"),
                                         (320, 4096, 1024, "48x32"), (375, 4096, 1024, "48x32"),
                                         (500, 4096, 1024, "32x64"), (130, 1028, 272, "16x16"),
                                         (9, 1024, 4096, "16x16"), (38, 1024, 1024, "16x16"), (38, 1024, 4096, "32x32"),
                                         (1, 1024, 1024, "16x16"), (17, 256, 48, "16x16"), (100, 1024, 1024, "16x16"),
                                         (38, 1024, 3072, "32x32")])
def test_small_m_plans(M, K, N, plan):
    """The planner's small-M tiles where they fit the CUs in one round: sixteen rows (16 x 16, then 16 x 32 with eight
    waves for K > 1024; 16 x 16 with four waves, two workgroups per CU, for K <= 1024), then for K > 1024 the
    eight-wave 32 x 32 and 48 x 32, then the four- or eight-wave 32 x 64; each bit-exact against the oracle on a
    down- or up-projection's weights."""
    assert P.plan("int8w", M, N, K).startswith(f"tile {plan},")
    signs, flags, lo, hi = _weight(K, N, 960 + M)
    w = P.FvWeight(signs, flags, lo, hi, K, N)
    A = P.gen_activations(SEED, 961 + M, M, K)
    q, sc = O.quant_rows(A)
    C0 = P.gen_activations(SEED, 962 + M, M, N)
    ref = O.gemm_i8_run("int8w", q, sc, signs, flags, lo, hi, N, alpha=-0.5, C0=C0, beta_zero=False)
    _assert_fp32(P.fvb_gemm_q8a("int8w", q, sc, w, alpha=-0.5, beta=1.0, C0=C0), ref)


@pytest.mark.parametrize("tile", [0, 1, 2, 3, 10, 13, 14, 15, 16, 17])
@pytest.mark.parametrize("split_rows", [0, 256, 1024])
def test_tiles_and_splits_int8(monkeypatch, tile, split_rows):
    monkeypatch.setenv("P2H_TILE", str(tile))
    monkeypatch.setenv("P2H_SPLIT_ROWS", str(split_rows))
    M, K, N = 200, 2052, 144
    signs, flags, lo, hi = _weight(K, N, 950)
    w = P.FvWeight(signs, flags, lo, hi, K, N)
    A = P.gen_activations(SEED, 951, M, K)
    q, sc = O.quant_rows(A)
    ref = O.gemm_i8_run("int8", q, sc, signs, flags, lo, hi, N)
    _assert_fp32(P.fvb_gemm_q8a("int8", q, sc, w), ref)
    _assert_fp32(P.fvb_gemm_q8a("int8", q, sc, w, split=False), ref)


def test_one_workspace_across_shapes():
    """A workspace reused by calls of different shapes, split and unsplit in turn: no call may depend on what an
    earlier call left in it."""
    shapes = [(38, 4096, 1024), (9, 256, 32), (375, 1024, 1024), (38, 1024, 4096), (9, 256, 32)]
    need = max(P.q8a_workspace_bytes("int8w", M, N, K) for M, K, N in shapes)
    ws = P.Workspace(need)
    for i, (M, K, N) in enumerate(shapes):
        signs, flags, lo, hi = _weight(K, N, 960 + i)
        w = P.FvWeight(signs, flags, lo, hi, K, N)
        A = P.gen_activations(SEED, 970 + i, M, K)
        q, sc = O.quant_rows(A)
        ref = O.gemm_i8_run("int8w", q, sc, signs, flags, lo, hi, N)
        _assert_fp32(P.fvb_gemm_q8a("int8w", q, sc, w, ws=ws), ref)


@pytest.mark.parametrize("mode", ["int8w", "int8"])
def test_one_fp32_workspace_across_shapes(mode):
    """The fp32-input entry with one workspace for calls of different M, K and N, split and unsplit in turn (the
    blas.h drop-in reuses its per-thread workspace exactly like this)."""
    shapes = [(375, 1024, 1024), (38, 4096, 1024), (9, 256, 32), (2000, 1024, 2048), (38, 1024, 1024),
              (9, 256, 32)]
    ws = P.Workspace(max(P.workspace_bytes(mode, M, N, K) for M, K, N in shapes))
    for i, (M, K, N) in enumerate(shapes):
        signs, flags, lo, hi = _weight(K, N, 980 + i)
        w = P.FvWeight(signs, flags, lo, hi, K, N)
        A = P.gen_activations(SEED, 990 + i, M, K)
        rows = np.arange(M) if M <= 400 else np.random.default_rng(i).choice(M, 64, replace=False)
        got = P.fvb_gemm(mode, A, w, ws=ws)
        _assert_fp32(got[rows], O.sgemm_fvb(mode, A[rows], signs, flags, lo, hi, N))
