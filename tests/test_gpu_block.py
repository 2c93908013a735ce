"""The conformer block on the GPU (encoder.c:252-625): its pieces between the linears through the C ABI against the
oracle, and one whole block (p2h_conformer_block) against the reference engine's own conformer_block built from its
sources (oracle/_ref/libp2refblock*.so), on the seeded synthetic block of p2gemm.block_params.

Pieces. Index moves (head gather, transposes, concatenation), the residual fmadd, the depthwise convolution with its
SiLU, and the LayerNorm rows are bit-exact with the oracle: every operation is rounded once in the source's order on
both sides. The softmax and the GLU call expf (the softmax for its last T mod 8 elements, the GLU everywhere); the
device's expf and the host's libm may differ in the last place, so those are held to 4 ulp, and rows of the softmax
without a tail (T % 8 == 0) are bit-exact.

Whole block. int8w and int8: the reference block runs with the oracle's GEMMs (the reference's x86 blas.c has only
the exact route, blas.c:1043-1045), which the device's GEMMs equal bit for bit on the same quantised rows. Between
them the block's fp32 pieces may differ in the last bits (the reference's -ffast-math build divides through
approximate reciprocals and reassociates the convolution's scalar edges; its heads' fp32 GEMMs sum in another
order than the matrix cores), and a last-bit difference moves a quantisation code wherever a value sits on a
rounding boundary; the steps after it carry the moved code on. The reference block itself, run on its input with
every element moved one ulp, moves by 3.3e-3 (relative L2) at T = 375 on this block; the int8 and int8w blocks
differ by 6e-3. So the whole quantised block is held to 1e-2 over the block and 2e-2 per frame, which catches
wiring mistakes but not last-bit ones, and each step is also tested alone (test_block_step_against_reference):
the other three steps' residual linears get all-zero weights, so both sides compute LayerNorm(x + step(x)) from the
same x and a moved code stays a local effect. There the step's contribution agrees with the reference's to fp32
rounding on most frames (median per frame at most 1e-4 of its size; measured 3e-7 to 2e-5), and on the frames where
a code moved (one code of a 1024-element row is about 1e-3 of the row) within 1e-2.
exact: the reference block with the reference's own blas.c, no quantisation: at most 2e-5 per frame, which holds
every piece of the attention and convolution modules to fp32 rounding.
"""
import os
import subprocess
import sys

import numpy as np
import pytest

import _oracle as O
import p2gemm as P

pytestmark = pytest.mark.gpu

SEED = 20261202
HERE = os.path.dirname(os.path.abspath(__file__))
CHILD = os.path.join(HERE, "refblock_child.py")
H, Dh, D = 8, 128, 1024


@pytest.fixture(scope="module", autouse=True)
def device():
    name = P.init()
    assert name.startswith("gfx950"), name
    return name


def _ulps(a, b):
    a, b = np.asarray(a, np.float32), np.asarray(b, np.float32)
    spacing = np.spacing(np.abs(b)).astype(np.float64)
    return np.abs(a.astype(np.float64) - b.astype(np.float64)) / np.maximum(spacing, np.finfo(np.float32).tiny)


@pytest.mark.parametrize("T", [375, 17, 1])
def test_gather_and_transposes(T):
    print(f"gather/transpose T={T}", flush=True)
    rng = np.random.default_rng(SEED + T)
    qkv = rng.standard_normal((T, 3 * D)).astype(np.float32)
    bu, bv = (rng.standard_normal(D) * 0.1).astype(np.float32), (rng.standard_normal(D) * 0.1).astype(np.float32)
    qu, qv, kt, vh = P.gather_heads(qkv, bu, bv)
    q, k, v = (qkv[:, i * D:(i + 1) * D].reshape(T, H, Dh) for i in range(3))
    assert np.array_equal(qu, (q + bu.reshape(H, Dh)).transpose(1, 0, 2))
    assert np.array_equal(qv, (q + bv.reshape(H, Dh)).transpose(1, 0, 2))
    assert np.array_equal(kt, k.transpose(1, 2, 0))
    assert np.array_equal(vh, v.transpose(1, 0, 2))
    L = 2 * T - 1
    Pm = rng.standard_normal((L, D)).astype(np.float32)
    assert np.array_equal(P.transpose_pos(Pm), Pm.reshape(L, H, Dh).transpose(1, 2, 0))
    attn_h = rng.standard_normal((H, T, Dh)).astype(np.float32)
    assert np.array_equal(P.concat_heads_rows(attn_h), attn_h.transpose(1, 0, 2).reshape(T, D))
    dw = rng.standard_normal((D, T)).astype(np.float32)
    assert np.array_equal(P.channel_major_rows(dw), dw.T)


@pytest.mark.parametrize("T", [376, 375, 9, 5, 1, 700, 1030, 2100])
def test_combine_softmax(T):
    """One wave per row up to T = 2048 (the row in registers, 6, 12 or 32 values per lane), eight threads per row
    beyond; the same bits either way."""
    print(f"combine_softmax T={T}", flush=True)
    rng = np.random.default_rng(SEED + 7 * T)
    ac = (rng.standard_normal((H * T, T)) * 3).astype(np.float32)
    bd = (rng.standard_normal((H * T, 2 * T - 1)) * 3).astype(np.float32)
    ac[0, :] = -200.0   # a row far below zero: exp of (a − max) still sums from 1
    got, ref = P.combine_softmax(ac, bd), O.combine_softmax(ac, bd)
    if T % 8 == 0:
        assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))
    else:
        assert _ulps(got, ref).max() <= 4


def _attention_reference(qkv, bu, bv, pos):
    """encoder.c:495-523 on the CPU: float64 score and output products (rounded to float32 where the reference
    stores them), the oracle's combine_softmax (the reference's order) in between."""
    T = qkv.shape[0]
    q, k, v = (qkv[:, i * D:(i + 1) * D].reshape(T, H, Dh).transpose(1, 0, 2) for i in range(3))
    qu = (q + bu.reshape(H, 1, Dh)).astype(np.float32)
    qv = (q + bv.reshape(H, 1, Dh)).astype(np.float32)
    Ph = pos.reshape(2 * T - 1, H, Dh).transpose(1, 0, 2)
    ac = np.matmul(qu.astype(np.float64), k.transpose(0, 2, 1).astype(np.float64)).astype(np.float32)
    bd = np.matmul(qv.astype(np.float64), Ph.transpose(0, 2, 1).astype(np.float64)).astype(np.float32)
    p = O.combine_softmax(ac.reshape(H * T, T), bd.reshape(H * T, 2 * T - 1)).reshape(H, T, T)
    return np.matmul(p.astype(np.float64), v.astype(np.float64))


@pytest.mark.parametrize("T,gain", [(375, 1.0), (375, 3.0), (1, 1.0), (17, 1.0), (100, 2.0), (384, 1.0), (385, 1.0),
                                    (700, 1.0)])
def test_attention_heads(T, gain):
    """p2h_attention_heads (one kernel: scores, relative shift, softmax, product with V) against float64 products
    around the oracle's softmax: the kernel's products are fp32 matrix-core sums, so per output row (128 values) the
    relative L2 difference is at most 2e-5 (gain 3 makes the softmax peaked: scores up to ~±40)."""
    print(f"attention_heads T={T} gain={gain}", flush=True)
    rng = np.random.default_rng(SEED + 17 * T)
    qkv = (rng.standard_normal((T, 3 * D)) * gain).astype(np.float32)
    bu, bv = (rng.standard_normal(D) * 0.1).astype(np.float32), (rng.standard_normal(D) * 0.1).astype(np.float32)
    pos = rng.standard_normal((2 * T - 1, D)).astype(np.float32)
    got = P.attention_heads(qkv, bu, bv, pos)
    ref = _attention_reference(qkv, bu, bv, pos)
    d = np.linalg.norm(got - ref, axis=2) / np.linalg.norm(ref, axis=2)
    print(f"  per-row relative L2: max {d.max():.3g}, median {np.median(d):.3g}", flush=True)
    assert np.isfinite(got).all()
    assert d.max() <= 2e-5


@pytest.mark.parametrize("T", [375, 17, 385])
def test_attention_rows(T):
    """p2h_attention_rows is p2h_attention_heads' output concatenated by head (concat_heads' rows), bit for bit, and
    its rows quantised by the plain quantiser equal the concatenation→int8 producer's codes and scales."""
    print(f"attention_rows T={T}", flush=True)
    rng = np.random.default_rng(SEED + 29 * T)
    qkv = rng.standard_normal((T, 3 * D)).astype(np.float32)
    bu, bv = (rng.standard_normal(D) * 0.1).astype(np.float32), (rng.standard_normal(D) * 0.1).astype(np.float32)
    pos = rng.standard_normal((2 * T - 1, D)).astype(np.float32)
    heads = P.attention_heads(qkv, bu, bv, pos)
    rows = P.attention_heads(qkv, bu, bv, pos, rows=True)
    cat = np.ascontiguousarray(heads.transpose(1, 0, 2).reshape(T, D))
    assert np.array_equal(rows.view(np.uint32), cat.view(np.uint32))
    q1, s1 = P.quant_rows(rows)
    q2, s2 = P.concat_heads_quant_rows(heads)
    assert np.array_equal(q1, q2)
    assert np.array_equal(s1.view(np.uint32), s2.view(np.uint32))


@pytest.mark.parametrize("M", [375, 3000, 1])
@pytest.mark.parametrize("in_place", [False, True])
def test_layer_norm2_quant_rows(M, in_place):
    """Two LayerNorms in one kernel equal p2h_layer_norm_rows followed by p2h_layer_norm_quant_rows, bit for bit:
    the fp32 rows of the first and the codes and scales of the second (375 rows: sums from registers; 3000: from
    LDS batches)."""
    print(f"layer_norm2_quant_rows M={M} in_place={in_place}", flush=True)
    rng = np.random.default_rng(SEED + 31 * M)
    x = (rng.standard_normal((M, D)) * 3 + 0.5).astype(np.float32)
    g1, g2 = (rng.uniform(0.5, 1.5, D).astype(np.float32) for _ in range(2))
    b1, b2 = ((rng.uniform(-0.2, 0.2, D)).astype(np.float32) for _ in range(2))
    y, q, s = P.layer_norm2_quant_rows(x, g1, b1, g2, b2, in_place=in_place)
    y_ref = P.layer_norm_rows(x, g1, b1)
    q_ref, s_ref = P.layer_norm_quant_rows(y_ref, g2, b2)
    assert np.array_equal(y.view(np.uint32), y_ref.view(np.uint32))
    assert np.array_equal(q, q_ref)
    assert np.array_equal(s.view(np.uint32), s_ref.view(np.uint32))


@pytest.mark.parametrize("T", [375, 7])
def test_glu_channel_major(T):
    print(f"glu T={T}", flush=True)
    rng = np.random.default_rng(SEED + 11 * T)
    pw1 = (rng.standard_normal((T, 2 * D)) * 2).astype(np.float32)
    pw1[0, D:D + 4] = [-100.0, 100.0, -87.5, 88.0]
    assert _ulps(P.glu_channel_major(pw1), O.glu_channel_major(pw1)).max() <= 4


@pytest.mark.parametrize("T", [375, 300, 9, 4, 1])
def test_depthwise_conv_silu(T):
    print(f"depthwise_conv_silu T={T}", flush=True)
    rng = np.random.default_rng(SEED + 13 * T)
    x = rng.standard_normal((D, T)).astype(np.float32)
    w = (rng.standard_normal((D, 9)) * 0.3).astype(np.float32)
    b = (rng.standard_normal(D) * 0.1).astype(np.float32)
    got = P.depthwise_conv_silu(x, w, b)
    assert np.array_equal(got.view(np.uint32), O.dwconv_silu(x, w, b).view(np.uint32))


@pytest.mark.parametrize("T", [375, 300, 9, 4, 1, 33])
def test_glu_depthwise_conv_silu_fused(T):
    """The fused kernel equals the GLU kernel followed by the convolution kernel, bit for bit."""
    print(f"glu_depthwise_conv_silu T={T}", flush=True)
    rng = np.random.default_rng(SEED + 19 * T)
    pw1 = (rng.standard_normal((T, 2 * D)) * 2).astype(np.float32)
    pw1[0, D:D + 4] = [-100.0, 100.0, -87.5, 88.0]
    w = (rng.standard_normal((D, 9)) * 0.3).astype(np.float32)
    b = (rng.standard_normal(D) * 0.1).astype(np.float32)
    got = P.glu_depthwise_conv_silu(pw1, w, b)
    two = P.depthwise_conv_silu(P.glu_channel_major(pw1), w, b)
    assert np.array_equal(got.view(np.uint32), two.view(np.uint32))


@pytest.mark.parametrize("tt", ["1", "2", "4", "8"])
@pytest.mark.parametrize("T,ldq", [(375, 1024), (1, 1024), (4, 1024), (9, 1152), (17, 1024), (300, 1024),
                                   (760, 1152)])
def test_glu_depthwise_conv_silu_quant_rows(monkeypatch, tt, T, ldq):
    """The int8 modes' convolution kernel (GLU, convolution, SiLU and the rows' quantisation in one pass), at every
    frames-per-workgroup setting (P2H_CONV_TT), equals the rows kernel followed by the plain quantiser bit for bit:
    codes, scales, zero pad rows up to the next multiple of 16 and zero columns beyond 1024; with the GLU's clamp
    values and a zero frame."""
    monkeypatch.setenv("P2H_CONV_TT", tt)
    print(f"glu_depthwise_conv_silu_quant_rows T={T} ldq={ldq} frames per workgroup {tt}", flush=True)
    rng = np.random.default_rng(SEED + 29 * T)
    pw1 = (rng.standard_normal((T, 2 * D)) * 2).astype(np.float32)
    pw1[0, D:D + 4] = [-100.0, 100.0, -87.5, 88.0]
    if T > 3:
        pw1[2] = 0.0
    w = (rng.standard_normal((D, 9)) * 0.3).astype(np.float32)
    b = (rng.standard_normal(D) * 0.1).astype(np.float32)
    q, s = P.glu_depthwise_conv_silu_quant_rows(pw1, w, b, ldq)
    q_ref, s_ref = P.quant_rows(P.glu_depthwise_conv_silu(pw1, w, b, rows=True))
    Mp = (T + 15) // 16 * 16
    assert q.shape == (Mp, ldq)
    assert np.array_equal(s.view(np.uint32), s_ref.view(np.uint32))
    assert np.array_equal(q[:, :D], q_ref[:, :D])
    assert not q[:, D:].any() and not q[T:].any()


@pytest.mark.parametrize("mode", ["int8w", "int8"])
def test_conv_quant_same_bits(monkeypatch, mode):
    """The block with the convolution's rows quantised in the convolution kernel equals the block with the rows
    kernel and the plain quantiser (P2H_CONV_QUANT=0) bit for bit."""
    print(f"conv quant mode={mode}", flush=True)
    sys.path.insert(0, HERE)
    import refblock_child as RC
    x, pe = RC.block_input(SEED, 375)
    blk = _device_block(SEED)
    fused = blk.run(mode, x, pe)
    monkeypatch.setenv("P2H_CONV_QUANT", "0")
    separate = blk.run(mode, x, pe)
    assert np.isfinite(fused).all()
    assert np.array_equal(fused.view(np.uint32), separate.view(np.uint32))


@pytest.mark.parametrize("T", [375, 33, 32, 31, 1])
def test_glu_depthwise_conv_silu_rows(T):
    """The row-major variant is the transpose of the channel-major output bit for bit, and its rows quantised by
    the plain quantiser equal the channel-major→int8 producer's codes and scales (the block's int8 route)."""
    print(f"glu_depthwise_conv_silu_rows T={T}", flush=True)
    rng = np.random.default_rng(SEED + 23 * T)
    pw1 = (rng.standard_normal((T, 2 * D)) * 2).astype(np.float32)
    w = (rng.standard_normal((D, 9)) * 0.3).astype(np.float32)
    b = (rng.standard_normal(D) * 0.1).astype(np.float32)
    cm = P.glu_depthwise_conv_silu(pw1, w, b)
    rows = P.glu_depthwise_conv_silu(pw1, w, b, rows=True)
    assert rows.shape == (T, D)
    assert np.array_equal(rows.view(np.uint32), np.ascontiguousarray(cm.T).view(np.uint32))
    q1, s1 = P.quant_rows(rows)
    q2, s2 = P.channel_major_quant_rows(cm)
    assert np.array_equal(q1, q2)
    assert np.array_equal(s1.view(np.uint32), s2.view(np.uint32))


@pytest.mark.parametrize("n", [375 * 4096, 1001])
def test_silu_flat(n):
    """The eight-wide body bit-exact; the tail (n mod 8 elements, expf) within 4 ulp."""
    print(f"silu n={n}", flush=True)
    rng = np.random.default_rng(SEED + n)
    x = (rng.standard_normal(n) * 4).astype(np.float32)
    x[:6] = [0.0, 100.0, -100.0, 87.0, -87.5, 30.0]
    x[-3:] = [-100.0, 0.5, -2.0]
    got = P.silu(x)
    ref = x.copy()
    O.lib().p2o_swish_row(ref, n)
    body = n // 8 * 8
    assert np.array_equal(got[:body].view(np.uint32), ref[:body].view(np.uint32))
    assert body == n or _ulps(got[body:], ref[body:]).max() <= 4


def test_add_residual():
    rng = np.random.default_rng(SEED + 5)
    X, Y = (rng.standard_normal((37, D)).astype(np.float32) for _ in range(2))
    ref = (Y.astype(np.float64) * 0.5 + X.astype(np.float64)).astype(np.float32)
    assert np.array_equal(P.add_residual(X, Y, 0.5), ref)


@pytest.mark.parametrize("M", [375, 6000, 3])
def test_layer_norm_rows(M):
    print(f"layer_norm_rows M={M}", flush=True)
    rng = np.random.default_rng(SEED + M)
    X = (rng.standard_normal((M, D)) * 1.7 + 0.3).astype(np.float32)
    g = rng.uniform(0.5, 1.5, D).astype(np.float32)
    b = rng.uniform(-0.2, 0.2, D).astype(np.float32)
    ref = O.layer_norm_rows(X, g, b)
    assert np.array_equal(P.layer_norm_rows(X, g, b).view(np.uint32), ref.view(np.uint32))
    assert np.array_equal(P.layer_norm_rows(X, g, b, in_place=True).view(np.uint32), ref.view(np.uint32))


# ── the whole block ───────────────────────────────────────────────────────────────────────────────────────────

_BLOCK = {}


def _device_block(seed):
    if seed not in _BLOCK:
        _BLOCK.clear()
        sys.path.insert(0, HERE)
        _BLOCK[seed] = P.Block(P.block_params(seed, 100))
    return _BLOCK[seed]


def _reference_block(mode, seed, T, tmp_path, stage=None):
    """The reference's conformer_block in a child process (the GEMM mode is latched once per process)."""
    out = tmp_path / f"ref_{mode}_{seed}_{T}_{stage}.npy"
    env = dict(os.environ)
    env["P2_GEMM"] = mode
    env.pop("P2_EXACT", None)
    gemms = "reference" if mode == "exact" else "oracle"
    args = [sys.executable, CHILD, str(seed), str(T), str(out), gemms] + ([] if stage is None else [str(stage)])
    r = subprocess.run(args, env=env, capture_output=True, text=True, timeout=300)
    assert r.returncode == 0, r.stdout + r.stderr
    return np.load(out)


def _distance(a, ref):
    d = (a - ref).astype(np.float64)
    r64 = ref.astype(np.float64)
    return np.linalg.norm(d, axis=1) / np.linalg.norm(r64, axis=1), np.linalg.norm(d) / np.linalg.norm(r64)


@pytest.mark.skipif(not O.refblock_available(), reason="reference block library not built")
@pytest.mark.parametrize("mode,T", [("int8w", 375), ("int8", 375), ("exact", 375), ("int8w", 40), ("exact", 9),
                                    ("int8", 1), ("int8w", 500), ("exact", 520), ("int8w", 800)])
def test_block_against_reference(mode, T, tmp_path):
    """The device block against the reference engine's conformer_block (built from its sources) at T where the
    attention runs in each of its forms: T <= 384 the fused kernel with its tiles in LDS, 385..768 the fused kernel
    with its tiles in registers, beyond the separate products and softmax."""
    print(f"conformer block mode={mode} T={T}", flush=True)
    sys.path.insert(0, HERE)
    import refblock_child as RC
    ref = _reference_block(mode, SEED, T, tmp_path)
    x, pe = RC.block_input(SEED, T)
    got = _device_block(SEED).run(mode, x, pe)
    assert np.isfinite(got).all()
    row_rel, total_rel = _distance(got, ref)
    print(f"  per-frame max {row_rel.max():.3g}, block {total_rel:.3g}", flush=True)
    if mode == "exact":
        assert row_rel.max() <= 2e-5
    else:   # measured on MI355X: per frame at most 5.8e-3, over the block 2.9e-3 to 3.4e-3 (T = 375, 500, 800)
        assert row_rel.max() <= 8e-3 and total_rel <= 5e-3


@pytest.mark.skipif(not O.refblock_available(), reason="reference block library not built")
@pytest.mark.parametrize("mode", ["int8w", "int8"])
@pytest.mark.parametrize("stage", [0, 1, 2, 3])
def test_block_step_against_reference(mode, stage, tmp_path):
    """One step of the block alone (the others' residual linears zero): the device's step contribution
    LayerNorm⁻¹-free form — the block output minus LayerNorm(x) — against the reference's, per frame."""
    print(f"conformer block step {stage} mode={mode} T=375", flush=True)
    sys.path.insert(0, HERE)
    import refblock_child as RC
    T = 375
    ref = _reference_block(mode, SEED, T, tmp_path, stage)
    x, pe = RC.block_input(SEED, T)
    params = RC.isolated_params(P.block_params(SEED, RC.BLOCK_TID0), stage)
    got = P.Block(params).run(mode, x, pe)
    base = O.layer_norm_rows(x, params["norm_out_w"], params["norm_out_b"])   # the block with the step removed
    contrib = (ref - base).astype(np.float64)
    d = (got - ref).astype(np.float64)
    rel = np.linalg.norm(d, axis=1) / np.linalg.norm(contrib, axis=1)
    print(f"  step contribution / output {np.linalg.norm(contrib) / np.linalg.norm(ref):.3g}; device vs reference "
          f"per frame max {rel.max():.3g} median {np.median(rel):.3g} of the contribution", flush=True)
    print(f"  percentiles 90 / 99: {np.percentile(rel, 90):.3g} / {np.percentile(rel, 99):.3g}", flush=True)
    assert np.linalg.norm(contrib) > 1e-2 * np.linalg.norm(ref)   # the step does contribute
    # measured on MI355X (both int8 modes): the median frame within 1.6e-5 of the contribution on every step; the
    # 99th percentile 1.8e-3 on step 1 (where a moved code propagates through the convolution) and at most 2.2e-6
    # on the others; the worst frame 3.0e-3, 1.7e-3 on step 2, 1.6e-6 on step 3
    p99_bound, max_bound = {0: (1e-5, 2e-3), 1: (3e-3, 5e-3), 2: (1e-5, 3e-3), 3: (1e-5, 1e-4)}[stage]
    assert np.median(rel) <= 5e-5
    assert np.percentile(rel, 99) <= p99_bound and rel.max() <= max_bound


@pytest.mark.parametrize("T", [375, 520])
def test_exact_epilogues_same_bits(monkeypatch, T):
    """Exact mode adds its three residuals (x = fmaf(y, α, x) over the linear's output y) in the matrix-core GEMM's
    epilogue, fmaf(α, sum, x) with β = 1, and applies the feed-forward's SiLU there; the block equals the one with
    the separate passes (P2H_EXACT_EPILOGUE=0) bit for bit."""
    print(f"exact residual epilogue T={T}", flush=True)
    sys.path.insert(0, HERE)
    import refblock_child as RC
    x, pe = RC.block_input(SEED, T)
    blk = _device_block(SEED)
    fused = blk.run("exact", x, pe)
    monkeypatch.setenv("P2H_EXACT_EPILOGUE", "0")
    separate = blk.run("exact", x, pe)
    assert np.isfinite(fused).all()
    assert np.array_equal(fused.view(np.uint32), separate.view(np.uint32))


@pytest.mark.parametrize("mode,T", [("int8w", 375), ("int8", 375), ("int8w", 40)])
def test_silu_epilogue_same_bits(monkeypatch, mode, T):
    """The int8 modes apply the feed-forward's SiLU in the up-projection's epilogue and quantise its rows with the
    plain quantiser; the block equals the one with the SiLU→int8 producer after a plain GEMM (P2H_SILU_EPILOGUE=0,
    p2_swish_quant_rows' order, tensor_ops.c:491-511) bit for bit."""
    print(f"SiLU epilogue mode={mode} T={T}", flush=True)
    sys.path.insert(0, HERE)
    import refblock_child as RC
    x, pe = RC.block_input(SEED, T)
    blk = _device_block(SEED)
    fused = blk.run(mode, x, pe)
    monkeypatch.setenv("P2H_SILU_EPILOGUE", "0")
    separate = blk.run(mode, x, pe)
    assert np.isfinite(fused).all()
    assert np.array_equal(fused.view(np.uint32), separate.view(np.uint32))


@pytest.mark.parametrize("mode", ["int8w", "int8", "exact"])
def test_stack_equals_blocks_one_by_one(mode):
    """p2h_conformer_stack over three distinct blocks equals p2h_conformer_block called block after block, bit for
    bit (in the int8 modes the stack quantises the positional rows once and projects them for all blocks in a
    grouped launch; the products are the same)."""
    print(f"conformer stack of 3 blocks, mode={mode}, T=375", flush=True)
    sys.path.insert(0, HERE)
    import refblock_child as RC
    T = 375
    blocks = [P.Block(P.block_params(SEED, 200 + 20 * b)) for b in range(3)]
    x, pe = RC.block_input(SEED, T)
    one_by_one = x
    for b in blocks:
        one_by_one = b.run(mode, one_by_one, pe)
    stacked = P.Stack(blocks).run(mode, x, pe)
    assert np.isfinite(stacked).all()
    assert np.array_equal(stacked.view(np.uint32), one_by_one.view(np.uint32))
