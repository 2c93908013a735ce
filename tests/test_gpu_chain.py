"""The 216-linear encoder sweep that bench.py times, checked as a chain against the oracle.

bench.py's Chain runs one 30 s window's five-value linears (24 blocks × 9 at their real shapes, encoder.c:333-613)
the way the timed step does: each linear quantises its input rows and runs the q8a GEMM that reads the next weight's
records ahead, the 24 positional projections are one quantisation and one grouped launch, and the whole window is
replayed from one HIP graph. Every linear's output is compared with the oracle's p2_sgemm_fvb (int8w: quantise, then
the int8 GEMM, blas.c:1404-1428) on sampled rows, fed layer to layer from the oracle's own outputs: bit for bit.
Rows are independent through the chain (every step is row-wise), so a row sample checks the whole chain exactly.
"""
import os
import sys

import numpy as np
import pytest

import _oracle as O
import p2gemm as P

sys.path.insert(0, os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
import bench  # noqa: E402

pytestmark = pytest.mark.gpu


def _oracle_chain(spec, linears, rows, pos_rows):
    """Each linear's output rows through the oracle, inputs taken from the oracle's earlier outputs."""
    seed = bench.SEED
    outs = []
    for (tid, K, N, M, src), lin in zip(spec, linears):
        signs, flags, lo, hi = P.gen_fv_weight(seed, tid, K, N)
        if src in ("x", "pos"):
            A = P.gen_activations(seed, 10_000 + K + M, M, K)[pos_rows if src == "pos" else rows]
        else:
            A = outs[src]
        alpha = 1.0 if src == "pos" else lin.alpha
        outs.append(O.sgemm_fvb("int8w", A, signs, flags, lo, hi, N, alpha=alpha))
    return outs


@pytest.mark.parametrize("blocks", [2, 24])
def test_sweep_chain_matches_oracle(blocks):
    assert P.init().startswith("gfx950")
    T = 375
    spec = bench.sweep_spec(T)[: 9 * blocks]
    stream = P.Stream()
    print(f"sweep chain: {blocks} blocks, {len(spec)} linears", flush=True)
    ch = bench.Chain(spec)
    graphs = bench.StepGraphs(stream, lambda: ch.body(stream), 1, 1)
    for _ in range(2):   # the second replay's first loads find the records the first read ahead
        graphs.full.launch()
    stream.sync()
    rng = np.random.default_rng(blocks)
    rows = np.unique(np.concatenate([[0, T - 1], rng.choice(T, 6, replace=False)]))
    pos_rows = np.unique(np.concatenate([[0, 2 * T - 2], rng.choice(2 * T - 1, 4, replace=False)]))
    want = _oracle_chain(spec, ch.linears, rows, pos_rows)
    for i, ((tid, K, N, M, src), lin) in enumerate(zip(spec, ch.linears)):
        got = lin.out.download((M, N), np.float32)[pos_rows if src == "pos" else rows]
        neq = got.view(np.uint32) != want[i].view(np.uint32)
        assert not neq.any(), f"linear {i} (block {i // 9}, {K}->{N}, input {src}): {neq.sum()} outputs differ"


def _assert_exact(got, ref):
    """The exact-mode bar: within 1e-4 of the reference's exact route, elementwise relative to max(|ref|, row rms)."""
    rms = np.sqrt(np.mean(ref.astype(np.float64) ** 2, axis=1, keepdims=True))
    tol = 1e-4 * np.maximum(np.abs(ref), rms)
    bad = np.abs(got.astype(np.float64) - ref) > tol
    assert not bad.any(), f"{bad.sum()} of {bad.size} outside 1e-4 relative; first at {np.argwhere(bad)[0]}"


@pytest.mark.parametrize("blocks", [2, 24])
def test_exact_sweep_chain(monkeypatch, blocks):
    """The exact-mode sweep bench.py times (ExactChain: 9 linears per block at their real shapes, one graph per
    window), on sampled rows. The fp32 matrix-core route: every linear within 1e-4 of the oracle's exact route
    (blas.c:929-987) applied to the same input rows the device read (the chain's own earlier outputs), so each
    linear is held to the bar without the earlier linears' rounding compounding. The fmaf-chain route
    (P2H_EXACT_CHAIN=1 at capture): bit for bit the oracle's exact chain fed from its own outputs, every linear."""
    assert P.init().startswith("gfx950")
    T = 375
    spec = bench.sweep_spec(T)[: 9 * blocks]
    seed = bench.SEED
    rng = np.random.default_rng(100 + blocks)
    rows = np.unique(np.concatenate([[0, T - 1], rng.choice(T, 6, replace=False)]))
    pos_rows = np.unique(np.concatenate([[0, 2 * T - 2], rng.choice(2 * T - 1, 4, replace=False)]))
    stream = P.Stream()
    print(f"exact sweep chain: {blocks} blocks, {len(spec)} linears, matrix-core route", flush=True)
    ch = bench.ExactChain(spec)
    graphs = bench.StepGraphs(stream, lambda: ch.body(stream), 1, 1)
    graphs.full.launch()
    stream.sync()
    outs = [lin.out.download((lin.M, lin.N), np.float32) for lin in ch.linears]
    weights = [P.gen_fv_weight(seed, sp[0], sp[1], sp[2]) for sp in spec]
    fresh = {}
    for i, ((tid, K, N, M, src), lin) in enumerate(zip(spec, ch.linears)):
        r = pos_rows if src == "pos" else rows
        if src in ("x", "pos"):
            fresh.setdefault((M, K), P.gen_activations(seed, 10_000 + K + M, M, K))
            A = fresh[(M, K)][r]
        else:
            A = outs[src][r]
        ref = O.sgemm_fvb("exact", A, *weights[i], N, alpha=lin.alpha)
        try:
            _assert_exact(outs[i][r], ref)
        except AssertionError as e:
            raise AssertionError(f"linear {i} (block {i // 9}, {K}->{N}, input {src}): {e}") from None

    print(f"exact sweep chain: {blocks} blocks, fmaf-chain route", flush=True)
    monkeypatch.setenv("P2H_EXACT_CHAIN", "1")
    P.reload_switches()
    try:
        ch2 = bench.ExactChain(spec)
        graphs2 = bench.StepGraphs(stream, lambda: ch2.body(stream), 1, 1)
    finally:
        monkeypatch.delenv("P2H_EXACT_CHAIN")
        P.reload_switches()
    graphs2.full.launch()
    stream.sync()
    want = []
    for i, ((tid, K, N, M, src), lin) in enumerate(zip(spec, ch2.linears)):
        r = pos_rows if src == "pos" else rows
        A = fresh[(M, K)][r] if src in ("x", "pos") else want[src]
        want.append(O.sgemm_fvb("exact", A, *weights[i], N, alpha=lin.alpha))
        got = lin.out.download((M, N), np.float32)[r]
        neq = got.view(np.uint32) != want[i].view(np.uint32)
        assert not neq.any(), f"linear {i} (block {i // 9}, {K}->{N}, input {src}): {neq.sum()} outputs differ"
