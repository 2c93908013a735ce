#!/usr/bin/env python3
"""Throughput of the five-value int8 GEMM on one MI355X.

    python bench.py [--steps K] [--warmup W] [--workload gemm6000|ffn375|m6000|m38|sweep] [--no-cpu-baseline]

Default workload (`gemm6000`): the int8w five-value GEMM at M = 6000 (16 stacked 30 s windows), K = 1024, N = 4096,
the shape the metric's TOPS and % of int8 MFMA peak are quoted on. A step is one GEMM launch on rows already
quantised per row (the p2_sgemm_fvb_q8a route: the encoder's producers quantise as they produce, so the quantise
pass is NOT inside the timed step; the fp32-input route, quantise + GEMM, is reported beside it in `roofline`).
Operands are device-resident before the timed region; the steps are launched back to back on one stream.

Prints ONE JSON line. `value` is int8 TOPS (2·M·N·K per GEMM) and `pct_int8_peak` its share of 5.0 POP/s; `roofline`
is the same GEMM step against the roof that binds it by its algorithmic bytes and ops (HBM at this shape: 106.1 MB
take 13.26 µs at 8 TB/s, the ops 10.07 µs at the int8 peak), with the int8 fraction beside it and, as
`roofline.fp32_in_route`, the fp32-input route (quantise + GEMM per call) against its own roof; all measured live
with HIP events on the stream the kernels run on;
`cpu_baseline` is the reference's own p2_sgemm_fvb (built from its C sources into oracle/_ref/) at the same shape
on this host's cores. `sweep_ms_per_30s_window` is the 216-linear encoder sweep of one 30 s window; `extra` carries
the other configurations of the workload set, each measured the same way, and the other CPU baselines.
"""
import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "phonon-2-c_amd"))

import p2gemm as P  # noqa: E402

PEAK_INT8_TOPS = 5000.0     # MI355X dense int8 MFMA, TOPS
PEAK_HBM_GBS = 8000.0       # MI355X HBM3E, GB/s
PEAK_FP32_TFLOPS = 157.3    # MI355X fp32
SEED = 20261201


def gemm_ops(M, N, K):
    return 2.0 * M * N * K


def gemm_bytes(M, N, K, a_bytes_per_elem, beta1=False):
    """Algorithmic HBM bytes of one five-value GEMM: packed planes K·N·3/8, lo/hi 8N, activations, fp32 C."""
    return K * N * 3 / 8 + 8 * N + a_bytes_per_elem * M * K + (4 * M if a_bytes_per_elem == 1 else 0) \
        + 4 * M * N * (2 if beta1 else 1)


def quant_bytes(M, K):
    return 4 * M * K + M * K + 4 * M


class Linear:
    """One device-resident five-value linear [K, N] with its output buffer."""

    def __init__(self, tid, K, N, M):
        signs, flags, lo, hi = P.gen_fv_weight(SEED, tid, K, N)
        self.K, self.N, self.M = K, N, M
        self.w = P.FvWeight(signs, flags, lo, hi, K, N)
        ew2 = float(np.mean(0.4 * lo.astype(np.float64) ** 2 + 0.2 * hi.astype(np.float64) ** 2))
        self.alpha = float(np.float32(1.0 / np.sqrt(K * ew2)))   # keeps a chain of layers at unit variance
        self.out = P.DeviceBuffer(M * N * 4)


class Scratch:
    """Quantised rows, their scales, and the split-K workspace shared by a chain of linears (stream-ordered)."""

    def __init__(self, M, K, split_bytes):
        self.ldq = P.q_ld(K)
        self.q = P.DeviceBuffer(P.q_bytes(M, K))
        self.s = P.DeviceBuffer(M * 4)
        self.ws = P.Workspace(split_bytes)


def run_linear(lin, dA, lda, ws, stream, alpha=None, next_w=None):
    """Quantise A, then the q8a GEMM (which reads the records of next_w, the chain's next weight, ahead)."""
    a = lin.alpha if alpha is None else alpha
    ldq = P.q_ld(lin.K)   # the linear's own row pitch: the shared buffer is sized for the widest
    P.quant_rows_dev(lin.M, lin.K, dA, lda, ws.q.ptr, ldq, ws.s.ptr, stream.ptr)
    P.fvb_gemm_q8a_next_dev("int8w", lin.M, lin.N, lin.K, a, ws.q.ptr, ldq, ws.s.ptr, lin.w, 0.0, lin.out.ptr,
                            lin.N, ws.ws.ptr, ws.ws.nbytes, next_w, stream.ptr)


STEPS_PER_REPLAY = 10   # short chains: steps captured per graph (a window's graph holds all its linears)


class StepGraphs:
    """One step's launches (`body`) captured `per` times into one graph, and `steps % per` times into a second, so
    that timing exactly `steps` steps replays whole graphs. Launching a graph costs about 6.5 us of submission on
    its own (four-kernel FFN step: 30.0 us at one step per replay, 23.5 us at ten, MI355X); a caller that runs a
    window's linears from one graph pays it once per window, not once per linear pair."""

    def __init__(self, stream, body, per, steps):
        self.stream, self.per, self.rest = stream, max(1, per), steps % max(1, per)
        self.full = self._capture(body, self.per)
        self.part = self._capture(body, self.rest) if self.rest else None

    def _capture(self, body, n):
        with P.Graph(self.stream) as g:
            for _ in range(n):
                body()
        return g

    def time(self, steps, warmup):
        for _ in range(-(-warmup // self.per)):
            self.full.launch()
        self.stream.sync()
        e0, e1 = P.Event(), P.Event()
        e0.record(self.stream.ptr)
        t0 = time.perf_counter()
        for _ in range(steps // self.per):
            self.full.launch()
        if self.rest:
            self.part.launch()
        e1.record(self.stream.ptr)
        e1.sync()
        return e0.elapsed_ms(e1) / steps, time.perf_counter() - t0


def time_launches(launch, stream, reps):
    """Average duration (ms) of one kernel launched `reps` times on `stream` behind a stream hold, between two HIP
    events: the hold keeps the GPU busy while the host queues the launches, so they run back to back and the
    figure is the kernel time plus the dispatch gap between consecutive kernels. If the host took longer to queue
    them than the hold lasted, the measurement is repeated with a longer hold."""
    launch()
    stream.sync()
    hold_us = 2000
    for _ in range(4):
        e0, e1 = P.Event(), P.Event()
        stream.hold(hold_us)
        e0.record(stream.ptr)
        t0 = time.perf_counter()
        for _ in range(reps):
            launch()
        host_us = (time.perf_counter() - t0) * 1e6
        e1.record(stream.ptr)
        e1.sync()
        if host_us < 0.8 * hold_us:
            return e0.elapsed_ms(e1) / reps
        hold_us = min(1_000_000, int(2 * host_us) + 1000)
    raise RuntimeError(f"host queued {reps} launches more slowly than a {hold_us} us hold")


def kernel_name(plan):
    return "gemm_fvs" if "waves" in plan else "gemm_fv_rb" if "records in registers" in plan else "gemm_fv"


# ── workloads ──────────────────────────────────────────────────────────────────────────────────────────────────

def build_chain(spec, M_default):
    """spec: list of (tid, K, N, M, input) with input an index into the chain's outputs or 'x' for the fresh
    activation buffer of width K. Returns linears, their input pointers, and the workspace."""
    linears, inputs, fresh = [], [], {}
    for tid, K, N, M, src in spec:
        lin = Linear(tid, K, N, M)
        if src in ("x", "pos"):
            if (M, K) not in fresh:
                fresh[(M, K)] = P.to_device(P.gen_activations(SEED, 10_000 + K + M, M, K))
            inputs.append((fresh[(M, K)].ptr, K))
        else:
            inputs.append((linears[src].out.ptr, linears[src].N))
        linears.append(lin)
    maxm = max(s[3] for s in spec)
    maxk = max(s[1] for s in spec)
    split = max(P.q8a_workspace_bytes("int8w", l.M, l.N, l.K) for l in linears)
    return linears, inputs, Scratch(maxm, maxk, split), fresh


def ffn_spec(M, base=1):
    return [(base, 1024, 4096, M, "x"), (base + 1, 4096, 1024, M, 0)]


def sweep_spec(M=375):
    """24 FastConformer blocks × 9 five-value linears at their real shapes (weights.c:371-379, encoder.c:333-613):
    ff1.l1, ff1.l2, qkv, pos (M = 2T−1), out, pw1, pw2, ff2.l1, ff2.l2. The d = 1024 stream chains through
    ff1 → out → pw2 → ff2; qkv and pw1 read it; pos reads the positional rows, the same for every block
    (encoder.c:500), so the 24 positional projections run as one quantisation and one grouped launch."""
    spec = []
    for b in range(24):
        t = 100 + 16 * b
        i = len(spec)
        prev = "x" if b == 0 else i - 1          # the previous block's ff2.l2 output
        spec += [
            (t + 0, 1024, 4096, M, prev),         # i+0 ff1.linear1
            (t + 1, 4096, 1024, M, i + 0),        # i+1 ff1.linear2
            (t + 2, 1024, 3072, M, i + 1),        # i+2 qkv
            (t + 3, 1024, 1024, 2 * M - 1, "pos"),  # i+3 pos
            (t + 4, 1024, 1024, M, i + 1),        # i+4 out
            (t + 5, 1024, 2048, M, i + 4),        # i+5 pw1
            (t + 6, 1024, 1024, M, i + 4),        # i+6 pw2
            (t + 7, 1024, 4096, M, i + 6),        # i+7 ff2.linear1
            (t + 8, 4096, 1024, M, i + 7),        # i+8 ff2.linear2
        ]
    return spec


class Chain:
    """A chain of five-value linears on one stream, as an encoder window runs them: each linear quantises its input
    rows and runs the q8a GEMM, reading the records of the chain's next weight ahead; the positional projections
    (spec input 'pos'), whose rows are the same for every block (encoder.c:500), are one quantisation and one grouped
    launch at the start. body() queues one pass; it can be captured into a graph. Every linear writes its own output
    buffer (beta 0) from inputs no linear overwrites, so passes are idempotent."""

    def __init__(self, spec):
        self.spec = spec
        self.linears, self.inputs, self.ws, self.keep = build_chain(spec, None)
        self.pos = [i for i, sp in enumerate(spec) if sp[4] == "pos"]
        if self.pos:
            P0 = self.linears[self.pos[0]]
            self.pq = P.DeviceBuffer(P.q_bytes(P0.M, P0.K))
            self.ps = P.DeviceBuffer(4 * P0.M)
        self.order = [i for i in range(len(self.linears)) if i not in self.pos]

    def pos_launch(self, stream):
        P0 = self.linears[self.pos[0]]
        P.fvb_gemm_q8a_grouped_dev("int8w", P0.M, P0.N, P0.K, 1.0, self.pq.ptr, P.q_ld(P0.K), self.ps.ptr,
                                   [self.linears[i].w for i in self.pos], 0.0,
                                   [self.linears[i].out.ptr for i in self.pos], P0.N, stream.ptr)

    def pos_quant(self, stream):
        P0 = self.linears[self.pos[0]]
        dA, lda = self.inputs[self.pos[0]]
        P.quant_rows_dev(P0.M, P0.K, dA, lda, self.pq.ptr, P.q_ld(P0.K), self.ps.ptr, stream.ptr)

    def next_w(self, x):
        return self.linears[self.order[(x + 1) % len(self.order)]].w

    def body(self, stream):
        if self.pos:   # the positional rows quantised once, every block's projection in one launch (alpha 1)
            self.pos_quant(stream)
            self.pos_launch(stream)
        for x, i in enumerate(self.order):   # each GEMM reads the next one's records ahead (the last, the first's)
            run_linear(self.linears[i], *self.inputs[i], self.ws, stream, next_w=self.next_w(x))

    def kernel_times(self, stream, reps):
        """Duration (ms) of each kernel of the chain on its own (time_launches): per linear its quantisation and its
        GEMM as the chain calls it (the positional linears: the one grouped launch, and its quantisation, shared)."""
        n = len(self.linears)
        q, t = np.full(n, np.nan), np.full(n, np.nan)
        ws = self.ws
        for x, i in enumerate(self.order):
            lin, (dA, lda), nxt = self.linears[i], self.inputs[i], self.next_w(x)
            ldq = P.q_ld(lin.K)
            q[i] = time_launches(lambda: P.quant_rows_dev(lin.M, lin.K, dA, lda, ws.q.ptr, ldq, ws.s.ptr, stream.ptr),
                                 stream, reps)
            t[i] = time_launches(lambda: P.fvb_gemm_q8a_next_dev("int8w", lin.M, lin.N, lin.K, lin.alpha, ws.q.ptr,
                                                                 ldq, ws.s.ptr, lin.w, 0.0, lin.out.ptr, lin.N,
                                                                 ws.ws.ptr, ws.ws.nbytes, nxt, stream.ptr),
                                 stream, reps)
        grouped = None
        if self.pos:
            gq = time_launches(lambda: self.pos_quant(stream), stream, reps)
            grouped = time_launches(lambda: self.pos_launch(stream), stream, reps)
            for i in self.pos:
                q[i], t[i] = gq / len(self.pos), grouped / len(self.pos)
        stream.sync()
        return q, t, grouped


def measure_chain(spec, stream, steps, warmup, kreps, per=1):
    """Capture the chain into a graph on one stream (`per` steps per graph) and time exactly `steps` steps; then,
    when kreps > 0, time each kernel on its own. (A parallel graph branch for the positional projections, whose
    input is the positional table rather than an earlier linear's output, measured slower on MI355X than the
    single chain.)"""
    ch = Chain(spec)
    ms, wall = StepGraphs(stream, lambda: ch.body(stream), per, steps).time(steps, warmup)
    grouped = None
    if kreps > 0:
        qt, gt, grouped = ch.kernel_times(stream, kreps)
    else:
        qt, gt = np.full(len(ch.linears), np.nan), np.full(len(ch.linears), np.nan)
    return ch.linears, ms, wall, qt, gt, grouped


class ExactChain:
    """A chain of five-value linears in exact mode, the reference's only route on x86 (blas.c:1021-1023): each
    linear's fp32 rows straight into the exact GEMM (p2h_fvb_gemm, no quantisation; the fp32 matrix cores, or the
    per-output fmaf chain when P2H_EXACT_CHAIN=1 at capture), every linear, the positional projections included,
    with its own alpha. body() queues one pass; it can be captured into a graph."""

    def __init__(self, spec):
        self.spec = spec
        self.linears, self.inputs, _, self.keep = build_chain(spec, None)

    def body(self, stream):
        for lin, (dA, lda) in zip(self.linears, self.inputs):
            P.fvb_gemm_dev("exact", lin.M, lin.N, lin.K, lin.alpha, dA, lda, lin.w, 0.0, lin.out.ptr, lin.N, None, 0,
                           stream.ptr)


def exact_sweep_config(stream, steps=20, warmup=3):
    """The 216 linears of one 30 s window in exact mode (ExactChain): the 24 positional projections one by one (the
    grouped launch is the int8 modes'), one graph per window."""
    ch = ExactChain(sweep_spec(375))
    linears = ch.linears
    ms, _ = StepGraphs(stream, lambda: ch.body(stream), 1, steps).time(steps, warmup)
    flops = sum(2.0 * l.M * l.N * l.K for l in linears)
    tf = flops / (ms * 1e-3) / 1e12
    return {"what": "216 encoder linears of one 30 s window (M=375, pos M=749), exact mode (fp32 matrix cores)",
            "ms_per_30s_window": round(ms, 4), "tflops": round(tf, 2),
            "pct_fp32_peak": round(100.0 * tf / PEAK_FP32_TFLOPS, 2)}


def summarize(linears, ms, qt, gt):
    ops = sum(gemm_ops(l.M, l.N, l.K) for l in linears)
    planes = sum(l.K * l.N * 3 / 8 + 8 * l.N for l in linears)
    gbytes = [gemm_bytes(l.M, l.N, l.K, 1) for l in linears]
    return {
        "ms_per_step": ms,
        "tops": ops / (ms * 1e-3) / 1e12,
        "pct_int8_peak": 100.0 * ops / (ms * 1e-3) / 1e12 / PEAK_INT8_TOPS,
        "planes_gbs": planes / (ms * 1e-3) / 1e9,
        "gemm_kernels_ms": None if np.isnan(gt).any() else [round(float(x), 5) for x in gt],
        "quant_kernels_ms": None if np.isnan(qt).any() else [round(float(x), 5) for x in qt],
        "gemm_kernel_gbs": None if np.isnan(gt).any() else [round(b / (t * 1e-3) / 1e9, 1)
                                                             for b, t in zip(gbytes, gt)],
        "gemm_kernel_tops": None if np.isnan(gt).any() else [round(gemm_ops(l.M, l.N, l.K) / (t * 1e-3) / 1e12, 1)
                                                              for l, t in zip(linears, gt)],
    }


def host_cores():
    """Host cores this process may use, at most 16 (one GPU's share of its host), for the reference's thread pool."""
    try:
        n = len(os.sched_getaffinity(0))
    except AttributeError:
        n = os.cpu_count() or 1
    return max(1, min(n, 16))


def engine_window(seconds=30.0, timeout=300):
    """The reference engine's encoder on one 30 s window (encdump: its log-mel, p2_encoder, encoder.c:725-751) on a
    synthetic model in its weights format (tests/e2e/model.py), wall time of p2_encoder: as the reference ships it
    on this host's cores (encdump_cpu, exact: the x86 build's only GEMM route), and the same engine with its
    quantised GEMMs bound to this library (encdump_gpu: every linear crosses PCIe both ways, the attention and
    convolution steps stay on the CPU), int8w and exact. The first GPU-linked run moves the weights to the device;
    the figure is the best of the runs after it. With P2_CACHE_CODES=1 the engine's loader calls p2_cache_codes
    (weights.c:525-529), whose p2_fv_pack_codes calls upload every weight at load, before the first window.
    `*_breakdown`: for the best run, the library's own accounting (p2_gpu_stats_take) of the time inside its GEMM
    entries (operand copies over PCIe and kernels), the weight uploads among it, the bytes moved each way, and the
    rest of the window: the engine's CPU steps."""
    import re
    import subprocess
    import tempfile
    exes = {v: os.path.join(ROOT, "oracle", "_ref", f"encdump_{v}") for v in ("cpu", "gpu")}
    if not all(os.path.exists(e) for e in exes.values()):
        return None
    sys.path.insert(0, os.path.join(ROOT, "tests"))
    from e2e import model
    cores = host_cores()
    res = {"cores": cores, "kind": "reference", "what": f"p2_encoder wall time, {seconds:g} s of synthetic audio"}
    with tempfile.TemporaryDirectory() as d:
        model.write_model(os.path.join(d, "model"))
        wav = os.path.join(d, "a.wav")
        model.write_wav(wav, seconds, seed=5)
        for name, exe, env_mode, repeat in (
                ("encdump_cpu_exact_ms", exes["cpu"], {"P2_EXACT": "1"}, 2),
                ("encdump_gpu_int8w_ms", exes["gpu"], {"P2_GEMM": "int8w"}, 4),
                ("encdump_gpu_int8w_cache_codes_ms", exes["gpu"], {"P2_GEMM": "int8w", "P2_CACHE_CODES": "1"}, 4),
                ("encdump_gpu_exact_ms", exes["gpu"], {"P2_EXACT": "1"}, 4)):
            env = {k: v for k, v in os.environ.items()
                   if k not in ("P2_GEMM", "P2_EXACT", "P2H_EXACT_CHAIN", "P2_CACHE_CODES")}
            env.update(env_mode, P2_THREADS=str(cores), ENCDUMP_REPEAT=str(repeat))
            try:
                r = subprocess.run([exe, os.path.join(d, "model"), wav, os.path.join(d, "out.f32")],
                                   capture_output=True, text=True, timeout=timeout, env=env)
            except subprocess.TimeoutExpired:
                res[name] = None
                continue
            ms = [float(x) for x in re.findall(r"^encoder_ms ([\d.]+)", r.stderr, re.M)]
            res[name] = round(min(ms[1:]), 2) if r.returncode == 0 and len(ms) > 1 else None
            if name.startswith("encdump_gpu") and len(ms) > 0:
                res[name.replace("_ms", "_first_run_ms")] = round(ms[0], 2)
            stats = [{k: float(v) for k, v in re.findall(r"(\w+) ([\d.]+)", line)}
                     for line in re.findall(r"^gpu_stats (.*)$", r.stderr, re.M)]
            load = re.findall(r"^gpu_stats_load upload_ms ([\d.]+)", r.stderr, re.M)
            if r.returncode == 0 and len(stats) == len(ms) and len(ms) > 1:
                best = 1 + int(np.argmin(ms[1:]))
                st = stats[best]
                gemm = st["fvb_ms"] + st["q8b_ms"] + st["sgemm_ms"]
                res[name.replace("_ms", "_breakdown")] = {
                    "window_ms": round(ms[best], 2), "gemm_entries_ms": round(gemm, 2),
                    "of_which_upload_ms": round(st["upload_ms"], 2), "other_ms": round(ms[best] - gemm, 2),
                    "fvb_calls": int(st["fvb_calls"]), "q8b_calls": int(st["q8b_calls"]),
                    "sgemm_calls": int(st["sgemm_calls"]), "h2d_mb": round(st["h2d_mb"], 1),
                    "d2h_mb": round(st["d2h_mb"], 1),
                    "load_upload_ms": round(float(load[0]), 2) if load else None,
                    "first_run": {"window_ms": round(ms[0], 2),
                                  "gemm_entries_ms": round(stats[0]["fvb_ms"] + stats[0]["q8b_ms"] +
                                                           stats[0]["sgemm_ms"], 2),
                                  "of_which_upload_ms": round(stats[0]["upload_ms"], 2)}}
    return res


def cpu_baseline(M, shapes, seconds=8.0):
    """The reference's p2_sgemm_fvb (oracle/_ref/libp2ref.so: exact fp32 AVX2 route; int8w compiles only for
    AArch64, blas.c:1021-1023) on this host's cores, over the same shapes and generator, one warm-up pass and then
    whole passes for about `seconds`. The output buffers are allocated once, outside the timed passes."""
    so = os.path.join(ROOT, "oracle", "_ref", "libp2ref.so")
    if not os.path.exists(so):
        return None
    cores = host_cores()
    os.environ["P2_THREADS"] = str(cores)
    sys.path.insert(0, os.path.join(ROOT, "tests"))
    import _oracle as O
    ref = O.ref()
    data = []
    for i, (K, N) in enumerate(shapes):
        signs, flags, lo, hi = P.gen_fv_weight(SEED, 900 + i, K, N)
        A = np.ascontiguousarray(P.gen_activations(SEED, 950 + i, M, K), np.float32)
        C = np.zeros((M, N), np.float32)
        b = O.FiveValueB(signs.ctypes.data, flags.ctypes.data, lo.ctypes.data, hi.ctypes.data, None)
        data.append((K, N, A, C, b, (signs, flags, lo, hi)))

    def one_pass():
        for K, N, A, C, b, _keep in data:
            ref.p2_sgemm_fvb(M, N, K, 1.0, A.ctypes.data, K, O.C.byref(b), 0.0, C.ctypes.data, N)

    one_pass()   # warm-up: builds the pool and touches the buffers
    reps, t0 = 0, time.perf_counter()
    while True:
        one_pass()
        reps += 1
        if time.perf_counter() - t0 >= seconds:
            break
    dt = (time.perf_counter() - t0) / reps
    ops = sum(gemm_ops(M, N, K) for K, N in shapes)
    return {"value": round(ops / dt / 1e12, 4), "unit": "TOPS", "cores": cores, "kind": "reference",
            "ms_per_pass": round(dt * 1e3, 3),
            "sample": f"{reps} passes of the same GEMMs (M={M}, " + ", ".join(f"{K}->{N}" for K, N in shapes)
            + ") through the reference's p2_sgemm_fvb, exact fp32 AVX2 route (the only one x86 compiles), "
            f"P2_THREADS={cores}; {dt * 1e3:.2f} ms per pass"}


def bench_gemm_as_shipped(timeout=240):
    """The reference's own bench_gemm (oracle/_ref/bench_gemm, built from its sources: M = 416, its five encoder
    shapes, 1 warm-up + 10 repetitions each, rand() inputs, bench_gemm.c:31-58) with P2_GEMM=exact on this host's
    cores; its per-shape lines parsed."""
    exe = os.path.join(ROOT, "oracle", "_ref", "bench_gemm")
    if not os.path.exists(exe):
        return None
    import re
    import subprocess
    cores = host_cores()
    env = dict(os.environ, P2_GEMM="exact", P2_THREADS=str(cores))
    try:
        r = subprocess.run([exe], capture_output=True, text=True, timeout=timeout, env=env)
    except subprocess.TimeoutExpired:
        return {"error": f"bench_gemm did not finish in {timeout} s"}
    if r.returncode != 0:
        return {"error": f"bench_gemm exited with {r.returncode}"}
    shapes = []
    for m in re.finditer(r"^\s+(.+?)\s+K=\s*(\d+)\s+N=\s*(\d+)\s+([\d.]+) ms\s+(\d+) GMAC/s", r.stdout, re.M):
        shapes.append({"name": m.group(1).strip(), "K": int(m.group(2)), "N": int(m.group(3)),
                       "ms": float(m.group(4)), "gmac_s": float(m.group(5))})
    head = r.stdout.splitlines()[0] if r.stdout else ""
    return {"cores": cores, "kind": "reference", "header": head, "M": 416, "shapes": shapes,
            "block_ms": round(sum(s["ms"] for s in shapes), 3)}


class GemmStep:
    """One device-resident int8w five-value GEMM [M, K] x [K, N]: its rows quantised once (quant_rows), so that a
    step is the GEMM launch alone, p2h_fvb_gemm_q8a as p2_sgemm_fvb_q8a runs it; also the fp32-input route
    (p2h_fvb_gemm: quantise + GEMM in one call)."""

    def __init__(self, stream, M, K, N, tid):
        self.M, self.K, self.N, self.stream = M, K, N, stream
        self.lin = Linear(tid, K, N, M)
        self.A = P.to_device(P.gen_activations(SEED, 10_000 + K + M, M, K))
        self.sc = Scratch(M, K, P.q8a_workspace_bytes("int8w", M, N, K))
        self.ldq = P.q_ld(K)
        self.fws = P.Workspace(P.workspace_bytes("int8w", M, N, K))
        P.quant_rows_dev(M, K, self.A.ptr, K, self.sc.q.ptr, self.ldq, self.sc.s.ptr, stream.ptr)
        stream.sync()

    def launch(self):
        s = self.sc
        P.fvb_gemm_q8a_dev("int8w", self.M, self.N, self.K, 1.0, s.q.ptr, self.ldq, s.s.ptr, self.lin.w, 0.0,
                           self.lin.out.ptr, self.N, s.ws.ptr, s.ws.nbytes, self.stream.ptr)

    def launch_fp32_in(self):
        P.fvb_gemm_dev("int8w", self.M, self.N, self.K, 1.0, self.A.ptr, self.K, self.lin.w, 0.0, self.lin.out.ptr,
                       self.N, self.fws.ptr, self.fws.nbytes, self.stream.ptr)

    def time(self, steps, warmup, fp32_in=False):
        """`warmup` untimed launches, then exactly `steps` launches back to back between two HIP events on the
        stream (time_launches); returns ms per step."""
        fn = self.launch_fp32_in if fp32_in else self.launch
        for _ in range(warmup):
            fn()
        self.stream.sync()
        return time_launches(fn, self.stream, steps)


def binding_roof(ops, alg_bytes):
    """The roof that binds a GEMM by its algorithmic work: the one whose time at peak is longer."""
    t_mfma = ops / (PEAK_INT8_TOPS * 1e12)
    t_hbm = alg_bytes / (PEAK_HBM_GBS * 1e9)
    return ("hbm" if t_hbm >= t_mfma else "mfma"), t_hbm, t_mfma


def gemm_roofline(M, K, N, ms, plan, a_bytes=1, kernel=None):
    """One GEMM step against the roof that binds it. Algorithmic bytes: planes K·N·3/8 + lo/hi 8N + the rows
    (int8 M·K + row scales 4M, or fp32 4·M·K for the fp32-input route) + fp32 C 4·M·N; ops = 2·M·N·K. At M = 6000,
    K = 1024, N = 4096 the bytes take 13.26 µs at 8 TB/s and the ops 10.07 µs at 5.0 POP/s, so the binding roof is
    HBM: `frac` is against it, and `pct_int8_peak` (the target's unit) and `mfma` give the same step against the
    int8 matrix-core peak. `avg_ms` is the step's own time, from the same HIP events as `ms_per_step`."""
    ops = gemm_ops(M, N, K)
    tops = ops / (ms * 1e-3) / 1e12
    alg = gemm_bytes(M, N, K, a_bytes)
    gbs = alg / (ms * 1e-3) / 1e9
    bound, t_hbm, t_mfma = binding_roof(ops, alg)
    fake = Linear.__new__(Linear)
    fake.M, fake.K, fake.N = M, K, N
    mfma = {"achieved": round(tops, 1), "peak": PEAK_INT8_TOPS, "unit": "TOPS", "frac": round(tops / PEAK_INT8_TOPS, 4)}
    hbm = {"achieved": round(gbs, 1), "peak": PEAK_HBM_GBS, "unit": "GB/s", "frac": round(gbs / PEAK_HBM_GBS, 4)}
    r = dict(hbm if bound == "hbm" else mfma)
    traffic = measured_traffic(fake, plan)
    if a_bytes == 4 and traffic is not None:
        q = measured_traffic(fake, "quant_rows")
        traffic = traffic + q if q is not None else None
    r.update({"bound": bound, "traffic": traffic,
              "kernel": kernel or f"{kernel_name(plan)}<int8w> M={M} K={K} N={N} ({plan})", "avg_ms": round(ms, 6),
              "ops": int(ops), "algorithmic_bytes": int(alg), "us_at_hbm_peak": round(t_hbm * 1e6, 2),
              "us_at_int8_peak": round(t_mfma * 1e6, 2), "pct_int8_peak": round(100 * tops / PEAK_INT8_TOPS, 2),
              "mfma": mfma, "hbm": hbm})
    return r


def headline_roofline(lins, gt):
    """The dominant GEMM of the headline chain (longest duration) against the HBM roofline."""
    i = int(np.argmax(gt))
    L = lins[i]
    alg = gemm_bytes(L.M, L.N, L.K, 1)
    achieved = alg / (gt[i] * 1e-3) / 1e9
    plan = P.plan("int8w", L.M, L.N, L.K)
    roofline = {"bound": "hbm", "achieved": round(achieved, 1), "peak": PEAK_HBM_GBS, "unit": "GB/s",
                "frac": round(achieved / PEAK_HBM_GBS, 4), "traffic": measured_traffic(L, plan),
                "kernel": f"{kernel_name(plan)}<int8w> M={L.M} K={L.K} N={L.N} ({plan})",
                "algorithmic_bytes": int(alg), "avg_ms": gt[i],
                "tops": round(gemm_ops(L.M, L.N, L.K) / (gt[i] * 1e-3) / 1e12, 1),
                "pct_int8_peak": round(100 * gemm_ops(L.M, L.N, L.K) / (gt[i] * 1e-3) / 1e12 / PEAK_INT8_TOPS, 2)}

    return roofline


def compact(obj, keep=12):
    """`extra` with every numeric list longer than `keep` replaced by its count, sum and order statistics, so that
    the one JSON line stays a few KB (its tail is what a log keeps)."""
    if isinstance(obj, dict):
        return {k: compact(v, keep) for k, v in obj.items()}
    if isinstance(obj, list) and len(obj) > keep and all(isinstance(x, (int, float)) for x in obj):
        a = np.asarray(obj, dtype=np.float64)
        return {"n": int(a.size), "sum": round(float(a.sum()), 5), "min": round(float(a.min()), 5),
                "median": round(float(np.median(a)), 5), "max": round(float(a.max()), 5)}
    if isinstance(obj, list):
        return [compact(v, keep) for v in obj]
    return obj


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=2000)
    ap.add_argument("--warmup", type=int, default=200)
    ap.add_argument("--workload", default="gemm6000", choices=["gemm6000", "ffn375", "m6000", "m38", "sweep"])
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-extra", action="store_true")
    ap.add_argument("--eager-extras", action="store_true",
                    help="extra configurations without HIP graphs: the device conformer block, the producers, the "
                         "attention products, the feed-forward module's kernels and the sweep's kernels, each "
                         "timed by back-to-back launches (what rocprofv3 traces)")
    ap.add_argument("--no-sweep", action="store_true",
                    help="leave the 216-linear sweep out of the extra configurations")
    ap.add_argument("--kernel-reps", type=int, default=200,
                    help="back-to-back launches of each kernel for the per-kernel durations (0: skip them)")
    ap.add_argument("--copy-mib", type=int, default=0,
                    help="only run device-to-device copies of this many MiB (the plain copy kernel that scales "
                         "FETCH_SIZE / WRITE_SIZE counter readings to bytes)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py runs on one GPU: the five-value GEMM path has no multi-GPU form here "
              f"(--gpus {args.gpus} requested)", file=sys.stderr)
        sys.exit(2)

    dev = P.init()
    stream = P.Stream()
    print(f"# device {dev}, {P.device_cu_count()} CUs", file=sys.stderr, flush=True)
    if args.copy_mib:
        nbytes = args.copy_mib << 20
        src, dst = P.DeviceBuffer(nbytes), P.DeviceBuffer(nbytes)
        for _ in range(5):
            P._ok(P.hip().p2h_memcpy_d2d(dst.ptr, src.ptr, nbytes, stream.ptr), "d2d")
        stream.sync()
        print(f"# copied {args.copy_mib} MiB x5", file=sys.stderr, flush=True)
        return

    results = {}

    def run(name, spec, steps, warmup, kreps):
        per = STEPS_PER_REPLAY if len(spec) <= 4 else 1   # a window's chain is one graph already
        lins, ms, wall, qt, gt, grouped = measure_chain(spec, stream, steps, warmup, kreps, per)
        r = summarize(lins, ms, qt, gt)
        if grouped is not None:
            r["grouped_pos_ms"] = round(float(grouped), 5)
        r["wall_s"] = round(wall, 3)
        results[name] = (lins, r)
        print(f"# {name}: {ms * 1e3:.2f} us/step, {r['tops']:.1f} TOPS", file=sys.stderr, flush=True)
        return lins, r

    specs = {
        "ffn375": lambda: ffn_spec(375),
        "m6000": lambda: ffn_spec(6000, base=3),
        "m38": lambda: ffn_spec(38, base=5),
        "sweep": lambda: sweep_spec(375),
    }
    main_wl = args.workload
    extra = {}
    kernels = None
    if main_wl == "gemm6000":
        M, K, N = 6000, 1024, 4096
        gs = GemmStep(stream, M, K, N, tid=3)
        ms = gs.time(args.steps, args.warmup)
        plan = P.plan("int8w", M, N, K)
        roofline = gemm_roofline(M, K, N, ms, plan)
        tops = roofline["mfma"]["achieved"]
        print(f"# gemm6000: {ms * 1e3:.2f} us/GEMM, {tops:.1f} TOPS ({100 * tops / PEAK_INT8_TOPS:.1f} % of int8 "
              f"peak, {100 * roofline['hbm']['frac']:.1f} % of HBM)", file=sys.stderr, flush=True)
        ms_f = gs.time(max(1, min(args.steps, 500)), 20, fp32_in=True)
        # the p2_sgemm_fvb route the reference's bench_gemm and sgemm_i8 run: fp32 rows in, quantised per call
        roofline["fp32_in_route"] = gemm_roofline(
            M, K, N, ms_f, plan, a_bytes=4,
            kernel=f"quant_rows + {kernel_name(plan)}<int8w> M={M} K={K} N={N} "
                   "(p2h_fvb_gemm: fp32 rows quantised in the step)")
        print(f"# gemm6000 fp32 in: {ms_f * 1e3:.2f} us/GEMM, "
              f"{roofline['fp32_in_route']['pct_int8_peak']:.1f} % of int8 peak", file=sys.stderr, flush=True)
        del gs
        step_ms, ops, value = ms, gemm_ops(M, N, K), tops
        pct = 100 * tops / PEAK_INT8_TOPS
        workload = ("int8w five-value GEMM M=6000 (16 stacked 30 s windows), K=1024, N=4096, from per-row "
                    "quantised int8 rows (p2_sgemm_fvb_q8a route; quantise pass not in the step), fp32 C")
        config = {"workload": workload, "M": M, "K": K, "N": N, "gemm_ops_per_step": ops,
                  "quantise_in_step": False, "launch": "back to back on one stream"}
        cpu_shapes = (M, [(K, N)])
    else:
        lins, r = run(main_wl, specs[main_wl](), args.steps, args.warmup, args.kernel_reps)
        gt = r["gemm_kernels_ms"]
        roofline = headline_roofline(lins, gt) if gt is not None else None
        step_ms, value, pct = r["ms_per_step"], r["tops"], r["pct_int8_peak"]
        ops = sum(gemm_ops(l.M, l.N, l.K) for l in lins)
        config = {"workload": {"ffn375": "FFN pair M=375: 1024->4096 then 4096->1024, int8w, fp32 A in HBM",
                               "m6000": "FFN pair M=6000: 1024->4096 then 4096->1024, int8w",
                               "m38": "FFN pair M=38: 1024->4096 then 4096->1024, int8w",
                               "sweep": "216 encoder linears of one 30 s window (M=375, pos M=749), int8w"}[main_wl],
                  "M": lins[0].M, "gemm_ops_per_step": ops, "quantise_in_step": True,
                  "graph": {"steps_per_replay": STEPS_PER_REPLAY if len(lins) <= 4 else 1}}
        kernels = {"gemm_ms": r["gemm_kernels_ms"], "quant_ms": r["quant_kernels_ms"],
                   "gemm_gbs": r["gemm_kernel_gbs"], "gemm_tops": r["gemm_kernel_tops"]}
        cpu_shapes = (lins[0].M, [(l.K, l.N) for l in lins])

    if not args.no_extra and args.eager_extras:
        extra["conformer_block375"] = conformer_block_config(stream, graph=False)
        extra["attention375"] = attention_config(stream, graph=False)
        extra["producers"] = producer_config(stream)
        extra["ffn_module375"] = ffn_module_config(stream, graph=False)
        if not args.no_sweep:
            extra["sweep_kernels"] = sweep_kernels_eager(stream, reps=20)
    elif not args.no_extra:
        for name in ("ffn375", "m6000", "m38", "sweep"):
            if name == main_wl or (name == "sweep" and args.no_sweep):
                continue
            steps = {"ffn375": 2000, "m6000": 200, "m38": 2000, "sweep": 50}[name]
            kreps = 20 if name == "sweep" else args.kernel_reps
            _, rr = run(name, specs[name](), steps, 20, kreps)
            extra[name] = rr
        extra["exact375"] = exact_config(stream)
        extra["q8b375"] = q8b_config(stream)
        if not args.no_sweep:
            extra["sweep_exact"] = exact_sweep_config(stream)
        extra["attention375"] = attention_config(stream)
        extra["producers"] = producer_config(stream)
        extra["ffn_module375"] = ffn_module_config(stream)
        extra["block375"] = block_config(stream)
        extra["conformer_block375"] = conformer_block_config(stream)
        extra["conformer_stack375"] = conformer_stack_config(stream)
        extra["m38_rotated"] = m38_rotated_config(stream)
    sweep_ms = results["sweep"][1]["ms_per_step"] if "sweep" in results else None

    cpu = None
    if not args.no_cpu_baseline:
        cpu = cpu_baseline(*cpu_shapes, seconds=12.0)
        if not args.no_extra:
            extra["cpu_baselines"] = {
                "exact375_1024x1024": cpu_baseline(375, [(1024, 1024)], seconds=4.0),
                "ffn375_pair": cpu_baseline(375, [(1024, 4096), (4096, 1024)], seconds=4.0),
                "bench_gemm_as_shipped": bench_gemm_as_shipped(),
                "engine_30s_window": engine_window(),
            }

    line = {
        "metric": "five-value int8 GEMM TOPS + % int8 MFMA peak; encoder linears ms per 30 s",
        "value": round(value, 3),
        "unit": "TOPS",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(step_ms, 6),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8",
        "data": "synthetic (seeded generator: N(0,1) activations with 0.1% x20 outliers; five-value weights "
                "P(0)=0.4, P(lo)=0.4, P(hi)=0.2, fp16 lo/hi)",
        "config": config,
        "pct_int8_peak": round(pct, 3),
        "sweep_ms_per_30s_window": round(sweep_ms, 5) if sweep_ms is not None else None,
        "roofline": roofline,
        "cpu_baseline": cpu,
        "kernels": kernels,
        "extra": compact(extra),
    }
    print(json.dumps(line), flush=True)


def sweep_kernels_eager(stream, reps=20):
    """The 216-linear sweep's kernels, each timed on its own by back-to-back launches (Chain.kernel_times), with
    no graph: what the profiler traces for the sweep."""
    ch = Chain(sweep_spec(375))
    q, t, grouped = ch.kernel_times(stream, reps)
    lins = ch.linears
    return {"gemm_ms_sum": round(float(np.nansum(t)), 5), "quant_ms_sum": round(float(np.nansum(q)), 5),
            "grouped_pos_ms": round(float(grouped), 5) if grouped is not None else None,
            "gemm_ms_first_block": [round(float(x), 5) for x in t[:9]],
            "shapes_first_block": [f"{l.M}x{l.K}->{l.N}" for l in lins[:9]]}


def measured_traffic(L, plan):
    """HBM bytes per launch of this GEMM from the committed rocprofv3 FETCH_SIZE / WRITE_SIZE runs
    (profiles/gemm_fv_traffic.json), when they were taken for the same shape and plan; otherwise None. The plan
    "quant_rows" names the row quantiser that feeds the GEMM on the fp32-input route (M rows of K)."""
    path = os.path.join(ROOT, "profiles", "gemm_fv_traffic.json")
    if not os.path.exists(path):
        return None
    for e in json.load(open(path))["entries"]:
        if (e["M"], e["K"], e["N"]) == (L.M, L.K, L.N) and e["plan"] == plan:
            return int(e["fetch_kib"] * 1024 * e["fetch_scale"] + e["write_kib"] * 1024 * e["write_scale"])
    return None


def exact_config(stream):
    """The exact-mode five-value GEMM at M=375, K=1024, N=1024 (bench_gemm.c's route) on the fp32 matrix cores and on
    the bit-exact fmaf-chain route (P2H_EXACT_CHAIN=1), and at the M=6000 FFN shapes on the matrix cores."""
    out = {}
    for name, (M, K, N), chain, reps in (("m375", (375, 1024, 1024), False, 200), ("m375_fmaf_chain", (375, 1024, 1024), True, 50),
                                         ("m6000_up", (6000, 1024, 4096), False, 10),
                                         ("m6000_down", (6000, 4096, 1024), False, 10)):
        signs, flags, lo, hi = P.gen_fv_weight(SEED, 77, K, N)
        w = P.FvWeight(signs, flags, lo, hi, K, N)
        dA = P.to_device(P.gen_activations(SEED, 78, M, K))
        dC = P.DeviceBuffer(M * N * 4)
        if chain:   # the library reads its switches once: reload them around the capture
            os.environ["P2H_EXACT_CHAIN"] = "1"
            P.reload_switches()
        try:
            sg = StepGraphs(stream, lambda: P.fvb_gemm_dev("exact", M, N, K, 1.0, dA.ptr, K, w, 0.0, dC.ptr, N, None,
                                                           0, stream.ptr), STEPS_PER_REPLAY, reps)
        finally:
            os.environ.pop("P2H_EXACT_CHAIN", None)
            P.reload_switches()
        ms, _ = sg.time(reps, 3)
        del sg
        tf = gemm_ops(M, N, K) / (ms * 1e-3) / 1e12
        out[name] = {"ms": round(ms, 5), "tflops": round(tf, 2), "pct_fp32_peak": round(100 * tf / PEAK_FP32_TFLOPS, 2)}
    return out


def q8b_config(stream, T=375, reps=500):
    """The encoder's two int8-table linears (p2_sgemm_q8b: one int8 plane with a per-column fp32 scale) at a 30 s
    window's T = 375 frames: the subsampling output linear 4096 -> 1024 (encoder.c:219) and the projector
    1024 -> 640 (encoder.c:744), each timed by time_launches as p2_wmatmul calls it: p2h_q8b_gemm on fp32 rows
    (quantise, GEMM, and for the subsampling K split at its four 1024-row blocks plus the fold), beside the
    quantiser alone and p2h_q8b_gemm_q8a (rows already quantised; no workspace, so never split). Algorithmic bytes
    of the fp32-row route: the fp32 rows 4·M·K, the int8 plane K·N, its scales 4N, fp32 C 4·M·N."""
    rng = np.random.default_rng(SEED + 11)
    out = {}
    for name, K, N in (("subsampling_4096x1024", 4096, 1024), ("projector_1024x640", 1024, 640)):
        B = P.to_device(rng.integers(-127, 128, (K, N), dtype=np.int8))
        bs = P.to_device(rng.uniform(0.5, 1.5, N).astype(np.float32) / 127.0)
        dA = P.to_device(P.gen_activations(SEED, 20_100 + K, T, K))
        ldq = P.q_ld(K)
        dQ, dS = P.DeviceBuffer(P.q_bytes(T, K)), P.DeviceBuffer(4 * T)
        dC = P.DeviceBuffer(T * N * 4)
        ws = P.Workspace(P.q8b_workspace_bytes("int8w", T, N, K))
        quant = time_launches(lambda: P.quant_rows_dev(T, K, dA.ptr, K, dQ.ptr, ldq, dS.ptr, stream.ptr), stream, reps)
        route = time_launches(lambda: P.q8b_gemm_dev("int8w", T, N, K, 1.0, dA.ptr, K, B.ptr, N, bs.ptr, 0.0, dC.ptr, N,
                                                     ws.ptr, ws.nbytes, stream.ptr), stream, reps)
        q8a = time_launches(lambda: P.q8b_gemm_q8a_dev(T, N, K, 1.0, dQ.ptr, ldq, dS.ptr, B.ptr, N, bs.ptr, 0.0, dC.ptr,
                                                       N, stream.ptr), stream, reps)
        alg = 4 * T * K + K * N + 4 * N + 4 * T * N
        out[name] = {"fp32_rows_us": round(route * 1e3, 3), "quant_us": round(quant * 1e3, 3),
                     "q8a_entry_us": round(q8a * 1e3, 3),
                     "gbs": round(alg / (route * 1e-3) / 1e9, 1),
                     "tops": round(gemm_ops(T, N, K) / (route * 1e-3) / 1e12, 1)}
    return out


def producer_config(stream, reps=200):
    """The four row producers (LayerNorm, SiLU, head concatenation, channel-major transpose, each quantised as
    produced) at the encoder's shapes for T = 375 and T = 6000, each timed on its own by time_launches, against the
    HBM roofline: algorithmic bytes = fp32 rows read + int8 rows and fp32 scales written (+ gamma, beta)."""
    rng = np.random.default_rng(SEED)
    out = {}
    for T in (375, 6000):
        D, FF, H, Dh = 1024, 4096, 8, 128
        x = P.to_device(rng.standard_normal((T, D)).astype(np.float32))
        h = P.to_device(rng.standard_normal((T, FF)).astype(np.float32))
        heads = P.to_device(rng.standard_normal((H, T, Dh)).astype(np.float32))
        cm = P.to_device(rng.standard_normal((D, T)).astype(np.float32))
        g = P.to_device(rng.uniform(0.5, 1.5, D).astype(np.float32))
        b = P.to_device(rng.uniform(-0.2, 0.2, D).astype(np.float32))
        q = P.DeviceBuffer(P.q_bytes(T, FF))
        s = P.DeviceBuffer(4 * T)
        ldD, ldF = P.q_ld(D), P.q_ld(FF)
        cases = (
            ("layer_norm", D, 8 * D,
             lambda: P.layer_norm_quant_rows_dev(T, D, x.ptr, D, g.ptr, b.ptr, q.ptr, ldD, s.ptr, stream.ptr)),
            ("silu", FF, 0, lambda: P.silu_quant_rows_dev(T, FF, h.ptr, FF, q.ptr, ldF, s.ptr, stream.ptr)),
            ("concat_heads", D, 0,
             lambda: P.concat_heads_quant_rows_dev(H, T, Dh, heads.ptr, q.ptr, ldD, s.ptr, stream.ptr)),
            ("channel_major", D, 0, lambda: P.channel_major_quant_rows_dev(D, T, cm.ptr, q.ptr, ldD, s.ptr, stream.ptr)),
            ("plain_quant", D, 0, lambda: P.quant_rows_dev(T, D, x.ptr, D, q.ptr, ldD, s.ptr, stream.ptr)),
        )
        for name, K, extra_bytes, fn in cases:
            ms = time_launches(fn, stream, reps)
            alg = quant_bytes(T, K) + extra_bytes
            out[f"{name}_T{T}"] = {"us": round(ms * 1e3, 2), "gbs": round(alg / (ms * 1e-3) / 1e9, 1),
                                   "frac_hbm": round(alg / (ms * 1e-3) / 1e9 / PEAK_HBM_GBS, 4),
                                   "algorithmic_bytes": int(alg)}
    stream.sync()
    return out


def ffn_module_config(stream, M=375, steps=2000, warmup=100, reps=200, graph=True):
    """One conformer feed-forward module as the encoder runs it in the int8 modes (encoder.c:340-348), every step on
    the device and replayed from one graph: LayerNorm quantised as produced, up-projection 1024 -> 4096, SiLU
    quantised as produced, down-projection 4096 -> 1024 with the residual in its epilogue (alpha 0.5, beta 1)."""
    D, FF = 1024, 4096
    rng = np.random.default_rng(SEED + 5)
    l1, l2 = Linear(41, D, FF, M), Linear(42, FF, D, M)
    x = P.to_device(P.gen_activations(SEED, 10_000 + D + M, M, D))
    g = P.to_device(rng.uniform(0.5, 1.5, D).astype(np.float32))
    b = P.to_device(rng.uniform(-0.2, 0.2, D).astype(np.float32))
    ws = Scratch(M, FF, max(P.q8a_workspace_bytes("int8w", M, FF, D), P.q8a_workspace_bytes("int8w", M, D, FF)))
    ldD, ldF = P.q_ld(D), P.q_ld(FF)
    steps_fns = (
        lambda: P.layer_norm_quant_rows_dev(M, D, x.ptr, D, g.ptr, b.ptr, ws.q.ptr, ldD, ws.s.ptr, stream.ptr),
        lambda: P.fvb_gemm_q8a_next_dev("int8w", M, FF, D, 1.0, ws.q.ptr, ldD, ws.s.ptr, l1.w, 0.0, l1.out.ptr, FF,
                                        ws.ws.ptr, ws.ws.nbytes, l2.w, stream.ptr),
        lambda: P.silu_quant_rows_dev(M, FF, l1.out.ptr, FF, ws.q.ptr, ldF, ws.s.ptr, stream.ptr),
        lambda: P.fvb_gemm_q8a_next_dev("int8w", M, D, FF, 0.5, ws.q.ptr, ldF, ws.s.ptr, l2.w, 1.0, x.ptr, D,
                                        ws.ws.ptr, ws.ws.nbytes, l1.w, stream.ptr),
    )
    ms = None
    if graph:
        def body():
            for fn in steps_fns:
                fn()
        ms, _ = StepGraphs(stream, body, STEPS_PER_REPLAY, steps).time(steps, warmup)
    kt = [round(time_launches(fn, stream, reps), 5) for fn in steps_fns] if reps > 0 else None
    ops = gemm_ops(M, FF, D) + gemm_ops(M, D, FF)
    return {"ms_per_step": round(ms, 6) if ms else None, "tops": round(ops / (ms * 1e-3) / 1e12, 2) if ms else None,
            "kernels_ms": dict(zip(("layer_norm_quant", "gemm_up", "silu_quant", "gemm_down_residual"), kt))
            if kt else None}


def m38_rotated_config(stream, pairs=188, steps=20, warmup=3):
    """The 3 s utterance's FFN pair (M = 38: 1024 -> 4096, then 4096 -> 1024, int8w) over `pairs` independently seeded
    weight pairs chained one after another (pair r's up-projection reads pair r - 1's output): 188 pairs hold 602 MB
    of packed planes (the reference's format) and 797 MB of device copies (4-bit records, lo, hi and the lo codes),
    far beyond the 256 MB Infinity Cache, so the weights stream from HBM: the weight-streaming bound of the small-M
    path.
    One graph replay runs all pairs; reported per pair,
    with GB/s on the packed planes (K·N·3/8 + 8N, the bytes the reference's format holds) and on the 4-bit operand
    records the kernels read (K·N/2 + 8N), against 8 TB/s."""
    M = 38
    spec = []
    for r in range(pairs):
        spec += [(2000 + 2 * r, 1024, 4096, M, "x" if r == 0 else 2 * r - 1), (2001 + 2 * r, 4096, 1024, M, 2 * r)]
    linears, ms, wall, qt, gt, _ = measure_chain(spec, stream, steps, warmup, 0)
    per_pair = ms / pairs
    planes = sum(l.K * l.N * 3 / 8 + 8 * l.N for l in linears) / pairs
    records = sum(l.K * l.N / 2 + 8 * l.N for l in linears) / pairs
    dev = sum(l.w.device_bytes() for l in linears)
    return {"ms_per_pair": round(per_pair, 6),
            "planes_gbs": round(planes / (per_pair * 1e-3) / 1e9, 1),
            "planes_frac_hbm": round(planes / (per_pair * 1e-3) / 1e9 / PEAK_HBM_GBS, 4),
            "records_gbs": round(records / (per_pair * 1e-3) / 1e9, 1),
            "weights_device_mb": round(dev / 1e6, 1),
            "what": f"{pairs} chained weight pairs, M={M}, int8w, one graph replay (quantise + GEMM per linear)"}


def block_config(stream, T=375, steps=500, warmup=50):
    """One conformer block's nine five-value linears as the encoder runs them in the int8 modes (encoder.c:333-613),
    every input made by its producer and every residual added in a GEMM epilogue, on the device and replayed from
    one graph: LN→int8, ff1.linear1 with SiLU, int8, ff1.linear2 (x += ½·), LN→int8, qkv, the positional
    projection (its rows quantised once per window, so not in the block), heads→int8, out (x += ), LN→int8, pw1,
    channel-major→int8, pw2 (x += ), LN→int8, ff2.linear1 with SiLU, int8, ff2.linear2 (x += ½·). The feed-forward's
    SiLU is applied as the up-projection stores its output and a plain quantiser follows, as p2h_conformer_block runs
    it (the same bits as the SiLU→int8 producer after a plain GEMM). What lies between the linears and is not on this
    path (attention scores and softmax, GLU, the depthwise convolution) is replaced by fixed buffers of the right
    shapes: the heads [8, T, 128] and the channel-major conv output [1024, T]."""
    D, FF, H, Dh = 1024, 4096, 8, 128
    rng = np.random.default_rng(SEED + 9)
    x = P.to_device(P.gen_activations(SEED, 10_000 + D + T, T, D))
    gb = [(P.to_device(rng.uniform(0.5, 1.5, D).astype(np.float32)),
           P.to_device(rng.uniform(-0.2, 0.2, D).astype(np.float32))) for _ in range(4)]
    heads = P.to_device((rng.standard_normal((H, T, Dh)) * 0.5).astype(np.float32))
    cm = P.to_device((rng.standard_normal((D, T)) * 0.5).astype(np.float32))
    lin = {name: Linear(60 + i, K, N, T) for i, (name, K, N) in enumerate(
        (("ff1_l1", D, FF), ("ff1_l2", FF, D), ("qkv", D, 3 * D), ("out", D, D), ("pw1", D, 2 * D), ("pw2", D, D),
         ("ff2_l1", D, FF), ("ff2_l2", FF, D)))}
    split = max(P.q8a_workspace_bytes("int8w", T, l.N, l.K) for l in lin.values())
    ws = Scratch(T, FF, split)
    ldD, ldF = P.q_ld(D), P.q_ld(FF)

    seq = ["ff1_l1", "ff1_l2", "qkv", "out", "pw1", "pw2", "ff2_l1", "ff2_l2"]   # the block's order of GEMMs

    def gemm(l, ldq, alpha, beta, out):   # reads the records of the block's next GEMM (the last, the first's) ahead
        name = next(k for k, v in lin.items() if v is l)
        nxt = lin[seq[(seq.index(name) + 1) % len(seq)]].w
        P.fvb_gemm_q8a_next_dev("int8w", T, l.N, l.K, alpha, ws.q.ptr, ldq, ws.s.ptr, l.w, beta, out, l.N,
                                ws.ws.ptr, ws.ws.nbytes, nxt, stream.ptr)

    def ln(i):
        P.layer_norm_quant_rows_dev(T, D, x.ptr, D, gb[i][0].ptr, gb[i][1].ptr, ws.q.ptr, ldD, ws.s.ptr, stream.ptr)

    def up_silu(l):   # SiLU as the up-projection stores, then the plain quantiser of its rows
        P.fvb_gemm_q8a_silu_dev("int8w", T, l.N, l.K, 1.0, ws.q.ptr, ldD, ws.s.ptr, l.w, l.out.ptr, ws.ws.ptr,
                                ws.ws.nbytes, stream.ptr)
        P.quant_rows_dev(T, FF, l.out.ptr, FF, ws.q.ptr, ldF, ws.s.ptr, stream.ptr)

    def block():
        ln(0); up_silu(lin["ff1_l1"]); gemm(lin["ff1_l2"], ldF, 0.5, 1.0, x.ptr)
        ln(1); gemm(lin["qkv"], ldD, 1.0, 0.0, lin["qkv"].out.ptr)
        P.concat_heads_quant_rows_dev(H, T, Dh, heads.ptr, ws.q.ptr, ldD, ws.s.ptr, stream.ptr)
        gemm(lin["out"], ldD, 1.0, 1.0, x.ptr)
        ln(2); gemm(lin["pw1"], ldD, 1.0, 0.0, lin["pw1"].out.ptr)
        P.channel_major_quant_rows_dev(D, T, cm.ptr, ws.q.ptr, ldD, ws.s.ptr, stream.ptr)
        gemm(lin["pw2"], ldD, 1.0, 1.0, x.ptr)
        ln(3); up_silu(lin["ff2_l1"]); gemm(lin["ff2_l2"], ldF, 0.5, 1.0, x.ptr)

    ms, _ = StepGraphs(stream, block, STEPS_PER_REPLAY, steps).time(steps, warmup)
    ops = sum(gemm_ops(T, l.N, l.K) for l in lin.values())
    return {"ms_per_block": round(ms, 6), "ms_per_30s_window_24_blocks": round(24 * ms, 4),
            "tops": round(ops / (ms * 1e-3) / 1e12, 2), "kernels_per_block": 16,
            "what": f"T={T}: 8 producers + 8 five-value GEMMs (int8w), residuals and the feed-forward's SiLU in the "
                    "epilogues"}


def conformer_block_config(stream, T=375, steps=200, warmup=20, graph=True):
    """One whole conformer block on the device (p2h_conformer_block: encoder.c:617-625, every step between the
    linears included — attention scores, relative shift and softmax, GLU, depthwise convolution and SiLU, the
    LayerNorms, the positional projection of its 2T − 1 rows) on a seeded synthetic block, replayed from one graph;
    x is carried from replay to replay (the final LayerNorm keeps it bounded). Per mode: ms per block and per 30 s
    window of 24 blocks. graph=False launches the block's kernels directly, block after block, between two HIP
    events (what the profiler traces)."""
    params = P.block_params(SEED, 100)
    blk = P.Block(params)
    D = P.D_MODEL
    x = P.to_device(P.gen_activations(SEED, 20_000 + T, T, D))
    pe = P.to_device(P.gen_activations(SEED, 20_001 + T, 2 * T - 1, D))
    res = {"what": f"T={T}: one device conformer block (9 five-value linears + attention + convolution module)"}
    for mode in ("int8w", "exact"):
        ws = P.Workspace(P.block_workspace_bytes(mode, T))
        body = lambda m=mode, w=ws: blk.run_dev(m, T, pe.ptr, x.ptr, w, stream.ptr)
        body()   # anything a first call prepares is made before the capture
        stream.sync()
        if graph:
            ms, _ = StepGraphs(stream, body, 1, steps).time(steps, warmup)
        else:
            for _ in range(warmup):
                body()
            e0, e1 = P.Event(), P.Event()
            e0.record(stream.ptr)
            for _ in range(steps):
                body()
            e1.record(stream.ptr)
            e1.sync()
            ms = e0.elapsed_ms(e1) / steps
        res[mode] = {"ms_per_block": round(ms, 5), "ms_per_30s_window_24_blocks": round(24 * ms, 4)}
    res["launch"] = "one graph per block" if graph else "direct launches, block after block"
    return res


def conformer_stack_config(stream, T=375, n_blocks=24, steps=20, warmup=3):
    """One 30 s window's 24 conformer blocks on the device (p2h_conformer_stack: encode_blocks, encoder.c:628-644),
    24 distinct seeded synthetic blocks (216 five-value linears, 0.53 GB of device weights), the positional rows
    quantised once and the 24 positional projections grouped; the whole window replayed from one graph, x carried
    from window to window. ms per 30 s window, int8w and exact."""
    blocks = [P.Block(P.block_params(SEED, 1000 + 20 * b)) for b in range(n_blocks)]
    stack = P.Stack(blocks)
    D = P.D_MODEL
    x = P.to_device(P.gen_activations(SEED, 30_000 + T, T, D))
    pe = P.to_device(P.gen_activations(SEED, 30_001 + T, 2 * T - 1, D))
    res = {"what": f"T={T}: {n_blocks} device conformer blocks, distinct weights, one graph per window"}
    for mode in ("int8w", "exact"):
        ws = P.Workspace(P.stack_workspace_bytes(mode, T, n_blocks))
        body = lambda m=mode, w=ws: stack.run_dev(m, T, pe.ptr, x.ptr, w, stream.ptr)
        body()
        stream.sync()
        ms, _ = StepGraphs(stream, body, 1, steps).time(steps, warmup)
        res[mode] = {"ms_per_30s_window": round(ms, 4), "ms_per_block": round(ms / n_blocks, 5)}
    res["weights_device_mb"] = round(sum(getattr(b._keep[f], "device_bytes", lambda: 0)() for b in blocks
                                         for f in P.BLOCK_LINEARS) / 1e6, 1)
    return res


def attention_config(stream, H=8, T=375, Dh=128, graph=True, reps=200):
    """The fp32 per-head products of one block's relative-position attention at T = 375 (encoder.c:505-519), every
    head in one p2h_sgemm_batched launch each: Q_u·K_t [T, T], Q_v·P_t [T, 2T−1], scores·V [T, Dh]."""
    rng = np.random.default_rng(SEED)
    L = 2 * T - 1
    bufs = {k: P.to_device(rng.standard_normal(sh).astype(np.float32)) for k, sh in
            (("qu", (H, T, Dh)), ("kt", (H, Dh, T)), ("pt", (H, Dh, L)), ("s", (H, T, T)), ("v", (H, T, Dh)))}
    out = {k: P.DeviceBuffer(H * T * n * 4) for k, n in (("ac", T), ("bd", L), ("ctx", Dh))}
    calls = ((T, T, Dh, "qu", "kt", "ac"), (T, L, Dh, "qu", "pt", "bd"), (T, Dh, T, "s", "v", "ctx"))
    fns = [lambda M=M, N=N, K=K, a=a, b=b, c=c: P.sgemm_batched_dev(
        False, False, M, N, K, 1.0, bufs[a].ptr, K, M * K, bufs[b].ptr, N, K * N, 0.0, out[c].ptr, N, M * N, H,
        stream.ptr) for M, N, K, a, b, c in calls]
    flops = sum(2.0 * H * M * N * K for M, N, K, *_ in calls)
    res = {"what": f"{H} heads, T={T}, Dh={Dh}: 3 batched fp32 products per block"}
    if graph:
        def body():
            for fn in fns:
                fn()
        ms, _ = StepGraphs(stream, body, STEPS_PER_REPLAY, 200).time(200, 10)
        res.update({"ms": round(ms, 5), "tflops": round(flops / (ms * 1e-3) / 1e12, 2),
                    "pct_fp32_peak": round(100 * flops / (ms * 1e-3) / 1e12 / PEAK_FP32_TFLOPS, 2)})
    res["products_ms_back_to_back"] = [round(time_launches(fn, stream, reps), 5) for fn in fns]
    return res


if __name__ == "__main__":
    main()
