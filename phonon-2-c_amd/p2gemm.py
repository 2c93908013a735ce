"""ctypes binding of the MI355X five-value GEMM (lib/libp2hip.so, include/p2hip.h) and the input generator
(lib/libp2gen.so, include/p2gen.h), with numpy host arrays.

Device memory, copies, streams and events all go through libp2hip.so itself, so a process that uses this module
holds exactly one HIP runtime. Every call raises P2Error when the library reports an error; nothing here computes
a product on the CPU.
"""
import ctypes as C
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIBDIR = os.path.join(HERE, "lib")
HIP_SO = os.path.join(LIBDIR, "libp2hip.so")
GEN_SO = os.path.join(LIBDIR, "libp2gen.so")
BLAS_SO = os.path.join(LIBDIR, "libphonon2_gemm.so")

INT8, EXACT, INT8W = 0, 1, 2
MODES = {"int8": INT8, "exact": EXACT, "int8w": INT8W}
Q_KALIGN = 128


class P2Error(RuntimeError):
    pass


_vp, _sz, _i, _f = C.c_void_p, C.c_size_t, C.c_int, C.c_float

_HIP_SIG = {
    "p2h_init": (_i, []),
    "p2h_reload_switches": (_i, []),
    "p2h_last_error": (C.c_char_p, []),
    "p2h_device_name": (C.c_char_p, []),
    "p2h_device_cu_count": (_i, []),
    "p2h_stream_create": (_vp, []),
    "p2h_stream_destroy": (_i, [_vp]),
    "p2h_stream_sync": (_i, [_vp]),
    "p2h_thread_stream": (_vp, []),
    "p2h_malloc": (_vp, [_sz]),
    "p2h_free": (_i, [_vp]),
    "p2h_host_malloc": (_vp, [_sz]),
    "p2h_host_free": (_i, [_vp]),
    "p2h_memset": (_i, [_vp, _i, _sz, _vp]),
    "p2h_memcpy_h2d": (_i, [_vp, _vp, _sz, _vp]),
    "p2h_memcpy_d2h": (_i, [_vp, _vp, _sz, _vp]),
    "p2h_memcpy_d2d": (_i, [_vp, _vp, _sz, _vp]),
    "p2h_memcpy2d_h2d": (_i, [_vp, _sz, _vp, _sz, _sz, _sz, _vp]),
    "p2h_memcpy2d_d2h": (_i, [_vp, _sz, _vp, _sz, _sz, _sz, _vp]),
    "p2h_capture_begin": (_i, [_vp]),
    "p2h_capture_end": (_i, [_vp, C.POINTER(_vp)]),
    "p2h_graph_launch": (_i, [_vp, _vp]),
    "p2h_graph_destroy": (_i, [_vp]),
    "p2h_event_create": (_vp, []),
    "p2h_event_destroy": (_i, [_vp]),
    "p2h_event_record": (_i, [_vp, _vp]),
    "p2h_event_sync": (_i, [_vp]),
    "p2h_stream_wait_event": (_i, [_vp, _vp]),
    "p2h_event_elapsed_ms": (_f, [_vp, _vp]),
    "p2h_stream_hold": (_i, [_vp, C.c_uint]),
    "p2h_fv_weight_upload": (_vp, [_vp, _vp, _vp, _vp, _i, _i]),
    "p2h_fv_weight_wrap": (_vp, [_vp, _vp, _vp, _vp, _i, _i]),
    "p2h_weight_free": (None, [_vp]),
    "p2h_weight_shape": (_i, [_vp, C.POINTER(_i), C.POINTER(_i)]),
    "p2h_weight_device_bytes": (_sz, [_vp]),
    "p2h_fv_pack_codes": (_i, [_vp, _vp, _vp]),
    "p2h_quant_rows": (_i, [_i, _i, _vp, _i, _vp, _i, _vp, _vp]),
    "p2h_q_ld": (_i, [_i]),
    "p2h_layer_norm_quant_rows": (_i, [_i, _i, _vp, _i, _vp, _vp, _vp, _i, _vp, _vp]),
    "p2h_layer_norm2_quant_rows": (_i, [_i, _i, _vp, _i, _vp, _vp, _vp, _i, _vp, _vp, _vp, _i, _vp, _vp]),
    "p2h_recip_selftest": (_i, [C.POINTER(C.c_ulonglong)]),
    "p2h_silu_quant_rows": (_i, [_i, _i, _vp, _i, _vp, _i, _vp, _vp]),
    "p2h_concat_heads_quant_rows": (_i, [_i, _i, _i, _vp, _vp, _i, _vp, _vp]),
    "p2h_channel_major_quant_rows": (_i, [_i, _i, _vp, _vp, _i, _vp, _vp]),
    "p2h_q_bytes": (C.c_size_t, [_i, _i]),
    "p2h_fvb_gemm_q8a": (_i, [_i, _i, _i, _i, _f, _vp, _i, _vp, _vp, _f, _vp, _i, _vp, _sz, _vp]),
    "p2h_fvb_gemm_q8a_next": (_i, [_i, _i, _i, _i, _f, _vp, _i, _vp, _vp, _f, _vp, _i, _vp, _sz, _vp, _vp]),
    "p2h_fvb_gemm_q8a_silu": (_i, [_i, _i, _i, _i, _f, _vp, _i, _vp, _vp, _vp, _vp, _sz, _vp]),
    "p2h_fvb_gemm_q8a_grouped": (_i, [_i, _i, _i, _i, _f, _vp, _i, _vp, _vp, _i, _f, _vp, _i, _vp]),
    "p2h_fvb_q8a_workspace_bytes": (_sz, [_i, _i, _i, _i]),
    "p2h_fvb_plan": (C.c_char_p, [_i, _i, _i, _i, _i]),
    "p2h_fvb_gemm": (_i, [_i, _i, _i, _i, _f, _vp, _i, _vp, _f, _vp, _i, _vp, _sz, _vp]),
    "p2h_fvb_workspace_bytes": (_sz, [_i, _i, _i, _i]),
    "p2h_fvb_acc_i32": (_i, [_i, _i, _i, _i, _vp, _i, _vp, _vp, _vp, _i, _vp]),
    "p2h_scale_c": (_i, [_i, _i, _f, _vp, _i, _vp]),
    "p2h_q8b_gemm_q8a": (_i, [_i, _i, _i, _f, _vp, _i, _vp, _vp, _i, _vp, _f, _vp, _i, _vp]),
    "p2h_q8b_gemm": (_i, [_i, _i, _i, _i, _f, _vp, _i, _vp, _i, _vp, _f, _vp, _i, _vp, _sz, _vp]),
    "p2h_q8b_workspace_bytes": (_sz, [_i, _i, _i, _i]),
    "p2h_sgemm": (_i, [_i, _i, _i, _i, _i, _f, _vp, _i, _vp, _i, _f, _vp, _i, _vp]),
    "p2h_sgemm_batched": (_i, [_i, _i, _i, _i, _i, _f, _vp, _i, C.c_longlong, _vp, _i, C.c_longlong, _f, _vp, _i,
                               C.c_longlong, _i, _vp]),
    "p2h_gather_heads": (_i, [_i, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp]),
    "p2h_transpose_pos": (_i, [_i, _vp, _vp, _vp]),
    "p2h_combine_softmax": (_i, [_i, _vp, _vp, _vp]),
    "p2h_attention_heads": (_i, [_i, _vp, _vp, _vp, _vp, _vp, _vp]),
    "p2h_attention_rows": (_i, [_i, _vp, _vp, _vp, _vp, _vp, _vp]),
    "p2h_glu_depthwise_conv_silu": (_i, [_i, _vp, _vp, _vp, _vp, _vp]),
    "p2h_glu_depthwise_conv_silu_rows": (_i, [_i, _vp, _vp, _vp, _vp, _vp]),
    "p2h_glu_depthwise_conv_silu_quant_rows": (_i, [_i, _vp, _vp, _vp, _vp, _i, _vp, _vp]),
    "p2h_conformer_stack_workspace_bytes": (_sz, [_i, _i, _i]),
    "p2h_conformer_stack": (_i, [_i, _vp, _i, _i, _vp, _vp, _vp, _sz, _vp]),
    "p2h_glu_channel_major": (_i, [_i, _vp, _vp, _vp]),
    "p2h_depthwise_conv_silu": (_i, [_i, _vp, _vp, _vp, _vp, _vp]),
    "p2h_silu": (_i, [_sz, _vp, _vp]),
    "p2h_add_residual": (_i, [_i, _vp, _vp, _f, _vp]),
    "p2h_layer_norm_rows": (_i, [_i, _i, _vp, _i, _vp, _vp, _vp, _i, _vp]),
    "p2h_concat_heads_rows": (_i, [_i, _vp, _vp, _vp]),
    "p2h_channel_major_rows": (_i, [_i, _vp, _vp, _vp]),
    "p2h_conformer_block_workspace_bytes": (_sz, [_i, _i]),
    "p2h_conformer_block": (_i, [_i, _vp, _i, _vp, _vp, _vp, _sz, _vp]),
}

_hip = None
_gen = None


def hip():
    """libp2hip.so with its prototypes declared; raises if the library is missing (no CPU fallback exists)."""
    global _hip
    if _hip is None:
        if not os.path.exists(HIP_SO):
            raise P2Error(f"{HIP_SO} is not built: run __graft_entry__.build() or make -C phonon-2-c_amd")
        L = C.CDLL(HIP_SO)
        for name, (res, args) in _HIP_SIG.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _hip = L
    return _hip


def last_error():
    return hip().p2h_last_error().decode(errors="replace")


def _ok(rc, what):
    if rc != 0:
        raise P2Error(f"{what}: {last_error()} (rc {rc})")


def reload_switches():
    """Re-read the library's P2H_* tuning and comparison switches from the environment (read once at init)."""
    _ok(hip().p2h_reload_switches(), "p2h_reload_switches")


def init():
    _ok(hip().p2h_init(), "p2h_init")
    return hip().p2h_device_name().decode()


def device_cu_count():
    return hip().p2h_device_cu_count()


# ── device memory ───────────────────────────────────────────────────────────────────────────────────────────────

class DeviceBuffer:
    """A device allocation; .ptr is the device address."""

    def __init__(self, nbytes):
        self.nbytes = int(nbytes)
        self.ptr = hip().p2h_malloc(max(self.nbytes, 1))
        if not self.ptr:
            raise P2Error(f"p2h_malloc({self.nbytes}): {last_error()}")

    def free(self):
        if self.ptr:
            hip().p2h_free(self.ptr)
            self.ptr = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass

    def upload(self, arr, stream=None, offset=0):
        arr = np.ascontiguousarray(arr)
        assert offset + arr.nbytes <= self.nbytes, "upload beyond the buffer"
        _ok(hip().p2h_memcpy_h2d(self.ptr + offset, arr.ctypes.data, arr.nbytes, stream), "h2d")
        sync(stream)
        return self

    def download(self, shape, dtype, stream=None, offset=0):
        out = np.empty(shape, dtype)
        assert offset + out.nbytes <= self.nbytes, "download beyond the buffer"
        sync(stream)
        _ok(hip().p2h_memcpy_d2h(out.ctypes.data, self.ptr + offset, out.nbytes, stream), "d2h")
        sync(stream)
        return out

    def zero(self, stream=None):
        _ok(hip().p2h_memset(self.ptr, 0, self.nbytes, stream), "memset")
        return self


def to_device(arr, stream=None, pad=0):
    arr = np.ascontiguousarray(arr)
    b = DeviceBuffer(arr.nbytes + pad)
    if pad:
        b.zero(stream)
    return b.upload(arr, stream)


def sync(stream=None):
    _ok(hip().p2h_stream_sync(stream), "stream sync")


class Stream:
    def __init__(self):
        self.ptr = hip().p2h_stream_create()
        if not self.ptr:
            raise P2Error(last_error())

    def sync(self):
        sync(self.ptr)

    def wait(self, event):
        """Work queued on this stream after this call waits for `event` (a dependency edge under capture)."""
        _ok(hip().p2h_stream_wait_event(self.ptr, event.ptr), "stream wait event")

    def hold(self, usec):
        """Keep the stream busy for about `usec` microseconds, so launches queued behind run back to back."""
        _ok(hip().p2h_stream_hold(self.ptr, int(usec)), "stream hold")

    def __del__(self):
        try:
            if self.ptr:
                hip().p2h_stream_destroy(self.ptr)
        except Exception:
            pass


class Graph:
    """Capture the calls made inside `with Graph(stream) as g:` on `stream`, then g.launch() replays them."""

    def __init__(self, stream):
        self.stream = stream
        self.ptr = None

    def __enter__(self):
        _ok(hip().p2h_capture_begin(self.stream.ptr), "p2h_capture_begin")
        return self

    def __exit__(self, et, ev, tb):
        out = C.c_void_p()
        rc = hip().p2h_capture_end(self.stream.ptr, C.byref(out))
        if et is None:
            _ok(rc, "p2h_capture_end")
            self.ptr = out.value
        return False

    def launch(self):
        _ok(hip().p2h_graph_launch(self.ptr, self.stream.ptr), "p2h_graph_launch")

    def __del__(self):
        try:
            if self.ptr:
                hip().p2h_graph_destroy(self.ptr)
        except Exception:
            pass


class Event:
    def __init__(self):
        self.ptr = hip().p2h_event_create()
        if not self.ptr:
            raise P2Error(last_error())

    def record(self, stream=None):
        _ok(hip().p2h_event_record(self.ptr, stream), "event record")

    def sync(self):
        _ok(hip().p2h_event_sync(self.ptr), "event sync")

    def elapsed_ms(self, end):
        ms = hip().p2h_event_elapsed_ms(self.ptr, end.ptr)
        if ms < 0:
            raise P2Error("hipEventElapsedTime failed")
        return ms

    def __del__(self):
        try:
            if self.ptr:
                hip().p2h_event_destroy(self.ptr)
        except Exception:
            pass


# ── weights ─────────────────────────────────────────────────────────────────────────────────────────────────────

class FvWeight:
    """A device-resident five-value weight [K, N] uploaded from host planes."""

    def __init__(self, signs, flags, lo, hi, K, N):
        s = np.ascontiguousarray(signs, np.uint8)
        f = np.ascontiguousarray(flags, np.uint8)
        l = np.ascontiguousarray(lo, np.float32)
        h = np.ascontiguousarray(hi, np.float32)
        assert s.size == K * N // 4 and f.size == K * N // 8 and l.size == N and h.size == N
        self.K, self.N = K, N
        self.ptr = hip().p2h_fv_weight_upload(s.ctypes.data, f.ctypes.data, l.ctypes.data, h.ctypes.data, K, N)
        if not self.ptr:
            raise P2Error(f"p2h_fv_weight_upload: {last_error()}")

    @classmethod
    def wrap(cls, d_signs, d_flags, d_lo, d_hi, K, N, keep=()):
        """A weight made from planes already in device memory (p2h_fv_weight_wrap); `keep` holds the device
        buffers whose lo and hi the weight goes on using."""
        self = cls.__new__(cls)
        self.K, self.N, self._keep = K, N, tuple(keep)
        self.ptr = hip().p2h_fv_weight_wrap(d_signs, d_flags, d_lo, d_hi, K, N)
        if not self.ptr:
            raise P2Error(f"p2h_fv_weight_wrap: {last_error()}")
        return self

    def device_bytes(self):
        return hip().p2h_weight_device_bytes(self.ptr)

    def free(self):
        if self.ptr:
            hip().p2h_weight_free(self.ptr)
            self.ptr = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


def q_ld(K):
    return hip().p2h_q_ld(K)


def q_bytes(M, K):
    """Bytes of a tiled quantised-activation buffer for M rows (rows padded to 16, columns to q_ld(K))."""
    return hip().p2h_q_bytes(M, K)


def q_tile(q, ldq):
    """Row-major int8 q [M, <= ldq] → the library's tiled layout (rows padded to 16, columns to ldq, with zeros):
    per 16 rows × 64 columns one 1 KB block of 64 lanes × 16 bytes, lane = (column/16 % 4)·16 + row % 16."""
    q = np.asarray(q, np.int8)
    M, K = q.shape
    Mp = (M + 15) // 16 * 16
    full = np.zeros((Mp, ldq), np.int8)
    full[:M, :K] = q
    return np.ascontiguousarray(full.reshape(Mp // 16, 16, ldq // 64, 4, 16).transpose(0, 2, 3, 1, 4)).reshape(-1)


def q_untile(t, M, ldq):
    """Inverse of q_tile: the tiled buffer → row-major [roundup(M, 16), ldq]."""
    Mp = (M + 15) // 16 * 16
    t = np.asarray(t, np.int8)[: Mp * ldq]
    return np.ascontiguousarray(t.reshape(Mp // 16, ldq // 64, 4, 16, 16).transpose(0, 3, 1, 2, 4)).reshape(Mp, ldq)


def workspace_bytes(mode, M, N, K):
    """Workspace of p2h_fvb_gemm (fp32 activations): quantised rows plus the split-K area."""
    return hip().p2h_fvb_workspace_bytes(MODES.get(mode, mode), M, N, K)


def plan(mode, M, N, K, with_workspace=True):
    """The tile and K split the library picks for this shape."""
    return hip().p2h_fvb_plan(MODES.get(mode, mode), M, N, K, 1 if with_workspace else 0).decode()


def q8a_workspace_bytes(mode, M, N, K):
    return hip().p2h_fvb_q8a_workspace_bytes(MODES.get(mode, mode), M, N, K)


class Workspace(DeviceBuffer):
    """Device scratch for the GEMM entries (quantised rows, split-K partial sums)."""

    def __init__(self, nbytes, stream=None):
        super().__init__(max(int(nbytes), 256))


# ── device-pointer entry points (asynchronous on `stream`) ───────────────────────────────────────────────────────

def quant_rows_dev(M, K, dA, lda, dQ, ldq, dS, stream=None):
    _ok(hip().p2h_quant_rows(M, K, dA, lda, dQ, ldq, dS, stream), "p2h_quant_rows")


def recip_selftest():
    """p2h_recip_selftest: (mismatches, smallest mismatching bit pattern or 2^64 - 1, values checked)."""
    r = (C.c_ulonglong * 3)()
    _ok(hip().p2h_recip_selftest(r), "p2h_recip_selftest")
    return int(r[0]), int(r[1]), int(r[2])


def layer_norm_quant_rows_dev(M, D, dX, ldx, dGamma, dBeta, dQ, ldq, dS, stream=None):
    _ok(hip().p2h_layer_norm_quant_rows(M, D, dX, ldx, dGamma, dBeta, dQ, ldq, dS, stream),
        "p2h_layer_norm_quant_rows")


def silu_quant_rows_dev(M, K, dH, ldh, dQ, ldq, dS, stream=None):
    _ok(hip().p2h_silu_quant_rows(M, K, dH, ldh, dQ, ldq, dS, stream), "p2h_silu_quant_rows")


def concat_heads_quant_rows_dev(H, T, Dh, dAttnH, dQ, ldq, dS, stream=None):
    _ok(hip().p2h_concat_heads_quant_rows(H, T, Dh, dAttnH, dQ, ldq, dS, stream), "p2h_concat_heads_quant_rows")


def channel_major_quant_rows_dev(D, T, dDW, dQ, ldq, dS, stream=None):
    _ok(hip().p2h_channel_major_quant_rows(D, T, dDW, dQ, ldq, dS, stream), "p2h_channel_major_quant_rows")


def fvb_gemm_q8a_dev(mode, M, N, K, alpha, dQ, ldq, dS, w, beta, dC, ldc, ws=None, ws_bytes=0, stream=None):
    _ok(hip().p2h_fvb_gemm_q8a(MODES.get(mode, mode), M, N, K, alpha, dQ, ldq, dS, w.ptr, beta, dC, ldc, ws,
                               ws_bytes, stream), "p2h_fvb_gemm_q8a")


def q8b_gemm_dev(mode, M, N, K, alpha, dA, lda, dB, ldb, dBs, beta, dC, ldc, ws=None, ws_bytes=0, stream=None):
    """p2h_q8b_gemm on device pointers: fp32 rows A [M][lda] (quantised in the call in the int8 modes)."""
    _ok(hip().p2h_q8b_gemm(MODES.get(mode, mode), M, N, K, alpha, dA, lda, dB, ldb, dBs, beta, dC, ldc, ws,
                           ws_bytes, stream), "p2h_q8b_gemm")


def q8b_gemm_q8a_dev(M, N, K, alpha, dQ, ldq, dS, dB, ldb, dBs, beta, dC, ldc, stream=None):
    """p2h_q8b_gemm_q8a on device pointers: rows already quantised (tiled, pitch ldq) with their scales."""
    _ok(hip().p2h_q8b_gemm_q8a(M, N, K, alpha, dQ, ldq, dS, dB, ldb, dBs, beta, dC, ldc, stream),
        "p2h_q8b_gemm_q8a")


def fvb_gemm_q8a_silu_dev(mode, M, N, K, alpha, dQ, ldq, dS, w, dC, ws=None, ws_bytes=0, stream=None):
    """SiLU(alpha·A·W) into dC [M, N] (ldc = N): the feed-forward up-projection with SiLU applied as C is stored."""
    _ok(hip().p2h_fvb_gemm_q8a_silu(MODES.get(mode, mode), M, N, K, alpha, dQ, ldq, dS, w.ptr, dC, ws, ws_bytes,
                                    stream), "p2h_fvb_gemm_q8a_silu")


def fvb_gemm_q8a_next_dev(mode, M, N, K, alpha, dQ, ldq, dS, w, beta, dC, ldc, ws=None, ws_bytes=0, next_w=None,
                          stream=None):
    """fvb_gemm_q8a_dev that also reads the records of `next_w` (the next weight the caller runs) ahead."""
    _ok(hip().p2h_fvb_gemm_q8a_next(MODES.get(mode, mode), M, N, K, alpha, dQ, ldq, dS, w.ptr, beta, dC, ldc, ws,
                                    ws_bytes, next_w.ptr if next_w is not None else None, stream),
        "p2h_fvb_gemm_q8a_next")


def fvb_gemm_q8a_grouped_dev(mode, M, N, K, alpha, dQ, ldq, dS, weights, beta, dCs, ldc, stream=None):
    """p2h_fvb_gemm_q8a_grouped: one product per weight against the same quantised rows, outputs dCs[i]."""
    n = len(weights)
    assert len(dCs) == n
    wa = (C.c_void_p * max(n, 1))(*[w.ptr for w in weights])
    ca = (C.c_void_p * max(n, 1))(*dCs)
    _ok(hip().p2h_fvb_gemm_q8a_grouped(MODES.get(mode, mode), M, N, K, alpha, dQ, ldq, dS, wa, n, beta, ca, ldc,
                                       stream), "p2h_fvb_gemm_q8a_grouped")


def fvb_gemm_dev(mode, M, N, K, alpha, dA, lda, w, beta, dC, ldc, ws, ws_bytes, stream=None):
    _ok(hip().p2h_fvb_gemm(MODES.get(mode, mode), M, N, K, alpha, dA, lda, w.ptr, beta, dC, ldc, ws, ws_bytes,
                           stream), "p2h_fvb_gemm")


# ── host-array conveniences (upload, run, download, synchronise) ─────────────────────────────────────────────────

def quant_rows(A, K=None):
    """p2h_quant_rows on a host matrix: q as row-major [roundup(M, 16), ldq] (untiled, pads included), scales [M]."""
    A = np.ascontiguousarray(A, np.float32)
    M, lda = A.shape
    K = lda if K is None else K
    ldq = q_ld(K)
    dA = to_device(A)
    nbytes = max(q_bytes(M, K), 16)
    dQ = DeviceBuffer(nbytes)
    dQ.upload(np.full(nbytes, 0x5A, np.uint8))   # every byte, pads included, must be written
    dS = DeviceBuffer(max(M, 1) * 4)
    quant_rows_dev(M, K, dA.ptr, lda, dQ.ptr, ldq, dS.ptr)
    q = q_untile(dQ.download((q_bytes(M, K),), np.int8), M, ldq) if M > 0 else np.zeros((0, ldq), np.int8)
    s = dS.download((M,), np.float32)
    return q, s


def _produced(M, K, run):
    """Run a producer into fresh device buffers (every byte preset, so pads must be written) and download."""
    ldq = q_ld(K)
    nbytes = max(q_bytes(M, K), 16)
    dQ = DeviceBuffer(nbytes)
    dQ.upload(np.full(nbytes, 0x5A, np.uint8))
    dS = DeviceBuffer(max(M, 1) * 4)
    run(dQ.ptr, ldq, dS.ptr)
    q = q_untile(dQ.download((q_bytes(M, K),), np.int8), M, ldq) if M > 0 else np.zeros((0, ldq), np.int8)
    return q, dS.download((M,), np.float32)


def layer_norm_quant_rows(X, gamma, beta, D=None):
    """p2h_layer_norm_quant_rows on host arrays X [M, ldx] (first D columns): q untiled [roundup(M, 16), ldq]."""
    X = np.ascontiguousarray(X, np.float32)
    M, ldx = X.shape
    D = ldx if D is None else D
    dX, dG, dB = to_device(X), to_device(np.ascontiguousarray(gamma, np.float32)), \
        to_device(np.ascontiguousarray(beta, np.float32))
    return _produced(M, D, lambda dQ, ldq, dS: layer_norm_quant_rows_dev(M, D, dX.ptr, ldx, dG.ptr, dB.ptr, dQ, ldq,
                                                                         dS))


def silu_quant_rows(H, K=None):
    H = np.ascontiguousarray(H, np.float32)
    M, ldh = H.shape
    K = ldh if K is None else K
    dH = to_device(H)
    return _produced(M, K, lambda dQ, ldq, dS: silu_quant_rows_dev(M, K, dH.ptr, ldh, dQ, ldq, dS))


def concat_heads_quant_rows(attn_h):
    attn_h = np.ascontiguousarray(attn_h, np.float32)
    H, T, Dh = attn_h.shape
    dA = to_device(attn_h)
    return _produced(T, H * Dh, lambda dQ, ldq, dS: concat_heads_quant_rows_dev(H, T, Dh, dA.ptr, dQ, ldq, dS))


def channel_major_quant_rows(dw):
    dw = np.ascontiguousarray(dw, np.float32)
    D, T = dw.shape
    dW = to_device(dw)
    return _produced(T, D, lambda dQ, ldq, dS: channel_major_quant_rows_dev(D, T, dW.ptr, dQ, ldq, dS))


def fvb_gemm(mode, A, w, alpha=1.0, beta=0.0, C0=None, K=None, ws=None):
    """p2h_fvb_gemm on host arrays: A [M, lda] (first K columns used), C0 [M, ldc] (ldc >= N) or None."""
    A = np.ascontiguousarray(A, np.float32)
    M, lda = A.shape
    K = w.K if K is None else K
    N = w.N
    C0 = np.zeros((M, N), np.float32) if C0 is None else np.ascontiguousarray(C0, np.float32)
    ldc = C0.shape[1]
    dA = to_device(A)
    dC = to_device(C0)
    if ws is None:
        ws = Workspace(workspace_bytes(mode, M, N, K))
    fvb_gemm_dev(mode, M, N, K, alpha, dA.ptr, lda, w, beta, dC.ptr, ldc, ws.ptr, ws.nbytes)
    return dC.download((M, ldc), np.float32)


def fvb_gemm_q8a(mode, q, scales, w, alpha=1.0, beta=0.0, C0=None, split=True, ws=None):
    """p2h_fvb_gemm_q8a on a quantised host matrix q [M, K] (re-padded to the library's ldq); split=False runs
    without a workspace (no K split)."""
    q = np.ascontiguousarray(q, np.int8)
    M, K = q.shape
    N = w.N
    ldq = q_ld(K)
    C0 = np.zeros((M, N), np.float32) if C0 is None else np.ascontiguousarray(C0, np.float32)
    dQ, dS, dC = to_device(q_tile(q, ldq)), to_device(np.ascontiguousarray(scales, np.float32)), to_device(C0)
    if ws is None and split:
        ws = Workspace(q8a_workspace_bytes(mode, M, N, K))
    fvb_gemm_q8a_dev(mode, M, N, K, alpha, dQ.ptr, ldq, dS.ptr, w, beta, dC.ptr, C0.shape[1],
                     ws.ptr if ws else None, ws.nbytes if ws else 0)
    return dC.download(C0.shape, np.float32)


def fvb_gemm_q8a_silu(mode, q, scales, w, alpha=1.0, ws=None):
    """p2h_fvb_gemm_q8a_silu on a quantised host matrix q [M, K]: SiLU(alpha·A·W) as [M, N]."""
    q = np.ascontiguousarray(q, np.int8)
    M, K = q.shape
    N = w.N
    ldq = q_ld(K)
    dQ, dS = to_device(q_tile(q, ldq)), to_device(np.ascontiguousarray(scales, np.float32))
    dC = DeviceBuffer(max(M * N, 1) * 4)
    dC.upload(np.full(max(M * N, 1), np.nan, np.float32))   # every output must be written
    if ws is None:
        ws = Workspace(q8a_workspace_bytes(mode, M, N, K))
    _ok(hip().p2h_fvb_gemm_q8a_silu(MODES.get(mode, mode), M, N, K, alpha, dQ.ptr, ldq, dS.ptr, w.ptr, dC.ptr,
                                    ws.ptr, ws.nbytes, None), "p2h_fvb_gemm_q8a_silu")
    return dC.download((M, N), np.float32)


def fvb_acc_i32(mode, q, w):
    """The raw int32 sums of the int8 kernel over all K: one matrix (int8w) or the S and T sums (int8)."""
    q = np.ascontiguousarray(q, np.int8)
    M, K = q.shape
    N = w.N
    ldq = q_ld(K)
    dQ = to_device(q_tile(q, ldq))
    d1 = DeviceBuffer(M * N * 4)
    d2 = DeviceBuffer(M * N * 4)
    m = MODES.get(mode, mode)
    _ok(hip().p2h_fvb_acc_i32(m, M, N, K, dQ.ptr, ldq, w.ptr, d1.ptr, d2.ptr if m == INT8 else None, N, None),
        "p2h_fvb_acc_i32")
    a1 = d1.download((M, N), np.int32)
    return (a1, d2.download((M, N), np.int32)) if m == INT8 else a1


def fv_pack_codes(w):
    d = DeviceBuffer(w.K * w.N)
    _ok(hip().p2h_fv_pack_codes(w.ptr, d.ptr, None), "p2h_fv_pack_codes")
    return d.download((w.K * w.N,), np.int8)


def q8b_workspace_bytes(mode, M, N, K):
    return hip().p2h_q8b_workspace_bytes(MODES.get(mode, mode), M, N, K)


def q8b_gemm(mode, A, B, scales, alpha=1.0, beta=0.0, C0=None, ws_bytes=None):
    """p2h_q8b_gemm on host arrays; ws_bytes overrides the workspace size (default: room to split K)."""
    A = np.ascontiguousarray(A, np.float32)
    B = np.ascontiguousarray(B, np.int8)
    M, K = A.shape
    N = B.shape[1]
    C0 = np.zeros((M, N), np.float32) if C0 is None else np.ascontiguousarray(C0, np.float32)
    dA, dB, dS, dC = to_device(A), to_device(B), to_device(np.ascontiguousarray(scales, np.float32)), to_device(C0)
    ws = Workspace(q8b_workspace_bytes(mode, M, N, K) if ws_bytes is None else ws_bytes)
    _ok(hip().p2h_q8b_gemm(MODES.get(mode, mode), M, N, K, alpha, dA.ptr, K, dB.ptr, N, dS.ptr, beta, dC.ptr,
                           C0.shape[1], ws.ptr, ws.nbytes, None), "p2h_q8b_gemm")
    return dC.download(C0.shape, np.float32)


def sgemm(A, B, transA=False, transB=False, alpha=1.0, beta=0.0, C0=None):
    A = np.ascontiguousarray(A, np.float32)
    B = np.ascontiguousarray(B, np.float32)
    M = A.shape[1] if transA else A.shape[0]
    K = A.shape[0] if transA else A.shape[1]
    N = B.shape[0] if transB else B.shape[1]
    C0 = np.zeros((M, N), np.float32) if C0 is None else np.ascontiguousarray(C0, np.float32)
    dA, dB, dC = to_device(A), to_device(B), to_device(C0)
    _ok(hip().p2h_sgemm(int(transA), int(transB), M, N, K, alpha, dA.ptr, A.shape[1], dB.ptr, B.shape[1], beta,
                        dC.ptr, C0.shape[1], None), "p2h_sgemm")
    return dC.download(C0.shape, np.float32)


def sgemm_batched_dev(transA, transB, M, N, K, alpha, dA, lda, sA, dB, ldb, sB, beta, dC, ldc, sC, batch,
                      stream=None):
    _ok(hip().p2h_sgemm_batched(int(transA), int(transB), M, N, K, alpha, dA, lda, sA, dB, ldb, sB, beta, dC, ldc,
                                sC, batch, stream), "p2h_sgemm_batched")


def sgemm_batched(A, B, transA=False, transB=False, alpha=1.0, beta=0.0, C0=None):
    """p2h_sgemm_batched on host arrays A [b, ., .], B [b, ., .] (contiguous per entry)."""
    A = np.ascontiguousarray(A, np.float32)
    B = np.ascontiguousarray(B, np.float32)
    b = A.shape[0]
    M = A.shape[2] if transA else A.shape[1]
    K = A.shape[1] if transA else A.shape[2]
    N = B.shape[1] if transB else B.shape[2]
    C0 = np.zeros((b, M, N), np.float32) if C0 is None else np.ascontiguousarray(C0, np.float32)
    dA, dB, dC = to_device(A), to_device(B), to_device(C0)
    sgemm_batched_dev(transA, transB, M, N, K, alpha, dA.ptr, A.shape[2], A.shape[1] * A.shape[2], dB.ptr,
                      B.shape[2], B.shape[1] * B.shape[2], beta, dC.ptr, N, M * N, b)
    return dC.download(C0.shape, np.float32)


# ── the conformer block between its linears (model widths D = 1024, 8 heads of 128) ─────────────────────────────

D_MODEL, N_HEADS, HEAD_DIM, CONV_K = 1024, 8, 128, 9


def _f32(a):
    return np.ascontiguousarray(a, np.float32)


def gather_heads(qkv, bias_u, bias_v):
    """p2h_gather_heads on host arrays: QKV [T, 3072] → (Q_u, Q_v, V_h [8, T, 128], K_t [8, 128, T])."""
    qkv = _f32(qkv)
    T = qkv.shape[0]
    dq, du, dv = to_device(qkv), to_device(_f32(bias_u)), to_device(_f32(bias_v))
    outs = [DeviceBuffer(T * D_MODEL * 4) for _ in range(4)]
    _ok(hip().p2h_gather_heads(T, dq.ptr, du.ptr, dv.ptr, outs[0].ptr, outs[1].ptr, outs[2].ptr, outs[3].ptr, None),
        "p2h_gather_heads")
    qu, qv, vh = (outs[i].download((N_HEADS, T, HEAD_DIM), np.float32) for i in (0, 1, 3))
    return qu, qv, outs[2].download((N_HEADS, HEAD_DIM, T), np.float32), vh


def transpose_pos(P):
    P = _f32(P)
    L = P.shape[0]
    dP, dPt = to_device(P), DeviceBuffer(P.nbytes)
    _ok(hip().p2h_transpose_pos(L, dP.ptr, dPt.ptr, None), "p2h_transpose_pos")
    return dPt.download((N_HEADS, HEAD_DIM, L), np.float32)


def combine_softmax(ac, bd):
    """ac [8·T, T], bd [8·T, 2T−1] → softmax((ac + shift(bd)) / sqrt(128)) per row."""
    ac = _f32(ac)
    T = ac.shape[1]
    dA, dB = to_device(ac), to_device(_f32(bd))
    _ok(hip().p2h_combine_softmax(T, dA.ptr, dB.ptr, None), "p2h_combine_softmax")
    return dA.download(ac.shape, np.float32)


def attention_heads(qkv, bias_u, bias_v, P, rows=False):
    """p2h_attention_heads on host arrays: QKV [T, 3072], bias_u / bias_v [1024], P [2T − 1, 1024] → [8, T, 128]
    (rows: p2h_attention_rows → [T, 1024])."""
    qkv = _f32(qkv)
    T = qkv.shape[0]
    dq, du, dv, dp = to_device(qkv), to_device(_f32(bias_u)), to_device(_f32(bias_v)), to_device(_f32(P))
    dO = DeviceBuffer(T * D_MODEL * 4)
    if rows:
        _ok(hip().p2h_attention_rows(T, dq.ptr, du.ptr, dv.ptr, dp.ptr, dO.ptr, None), "p2h_attention_rows")
        return dO.download((T, D_MODEL), np.float32)
    _ok(hip().p2h_attention_heads(T, dq.ptr, du.ptr, dv.ptr, dp.ptr, dO.ptr, None), "p2h_attention_heads")
    return dO.download((N_HEADS, T, HEAD_DIM), np.float32)


def glu_channel_major(pw1):
    pw1 = _f32(pw1)
    T = pw1.shape[0]
    dP, dG = to_device(pw1), DeviceBuffer(T * D_MODEL * 4)
    _ok(hip().p2h_glu_channel_major(T, dP.ptr, dG.ptr, None), "p2h_glu_channel_major")
    return dG.download((D_MODEL, T), np.float32)


def depthwise_conv_silu(gated, w, b):
    gated = _f32(gated)
    T = gated.shape[1]
    dX, dW, dB, dO = to_device(gated), to_device(_f32(w)), to_device(_f32(b)), DeviceBuffer(gated.nbytes)
    _ok(hip().p2h_depthwise_conv_silu(T, dX.ptr, dW.ptr, dB.ptr, dO.ptr, None), "p2h_depthwise_conv_silu")
    return dO.download(gated.shape, np.float32)


def glu_depthwise_conv_silu(pw1, w, b, rows=False):
    """pw1 [T, 2048] → SiLU(depthwise conv(GLU(pw1))) as [1024, T] (rows: as [T, 1024]), one kernel."""
    pw1 = _f32(pw1)
    T = pw1.shape[0]
    dP, dW, dB, dO = to_device(pw1), to_device(_f32(w)), to_device(_f32(b)), DeviceBuffer(T * D_MODEL * 4)
    if rows:
        _ok(hip().p2h_glu_depthwise_conv_silu_rows(T, dP.ptr, dW.ptr, dB.ptr, dO.ptr, None),
            "p2h_glu_depthwise_conv_silu_rows")
        return dO.download((T, D_MODEL), np.float32)
    _ok(hip().p2h_glu_depthwise_conv_silu(T, dP.ptr, dW.ptr, dB.ptr, dO.ptr, None), "p2h_glu_depthwise_conv_silu")
    return dO.download((D_MODEL, T), np.float32)


def glu_depthwise_conv_silu_quant_rows(pw1, w, b, ldq=None):
    """pw1 [T, 2048] → SiLU(depthwise conv(GLU(pw1))) rows quantised in the same kernel: (q untiled
    [roundup(T, 16), ldq], scales [T]). Every byte of Q is preset, so its pads must be written."""
    pw1 = _f32(pw1)
    T = pw1.shape[0]
    ldq = q_ld(D_MODEL) if ldq is None else ldq
    nbytes = (T + 15) // 16 * 16 * ldq
    dP, dW, dB = to_device(pw1), to_device(_f32(w)), to_device(_f32(b))
    dQ = DeviceBuffer(max(nbytes, 16))
    dQ.upload(np.full(max(nbytes, 16), 0x5A, np.uint8))
    dS = DeviceBuffer(max(T, 1) * 4)
    _ok(hip().p2h_glu_depthwise_conv_silu_quant_rows(T, dP.ptr, dW.ptr, dB.ptr, dQ.ptr, ldq, dS.ptr, None),
        "p2h_glu_depthwise_conv_silu_quant_rows")
    return q_untile(dQ.download((nbytes,), np.int8), T, ldq), dS.download((T,), np.float32)


def silu(x):
    x = _f32(x)
    d = to_device(x)
    _ok(hip().p2h_silu(x.size, d.ptr, None), "p2h_silu")
    return d.download(x.shape, np.float32)


def add_residual(X, Y, alpha):
    X = _f32(X)
    dX, dY = to_device(X), to_device(_f32(Y))
    _ok(hip().p2h_add_residual(X.shape[0], dX.ptr, dY.ptr, alpha, None), "p2h_add_residual")
    return dX.download(X.shape, np.float32)


def layer_norm2_quant_rows(X, gamma1, beta1, gamma2, beta2, in_place=False):
    """p2h_layer_norm2_quant_rows on host arrays X [M, D]: (Y = LayerNorm(X; gamma1, beta1) as fp32 [M, D],
    q untiled [roundup(M, 16), ldq], scales [M]) of LayerNorm(Y; gamma2, beta2)."""
    X = _f32(X)
    M, D = X.shape
    dX = to_device(X)
    dY = dX if in_place else DeviceBuffer(X.nbytes)
    g1, b1, g2, b2 = (to_device(_f32(v)) for v in (gamma1, beta1, gamma2, beta2))
    q, s = _produced(M, D, lambda dQ, ldq, dS: _ok(hip().p2h_layer_norm2_quant_rows(
        M, D, dX.ptr, D, g1.ptr, b1.ptr, dY.ptr, D, g2.ptr, b2.ptr, dQ, ldq, dS, None), "p2h_layer_norm2_quant_rows"))
    return dY.download(X.shape, np.float32), q, s


def layer_norm_rows(X, gamma, beta, in_place=False):
    X = _f32(X)
    M, D = X.shape
    dX, dg, db = to_device(X), to_device(_f32(gamma)), to_device(_f32(beta))
    dY = dX if in_place else DeviceBuffer(X.nbytes)
    _ok(hip().p2h_layer_norm_rows(M, D, dX.ptr, D, dg.ptr, db.ptr, dY.ptr, D, None), "p2h_layer_norm_rows")
    return dY.download(X.shape, np.float32)


def concat_heads_rows(attn_h):
    attn_h = _f32(attn_h)
    T = attn_h.shape[1]
    dA, dY = to_device(attn_h), DeviceBuffer(T * D_MODEL * 4)
    _ok(hip().p2h_concat_heads_rows(T, dA.ptr, dY.ptr, None), "p2h_concat_heads_rows")
    return dY.download((T, D_MODEL), np.float32)


def channel_major_rows(dw):
    dw = _f32(dw)
    T = dw.shape[1]
    dA, dY = to_device(dw), DeviceBuffer(T * D_MODEL * 4)
    _ok(hip().p2h_channel_major_rows(T, dA.ptr, dY.ptr, None), "p2h_channel_major_rows")
    return dY.download((T, D_MODEL), np.float32)


BLOCK_FIELDS = ("norm_ff1_w", "norm_ff1_b", "ff1_l1", "ff1_l2", "norm_sa_w", "norm_sa_b", "qkv", "pos", "out",
                "bias_u", "bias_v", "norm_conv_w", "norm_conv_b", "pw1", "pw2", "dw_w", "dw_b", "norm_ff2_w",
                "norm_ff2_b", "ff2_l1", "ff2_l2", "norm_out_w", "norm_out_b")
BLOCK_LINEARS = {"ff1_l1": (1024, 4096), "ff1_l2": (4096, 1024), "qkv": (1024, 3072), "pos": (1024, 1024),
                 "out": (1024, 1024), "pw1": (1024, 2048), "pw2": (1024, 1024), "ff2_l1": (1024, 4096),
                 "ff2_l2": (4096, 1024)}


class _P2hBlock(C.Structure):
    _fields_ = [(f, C.c_void_p) for f in BLOCK_FIELDS]


class Block:
    """One conformer block's weights on the device (P2hBlock): `params` maps each vector name to a float32 array and
    each linear name to (signs, flags, lo, hi)."""

    def __init__(self, params):
        self._keep = {}
        vals = {}
        for f in BLOCK_FIELDS:
            if f in BLOCK_LINEARS:
                K, N = BLOCK_LINEARS[f]
                w = FvWeight(*params[f], K, N)
                self._keep[f] = w
                vals[f] = w.ptr
            else:
                d = to_device(_f32(params[f]))
                self._keep[f] = d
                vals[f] = d.ptr
        self.c = _P2hBlock(**vals)

    def run_dev(self, mode, T, dPE, dX, ws, stream=None):
        _ok(hip().p2h_conformer_block(MODES.get(mode, mode), C.byref(self.c), T, dPE, dX, ws.ptr, ws.nbytes, stream),
            "p2h_conformer_block")

    def run(self, mode, x, pe):
        """x [T, 1024] through the block; pe [2T−1, 1024]."""
        x = _f32(x)
        T = x.shape[0]
        dX, dPE = to_device(x), to_device(_f32(pe))
        ws = Workspace(block_workspace_bytes(mode, T))
        self.run_dev(mode, T, dPE.ptr, dX.ptr, ws)
        return dX.download(x.shape, np.float32)


class Stack:
    """The blocks of one window on the device (p2h_conformer_stack): a list of Block."""

    def __init__(self, blocks):
        self.blocks = list(blocks)
        self.arr = (_P2hBlock * len(self.blocks))(*[b.c for b in self.blocks])

    def run_dev(self, mode, T, dPE, dX, ws, stream=None):
        _ok(hip().p2h_conformer_stack(MODES.get(mode, mode), C.byref(self.arr), len(self.blocks), T, dPE, dX, ws.ptr,
                                      ws.nbytes, stream), "p2h_conformer_stack")

    def run(self, mode, x, pe):
        x = _f32(x)
        T = x.shape[0]
        dX, dPE = to_device(x), to_device(_f32(pe))
        ws = Workspace(stack_workspace_bytes(mode, T, len(self.blocks)))
        self.run_dev(mode, T, dPE.ptr, dX.ptr, ws)
        return dX.download(x.shape, np.float32)


def stack_workspace_bytes(mode, T, n_blocks):
    return hip().p2h_conformer_stack_workspace_bytes(MODES.get(mode, mode), T, n_blocks)


def block_workspace_bytes(mode, T):
    return hip().p2h_conformer_block_workspace_bytes(MODES.get(mode, mode), T)


# ── the generator ───────────────────────────────────────────────────────────────────────────────────────────────

def gen():
    global _gen
    if _gen is None:
        if not os.path.exists(GEN_SO):
            raise P2Error(f"{GEN_SO} is not built")
        L = C.CDLL(GEN_SO)
        u64 = C.c_uint64
        L.p2g_activations.argtypes = [u64, u64, _i, _i, _vp]
        L.p2g_fv_weight.argtypes = [u64, u64, _i, _i, _vp, _vp, _vp, _vp]
        L.p2g_i8_weight.argtypes = [u64, u64, _i, _i, _vp, _vp]
        L.p2g_round_fp16.argtypes = [C.c_double]
        L.p2g_round_fp16.restype = C.c_float
        for n in ("p2g_activations", "p2g_fv_weight", "p2g_i8_weight"):
            getattr(L, n).restype = None
        _gen = L
    return _gen


def gen_activations(seed, tensor_id, M, K):
    A = np.empty((M, K), np.float32)
    gen().p2g_activations(seed, tensor_id, M, K, A.ctypes.data)
    return A


def gen_fv_weight(seed, tensor_id, K, N):
    signs = np.empty((K, N // 4), np.uint8)
    flags = np.empty((K, N // 8), np.uint8)
    lo = np.empty(N, np.float32)
    hi = np.empty(N, np.float32)
    gen().p2g_fv_weight(seed, tensor_id, K, N, signs.ctypes.data, flags.ctypes.data, lo.ctypes.data, hi.ctypes.data)
    return signs, flags, lo, hi


def gen_i8_weight(seed, tensor_id, K, N):
    q8 = np.empty((K, N), np.int8)
    sc = np.empty(N, np.float32)
    gen().p2g_i8_weight(seed, tensor_id, K, N, q8.ctypes.data, sc.ctypes.data)
    return q8, sc


def block_params(seed, tid0):
    """Seeded synthetic weights of one conformer block in the shapes of P2hBlock: the nine five-value linears from
    the generator (tensor ids tid0 .. tid0 + 8), norms gamma ~ U(0.5, 1.5) and beta ~ U(−0.2, 0.2), bias_u / bias_v
    ~ N(0, 0.1²), depthwise kernel ~ N(0, 0.3²) and bias ~ N(0, 0.1²)."""
    rng = np.random.default_rng(seed * 1000 + tid0)
    p = {}
    for i, (name, (K, N)) in enumerate(BLOCK_LINEARS.items()):
        p[name] = gen_fv_weight(seed, tid0 + i, K, N)
    for name in ("norm_ff1", "norm_sa", "norm_conv", "norm_ff2", "norm_out"):
        p[name + "_w"] = rng.uniform(0.5, 1.5, D_MODEL).astype(np.float32)
        p[name + "_b"] = rng.uniform(-0.2, 0.2, D_MODEL).astype(np.float32)
    p["bias_u"] = (rng.standard_normal(D_MODEL) * 0.1).astype(np.float32)
    p["bias_v"] = (rng.standard_normal(D_MODEL) * 0.1).astype(np.float32)
    p["dw_w"] = (rng.standard_normal(D_MODEL * CONV_K) * 0.3).astype(np.float32)
    p["dw_b"] = (rng.standard_normal(D_MODEL) * 0.1).astype(np.float32)
    return p
