"""ctypes wrapper over the CPU oracle (oracle/liboracle.so) and the reference build (oracle/_ref/libp2ref.so).

Test infrastructure: the reference for the HIP path's results. Only tests/, __graft_entry__.smoke() and bench.py's
cpu_baseline leg use it.
"""
import ctypes as C
import os

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
ORACLE_SO = os.path.join(ROOT, "oracle", "liboracle.so")
REF_SO = os.path.join(ROOT, "oracle", "_ref", "libp2ref.so")

INT8, EXACT, INT8W = 0, 1, 2
MODES = {"int8": INT8, "exact": EXACT, "int8w": INT8W}

_f32p = np.ctypeslib.ndpointer(np.float32, flags="C_CONTIGUOUS")
_u8p = np.ctypeslib.ndpointer(np.uint8, flags="C_CONTIGUOUS")
_i8p = np.ctypeslib.ndpointer(np.int8, flags="C_CONTIGUOUS")
_i32p = np.ctypeslib.ndpointer(np.int32, flags="C_CONTIGUOUS")
_i, _f = C.c_int, C.c_float

_lib = None


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(ORACLE_SO):
            raise RuntimeError(f"{ORACLE_SO} missing: run `make -C oracle`")
        L = C.CDLL(ORACLE_SO)
        sig = {
            "p2o_pack_planes": [_i8p, _u8p, _i, _i, _u8p, _u8p],
            "p2o_unpack_planes": [_u8p, _u8p, _i, _i, _u8p, _u8p],
            "p2o_expand_exact": [_u8p, _u8p, _f32p, _f32p, _i, _i, _f32p],
            "p2o_sgemm_fvb_exact": [_i, _i, _i, _f, _f32p, _i, _u8p, _u8p, _f32p, _f32p, _f, _f32p, _i],
            "p2o_quant_rows": [_f32p, _i, _i, _i, _i8p, _f32p],
            "p2o_clo": [_f32p, _f32p, _i, _u8p],
            "p2o_codes_i8w": [_u8p, _u8p, _f32p, _f32p, _i, _i, _i8p],
            "p2o_fv_pack_codes": [_u8p, _u8p, _f32p, _f32p, _i, _i, _i8p],
            "p2o_planes_i8": [_u8p, _u8p, _i, _i, _i8p, _i8p],
            "p2o_acc_i32": [_i8p, _i, _i, _i8p, _i, _i, _i, _i32p],
            "p2o_gemm_i8_run": [_i, _i, _i, _i, _f, _i8p, _f32p, _u8p, _u8p, _f32p, _f32p, _i, _f32p, _i],
            "p2o_gemm_q8b_run": [_i, _i, _i, _f, _i8p, _f32p, _i8p, _i, _f32p, _i, _f32p, _i],
            "p2o_sgemm_fvb": [_i, _i, _i, _i, _f, _f32p, _i, _u8p, _u8p, _f32p, _f32p, _f, _f32p, _i],
            "p2o_sgemm_q8b": [_i, _i, _i, _i, _f, _f32p, _i, _i8p, _f32p, _i, _f, _f32p, _i],
            "p2o_mode_from_env": [C.c_char_p, C.c_char_p],
            "p2o_layer_norm_row": [_f32p, _f32p, _f32p, _f32p, _i],
            "p2o_swish_row": [_f32p, _i],
            "p2o_ln_quant_rows": [_f32p, _i, _i, _i, _f32p, _f32p, _i8p, _f32p],
            "p2o_silu_quant_rows": [_f32p, _i, _i, _i, _i8p, _f32p],
            "p2o_concat_heads_quant_rows": [_f32p, _i, _i, _i, _i8p, _f32p],
            "p2o_channel_major_quant_rows": [_f32p, _i, _i, _i8p, _f32p],
            "p2o_combine_softmax": [_f32p, _f32p, _i, _i, _f],
            "p2o_glu_channel_major": [_f32p, _f32p, _i, _i],
            "p2o_dwconv": [_f32p, _f32p, _f32p, _f32p, _i, _i, _i],
            "p2o_dwconv_silu": [_f32p, _f32p, _f32p, _f32p, _i, _i, _i],
        }
        for name, args in sig.items():
            fn = getattr(L, name)
            fn.argtypes = args
            fn.restype = C.c_int if name == "p2o_mode_from_env" else None
        _lib = L
    return _lib


def _c(a, dt):
    return np.ascontiguousarray(a, dtype=dt)


def pack_planes(sign, is_hi):
    K, N = sign.shape
    s = np.zeros((K, N // 4), np.uint8)
    f = np.zeros((K, N // 8), np.uint8)
    lib().p2o_pack_planes(_c(sign, np.int8), _c(is_hi, np.uint8), K, N, s, f)
    return s, f


def unpack_planes(signs, flags, K, N):
    code = np.zeros((K, N), np.uint8)
    flag = np.zeros((K, N), np.uint8)
    lib().p2o_unpack_planes(_c(signs, np.uint8), _c(flags, np.uint8), K, N, code, flag)
    return code, flag


def expand_exact(signs, flags, lo, hi, K, N):
    W = np.zeros((K, N), np.float32)
    lib().p2o_expand_exact(_c(signs, np.uint8), _c(flags, np.uint8), _c(lo, np.float32), _c(hi, np.float32), K, N, W)
    return W


def quant_rows(A, K=None):
    A = _c(A, np.float32)
    M, lda = A.shape
    K = lda if K is None else K
    q = np.zeros((M, K), np.int8)
    sc = np.zeros(max(M, 1), np.float32)
    lib().p2o_quant_rows(A, M, K, lda, q, sc)
    return q, sc[:M]


def clo(lo, hi):
    N = len(lo)
    out = np.zeros(N, np.uint8)
    lib().p2o_clo(_c(lo, np.float32), _c(hi, np.float32), N, out)
    return out


def codes_i8w(signs, flags, lo, hi, K, N):
    out = np.zeros((K, N), np.int8)
    lib().p2o_codes_i8w(_c(signs, np.uint8), _c(flags, np.uint8), _c(lo, np.float32), _c(hi, np.float32), K, N, out)
    return out


def fv_pack_codes(signs, flags, lo, hi, K, N):
    out = np.zeros(K * N, np.int8)
    lib().p2o_fv_pack_codes(_c(signs, np.uint8), _c(flags, np.uint8), _c(lo, np.float32), _c(hi, np.float32),
                            K, N, out)
    return out


def planes_i8(signs, flags, K, N):
    S = np.zeros((K, N), np.int8)
    T = np.zeros((K, N), np.int8)
    lib().p2o_planes_i8(_c(signs, np.uint8), _c(flags, np.uint8), K, N, S, T)
    return S, T


def acc_i32(q, B, k0=0, k1=None):
    q = _c(q, np.int8)
    B = _c(B, np.int8)
    M, K = q.shape
    N = B.shape[1]
    k1 = K if k1 is None else k1
    acc = np.zeros((M, N), np.int32)
    lib().p2o_acc_i32(q, M, K, B, N, k0, k1, acc)
    return acc


def gemm_i8_run(mode, q, a_scales, signs, flags, lo, hi, N, alpha=1.0, C0=None, beta_zero=True):
    q = _c(q, np.int8)
    M, K = q.shape
    C = np.zeros((M, N), np.float32) if C0 is None else _c(C0, np.float32).copy()
    lib().p2o_gemm_i8_run(MODES[mode] if isinstance(mode, str) else mode, M, N, K, alpha, q,
                          _c(a_scales, np.float32), _c(signs, np.uint8), _c(flags, np.uint8),
                          _c(lo, np.float32), _c(hi, np.float32), 1 if beta_zero else 0, C, C.shape[1])
    return C


def sgemm_fvb(mode, A, signs, flags, lo, hi, N, alpha=1.0, beta=0.0, C0=None, K=None, ldc=None):
    """p2_sgemm_fvb in `mode`; A is [M, lda] with the first K columns used; C0 is [M, ldc]."""
    A = _c(A, np.float32)
    M, lda = A.shape
    K = lda if K is None else K
    if C0 is None:
        C = np.zeros((M, N if ldc is None else ldc), np.float32)
    else:
        C = _c(C0, np.float32).copy()
    lib().p2o_sgemm_fvb(MODES[mode] if isinstance(mode, str) else mode, M, N, K, alpha, A, lda,
                        _c(signs, np.uint8), _c(flags, np.uint8), _c(lo, np.float32), _c(hi, np.float32),
                        beta, C, C.shape[1])
    return C


def sgemm_q8b(mode, A, B, scales, N, alpha=1.0, beta=0.0, C0=None, K=None):
    A = _c(A, np.float32)
    B = _c(B, np.int8)
    M, lda = A.shape
    K = lda if K is None else K
    C = np.zeros((M, N), np.float32) if C0 is None else _c(C0, np.float32).copy()
    lib().p2o_sgemm_q8b(MODES[mode] if isinstance(mode, str) else mode, M, N, K, alpha, A, lda, B,
                        _c(scales, np.float32), B.shape[1], beta, C, C.shape[1])
    return C


def mode_from_env(p2_gemm, p2_exact):
    enc = lambda s: None if s is None else s.encode()
    return lib().p2o_mode_from_env(enc(p2_gemm), enc(p2_exact))


# ── the reference's own library, built from its C sources by oracle/Makefile ─────────────────────────────────

class FiveValueB(C.Structure):
    """The reference's FiveValueB (blas.h:39-45)."""
    _fields_ = [("signs", C.c_void_p), ("flags", C.c_void_p), ("lo", C.c_void_p), ("hi", C.c_void_p),
                ("codes", C.c_void_p)]


_ref = None


def ref_available():
    return os.path.exists(REF_SO)


def layer_norm_rows(X, gamma, beta):
    X = _c(X, np.float32)
    out = np.empty_like(X)
    g, b = _c(gamma, np.float32), _c(beta, np.float32)
    for m in range(X.shape[0]):
        row = np.empty(X.shape[1], np.float32)
        lib().p2o_layer_norm_row(_c(X[m], np.float32), g, b, row, X.shape[1])
        out[m] = row
    return out


def swish_rows(X):
    out = _c(X, np.float32).copy()
    for m in range(out.shape[0]):
        row = out[m].copy()
        lib().p2o_swish_row(row, row.size)
        out[m] = row
    return out


def ln_quant_rows(X, gamma, beta, D=None):
    X = _c(X, np.float32)
    M, ldx = X.shape
    D = ldx if D is None else D
    q, sc = np.zeros((M, D), np.int8), np.zeros(M, np.float32)
    lib().p2o_ln_quant_rows(X, M, D, ldx, _c(gamma, np.float32), _c(beta, np.float32), q, sc)
    return q, sc


def silu_quant_rows(H, K=None):
    H = _c(H, np.float32)
    M, ldh = H.shape
    K = ldh if K is None else K
    q, sc = np.zeros((M, K), np.int8), np.zeros(M, np.float32)
    lib().p2o_silu_quant_rows(H, M, K, ldh, q, sc)
    return q, sc


def concat_heads_quant_rows(attn_h):
    attn_h = _c(attn_h, np.float32)
    H, T, Dh = attn_h.shape
    q, sc = np.zeros((T, H * Dh), np.int8), np.zeros(T, np.float32)
    lib().p2o_concat_heads_quant_rows(attn_h, H, T, Dh, q, sc)
    return q, sc


def channel_major_quant_rows(dw):
    dw = _c(dw, np.float32)
    D, T = dw.shape
    q, sc = np.zeros((T, D), np.int8), np.zeros(T, np.float32)
    lib().p2o_channel_major_quant_rows(dw, D, T, q, sc)
    return q, sc


def ref():
    """The reference's p2_sgemm_fvb / p2_sgemm_q8b (x86: the exact fp32 AVX2 route, blas.c:1043-1045), and its
    p2_layer_norm / p2_swish (tensor_ops.c, AVX2 routes)."""
    global _ref
    if _ref is None:
        L = C.CDLL(REF_SO)
        L.p2_layer_norm.argtypes = [C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p, _i]
        L.p2_layer_norm.restype = None
        L.p2_swish.argtypes = [C.c_void_p, _i]
        L.p2_swish.restype = None
        L.p2_sgemm_fvb.argtypes = [_i, _i, _i, _f, C.c_void_p, _i, C.POINTER(FiveValueB), _f, C.c_void_p, _i]
        L.p2_sgemm_fvb.restype = None
        L.p2_sgemm_q8b.argtypes = [_i, _i, _i, _f, C.c_void_p, _i, C.c_void_p, C.c_void_p, _i, _f, C.c_void_p, _i]
        L.p2_sgemm_q8b.restype = None
        L.p2_gemm_mode.restype = C.c_char_p
        _ref = L
    return _ref


def ref_sgemm_fvb(A, signs, flags, lo, hi, N, alpha, beta, C0, K=None):
    A = _c(A, np.float32)
    M, lda = A.shape
    K = lda if K is None else K
    out = _c(C0, np.float32).copy()
    s, f, l, h = _c(signs, np.uint8), _c(flags, np.uint8), _c(lo, np.float32), _c(hi, np.float32)
    b = FiveValueB(s.ctypes.data, f.ctypes.data, l.ctypes.data, h.ctypes.data, None)
    ref().p2_sgemm_fvb(M, N, K, alpha, A.ctypes.data, lda, C.byref(b), beta, out.ctypes.data, out.shape[1])
    return out


def ref_sgemm_q8b(A, B, scales, N, alpha, beta, C0, K=None):
    A = _c(A, np.float32)
    B = _c(B, np.int8)
    M, lda = A.shape
    K = lda if K is None else K
    out = _c(C0, np.float32).copy()
    sc = _c(scales, np.float32)
    ref().p2_sgemm_q8b(M, N, K, alpha, A.ctypes.data, lda, B.ctypes.data, sc.ctypes.data, B.shape[1],
                       beta, out.ctypes.data, out.shape[1])
    return out


def ref_layer_norm_rows(X, gamma, beta):
    X = _c(X, np.float32)
    out = np.empty_like(X)
    g, b = _c(gamma, np.float32), _c(beta, np.float32)
    for m in range(X.shape[0]):
        row = _c(X[m], np.float32)
        o = np.empty(X.shape[1], np.float32)
        ref().p2_layer_norm(row.ctypes.data, g.ctypes.data, b.ctypes.data, o.ctypes.data, X.shape[1])
        out[m] = o
    return out


def ref_swish_rows(X):
    """p2_swish row by row (rows below its 32768-element threading threshold run swish_range directly)."""
    out = _c(X, np.float32).copy()
    for m in range(out.shape[0]):
        row = out[m].copy()
        ref().p2_swish(row.ctypes.data, row.size)
        out[m] = row
    return out


# ── the conformer block between its linears ─────────────────────────────────────────────────────────────────────

SCORE_SCALE = np.float32(1.0) / np.sqrt(np.float32(128.0), dtype=np.float32)   # 1/sqrtf(128), encoder.c:521


def combine_softmax(ac, bd, H=8):
    ac = _c(ac, np.float32).copy()
    T = ac.shape[1]
    lib().p2o_combine_softmax(ac, _c(bd, np.float32), H, T, float(SCORE_SCALE))
    return ac


def glu_channel_major(pw1, D=1024):
    pw1 = _c(pw1, np.float32)
    T = pw1.shape[0]
    out = np.zeros((D, T), np.float32)
    lib().p2o_glu_channel_major(pw1, out, T, D)
    return out


def dwconv(x, w, b, K=9):
    x = _c(x, np.float32)
    D, T = x.shape
    out = np.zeros((D, T), np.float32)
    lib().p2o_dwconv(x, _c(w, np.float32), _c(b, np.float32), out, D, T, K)
    return out


def dwconv_silu(x, w, b, K=9):
    x = _c(x, np.float32)
    D, T = x.shape
    out = np.zeros((D, T), np.float32)
    lib().p2o_dwconv_silu(x, _c(w, np.float32), _c(b, np.float32), out, D, T, K)
    return out


REFBLOCK_SO = os.path.join(ROOT, "oracle", "_ref", "libp2refblock.so")
REFBLOCK_ORACLE_SO = os.path.join(ROOT, "oracle", "_ref", "libp2refblock_oracle.so")


class RefFv(C.Structure):
    _fields_ = [("signs", C.c_void_p), ("flags", C.c_void_p), ("lo", C.c_void_p), ("hi", C.c_void_p),
                ("K", C.c_int), ("N", C.c_int)]


_BLOCK_ORDER = [("norm_ff1_w", 0), ("norm_ff1_b", 0), ("ff1_l1", 1), ("ff1_l2", 1), ("norm_sa_w", 0),
                ("norm_sa_b", 0), ("qkv", 1), ("pos", 1), ("out", 1), ("bias_u", 0), ("bias_v", 0),
                ("norm_conv_w", 0), ("norm_conv_b", 0), ("pw1", 1), ("pw2", 1), ("dw_w", 0), ("dw_b", 0),
                ("norm_ff2_w", 0), ("norm_ff2_b", 0), ("ff2_l1", 1), ("ff2_l2", 1), ("norm_out_w", 0),
                ("norm_out_b", 0)]


class RefBlock(C.Structure):
    _fields_ = [(n, RefFv if fv else C.c_void_p) for n, fv in _BLOCK_ORDER]


_refblock = {}


def refblock(oracle_gemms=False):
    """The reference's own conformer block (oracle/_ref/libp2refblock*.so, built from its encoder.c by
    oracle/ref_block.c): with its blas.c (x86: the fp32 path) or with the oracle's quantised GEMMs (the int8 path in
    the mode P2_GEMM names when the first GEMM runs; int8w when unset)."""
    key = bool(oracle_gemms)
    if key not in _refblock:
        L = C.CDLL(REFBLOCK_ORACLE_SO if key else REFBLOCK_SO)
        vp = C.c_void_p
        L.refblock_run.argtypes = [C.POINTER(RefBlock), vp, vp, _i, _i]
        L.refblock_run.restype = _i
        L.refblock_pos_encoding.argtypes = [_i, vp]
        L.refblock_gather_heads.argtypes = [vp, vp, vp, vp, vp, vp, vp, _i]
        L.refblock_transpose_pos.argtypes = [vp, vp, _i]
        L.refblock_combine_softmax.argtypes = [vp, vp, _i]
        L.refblock_concat_heads.argtypes = [vp, vp, _i]
        L.refblock_glu.argtypes = [vp, vp, _i]
        L.refblock_cm_to_rows.argtypes = [vp, vp, _i]
        L.refblock_add_residual.argtypes = [vp, vp, _i, _f]
        L.p2_depthwise_conv1d.argtypes = [vp, vp, vp, vp, _i, _i, _i]
        L.p2_swish.argtypes = [vp, _i]
        L.p2_layer_norm_rows_inplace.argtypes = [vp, vp, vp, _i, _i]
        _refblock[key] = L
    return _refblock[key]


def refblock_available():
    return os.path.exists(REFBLOCK_SO) and os.path.exists(REFBLOCK_ORACLE_SO)


def ref_pos_encoding(T):
    out = np.zeros((2 * T - 1, 1024), np.float32)
    refblock().refblock_pos_encoding(T, out.ctypes.data)
    return out


def ref_block_run(params, x, pe, oracle_gemms=False, stage=-1):
    """x [T, 1024] through the reference's conformer_block (encoder.c:617-625), or one of its five steps (stage 0..4,
    encoder.c:619-623); params as for p2gemm.Block."""
    x = _c(x, np.float32).copy()
    T = x.shape[0]
    keep, vals = [], {}
    for n, fv in _BLOCK_ORDER:
        if fv:
            s, f, lo, hi = (_c(a, t) for a, t in zip(params[n], (np.uint8, np.uint8, np.float32, np.float32)))
            keep += [s, f, lo, hi]
            vals[n] = RefFv(s.ctypes.data, f.ctypes.data, lo.ctypes.data, hi.ctypes.data, hi.size and
                            (s.size * 4 // hi.size), hi.size)
        else:
            a = _c(params[n], np.float32)
            keep.append(a)
            vals[n] = a.ctypes.data
    blk = RefBlock(**vals)
    pe = _c(pe, np.float32)
    rc = refblock(oracle_gemms).refblock_run(C.byref(blk), pe.ctypes.data, x.ctypes.data, T, stage)
    if rc != 0:
        raise RuntimeError("refblock_run failed")
    return x
