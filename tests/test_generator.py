"""The seeded generator (libp2gen.so): pinned bytes, the statistics the workload specifies, and plane packing that
agrees with the oracle's restatement of the reference's packer (convert_weights.py:114-125)."""
import hashlib

import numpy as np

import _oracle as O
import p2gemm as P


def _sha(*arrs):
    h = hashlib.sha256()
    for a in arrs:
        h.update(np.ascontiguousarray(a).tobytes())
    return h.hexdigest()


# SHA-256 of generator outputs; any change to the generator's arithmetic changes these.
GENERATOR_SHA256 = {
    "act_1_2_64x256": "238974db0d89316fbe7ae8acef4dbcfa5dbda464c5b3dd0295f1fd56c989fb37",
    "fv_7_3_64x128": "b61aee9ec6771fbdbe027bab374fcd2e6fcc2accdfe873bb14c5701a9459656e",
}


def test_generator_is_deterministic():
    a = P.gen_activations(1, 2, 64, 256)
    b = P.gen_activations(1, 2, 64, 256)
    c = P.gen_activations(1, 3, 64, 256)
    assert np.array_equal(a, b) and not np.array_equal(a, c)
    w1 = P.gen_fv_weight(7, 3, 64, 128)
    w2 = P.gen_fv_weight(7, 3, 64, 128)
    assert all(np.array_equal(x, y) for x, y in zip(w1, w2))


def test_generator_pinned_bytes():
    got = {
        "act_1_2_64x256": _sha(P.gen_activations(1, 2, 64, 256)),
        "fv_7_3_64x128": _sha(*P.gen_fv_weight(7, 3, 64, 128)),
    }
    assert got == GENERATOR_SHA256


def test_activation_statistics():
    A = P.gen_activations(11, 1, 1000, 1024).astype(np.float64)
    big = np.abs(A) > 6.0   # Irwin–Hall(12) is bounded by 6: only the ×20 outliers exceed it
    frac_out = big.mean()
    assert 0.0006 < frac_out < 0.0013
    core = A[~big]
    assert abs(core.mean()) < 0.01 and abs(core.var() - 1.0) < 0.02


def test_weight_statistics_and_fp16():
    K, N = 512, 1024
    signs, flags, lo, hi = P.gen_fv_weight(13, 2, K, N)
    code, flag = O.unpack_planes(signs, flags, K, N)
    assert not (code == 3).any()
    assert not flag[code == 1].any(), "flag must be 0 on zero weights"
    zero = (code == 1).mean()
    hi_frac = flag.mean()
    assert abs(zero - 0.4) < 0.005 and abs(hi_frac - 0.2) < 0.005
    pos = (code == 2).mean()
    assert abs(pos - 0.3) < 0.005
    for v in (lo, hi):
        assert np.array_equal(v, v.astype(np.float16).astype(np.float32)), "lo/hi must be fp16 values"
    assert lo.min() >= 0.005 * (1 - 1e-3) and lo.max() <= 0.02 * (1 + 1e-3)
    r = hi / lo
    assert r.min() >= 2 * (1 - 2e-3) and r.max() <= 4 * (1 + 2e-3)


def test_packing_agrees_with_the_oracle_packer():
    K, N = 32, 64
    signs, flags, lo, hi = P.gen_fv_weight(17, 4, K, N)
    code, flag = O.unpack_planes(signs, flags, K, N)
    s2, f2 = O.pack_planes(code.astype(np.int8) - 1, flag)
    assert np.array_equal(s2, signs) and np.array_equal(f2, flags)


def test_round_fp16():
    gen = P.gen()
    for x in (0.1, 1.0 / 3, 0.0123456, 65504.0, 1e-7, -2.5e-3):
        assert gen.p2g_round_fp16(x) == np.float32(np.float16(x))

