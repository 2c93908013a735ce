"""Child process for tests/test_gpu_block.py: one conformer block through the reference's own conformer_block
(encoder.c:617-625, built from its sources into oracle/_ref) on the seeded synthetic block of p2gemm.block_params.
The GEMM mode is latched from P2_GEMM once per process (blas.c:1027-1066), hence a process per mode.

    P2_GEMM=int8w python tests/refblock_child.py SEED T OUT.npy oracle [STAGE]  the oracle's int8w GEMMs
    python tests/refblock_child.py SEED T OUT.npy reference                the reference's blas.c (x86: exact route)

STAGE (optional, 0..3): keep only that step of the block (feed_forward, self_attention, conv_module, the second
feed_forward): the linears whose products are added to the residual in the other three steps get all-zero weights
(isolated_params), so x passes them unchanged and the block is LayerNorm(x + step(x)).
"""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, HERE)
sys.path.insert(0, os.path.join(os.path.dirname(HERE), "phonon-2-c_amd"))

import _oracle as O  # noqa: E402
import p2gemm as P  # noqa: E402

BLOCK_TID0 = 100


def block_input(seed, T):
    """The block's input rows and positional rows: generator activations [T, 1024], rel_pos_encoding (encoder.c:79-96)."""
    return P.gen_activations(seed, BLOCK_TID0 - 1, T, P.D_MODEL), O.ref_pos_encoding(T)


RESIDUAL_LINEARS = ("ff1_l2", "out", "pw2", "ff2_l2")   # encoder.c:347, 530, 602, 347: the products added to x


def isolated_params(params, stage):
    """The block with every step but `stage` reduced to x += 0: the sign plane of a zero weight is 01 in every
    two-bit field (0x55 per byte)."""
    if stage is None:
        return params
    p = dict(params)
    for i, name in enumerate(RESIDUAL_LINEARS):
        if i != stage:
            s, f, lo, hi = p[name]
            p[name] = (np.full_like(s, 0x55), np.zeros_like(f), lo, hi)
    return p


def main():
    seed, T, out, gemms = int(sys.argv[1]), int(sys.argv[2]), sys.argv[3], sys.argv[4]
    stage = int(sys.argv[5]) if len(sys.argv) > 5 else None
    params = isolated_params(P.block_params(seed, BLOCK_TID0), stage)
    x, pe = block_input(seed, T)
    y = O.ref_block_run(params, x, pe, oracle_gemms=(gemms == "oracle"))
    np.save(out, y)
    return 0


if __name__ == "__main__":
    sys.exit(main())
