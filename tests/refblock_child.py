"""Child process for tests/test_gpu_block.py: one conformer block through the reference's own conformer_block
(encoder.c:617-625, built from its sources into oracle/_ref) on the seeded synthetic block of p2gemm.block_params.
The GEMM mode is latched from P2_GEMM once per process (blas.c:1027-1066), hence a process per mode.

    P2_GEMM=int8w python tests/refblock_child.py SEED T OUT.npy oracle     the oracle's int8w GEMMs
    python tests/refblock_child.py SEED T OUT.npy reference                the reference's blas.c (x86: exact route)
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


def main():
    seed, T, out, gemms = int(sys.argv[1]), int(sys.argv[2]), sys.argv[3], sys.argv[4]
    params = P.block_params(seed, BLOCK_TID0)
    x, pe = block_input(seed, T)
    y = O.ref_block_run(params, x, pe, oracle_gemms=(gemms == "oracle"))
    np.save(out, y)
    return 0


if __name__ == "__main__":
    sys.exit(main())
