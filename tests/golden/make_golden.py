"""Writes quant_golden.npz: dequantised values and dot_row results computed by
the reference's own src/native/quant.cpp (oracle/_ref/libns_ref_quant.so,
built by oracle/Makefile from the reference checkout) for a few Q4_K / Q6_K
blocks, so that the oracle stays pinned where the reference is absent.

Inputs: seeded blocks from the build's generator plus hand-built extremes
(zero scales, maximal scales/mins, fp16-subnormal d, sc = -32).  Run from the
repository root:  python tests/golden/make_golden.py
"""
import os
import sys

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path[:0] = [os.path.join(ROOT, "tests"), os.path.join(ROOT, "oracle"), os.path.join(ROOT, "neutron-star_amd")]

import ns_oracle as O  # noqa: E402
import nsffn  # noqa: E402
from helpers import q4k_block, q6k_block  # noqa: E402


def main():
    assert O.ref() is not None, "build oracle/_ref first (make -C oracle)"
    out = {}
    rng = np.random.default_rng(2024)
    # Q4_K: 2 rows x 512 cols = 4 blocks
    q4 = [nsffn.synth_blocks(nsffn.Q4_K, 77, 2),
          q4k_block(2.0**-20, 1e-3, [63] * 8, [63] * 8, [15] * 256).reshape(1, -1),
          q4k_block(0.5, 0.0, [0, 1, 2, 63, 16, 32, 48, 31], [5] * 8, list(range(16)) * 16).reshape(1, -1)]
    q4 = np.ascontiguousarray(np.concatenate([a.reshape(-1) for a in q4]))
    # Q6_K: 2 rows x 512 cols = 4 blocks
    q6 = [nsffn.synth_blocks(nsffn.Q6_K, 78, 2),
          q6k_block(3.0e-6, [-32] * 16, [0] * 256).reshape(1, -1),
          q6k_block(0.75, list(range(-8, 8)), [63 - (i % 64) for i in range(256)]).reshape(1, -1)]
    q6 = np.ascontiguousarray(np.concatenate([a.reshape(-1) for a in q6]))
    for name, qtype, w in (("q4k", nsffn.Q4_K, q4), ("q6k", nsffn.Q6_K, q6)):
        cols, rows = 512, 2
        rc, vals = O.ref_dequant(qtype, w, cols, rows, 0, cols * rows)
        assert rc == 0
        x = rng.standard_normal(cols).astype(np.float32)
        dots = []
        for r in range(rows):
            rc, d = O.ref_dot_row(qtype, w, cols, rows, r, x)
            assert rc == 0
            dots.append(d)
        out[f"{name}_bytes"] = w
        out[f"{name}_shape"] = np.array([cols, rows], dtype=np.int64)
        out[f"{name}_values"] = vals
        out[f"{name}_x"] = x
        out[f"{name}_dot"] = np.array(dots, dtype=np.float32)
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "quant_golden.npz")
    np.savez_compressed(path, **out)
    print("wrote", path)


if __name__ == "__main__":
    main()
