"""Writes the small golden fixtures under tests/golden/ from the CPU oracle.

The reference ships no fixtures or golden vectors, so these are regression
vectors of the oracle (itself pinned by the hand-worked example, the
independent canonical checks and the restated validators).  Each SWTCF
fixture holds a COO, its canonical SWTCF arrays at their valid extents, a
seeded feature matrix X and the oracle's SpMM output at tc = 12.

Run from the repo root:  python tests/golden/make_fixtures.py
"""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

import oracle  # noqa: E402

CASES = [
    # name, n_dst, n_src, nnz, S, F, seed
    ("swtcf_small_s16", 50, 100, 400, 16, 8, 11),
    ("swtcf_ragged_s3", 37, 61, 300, 3, 5, 12),
    ("swtcf_dense_s1", 16, 16, 200, 1, 4, 13),
]


def main():
    for name, nd, ns, nnz, S, F, seed in CASES:
        rng = np.random.default_rng(seed)
        keys = rng.choice(nd * ns, size=nnz, replace=False)
        dst = (keys // ns).astype(np.uint32)
        src = (keys % ns).astype(np.uint32)
        m = oracle.swtcf_convert(dst, src, nd, ns, S)
        assert m["err"] == 0
        v = oracle.swtcf_valid_extents(m)
        X = rng.standard_normal((ns, F)).astype(np.float32)
        Y = oracle.swtcf_spmm(m, X, tc=12, rows=nd)
        np.savez_compressed(os.path.join(HERE, name + ".npz"), dst=dst, src=src, rows=nd, cols=ns, S=S, X=X,
                            Y_tc12=Y, **v)
        print("wrote", name)


if __name__ == "__main__":
    main()
