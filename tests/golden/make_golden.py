"""Writes the seeded golden fixtures in this folder from the oracle (oracle/).

The reference ships no golden vectors for this path (its tests pin by properties and
thresholds, simd_lut.rs:8710-8940), so these fixtures freeze the oracle's outputs on
seeded inputs.  Inputs are regenerable from the stored seed (numpy PCG64), so a test
can also check the compilers byte for byte.  Run: python tests/golden/make_golden.py
"""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(HERE, "..", "..", "oracle"))
import oracle as O  # noqa: E402

# name: (fmt, rows, cols, planes_or_sgc, seed)
CASES = {
    "config1_b4_1536x576": ("n4", 1536, 576, 4, 101),
    "b6_200x384_tail": ("n4", 200, 384, 6, 103),
    "b5_96x640": ("n4", 96, 640, 5, 104),
    "nf4g128_272x1024_tail": ("nf4", 272, 1024, 2, 102),
}


def inputs(rows, cols, seed):
    """W ~ N(0, 0.02); x ~ N(0, 1) with max(4, cols/1000) outlier channels x20 and chunk 1 zero."""
    rng = np.random.default_rng(seed)
    W = (rng.standard_normal((rows, cols)) * 0.02).astype(np.float32)
    x = rng.standard_normal(cols).astype(np.float32)
    idx = rng.choice(cols, max(4, cols // 1000), replace=False)
    x[idx] *= 20.0
    x[64:128] = 0.0
    return W, x


def make(name):
    fmt, rows, cols, p, seed = CASES[name]
    W, x = inputs(rows, cols, seed)
    q, s, sm = O.populate_fwht(x)
    if fmt == "n4":
        u, sc = O.bipolar_rtn(W, p)
        pair, tail = O.nibble4_repack(O.pack_interleaved(u, p), sc, rows, cols, p)
        out, dots = O.nibble4_gemv(pair, tail, rows, cols, p - 4, q, s, sm, want_dots=True)
        cb = np.zeros(16, np.int8)
    else:
        cb, mu = O.nf_fit_codebook(W, 4, p)
        idx, sc = O.nf_rtn(W, 4, p, cb, mu)
        pair, tail = O.nf_from_indices(idx, sc, rows, cols, 4, p)
        out, dots = O.nf_gemv(pair, tail, rows, cols, 4, p, cb, q, s, want_dots=True)
    return dict(fmt=np.array(fmt), rows=rows, cols=cols, p=p, seed=seed, x=x, q=q, s=s, sm=sm, pair=pair,
                tail=tail, cb=np.asarray(cb, np.int8), out=out, dots=dots)


def fwht_vectors():
    rng = np.random.default_rng(7)
    x = rng.standard_normal(64 * 5).astype(np.float32)
    x[64 * 3:64 * 4] *= 1e3
    return dict(x=x, y=O.fwht64(x))


if __name__ == "__main__":
    O.build()
    for n in CASES:
        np.savez_compressed(os.path.join(HERE, n + ".npz"), **make(n))
    np.savez_compressed(os.path.join(HERE, "fwht64_5blocks.npz"), **fwht_vectors())
    for f in sorted(os.listdir(HERE)):
        print(f, os.path.getsize(os.path.join(HERE, f)))
