"""Committed golden fixtures (tests/golden/*.npz, written by make_golden.py): the oracle
and the product's host compiler must reproduce them byte for byte on CPU; the GPU path
is checked against the same files in test_gpu_golden.py."""
import os

import numpy as np
import pytest

import oracle as O

GOLD = os.path.join(os.path.dirname(__file__), "golden")
NAMES = ["config1_b4_1536x576", "b6_200x384_tail", "b5_96x640", "nf4g128_272x1024_tail"]


def load(name):
    with np.load(os.path.join(GOLD, name + ".npz"), allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


def regen_inputs(g):
    import sys
    sys.path.insert(0, GOLD)
    from make_golden import inputs
    return inputs(int(g["rows"]), int(g["cols"]), int(g["seed"]))


def test_fwht_fixture():
    g = load("fwht64_5blocks")
    assert np.array_equal(O.fwht64(g["x"]).view(np.uint32), g["y"].view(np.uint32))


@pytest.mark.parametrize("name", NAMES)
def test_oracle_reproduces_fixture(name):
    g = load(name)
    rows, cols, p = int(g["rows"]), int(g["cols"]), int(g["p"])
    q, s, sm = O.populate_fwht(g["x"])
    assert np.array_equal(q, g["q"]) and np.array_equal(s.view(np.uint32), g["s"].view(np.uint32))
    assert np.array_equal(sm, g["sm"])
    if str(g["fmt"]) == "n4":
        out, dots = O.nibble4_gemv(g["pair"], g["tail"], rows, cols, p - 4, q, s, sm, want_dots=True)
    else:
        out, dots = O.nf_gemv(g["pair"], g["tail"], rows, cols, 4, p, g["cb"], q, s, want_dots=True)
    assert np.array_equal(dots, g["dots"])
    assert np.array_equal(out.view(np.uint32), g["out"].view(np.uint32))


@pytest.mark.parametrize("name", NAMES)
def test_product_compiler_reproduces_fixture(name):
    import k2t
    g = load(name)
    W, x = regen_inputs(g)
    assert np.array_equal(x.view(np.uint32), g["x"].view(np.uint32))
    if str(g["fmt"]) == "n4":
        pair, tail = k2t.compile_bipolar(W, int(g["p"]))
    else:
        cb, _, pair, tail = k2t.compile_nf4(W, int(g["p"]))
        assert np.array_equal(np.asarray(cb, np.int8), g["cb"])
    assert np.array_equal(pair, g["pair"]) and np.array_equal(tail, g["tail"])
