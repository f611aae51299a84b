"""The product's host weight compiler produces byte-identical streams to the
oracle's two-step path (RTN quantize -> FusedBipolar/indices -> Nibble4/NF layout)."""
import numpy as np
import pytest

import k2t
import oracle as O


@pytest.mark.parametrize("rows,cols,planes,inter", [(40, 192, 4, False), (256, 256, 5, True), (56, 128, 6, False),
                                                    (200, 512, 4, False)])
def test_compile_bipolar_matches_oracle(rows, cols, planes, inter):
    W = k2t.synth_normal(rows * cols + planes, rows * cols, 0.02).reshape(rows, cols)
    pair, tail = k2t.compile_bipolar(W, planes, inter, threads=3)
    u, sc = O.bipolar_rtn(W, planes)
    rp, rt = O.nibble4_repack(O.pack_interleaved(u, planes), sc, rows, cols, planes, inter)
    assert np.array_equal(pair, rp) and np.array_equal(tail, rt)


@pytest.mark.parametrize("bits", [4, 3])
@pytest.mark.parametrize("rows,cols,sgc,inter", [(40, 256, 2, False), (256, 512, 2, True), (48, 192, 1, False),
                                                 (600, 384, 2, False)])
def test_compile_nf_matches_oracle(rows, cols, sgc, inter, bits):
    W = k2t.synth_normal(rows + cols + sgc, rows * cols, 0.02).reshape(rows, cols)
    W[3, :64] = 0.0  # an all-zero scale group takes the rms <= 1e-12 branch
    cb, mu, pair, tail = k2t.compile_nf4(W, sgc, inter, threads=3, bits=bits)
    rcb, rmu = O.nf_fit_codebook(W, bits, sgc)
    assert np.array_equal(cb, rcb) and mu == pytest.approx(rmu, abs=0)
    idx, sc = O.nf_rtn(W, bits, sgc, rcb, rmu)
    if inter:
        inter_dim = rows // 2
        perm = [(b // 2) * 64 + o + (inter_dim if b % 2 else 0) for b in range(rows // 64) for o in range(64)]
        idx = idx[perm]
        nsg = (cols // 64 + sgc - 1) // sgc
        s3 = np.zeros((rows, nsg), np.uint16)
        for r in range(rows):
            s3[r] = sc.reshape(-1, nsg, 16)[r // 16, :, r % 16]
        s3 = s3[perm]
        sc = np.stack([s3[s * 16:(s + 1) * 16].T for s in range(rows // 16)]).ravel()
    rp, rt = O.nf_from_indices(idx, sc, rows, cols, bits, sgc)
    assert np.array_equal(pair, rp) and np.array_equal(tail, rt)


def test_synth_normal_is_deterministic_and_normal():
    a = k2t.synth_normal(7, 100001, 0.02, threads=1)
    b = k2t.synth_normal(7, 100001, 0.02, threads=5)
    assert np.array_equal(a, b)
    assert abs(a.mean()) < 5e-4 and abs(a.std() - 0.02) < 5e-4
