"""Pins the CPU oracle (oracle/k2t_oracle.c) against what the reference's own tests
assert and against what the mathematics fixes -- so that a plausible mistake in the
restatement (a dropped term, a wrong sign mask, a transposed operand, a wrong
rounding mode) fails here.  The reference ships no golden vectors for this path
(its tests assert parity and thresholds only); the closed forms used below are
independent of the restatement.
"""
import numpy as np
import pytest

import oracle as O
from helpers import activation, normal

H64 = np.array([[1.0]])
for _ in range(6):
    H64 = np.block([[H64, H64], [H64, -H64]])


def _signs(block):
    b = O.sign_bits(block)
    return np.array([-1.0 if (b >> i) & 1 else 1.0 for i in range(64)])


# ----------------------------------------------------------------------------- FWHT
def test_fwht_is_scaled_hadamard_times_signs():
    rng = np.random.default_rng(0)
    x = normal(rng, 64 * 300)  # beyond the reference's 256-block table (fallback masks)
    y = O.fwht64(x)
    for b in (0, 1, 7, 255, 256, 299):
        ref = H64 @ (_signs(b) * x[64 * b:64 * b + 64].astype(np.float64)) / 8.0
        assert np.abs(ref - y[64 * b:64 * b + 64]).max() < 1e-5


def test_fwht_orthogonal_self_inverse_and_distinct_masks():
    rng = np.random.default_rng(1)
    x = normal(rng, 640)
    assert np.abs(O.ifwht64(O.fwht64(x)) - x).max() < 1e-5
    assert abs(np.linalg.norm(O.fwht64(x)) - np.linalg.norm(x)) < 1e-3
    masks = {O.sign_bits(b) for b in range(256)}
    assert len(masks) == 256  # every block has its own Rademacher diagonal
    # roughly balanced +-1
    ones = sum(bin(O.sign_bits(b)).count("1") for b in range(256)) / (256 * 64)
    assert 0.45 < ones < 0.55


def test_fwht_reference_unit_test_vectors():
    """hadamard.rs:300-330: outlier flattening and inner-product invariance."""
    i = np.arange(128, dtype=np.float32)
    x = np.where(i == 17, 80.0, np.sin(i * np.float32(0.37))).astype(np.float32)
    w = np.where(i == 99, -25.0, np.cos(i * np.float32(0.19))).astype(np.float32)
    dot_before = float(np.dot(x, w))
    xr, wr = O.fwht64(x), O.fwht64(w)
    assert np.abs(xr).max() < 15.0
    assert abs(dot_before - float(np.dot(xr, wr))) < 1e-3


def test_bf16_round_to_nearest_even():
    assert O.f32_to_bf16(1.0) == 0x3F80
    # 1 + 2^-8 is exactly half-way between bf16 1.0 and 1.0078125 -> even (1.0)
    assert O.f32_to_bf16(1.0 + 2.0 ** -8) == 0x3F80
    assert O.f32_to_bf16(1.0 + 3 * 2.0 ** -8) == 0x3F82  # half-way to odd 0x3F81 -> 0x3F82
    assert O.f32_to_bf16(float("nan")) & 0x7FC0 == 0x7FC0


# ----------------------------------------------------------------------------- populate
def _brute_populate(x, w=None, inv=1.0):
    K = x.size
    q = np.zeros(K, np.int8)
    s = np.zeros(K // 64, np.float32)
    m = np.zeros(K // 64, np.int32)
    for c in range(K // 64):
        blk = x[64 * c:64 * c + 64].astype(np.float32)
        if w is not None:
            blk = (blk * np.float32(inv)) * w[64 * c:64 * c + 64]
        rot = (H64 @ (_signs(c) * blk.astype(np.float64)) / 8.0)
        mx = np.abs(rot).max()
        if mx <= np.finfo(np.float32).eps:
            continue
        q[64 * c:64 * c + 64] = np.rint(rot * 127.0 / mx).astype(np.int8)
        s[c] = mx / 127.0
        m[c] = int(q[64 * c:64 * c + 64].astype(np.int64).sum())
    return q, s, m


def test_populate_against_f64_closed_form():
    rng = np.random.default_rng(2)
    x = activation(rng, 1536, n_outliers=4, zero_chunk=5)
    q, s, m = O.populate_fwht(x)
    bq, bs, bm = _brute_populate(x)
    # f64 rotation vs f32 butterflies can move a value across a rounding boundary.
    assert np.abs(q.astype(int) - bq).max() <= 1
    assert (q != bq).mean() < 0.01
    np.testing.assert_allclose(s, bs, rtol=1e-5)
    assert np.array_equal(m, q.reshape(-1, 64).astype(np.int64).sum(1))
    assert np.all(np.abs(q.reshape(-1, 64)).max(1)[s > 0] == 127)
    assert s[5] == 0 and m[5] == 0 and not q[320:384].any()


def test_populate_reference_unit_tests():
    """simd_lut.rs:8843-8905: fused == FWHT then plain populate (bit-exact), zero chunks."""
    cols = 1536
    c = np.arange(cols, dtype=np.float32)
    x = np.where(c // 64 == 5, 0.0, np.sin(c * np.float32(0.43)) * np.float32(2.1)).astype(np.float32)
    w = (0.75 + np.cos(c * np.float32(0.13)) * np.float32(0.4)).astype(np.float32)
    inv = 0.8125
    a = O.populate_fwht(x)
    b = O.populate_plain(O.fwht64(x))
    for u, v in zip(a, b):
        assert np.array_equal(u, v)
    xn = ((x * np.float32(inv)) * w).astype(np.float32)
    a = O.populate_fwht(x, w, inv)
    b = O.populate_plain(O.fwht64(xn))
    for u, v in zip(a, b):
        assert np.array_equal(u, v)
    assert a[1][5] == 0 and a[2][5] == 0


def test_populate_ties_round_to_even():
    # a chunk whose scaled values hit exact .5 ties: max 127 -> inv = 1, values k + 0.5
    x = np.zeros(64, np.float32)
    x[0] = 127.0
    x[1] = 2.5
    x[2] = -3.5
    x[3] = 0.5
    q, s, m = O.populate_plain(x)
    assert list(q[:4]) == [127, 2, -4, 0]
    assert m[0] == 125


# ----------------------------------------------------------------------------- bipolar RTN + layout
def test_bipolar_rtn_reference_unit_test():
    """simd_lut.rs:8710-8743: reconstruction cosine > 0.99 for 4 and 5 planes."""
    rows, cols = 40, 192
    idx = np.arange(rows * cols)
    W = ((((idx * 7919 + 13) % 1009).astype(np.float32) / 1009.0 - 0.5) * 0.3).astype(np.float32).reshape(rows, cols)
    for planes in (4, 5):
        u, sc = O.bipolar_rtn(W, planes)
        inter = O.pack_interleaved(u, planes)
        pair, tail = O.nibble4_repack(inter, sc, rows, cols, planes)
        rec = np.stack([O.ifwht64(O.nibble4_dequant_row(pair, tail, rows, cols, planes - 4, r)) for r in range(rows)])
        cos = np.dot(rec.ravel(), W.ravel()) / (np.linalg.norm(rec) * np.linalg.norm(W))
        assert cos > 0.99


def test_bipolar_rtn_picks_best_ratio():
    """Brute-force the 12-candidate search of compiler.rs:1038-1084 on a small matrix."""
    rng = np.random.default_rng(4)
    rows, cols, planes = 16, 128, 4
    W = normal(rng, (rows, cols), 0.02)
    u, sc = O.bipolar_rtn(W, planes)
    M = (1 << planes) - 1
    ratios = np.array([0.62, 0.67, 0.72, 0.77, 0.82, 0.87, 0.92, 0.97, 1.02, 1.07, 1.12, 1.18], np.float32)
    for r in range(rows):
        rot = O.fwht64(W[r])
        for c in range(cols // 64):
            sub = rot[64 * c:64 * c + 64].astype(np.float64)
            delta = float(np.frombuffer(np.uint32(int(sc[(c) * 16 + r]) << 16).tobytes(), np.float32)[0])
            uu = u[r, 64 * c:64 * c + 64].astype(np.int64)
            err = np.sum((sub - (2 * uu - M) * delta) ** 2)
            best = np.inf
            for rat in ratios:
                d = float(np.float32(np.abs(sub).max().astype(np.float32) * rat) / np.float32(M))
                d = float(np.frombuffer(np.uint32(O.f32_to_bf16(d) << 16).tobytes(), np.float32)[0])
                uc = np.clip(np.floor(sub / (2 * d) + M / 2 + 0.5), 0, M)
                best = min(best, np.sum((sub - (2 * uc - M) * d) ** 2))
            assert err <= best * (1 + 1e-4) + 1e-12


def test_nibble4_layout_roundtrip_all_planes():
    """Repack invariance (simd_lut.rs:8745-8766) + code round trip on random codes."""
    rng = np.random.default_rng(5)
    for planes in (4, 5, 6):
        rows, cols = 56, 256  # 4 stripes; and 40 rows (odd stripes) below
        for rows in (56, 40):
            u = rng.integers(0, 1 << planes, (rows, cols), dtype=np.uint8)
            sc = rng.integers(0x3A00, 0x3C00, ((rows + 15) // 16) * (cols // 64) * 16).astype(np.uint16)
            inter = O.pack_interleaved(u, planes)
            pair, tail = O.nibble4_repack(inter, sc, rows, cols, planes)
            assert pair.size + tail.size == inter.size + sc.size * 2  # physical bytes unchanged
            M = (1 << planes) - 1
            for r in range(rows):
                assert np.array_equal(O.nibble4_row_codes(pair, tail, rows, cols, planes - 4, r), u[r])
                row = O.nibble4_dequant_row(pair, tail, rows, cols, planes - 4, r)
                s, lane = r // 16, r % 16
                delta = np.repeat(np.array([sc[(s * (cols // 64) + c) * 16 + lane] for c in range(cols // 64)],
                                           np.uint32) << 16, 64).view(np.float32)
                assert np.array_equal(row, ((2 * u[r].astype(np.int32) - M).astype(np.float32) * delta))


def test_gate_up_interleave_permutation():
    rng = np.random.default_rng(6)
    rows, cols, planes = 256, 128, 4
    u = rng.integers(0, 16, (rows, cols), dtype=np.uint8)
    sc = rng.integers(0x3A00, 0x3C00, (rows // 16) * (cols // 64) * 16).astype(np.uint16)
    inter = O.pack_interleaved(u, planes)
    pair, tail = O.nibble4_repack(inter, sc, rows, cols, planes, interleave_gate_up=True)
    inter_dim = rows // 2
    for r in range(rows):
        blk, off = divmod(r, 64)
        src = (blk // 2) * 64 + off + (inter_dim if blk % 2 else 0)
        assert np.array_equal(O.nibble4_row_codes(pair, tail, rows, cols, 0, r), u[src])


# ----------------------------------------------------------------------------- GEMV semantics
def _bf16(b):
    return (np.asarray(b, np.uint32) << 16).view(np.float32)


@pytest.mark.parametrize("hp", [0, 1, 2])
def test_nibble4_gemv_integer_dots_and_epilogue(hp):
    rng = np.random.default_rng(10 + hp)
    rows, cols = 40, 256
    planes = 4 + hp
    M = (1 << planes) - 1
    u = rng.integers(0, M + 1, (rows, cols), dtype=np.uint8)
    sc = rng.integers(0x3A00, 0x3C00, ((rows + 15) // 16) * (cols // 64) * 16).astype(np.uint16)
    pair, tail = O.nibble4_repack(O.pack_interleaved(u, planes), sc, rows, cols, planes)
    x = activation(rng, cols, n_outliers=2, zero_chunk=2)
    xq, xs, xsum = O.populate_fwht(x)
    out, dots = O.nibble4_gemv(pair, tail, rows, cols, hp, xq, xs, xsum, want_dots=True)
    qgrid = 2 * u.astype(np.int64) - M
    brute = (qgrid.reshape(rows, -1, 64) * xq.astype(np.int64).reshape(1, -1, 64)).sum(2)
    assert np.array_equal(dots, brute)
    ws = np.array([[_bf16(sc[((r // 16) * (cols // 64) + c) * 16 + r % 16]) for c in range(cols // 64)]
                   for r in range(rows)], np.float64)
    y = (brute * xs.astype(np.float64)[None, :] * ws).sum(1)
    assert np.all(np.abs(out - y) <= 1e-5 * (1 + np.abs(y)))
    port = O.nibble4_gemv_portable(pair, tail, rows, cols, hp, xq, xs)
    assert np.all(np.abs(port - out) <= 1e-4 * (1 + np.abs(out)))


def test_nibble4_gemv_skips_zero_scale_chunks():
    rng = np.random.default_rng(11)
    rows, cols = 32, 128
    u = rng.integers(0, 16, (rows, cols), dtype=np.uint8)
    sc = np.full((rows // 16, 2, 16), 0x7F80, np.uint16)  # +inf weights in chunk 1
    sc[:, 0, :] = 0x3C00
    sc = sc.ravel()
    pair, tail = O.nibble4_repack(O.pack_interleaved(u, 4), sc, rows, cols, 4)
    xq = np.zeros(cols, np.int8)
    xq[:64] = 3
    out = O.nibble4_gemv(pair, tail, rows, cols, 0, xq, np.array([0.5, 0.0], np.float32),
                         np.array([192, 0], np.int32))
    assert np.all(np.isfinite(out))


# ----------------------------------------------------------------------------- NF
def test_nf_codebook_default_for_tiny_and_fitted_shape():
    W = np.zeros((1, 64), np.float32)
    cb, mu = O.nf_fit_codebook(W, 4, 2)
    assert list(cb) == [-127, -96, -75, -58, -44, -31, -18, -6, 6, 18, 31, 44, 58, 75, 96, 127]
    rng = np.random.default_rng(12)
    cb, mu = O.nf_fit_codebook(normal(rng, (256, 1024), 0.02), 4, 2)
    assert np.all(np.diff(cb.astype(int)) > 0) and cb[15] == 127 and cb[0] == -127
    assert np.array_equal(cb[:8], -cb[::-1][:8])
    # a Gaussian's Lloyd-Max 16-level top centroid is about 2.73 sigma
    assert 2.3 < mu < 3.1
    cb3, _ = O.nf_fit_codebook(normal(rng, (256, 1024), 0.02), 3, 2)
    assert np.all(cb3[8:] == 0) and np.all(np.diff(cb3[:8].astype(int)) > 0)


def test_nf_rtn_nearest_centroid_and_layout():
    rng = np.random.default_rng(13)
    rows, cols, sgc = 48, 256, 2
    W = normal(rng, (rows, cols), 0.02)
    cb, mu = O.nf_fit_codebook(W, 4, sgc)
    idx, sc = O.nf_rtn(W, 4, sgc, cb, mu)
    nsg = cols // 64 // sgc
    for r in range(rows):
        rot = O.fwht64(W[r])
        for g in range(nsg):
            d = float(_bf16(sc[((r // 16) * nsg + g) * 16 + r % 16]))
            seg = rot[g * 128:(g + 1) * 128] / d
            k = idx[r, g * 128:(g + 1) * 128]
            err = np.abs(seg - cb[k])
            best = np.abs(seg[:, None] - cb[None, :].astype(np.float64)).min(1)
            assert np.all(err <= best + 1e-3)
    pair, tail = O.nf_from_indices(idx, sc, rows, cols, 4, sgc)
    for r in range(rows):
        assert np.array_equal(O.nf_row_indices(pair, tail, rows, cols, 4, sgc, r), idx[r])


@pytest.mark.parametrize("bits,sgc", [(4, 2), (4, 1), (3, 2), (5, 2)])
def test_nf_gemv_integer_dots(bits, sgc):
    rng = np.random.default_rng(14 + bits)
    rows, cols = 40, 256
    levels = 1 << bits
    idx = rng.integers(0, levels, (rows, cols), dtype=np.uint8)
    nsg = cols // 64 // sgc
    sc = rng.integers(0x3A00, 0x3C00, ((rows + 15) // 16) * nsg * 16).astype(np.uint16)
    cb = np.sort(rng.integers(-127, 128, 16)).astype(np.int8)
    pair, tail = O.nf_from_indices(idx, sc, rows, cols, bits, sgc)
    for r in range(rows):
        assert np.array_equal(O.nf_row_indices(pair, tail, rows, cols, bits, sgc, r), idx[r])
    xq, xs, _ = O.populate_fwht(activation(rng, cols, n_outliers=2))
    out, dots = O.nf_gemv(pair, tail, rows, cols, bits, sgc, cb, xq, xs, want_dots=True)
    full = np.zeros(32, np.int64)
    if bits == 5:
        full[15 - np.arange(16)] = -cb.astype(np.int64)
        full[16 + np.arange(16)] = cb
    else:
        full[:16] = cb
    vals = full[idx]
    brute = (vals.reshape(rows, -1, 64) * xq.astype(np.int64).reshape(1, -1, 64)).sum(2)
    assert np.array_equal(dots, brute)
    port = O.nf_gemv_portable(pair, tail, rows, cols, bits, sgc, cb, xq, xs)
    assert np.all(np.abs(port - out) <= 1e-4 * (1 + np.abs(out)))


# ----------------------------------------------------------------------------- KV + attention
@pytest.mark.parametrize("hd", [64, 128])
def test_kv_quant_head(hd):
    rng = np.random.default_rng(hd)
    v = normal(rng, hd)
    q, s = O.kv_quant_head(v)
    rot = np.concatenate([H64 @ (_signs(b) * v[64 * b:64 * b + 64].astype(np.float64)) / 8 for b in range(hd // 64)])
    assert abs(s - np.abs(rot).max() / 127) < 1e-6
    assert np.abs(q * s - rot).max() <= 0.5 * s + 1e-6
    q0, s0 = O.kv_quant_head(np.zeros(hd, np.float32))
    assert s0 == 0.0 and not q0.any()


@pytest.mark.parametrize("hd,seq", [(64, 37), (128, 300)])
def test_attention_q8_against_f64(hd, seq):
    """real_llm.rs:10190-10284 spirit: q8 Hadamard attention vs exact attention on the
    same (dequantized) operands in f64, then vs fp32 attention by cosine."""
    rng = np.random.default_rng(seq)
    K = normal(rng, (seq, hd))
    V = normal(rng, (seq, hd))
    K[:, 5] *= 12.0  # outlier channel
    qh = normal(rng, hd)
    kq, ks, vq, vs = [], [], [], []
    for t in range(seq):
        a, b = O.kv_quant_head(K[t])
        kq.append(a)
        ks.append(b)
        a, b = O.kv_quant_head(V[t])
        vq.append(a)
        vs.append(b)
    kq, vq = np.stack(kq), np.stack(vq)
    ks, vs = np.array(ks, np.float32), np.array(vs, np.float32)
    scale = 1.0 / np.sqrt(hd)
    out = O.attn_q8_head(qh, kq, ks, vq, vs, scale)
    qi, qs = O.kv_quant_head(qh)
    sc = (kq.astype(np.float64) @ qi.astype(np.float64)) * ks * qs * scale
    p = np.exp(sc - sc.max())
    p /= p.sum()
    o_rot = (p * vs) @ vq.astype(np.float64)
    ref = O.ifwht64(o_rot.astype(np.float32))
    assert np.abs(out - ref).max() < 1e-4 * (1 + np.abs(ref).max())
    s2 = K.astype(np.float64) @ qh * scale
    p2 = np.exp(s2 - s2.max())
    p2 /= p2.sum()
    fp = p2 @ V
    cos = np.dot(out, fp) / (np.linalg.norm(out) * np.linalg.norm(fp))
    assert cos > 0.998


def test_rope_and_swiglu_closed_forms():
    row = O.rope_row(64, 10000.0, 7)
    i = np.arange(32)
    freq = (1.0 / 10000.0 ** (2 * i / 64)).astype(np.float32)
    np.testing.assert_allclose(row[:32], np.cos(np.float32(7) * freq), rtol=1e-6, atol=1e-6)
    h = np.arange(64, dtype=np.float32)
    r = O.rope_apply(h, row)
    # rotation preserves each (x0, x1) pair's norm
    np.testing.assert_allclose(r[:32] ** 2 + r[32:] ** 2, h[:32] ** 2 + h[32:] ** 2, rtol=1e-5)
    g = np.array([-2.0, 0.0, 3.0], np.float32)
    u = np.array([1.0, 5.0, 2.0], np.float32)
    np.testing.assert_allclose(O.swiglu(g, u), g / (1 + np.exp(-g)) * u, rtol=1e-6)


def test_nf4_kv_store_pins():
    """store_hadamard_q4_head_raw (real_llm.rs:8646-8700): nearest-codebook thresholds are
    the midpoints of NF4_DEFAULT_CODEBOOK_I8 (brute force), codes are the nearest entries
    to v / s for the stored BF16 scale, the refined scale is the least-squares fit of
    the first-pass codes (closed form in f64, then BF16), zero blocks store 0x88 / 0."""
    import oracle as O
    cb = np.array([-127, -96, -75, -58, -44, -31, -18, -6, 6, 18, 31, 44, 58, 75, 96, 127], np.float64)
    for y in np.linspace(-140, 140, 5601):
        i = O.nf4_nearest_idx(np.float32(y))
        d = np.abs(cb - y)
        assert d[i] <= d.min() + 1e-9, (y, i)
    rng = np.random.default_rng(4)
    for hd in (64, 128):
        for trial in range(20):
            head = (rng.standard_normal(hd) * rng.uniform(0.01, 3.0)).astype(np.float32)
            q4, s16 = O.kv_quant_head_q4(head)
            rot = O.fwht64(head)
            for g in range(hd // 64):
                blk = rot[g * 64:(g + 1) * 64].astype(np.float64)
                mx = np.abs(blk).max()
                c0 = cb[[O.nf4_nearest_idx(np.float32(v) * np.float32(127.0 / np.float32(mx))) for v in blk]]
                s_ls = (blk * c0).sum() / (c0 * c0).sum()
                s = (np.uint32(s16[g]) << 16).view(np.float32)
                assert abs(float(s) - s_ls) <= 2 ** -7 * s_ls  # one BF16 ulp of the LS scale
                codes = np.zeros(64, np.int64)
                for h in range(2):
                    for i in range(16):
                        b = q4[g * 32 + h * 16 + i]
                        codes[h * 32 + i], codes[h * 32 + 16 + i] = b & 15, b >> 4
                # every code is the nearest codebook entry to v / s
                err = np.abs(cb[codes] * float(s) - blk)
                best = np.abs(cb[None, :] * float(s) - blk[:, None]).min(axis=1)
                assert np.all(err <= best + 1e-6 * max(1.0, float(s) * 127))
    q4, s16 = O.kv_quant_head_q4(np.zeros(64, np.float32))
    assert np.all(q4 == 0x88) and s16[0] == 0


def test_nf4_kv_attention_against_f64():
    """The NF4-KV attention restatement against f64 softmax attention on the dequantized
    K / V (codebook value x BF16 block scale, inverse-rotated) with the unquantized
    query: a dropped scale, a swapped nibble half or a wrong block index fails."""
    import oracle as O
    cb = np.array([-127, -96, -75, -58, -44, -31, -18, -6, 6, 18, 31, 44, 58, 75, 96, 127], np.float64)
    rng = np.random.default_rng(9)

    def deq(q4, s16, hd):
        out = np.zeros(hd)
        for g in range(hd // 64):
            s = float((np.uint32(s16[g]) << 16).view(np.float32))
            for h in range(2):
                for i in range(16):
                    b = q4[g * 32 + h * 16 + i]
                    out[g * 64 + h * 32 + i] = cb[b & 15] * s
                    out[g * 64 + h * 32 + 16 + i] = cb[b >> 4] * s
        return O.ifwht64(out.astype(np.float32)).astype(np.float64)

    for hd in (64, 128):
        n = 50
        K = rng.standard_normal((n, hd)).astype(np.float32)
        V = rng.standard_normal((n, hd)).astype(np.float32)
        q = rng.standard_normal(hd).astype(np.float32)
        k4, ks, v4, vs = [], [], [], []
        for t in range(n):
            a, b = O.kv_quant_head_q4(K[t])
            c, d = O.kv_quant_head_q4(V[t])
            k4.append(a), ks.append(b), v4.append(c), vs.append(d)
        scale = 1.0 / np.sqrt(hd)
        got = O.attn_q4_head(q, np.array(k4), np.array(ks), np.array(v4), np.array(vs), scale)
        Kd = np.stack([deq(k4[t], ks[t], hd) for t in range(n)])
        Vd = np.stack([deq(v4[t], vs[t], hd) for t in range(n)])
        z = Kd @ q.astype(np.float64) * scale
        p = np.exp(z - z.max())
        want = (p / p.sum()) @ Vd
        cos = np.dot(got, want) / (np.linalg.norm(got) * np.linalg.norm(want))
        assert cos > 0.999, (hd, cos)


def test_inv_rms_two_reference_orders():
    """or_inv_rms (x86 portable, real_llm.rs:910-925) and or_inv_rms_neon (aarch64,
    929-962) against the f64 closed form, equal to each other where every partial sum is
    exact (integer squares), and different summation orders (they disagree in the last
    bit on some random inputs)."""
    rng = np.random.default_rng(3)
    for n in (64, 576, 2048, 100):
        x = rng.standard_normal(n).astype(np.float32) * 3
        want = 1.0 / np.sqrt(np.mean(x.astype(np.float64) ** 2) + 1e-5)
        for order in ("x86", "neon"):
            assert abs(O.inv_rms(x, 1e-5, order) / want - 1) < 2e-6
    xi = np.arange(1, 65, dtype=np.float32)  # integer squares: every partial sum exact
    assert O.inv_rms(xi, 0.0, "x86") == O.inv_rms(xi, 0.0, "neon")
    assert O.inv_rms(xi, 0.0) == np.float32(1.0) / np.sqrt(np.float32(np.sum(xi.astype(np.float64) ** 2) / 64))
    diff = 0
    for s in range(200):
        x = np.random.default_rng(s).standard_normal(48).astype(np.float32)
        diff += O.inv_rms(x, 1e-5, "x86") != O.inv_rms(x, 1e-5, "neon")
    assert diff > 0
