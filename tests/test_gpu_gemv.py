"""GPU parity of the activation quantizer and the GEMV / 4-token tile (C ABI -> HIP).

Bar: int8 q / scales / sums and every per-(row, chunk) integer dot bit-exact against
the oracle; fp32 GEMV outputs bit-exact (same fmaf order as the reference's NEON
epilogue) in exact mode for every K split, because the per-chunk terms are staged in
LDS and the chain is replayed in chunk order; the default fast epilogue within
1e-5 * (1 + |y|) (the reference's own batch tolerance is 1e-4 * (1 + |y|),
simd_lut.rs:8936).
"""
import numpy as np
import pytest

import oracle as O
from helpers import acts, activation, quantized_nf4, quantized_nibble4, random_nf_streams, random_nibble4_streams

pytestmark = pytest.mark.gpu


def _t(a, dtype=None):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def _run_gemv(ctx, m, xq, xs, xsum, rows, ntok=1, s0=0, s1=-1, exact=True):
    import torch
    out = torch.full((ntok, rows), float("nan"), dtype=torch.float32, device="cuda")
    ctx.set_exact(exact)
    try:
        ctx.gemv(m, _t(xq), _t(xs), _t(xsum), out, ntok=ntok, s0=s0, s1=s1, out_stride=rows)
        ctx.sync()
    finally:
        ctx.set_exact(False)
    return out.cpu().numpy()


def _close(out, ref, tol=1e-5):
    """Fast epilogue: per-segment chains summed in a fixed order (a few ulp)."""
    return np.all(np.abs(out - ref) <= tol * (1 + np.abs(ref)))


@pytest.mark.parametrize("K,ntok,norm", [(576, 1, False), (2048, 1, True), (14336, 2, True), (8192, 3, False)])
def test_act_quant_bit_exact(gpu_ctx, K, ntok, norm):
    import torch
    rng = np.random.default_rng(K + ntok)
    x = np.stack([activation(rng, K, outlier_frac=0.001, outlier_scale=30.0, zero_chunk=t + 1) for t in range(ntok)])
    w = (0.75 + 0.4 * np.cos(np.arange(K) * 0.13)).astype(np.float32) if norm else None
    inv = np.array([0.8125, 1.3, 0.55][:ntok], np.float32) if norm else None
    q = torch.zeros((ntok, K), dtype=torch.int8, device="cuda")
    s = torch.zeros((ntok, K // 64), dtype=torch.float32, device="cuda")
    m = torch.zeros((ntok, K // 64), dtype=torch.int32, device="cuda")
    gpu_ctx.act_quant(_t(x), q, s, m, K, ntok, norm_w=None if w is None else _t(w),
                      inv_rms=None if inv is None else _t(inv))
    gpu_ctx.sync()
    for t in range(ntok):
        rq, rs, rm = O.populate_fwht(x[t], w, 1.0 if inv is None else inv[t])
        assert np.array_equal(q[t].cpu().numpy(), rq)
        assert np.array_equal(s[t].cpu().numpy().view(np.uint32), rs.view(np.uint32))
        assert np.array_equal(m[t].cpu().numpy(), rm)


def test_act_quant_rmsnorm_close(gpu_ctx):
    import torch
    rng = np.random.default_rng(7)
    K = 2048
    x = activation(rng, K, n_outliers=4)
    w = (1.0 + 0.1 * rng.standard_normal(K)).astype(np.float32)
    q = torch.zeros(K, dtype=torch.int8, device="cuda")
    s = torch.zeros(K // 64, dtype=torch.float32, device="cuda")
    m = torch.zeros(K // 64, dtype=torch.int32, device="cuda")
    gpu_ctx.act_quant_rmsnorm(_t(x), _t(w), 1e-5, q, s, m, K, 1)
    gpu_ctx.sync()
    rq, rs, rm = O.populate_fwht(x, w, O.inv_rms(x, 1e-5))
    assert np.abs(q.cpu().numpy().astype(int) - rq).max() <= 1
    np.testing.assert_allclose(s.cpu().numpy(), rs, rtol=1e-6)


NIBBLE_SHAPES = [(1536, 576), (40, 192), (54, 1536), (50, 256), (960, 576), (3072, 2048)]


@pytest.mark.parametrize("hp", [0, 1, 2])
@pytest.mark.parametrize("rows,cols", NIBBLE_SHAPES)
def test_nibble4_gemv_exact(gpu_ctx, hp, rows, cols):
    rng = np.random.default_rng(rows * 7 + cols + hp)
    pair, tail = random_nibble4_streams(rng, rows, cols, hp)
    m = gpu_ctx.upload_nibble4(rows, cols, hp, pair, tail)
    xq, xs, xsum = acts(rng, cols, 1, n_outliers=4, zero_chunk=1)
    ref, dots = O.nibble4_gemv(pair, tail, rows, cols, hp, xq[0], xs[0], xsum[0], want_dots=True)
    import torch
    d = torch.zeros((rows, cols // 64), dtype=torch.int32, device="cuda")
    gpu_ctx.gemv_chunk_dots(m, _t(xq[0]), _t(xsum[0]), d)
    assert np.array_equal(d.cpu().numpy(), dots), "integer chunk dots differ"
    out = _run_gemv(gpu_ctx, m, xq[0], xs[0], xsum[0], rows)[0]
    assert np.array_equal(out.view(np.uint32), ref.view(np.uint32)), "exact epilogue not bit-exact"
    gpu_ctx.set_splitk(1)
    try:
        out1 = _run_gemv(gpu_ctx, m, xq[0], xs[0], xsum[0], rows)[0]
    finally:
        gpu_ctx.set_splitk(0)
    assert np.array_equal(out1.view(np.uint32), ref.view(np.uint32)), "single-segment result not bit-exact"
    assert _close(_run_gemv(gpu_ctx, m, xq[0], xs[0], xsum[0], rows, exact=False)[0], ref)


def test_nibble4_config1_quantized(gpu_ctx):
    """Config 1: W 1536x576 ~N(0,0.02) Hadamard RTN b4, x with 4 outliers x20."""
    rng = np.random.default_rng(1)
    rows, cols = 1536, 576
    W, u, sc, pair, tail = quantized_nibble4(rng, rows, cols, 4)
    x = activation(rng, cols, n_outliers=4, outlier_scale=20.0)
    xq, xs, xsum = O.populate_fwht(x)
    m = gpu_ctx.upload_nibble4(rows, cols, 0, pair, tail)
    out = _run_gemv(gpu_ctx, m, xq, xs, xsum, rows)[0]
    ref = O.nibble4_gemv(pair, tail, rows, cols, 0, xq, xs, xsum)
    assert np.array_equal(out.view(np.uint32), ref.view(np.uint32))
    assert _close(_run_gemv(gpu_ctx, m, xq, xs, xsum, rows, exact=False)[0], ref)
    # and the quantized product approximates the fp32 one (W x)
    y = W.astype(np.float64) @ x.astype(np.float64)
    cos = float(np.dot(out, y) / (np.linalg.norm(out) * np.linalg.norm(y)))
    assert cos > 0.99


@pytest.mark.parametrize("sgc", [1, 2])
@pytest.mark.parametrize("rows,cols", [(1536, 576), (40, 256), (6144, 2048), (2048, 8192)])
def test_nf4_gemv_exact(gpu_ctx, sgc, rows, cols):
    import torch
    rng = np.random.default_rng(rows + cols + sgc)
    idx, sc, pair, tail = random_nf_streams(rng, rows, cols, sgc)
    cb = np.array([-127, -96, -75, -58, -44, -31, -18, -6, 6, 18, 31, 44, 58, 75, 96, 127], np.int8)
    if sgc == 1:
        cb = np.sort(rng.integers(-127, 128, 16)).astype(np.int8)  # asymmetric table
    m = gpu_ctx.upload_nf(rows, cols, 4, sgc, cb, pair, tail)
    xq, xs, xsum = acts(rng, cols, 1, n_outliers=3, zero_chunk=2)
    ref, dots = O.nf_gemv(pair, tail, rows, cols, 4, sgc, cb, xq[0], xs[0], want_dots=True)
    d = torch.zeros((rows, cols // 64), dtype=torch.int32, device="cuda")
    gpu_ctx.gemv_chunk_dots(m, _t(xq[0]), None, d)
    assert np.array_equal(d.cpu().numpy(), dots)
    out = _run_gemv(gpu_ctx, m, xq[0], xs[0], xsum[0], rows)[0]
    assert np.array_equal(out.view(np.uint32), ref.view(np.uint32))
    assert _close(_run_gemv(gpu_ctx, m, xq[0], xs[0], xsum[0], rows, exact=False)[0], ref)


@pytest.mark.parametrize("sgc", [1, 2])
@pytest.mark.parametrize("rows,cols", [(1536, 2048), (40, 256), (2048, 768)])
def test_nf3_gemv_exact(gpu_ctx, sgc, rows, cols):
    """NF3 stripes (simd_lut.rs:4932-4960, 6074-6364 with BITS = 3): 8-entry codebook,
    48-byte triplet blocks.  Integer dots and the exact epilogue bit-exact."""
    import torch
    rng = np.random.default_rng(rows + cols + sgc + 3)
    idx, sc, pair, tail = random_nf_streams(rng, rows, cols, sgc, bits=3)
    cb = np.zeros(16, np.int8)
    cb[:8] = np.sort(rng.choice(np.arange(-127, 128), 8, replace=False)).astype(np.int8)
    m = gpu_ctx.upload_nf(rows, cols, 3, sgc, cb, pair, tail)
    xq, xs, xsum = acts(rng, cols, 1, n_outliers=3, zero_chunk=1)
    ref, dots = O.nf_gemv(pair, tail, rows, cols, 3, sgc, cb, xq[0], xs[0], want_dots=True)
    d = torch.zeros((rows, cols // 64), dtype=torch.int32, device="cuda")
    gpu_ctx.gemv_chunk_dots(m, _t(xq[0]), None, d)
    assert np.array_equal(d.cpu().numpy(), dots)
    out = _run_gemv(gpu_ctx, m, xq[0], xs[0], xsum[0], rows)[0]
    assert np.array_equal(out.view(np.uint32), ref.view(np.uint32))
    assert _close(_run_gemv(gpu_ctx, m, xq[0], xs[0], xsum[0], rows, exact=False)[0], ref)


@pytest.mark.parametrize("rows,cols,sgc", [(40, 256, 1), (1536, 2048, 2)])
def test_nf3_lane_order_wrap_and_convert(gpu_ctx, rows, cols, sgc):
    """A wrapped NF3 matrix streams the reference layout (simd_lut.rs:4932-4960) as it
    lies; k2t_mat_nf3_lane_order rearranges it in place (16-byte piece k of triplet block
    (g, half) from 192*half + 48*g + 16*k to 128*k + 16*(2g + half) of each 384-byte
    stripe-chunk), and the GEMV gives the same bit-exact rows before and after, as does
    an uploaded copy (stored in lane order at upload).  A second conversion is a no-op."""
    import torch
    rng = np.random.default_rng(rows + sgc + 91)
    idx, sc, pair, tail = random_nf_streams(rng, rows, cols, sgc, bits=3)
    cb = np.zeros(16, np.int8)
    cb[:8] = np.sort(rng.choice(np.arange(-127, 128), 8, replace=False)).astype(np.int8)
    dp = torch.from_numpy(pair.copy()).cuda()
    dt = torch.from_numpy(tail.copy()).cuda() if tail.size else None
    m = gpu_ctx.wrap_nf(rows, cols, 3, sgc, cb, dp, pair.size, dt, tail.size)
    xq, xs, xsum = acts(rng, cols, 1, n_outliers=3, zero_chunk=1)
    ref = O.nf_gemv(pair, tail, rows, cols, 3, sgc, cb, xq[0], xs[0])
    before = _run_gemv(gpu_ctx, m, xq[0], xs[0], xsum[0], rows)[0]
    assert np.array_equal(before.view(np.uint32), ref.view(np.uint32))
    m.nf3_lane_order()
    got = dp.cpu().numpy()
    # literal positions inside the first pair record's chunk 0, side 0 (at byte 64, after
    # the 64-byte scale header), when the matrix has pair records
    if rows >= 32:
        c0 = 64
        for (g, h, k) in [(0, 0, 0), (1, 1, 2), (3, 0, 1), (2, 1, 0), (3, 1, 2)]:
            src = c0 + 192 * h + 48 * g + 16 * k
            dst = c0 + 128 * k + 16 * (2 * g + h)
            assert np.array_equal(got[dst:dst + 16], pair[src:src + 16]), (g, h, k)
        assert np.array_equal(got[:64], pair[:64])  # scale header untouched
    assert np.array_equal(np.sort(got), np.sort(pair))
    if dt is not None:
        assert np.array_equal(np.sort(dt.cpu().numpy()), np.sort(tail))
    after = _run_gemv(gpu_ctx, m, xq[0], xs[0], xsum[0], rows)[0]
    assert np.array_equal(after.view(np.uint32), ref.view(np.uint32))
    m.nf3_lane_order()
    assert np.array_equal(dp.cpu().numpy(), got)
    up = gpu_ctx.upload_nf(rows, cols, 3, sgc, cb, pair, tail)
    assert np.array_equal(_run_gemv(gpu_ctx, up, xq[0], xs[0], xsum[0], rows)[0].view(np.uint32),
                          ref.view(np.uint32))
    m.close()
    up.close()


def test_nf3_expert_slice_pair_range_and_batch(gpu_ctx):
    """nf_sdot_pair_stream_range_slices (simd_lut.rs:6372-6540): an expert's NF3 g128
    gate_up slice (rows % 32 == 0, no tail) run over a pair sub-range writes exactly those
    rows; 4-token tiles equal the per-token results."""
    rng = np.random.default_rng(21)
    rows, cols, sgc = 1536, 2048, 2
    W = (rng.standard_normal((rows, cols)) * 0.02).astype(np.float32)
    cb, mu = O.nf_fit_codebook(W, 3, sgc)
    idx, sc = O.nf_rtn(W, 3, sgc, cb, mu)
    pair, tail = O.nf_from_indices(idx, sc, rows, cols, 3, sgc)
    assert tail.size == 0
    m = gpu_ctx.upload_nf(rows, cols, 3, sgc, cb, pair, tail)
    xq, xs, xsum = acts(rng, cols, 4, outlier_frac=0.001, outlier_scale=30.0)
    p0, p1 = 7, 30  # pair range -> stripes [14, 60)
    out = _run_gemv(gpu_ctx, m, xq[0], xs[0], xsum[0], rows, s0=2 * p0, s1=2 * p1)[0]
    ref = O.nf_gemv(pair, tail, rows, cols, 3, sgc, cb, xq[0], xs[0], s0=2 * p0, s1=2 * p1)
    lo, hi = 32 * p0, 32 * p1
    assert np.array_equal(out[lo:hi].view(np.uint32), ref[lo:hi].view(np.uint32))
    assert np.isnan(out[:lo]).all() and np.isnan(out[hi:]).all()
    batch = _run_gemv(gpu_ctx, m, xq, xs, xsum, rows, ntok=4)
    for t in range(4):
        single = O.nf_gemv(pair, tail, rows, cols, 3, sgc, cb, xq[t], xs[t])
        assert np.array_equal(batch[t].view(np.uint32), single.view(np.uint32)), t


def test_nf4_quantized_model_matrix(gpu_ctx):
    rng = np.random.default_rng(3)
    rows, cols = 2048, 2048
    W, cb, idx, sc, pair, tail = quantized_nf4(rng, rows, cols, 2)
    x = activation(rng, cols, outlier_frac=0.001, outlier_scale=30.0)
    xq, xs, xsum = O.populate_fwht(x)
    m = gpu_ctx.upload_nf(rows, cols, 4, 2, cb, pair, tail)
    out = _run_gemv(gpu_ctx, m, xq, xs, xsum, rows)[0]
    ref = O.nf_gemv(pair, tail, rows, cols, 4, 2, cb, xq, xs)
    assert np.array_equal(out.view(np.uint32), ref.view(np.uint32))
    assert _close(_run_gemv(gpu_ctx, m, xq, xs, xsum, rows, exact=False)[0], ref)


@pytest.mark.parametrize("fmt", ["b5", "nf4"])
def test_batch_matches_single(gpu_ctx, fmt):
    """simd_lut.rs:8908-8940: 54 rows, K=1536, 15 tokens (every tile tail); batch == per token."""
    rng = np.random.default_rng(15)
    rows, cols, ntok = 54, 1536, 15
    if fmt == "b5":
        pair, tail = random_nibble4_streams(rng, rows, cols, 1)
        m = gpu_ctx.upload_nibble4(rows, cols, 1, pair, tail)
    else:
        _, _, pair, tail = random_nf_streams(rng, rows, cols, 2)
        cb = np.array([-127, -96, -75, -58, -44, -31, -18, -6, 6, 18, 31, 44, 58, 75, 96, 127], np.int8)
        m = gpu_ctx.upload_nf(rows, cols, 4, 2, cb, pair, tail)
    xq, xs, xsum = acts(rng, cols, ntok)
    batch = _run_gemv(gpu_ctx, m, xq, xs, xsum, rows, ntok=ntok)
    for t in range(ntok):
        one = _run_gemv(gpu_ctx, m, xq[t], xs[t], xsum[t], rows)[0]
        assert np.array_equal(batch[t].view(np.uint32), one.view(np.uint32)), f"token {t}"
    # fast epilogue: batch == per token bit for bit (same segment plan), and near exact
    fb = _run_gemv(gpu_ctx, m, xq, xs, xsum, rows, ntok=ntok, exact=False)
    for t in range(ntok):
        one = _run_gemv(gpu_ctx, m, xq[t], xs[t], xsum[t], rows, exact=False)[0]
        assert np.array_equal(fb[t].view(np.uint32), one.view(np.uint32)), f"token {t}"
    assert _close(fb, batch)


def test_stripe_subrange(gpu_ctx):
    """Odd start / end stripes (simd_lut.rs:3883-3888, 4086-4090) write only their rows."""
    rng = np.random.default_rng(5)
    rows, cols, hp = 200, 512, 2  # 13 stripes: 6 pairs + tail
    pair, tail = random_nibble4_streams(rng, rows, cols, hp)
    m = gpu_ctx.upload_nibble4(rows, cols, hp, pair, tail)
    xq, xs, xsum = acts(rng, cols, 1)
    ref = O.nibble4_gemv(pair, tail, rows, cols, hp, xq[0], xs[0], xsum[0])
    for s0, s1 in [(1, 12), (3, 13), (0, 1), (12, 13), (5, 6)]:
        for exact in (True, False):
            out = _run_gemv(gpu_ctx, m, xq[0], xs[0], xsum[0], rows, s0=s0, s1=s1, exact=exact)[0]
            lo, hi = s0 * 16, min(s1 * 16, rows)
            assert np.all(np.isnan(out[:lo])) and np.all(np.isnan(out[hi:]))
            if exact:
                assert np.array_equal(out[lo:hi].view(np.uint32), ref[lo:hi].view(np.uint32))
            else:
                assert _close(out[lo:hi], ref[lo:hi])


@pytest.mark.parametrize("rows,cols,hp", [(14336, 4096, 2), (4096, 14336, 2)])
def test_large_b6_dots_and_outputs(gpu_ctx, rows, cols, hp):
    """Config 4 shapes: integer dots exact over the full matrix, outputs within tolerance."""
    import torch
    rng = np.random.default_rng(rows)
    pair, tail = random_nibble4_streams(rng, rows, cols, hp)
    m = gpu_ctx.upload_nibble4(rows, cols, hp, pair, tail)
    xq, xs, xsum = acts(rng, cols, 1, outlier_frac=0.001, outlier_scale=30.0)
    ref, dots = O.nibble4_gemv(pair, tail, rows, cols, hp, xq[0], xs[0], xsum[0], want_dots=True)
    d = torch.zeros((rows, cols // 64), dtype=torch.int32, device="cuda")
    gpu_ctx.gemv_chunk_dots(m, _t(xq[0]), _t(xsum[0]), d)
    assert np.array_equal(d.cpu().numpy(), dots)
    out = _run_gemv(gpu_ctx, m, xq[0], xs[0], xsum[0], rows)[0]
    assert np.array_equal(out.view(np.uint32), ref.view(np.uint32))
    assert _close(_run_gemv(gpu_ctx, m, xq[0], xs[0], xsum[0], rows, exact=False)[0], ref)


def test_batch4_large_k(gpu_ctx):
    """4 tokens x K=14336: the kernel takes fewer tokens per weight pass so the staged
    per-chunk terms fit in LDS; results stay bit-exact."""
    rng = np.random.default_rng(21)
    rows, cols, ntok = 256, 14336, 4
    _, _, pair, tail = random_nf_streams(rng, rows, cols, 2)
    cb = np.array([-127, -96, -75, -58, -44, -31, -18, -6, 6, 18, 31, 44, 58, 75, 96, 127], np.int8)
    m = gpu_ctx.upload_nf(rows, cols, 4, 2, cb, pair, tail)
    xq, xs, xsum = acts(rng, cols, ntok)
    out = _run_gemv(gpu_ctx, m, xq, xs, xsum, rows, ntok=ntok)
    fast = _run_gemv(gpu_ctx, m, xq, xs, xsum, rows, ntok=ntok, exact=False)
    for t in range(ntok):
        ref = O.nf_gemv(pair, tail, rows, cols, 4, 2, cb, xq[t], xs[t])
        assert np.array_equal(out[t].view(np.uint32), ref.view(np.uint32))
        assert _close(fast[t], ref)
