"""test_nf3_nf4_sdot_neon_scalar_parity_and_quality (simd_lut.rs:9138-9320) on the GPU
GEMV, with the reference's own input generators (LCG weights with spike columns,
`sample_x` activations with every 23rd channel x6).  The reference compiles with GPTQ;
here the weights go through this repository's RTN compiler (same layouts).  Checks, at
the reference's tolerances:
  - exact-mode GEMV vs the scalar dequantize + fp32 dot path: |d| <= 1e-4 * max(|y|, 1)
    for rows 71 (odd stripe count, tail records) and 128, NF3 / NF4, sgc 1 / 2;
  - stripe range [0, 1) then [1, S) equals the full range (bit-exact);
  - 15-token batches vs single tokens: |d| <= 1e-4 * max(|y|, 1);
  - gate_up interleave (NF4 and 4-plane bit planes, 256 rows): interleaved outputs equal
    the plain outputs reordered, bit for bit."""
import numpy as np
import pytest
import torch

import k2t
import oracle as O

pytestmark = pytest.mark.gpu
M64 = (1 << 64) - 1
COLS = 256


def sample_x(seed):
    s = (seed ^ 0x9E3779B97F4A7C15) & M64
    out = np.zeros(COLS, np.float32)
    for c in range(COLS):
        s = (s * 6364136223846793005 + 1442695040888963407) & M64
        u = np.float32(s >> 40) / np.float32(1 << 24) - np.float32(0.5)
        out[c] = u * np.float32(6.0 if c % 23 == 0 else 1.0)
    return out


def lcg_weights(rows):
    ws = 0x517CC1B727220A95
    w = np.zeros(rows * COLS, np.float32)
    for idx in range(rows * COLS):
        ws = (ws * 6364136223846793005 + 1) & M64
        z1 = np.float32(ws >> 40) / np.float32(1 << 24) - np.float32(0.5)
        ws = (ws * 6364136223846793005 + 1) & M64
        z2 = np.float32(ws >> 40) / np.float32(1 << 24) - np.float32(0.5)
        w[idx] = ((z1 + z2) * np.float32(0.4)) * np.float32(3.5 if idx % 64 == 7 else 1.0)
    return w.reshape(rows, COLS)


def act_of(x):
    return O.populate_plain(O.fwht64(x))


def gemv(ctx, m, rows, xq, xs, xsum, ntok=1, s0=0, s1=-1, out=None):
    if out is None:
        out = torch.full((ntok, rows), float("nan"), dtype=torch.float32, device="cuda")
    dev = lambda a: torch.from_numpy(np.ascontiguousarray(a)).cuda()  # noqa: E731
    ctx.set_exact(True)
    try:
        ctx.gemv(m, dev(xq), dev(xs), dev(xsum), out, ntok=ntok, s0=s0, s1=s1, out_stride=rows)
        ctx.sync()
    finally:
        ctx.set_exact(False)
    return out


@pytest.mark.parametrize("rows", [71, 128])
@pytest.mark.parametrize("bits", [3, 4])
@pytest.mark.parametrize("sgc", [1, 2])
def test_reference_nf_parity(gpu_ctx, rows, bits, sgc):
    print(f"reference nf parity rows={rows} bits={bits} sgc={sgc}", flush=True)
    W = lcg_weights(rows)
    cb, _, pair, tail = k2t.compile_nf4(W, sgc, bits=bits)
    m = gpu_ctx.upload_nf(rows, COLS, bits, sgc, cb, pair, tail)
    xq, xs, xsum = act_of(sample_x(4242 + bits * 10 + sgc))
    y = gemv(gpu_ctx, m, rows, xq, xs, xsum).cpu().numpy()[0]
    y_scalar = O.nf_gemv_portable(pair, tail, rows, COLS, bits, sgc, cb, xq, xs)
    tol = 1e-4 * np.maximum(np.abs(y_scalar), 1.0)
    assert np.all(np.abs(y - y_scalar) <= tol), np.max(np.abs(y - y_scalar) / tol)
    # odd stripe split: [0, 1) then [1, S)
    S = (rows + 15) // 16
    out = torch.full((1, rows), float("nan"), dtype=torch.float32, device="cuda")
    gemv(gpu_ctx, m, rows, xq, xs, xsum, s0=0, s1=1, out=out)
    gemv(gpu_ctx, m, rows, xq, xs, xsum, s0=1, s1=S, out=out)
    assert np.array_equal(out.cpu().numpy()[0].view(np.uint32), y.view(np.uint32))
    # 15-token batch vs single tokens
    acts = [act_of(sample_x(7700 + t)) for t in range(15)]
    bq = np.stack([a[0] for a in acts])
    bs = np.stack([a[1] for a in acts])
    bm = np.stack([a[2] for a in acts])
    yb = gemv(gpu_ctx, m, rows, bq, bs, bm, ntok=15).cpu().numpy()
    for t in range(15):
        y1 = gemv(gpu_ctx, m, rows, bq[t], bs[t], bm[t]).cpu().numpy()[0]
        assert np.all(np.abs(yb[t] - y1) <= 1e-4 * np.maximum(np.abs(y1), 1.0)), t
    m.close()


def test_reference_gate_up_interleave(gpu_ctx):
    rows = 256
    i = np.arange(rows * COLS, dtype=np.float32)
    W = (np.sin(i * np.float32(0.137)) * np.float32(0.5)).astype(np.float32).reshape(rows, COLS)
    xq, xs, xsum = act_of(sample_x(9999))
    p_pair, p_tail = k2t.compile_bipolar(W, 4, interleave_gate_up=False)
    i_pair, i_tail = k2t.compile_bipolar(W, 4, interleave_gate_up=True)
    cbp, _, fp_pair, fp_tail = k2t.compile_nf4(W, 1)
    cbi, _, fi_pair, fi_tail = k2t.compile_nf4(W, 1, interleave_gate_up=True)
    assert np.array_equal(cbp, cbi)
    mats = [gpu_ctx.upload_nibble4(rows, COLS, 0, p_pair, p_tail), gpu_ctx.upload_nibble4(rows, COLS, 0, i_pair, i_tail),
            gpu_ctx.upload_nf(rows, COLS, 4, 1, cbp, fp_pair, fp_tail),
            gpu_ctx.upload_nf(rows, COLS, 4, 1, cbi, fi_pair, fi_tail)]
    yp_n, yi_n, yp_f, yi_f = (gemv(gpu_ctx, mm, rows, xq, xs, xsum).cpu().numpy()[0] for mm in mats)
    for ic in range(2):
        for yi, yp in ((yi_n, yp_n), (yi_f, yp_f)):
            assert np.array_equal(yi[ic * 128:ic * 128 + 64].view(np.uint32), yp[ic * 64:(ic + 1) * 64].view(np.uint32))
            assert np.array_equal(yi[ic * 128 + 64:ic * 128 + 128].view(np.uint32),
                                  yp[128 + ic * 64:128 + (ic + 1) * 64].view(np.uint32))
    for mm in mats:
        mm.close()
