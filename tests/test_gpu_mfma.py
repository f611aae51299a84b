"""Batched NF4 GEMV on the matrix cores (k2t_gemm_mfma.hip: 16 or more tokens per call,
one weight pass per 64 tokens).

Bar: every output bit-identical to the oracle's per-token NF4 GEMV (the reference's
per-row fmaf chain in chunk order, simd_lut.rs:4030-4059), in the fast and the exact
mode, for shapes with and without a tail stripe, scale groups of one and two chunks and
token counts that leave partial 16-token blocks; with the matrix cores off, the exact
mode's 4-token passes give the same bits.  Model level: a 40-token prefill through it
equals exact-order token-by-token decode and the oracle bit for bit, and the fast-mode
prefill stays within the fast path's bar.
"""
import numpy as np
import pytest

import k2t
import oracle as O
from helpers import acts, quantized_nf4, quantized_nibble4

pytestmark = pytest.mark.gpu


def _t(a):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def _batch(ctx, m, xq, xs, xsum, rows, ntok, exact, mfma=True):
    import torch
    out = torch.full((ntok, rows), float("nan"), dtype=torch.float32, device="cuda")
    ctx.set_exact(exact)
    ctx.set_mfma(mfma)
    try:
        ctx.gemv(m, _t(xq), _t(xs), _t(xsum), out, ntok=ntok, out_stride=rows)
        ctx.sync()
    finally:
        ctx.set_exact(False)
        ctx.set_mfma(True)
    return out.cpu().numpy()


@pytest.mark.parametrize("rows,cols,sgc,ntok", [(1040, 2048, 2, 16), (64, 576, 1, 17), (2048, 2048, 2, 64),
                                                (96, 1536, 2, 100), (1536, 4096, 2, 256)])
def test_mfma_gemv_equals_reference_chain(gpu_ctx, rows, cols, sgc, ntok):
    print(f"mfma gemv {rows}x{cols} sgc {sgc} ntok {ntok}", flush=True)
    rng = np.random.default_rng(rows + cols + ntok)
    _, cb, _, _, pair, tail = quantized_nf4(rng, rows, cols, sgc)
    m = gpu_ctx.upload_nf(rows, cols, 4, sgc, cb, pair, tail)
    xq, xs, xsum = acts(rng, cols, ntok, outlier_frac=0.001, outlier_scale=30.0)
    xs[min(3, ntok - 1), 1] = 0.0  # a chunk with scale 0 (skipped by the reference's chain)
    xq[min(3, ntok - 1), 64:128] = 0
    ref = np.stack([O.nf_gemv(pair, tail, rows, cols, 4, sgc, cb, xq[t], xs[t]) for t in range(ntok)])
    for exact in (False, True):
        out = _batch(gpu_ctx, m, xq, xs, xsum, rows, ntok, exact)
        bad = np.argwhere(out.view(np.uint32) != ref.view(np.uint32))
        assert bad.size == 0, f"exact={exact}: {len(bad)} outputs differ, first {bad[:3].tolist()}"
    if ntok <= 64:
        four = _batch(gpu_ctx, m, xq, xs, xsum, rows, ntok, True, mfma=False)
        assert np.array_equal(four.view(np.uint32), ref.view(np.uint32))
    m.close()


def test_mfma_gemv_strided_output_scale_groups_and_modes(gpu_ctx):
    """Output rows wider than the matrix (out_stride > rows: the gap stays untouched), NF4
    with 4-chunk scale groups (matrix cores) and 3-chunk groups (not a power of two: the
    4-token passes), both bit-identical to the oracle's chain in exact mode; an invalid
    k2t_ctx_set_mfma mode is refused."""
    import torch
    import k2t
    rng = np.random.default_rng(77)
    ntok = 20
    for rows, cols, sgc in [(64, 1024, 4), (48, 576, 3)]:
        _, cb, _, _, pair, tail = quantized_nf4(rng, rows, cols, sgc)
        m = gpu_ctx.upload_nf(rows, cols, 4, sgc, cb, pair, tail)
        xq, xs, xsum = acts(rng, cols, ntok)
        ref = np.stack([O.nf_gemv(pair, tail, rows, cols, 4, sgc, cb, xq[t], xs[t]) for t in range(ntok)])
        stride = rows + 13
        out = torch.full((ntok, stride), 7.0, dtype=torch.float32, device="cuda")
        gpu_ctx.set_exact(True)
        try:
            gpu_ctx.gemv(m, _t(xq), _t(xs), _t(xsum), out, ntok=ntok, out_stride=stride)
            gpu_ctx.sync()
        finally:
            gpu_ctx.set_exact(False)
        o = out.cpu().numpy()
        assert np.array_equal(o[:, :rows].view(np.uint32), ref.view(np.uint32)), (rows, cols, sgc)
        assert np.all(o[:, rows:] == 7.0)
        m.close()
    with pytest.raises(k2t.K2TError):
        gpu_ctx.set_mfma(3)
    gpu_ctx.set_mfma(1)


@pytest.mark.parametrize("planes,rows,cols,ntok", [(4, 1040, 2048, 16), (5, 96, 1536, 100), (6, 2048, 576, 64),
                                                   (4, 1536, 4096, 256), (6, 1040, 1536, 33)])
def test_mfma_bitplane_gemv_equals_reference_chain(gpu_ctx, planes, rows, cols, ntok):
    """Bit-plane matrices (b4 / b5 / b6, Nibble4SdotMatrix; rows % 32 == 16 has a tail
    stripe): every output bit-identical to the oracle's per-token chain of the odd-weight
    dots 2 * sum(u x) - max_odd * sum(x) (simd_lut.rs:4030-4045, 4304-4309), in both modes."""
    print(f"mfma bit-plane gemv b{planes} {rows}x{cols} ntok {ntok}", flush=True)
    rng = np.random.default_rng(planes * 1000 + rows + ntok)
    _, _, _, pair, tail = quantized_nibble4(rng, rows, cols, planes)
    hp = planes - 4
    m = gpu_ctx.upload_nibble4(rows, cols, hp, pair, tail)
    xq, xs, xsum = acts(rng, cols, ntok, outlier_frac=0.001, outlier_scale=30.0)
    xs[min(3, ntok - 1), 1] = 0.0
    xq[min(3, ntok - 1), 64:128] = 0
    xsum[min(3, ntok - 1), 1] = 0
    ref = np.stack([O.nibble4_gemv(pair, tail, rows, cols, hp, xq[t], xs[t], xsum[t]) for t in range(ntok)])
    for exact in (False, True):
        out = _batch(gpu_ctx, m, xq, xs, xsum, rows, ntok, exact)
        bad = np.argwhere(out.view(np.uint32) != ref.view(np.uint32))
        assert bad.size == 0, f"exact={exact}: {len(bad)} outputs differ, first {bad[:3].tolist()}"
    m.close()


@pytest.mark.parametrize("fmt,planes,max_seq,hd,n,ffn,qk", [("nf4", None, 64, 64, 40, 768, False),
                                                            ("nf4", None, 1100, 64, 40, 768, False),
                                                            ("n4", "p55454", 64, 64, 40, 768, False),
                                                            ("n4", "b6", 64, 64, 40, 768, False),
                                                            ("nf4", None, 300, 128, 40, 768, False),
                                                            ("nf4", None, 160, 64, 100, 8192, False),
                                                            ("n4", "p55454", 160, 64, 100, 8192, False),
                                                            ("nf4", None, 64, 64, 40, 768, True)])
def test_mfma_prefill_matches_exact_decode_and_oracle(gpu_ctx, fmt, planes, max_seq, hd, n, ffn, qk):
    """A 2-layer model (d 256, 256 / hd heads of hd 64 or 128, ffn 768 or 8192; nf4, p55454
    and b6 weights): an n-token prefill (qkv, o with the residual add, gate_up and down with the
    residual add on the matrix cores) in exact-order mode equals the oracle bit for bit,
    and so does the one with the matrix cores off, and one of 20 + (n - 20) tokens (the
    second batch appended at position 20).  In fast mode the batch's attention also runs
    on the matrix cores (attn_prefill_mfma_kernel), and the activation tiles written by
    their producers (RMSNorm, attention, SwiGLU or, with ffn 8192 and 100 tokens, gate_up's
    SwiGLU epilogue), with the qkv GEMV's q / k / v epilogue at head size 64 (also with a
    qkv bias and q / k norms), give the same logits as tiles copied by the GEMV (mode 2: separate SwiGLU),
    within the fast path's bar of the oracle, for one batch and for 20 + (n - 20)."""
    from model_oracle import OracleModel, random_model
    from test_gpu_model import P55454, _close, _gpu_model
    print(f"mfma prefill vs oracle, {fmt} {planes} max_seq {max_seq} hd {hd} n {n}", flush=True)
    plane_map = {"p55454": P55454, "b6": {k: 6 for k in P55454}, None: None}[planes]
    cfg = dict(n_layers=2, hidden=256, n_heads=256 // hd, n_kv_heads=128 // hd, head_dim=hd, intermediate=ffn,
               vocab=520, max_seq=max_seq, rms_eps=1e-5, rope_theta=10000.0)
    layers, head, fn = random_model(cfg, seed=41, fmt=fmt, planes=plane_map)
    if qk:  # a qkv bias and Qwen3 q / k norms (the q / k / v epilogue of the qkv GEMV applies them)
        rng = np.random.default_rng(5)
        nqkv = (cfg["n_heads"] + 2 * cfg["n_kv_heads"]) * hd
        for L in layers:
            L["bias"] = (0.05 * rng.standard_normal(nqkv)).astype(np.float32)
            L["q_norm"] = (1 + 0.1 * rng.standard_normal(hd)).astype(np.float32)
            L["k_norm"] = (1 + 0.1 * rng.standard_normal(hd)).astype(np.float32)
    ref = OracleModel(cfg, layers, head, fn)
    toks = np.random.default_rng(42).integers(0, cfg["vocab"], n)
    for t in toks[:-1]:
        ref.forward_token(int(t), want_logits=False)
    b = ref.forward_token(int(toks[-1]))
    gm, mats = _gpu_model(gpu_ctx, cfg, layers, head, fn, max_batch=128)
    if qk:
        for i, L in enumerate(layers):
            gm.set_qk_norm(i, L["q_norm"], L["k_norm"])
    try:
        gm.set_exact(True)
        for mfma in (True, False):
            gpu_ctx.set_mfma(mfma)
            gm.reset()
            pre = gm.prefill(toks, want_logits=True)
            assert np.array_equal(pre.view(np.uint32), b.view(np.uint32)), f"mfma={mfma}"
        gm.reset()
        gm.prefill(toks[:20], want_logits=False)
        pre = gm.prefill(toks[20:], want_logits=True)
        assert np.array_equal(pre.view(np.uint32), b.view(np.uint32)), "20 + 20"
        gm.set_exact(False)
        fast = {}
        for mode in (1, 2):  # tiles written by the activations' producers / copied by the GEMV
            gpu_ctx.set_mfma(mode)
            gm.reset()
            fast[mode] = gm.prefill(toks, want_logits=True)
        assert np.array_equal(fast[1].view(np.uint32), fast[2].view(np.uint32))
        ok, info = _close(fast[1], b, 0.9999)
        assert ok, info
        gpu_ctx.set_mfma(1)
        gm.reset()
        gm.prefill(toks[:20], want_logits=False)
        ok, info = _close(gm.prefill(toks[20:], want_logits=True), b, 0.9999)
        assert ok, ("20 + 20", info)
    finally:
        gpu_ctx.set_mfma(True)
        gm.close()
        for m in mats:
            m.close()
