"""Exact-order mode (k2t_model_set_exact): the GPU engine against the oracle's x86
restatement of the decode megakernel, at the north_star bar and bit for bit.

In this mode every step follows the x86 reference build's operation order:
  - RMSNorm and q / k norm: the sequential four-accumulator sum of squares
    (dot_f32_fast, real_llm.rs:911-926);
  - GEMVs: the in-order fmaf epilogue (simd_lut.rs:4030-4059, 6334-6335);
  - softmax and SwiGLU: glibc's expf results (f32::exp, real_llm.rs:9595, 9803), by the
    device routine that tests/test_expf.py compares with libm over all 2^32 inputs;
  - attention: sequential softmax and V sums (real_llm.rs:8533-8545, 8575-8585,
    9590-9600), the sliding-window variant with per-64-block score sums (8794-8937);
  - RoPE from the host table (build_rope_table, 9212-9232).
So the oracle's logits (OracleModel with rms_order "x86") are reproduced bit for bit; the
assertion is bit equality, which implies north_star's 1e-4 relative."""
import numpy as np
import pytest

import oracle as O
from model_oracle import OracleModel, random_model
from test_gpu_model import P55454, TINY, TINY128, _gpu_model

pytestmark = pytest.mark.gpu


def _same(a, b, what):
    a, b = np.asarray(a, np.float32), np.asarray(b, np.float32)
    ndiff = int(np.sum(a.view(np.uint32) != b.view(np.uint32)))
    rel = float(np.abs(a - b).max() / np.abs(b).max())
    print(f"  {what}: {ndiff} of {a.size} logits differ in any bit, max rel {rel:.2e}", flush=True)
    assert ndiff == 0, f"{what}: {ndiff} logits differ (max rel {rel:.2e})"


def test_expf_device_matches_libm(gpu_ctx):
    """The device routine on 2^24 + 2^22 inputs: every 256th fp32 bit pattern (the whole
    domain: NaN, inf, subnormal results, both overflow limits) and every pattern in
    [-16, -2^-8] (the softmax arguments s_t - max)."""
    import torch
    a = np.arange(0, 1 << 32, 256, dtype=np.uint64).astype(np.uint32)
    lo, hi = np.float32(-2.0 ** -8).view(np.uint32), np.float32(-16.0).view(np.uint32)
    b = np.arange(lo, hi, max(1, (int(hi) - int(lo)) // (1 << 22)), dtype=np.uint32)
    x = np.concatenate([a, b]).view(np.float32)
    want = np.empty_like(x)
    O.lib().or_expf_array(x, want, x.size)
    dx = torch.from_numpy(x).cuda()
    dy = torch.empty_like(dx)
    import k2t
    k2t.check(k2t.lib().k2t_expf_device(gpu_ctx.h, dx.data_ptr(), dy.data_ptr(), x.size))
    gpu_ctx.sync()
    got = dy.cpu().numpy()
    bad = np.flatnonzero(got.view(np.uint32) != want.view(np.uint32))
    assert bad.size == 0, f"{bad.size} differ, first x = {x[bad[0]]!r}"


CASES = [("nf4_hd64", TINY, "nf4", None, {}),
         ("p55454_hd64", TINY, "n4", P55454, {}),
         ("b6_hd128", TINY128, "n4", {k: 6 for k in P55454}, {}),
         ("nf4_hd128", TINY128, "nf4", None, {}),
         ("nf4_bias_qknorm", TINY, "nf4", None, {"bias": True, "qk_norm": True}),
         ("nf4_window", dict(TINY, max_seq=600), "nf4", None, {"window": (16, 4)})]


# decode steps of these run the persistent kernel's exact-order variant (one weight format
# family, int8 KV without a window, no q / k norm); the others the per-operation path
PERSISTENT = ("nf4_hd64", "p55454_hd64", "b6_hd128", "nf4_hd128")


@pytest.mark.parametrize("persistent", [1, 0])
@pytest.mark.parametrize("name,cfg,fmt,planes,opts", CASES, ids=[c[0] for c in CASES])
def test_exact_decode_bit_identical(gpu_ctx, name, cfg, fmt, planes, opts, persistent):
    """Small models of every weight family: a batched prefill (tokens of one batch share
    each weight pass) and then token-by-token decode, every logit bit-identical to the
    oracle's, with the persistent kernel allowed (1) or off (0).  Variants add a qkv bias
    and Qwen3 q / k norms, or a sliding-window ring (16 positions, 4 sinks) run past the
    ring's 528 slots."""
    print(f"exact decode {name} persistent={persistent}", flush=True)
    layers, head, fn = random_model(cfg, seed=len(name) + 3, fmt=fmt, planes=planes)
    rng = np.random.default_rng(21)
    d, hd, nq, nkv = cfg["hidden"], cfg["head_dim"], cfg["n_heads"], cfg["n_kv_heads"]
    if opts.get("bias"):
        for L in layers:
            L["bias"] = (0.05 * rng.standard_normal((nq + 2 * nkv) * hd)).astype(np.float32)
    if opts.get("qk_norm"):
        for L in layers:
            L["q_norm"] = (1 + 0.1 * rng.standard_normal(hd)).astype(np.float32)
            L["k_norm"] = (1 + 0.1 * rng.standard_normal(hd)).astype(np.float32)
    win = opts.get("window")
    ref = OracleModel(cfg, layers, head, fn, window=win[0] if win else 0, sinks=win[1] if win else 0)
    gm, mats = _gpu_model(gpu_ctx, cfg, layers, head, fn, max_batch=32)
    if opts.get("qk_norm"):
        for i, L in enumerate(layers):
            gm.set_qk_norm(i, L["q_norm"], L["k_norm"])
    if win:
        gm.set_kv_window(*win)
    gm.set_exact(True)
    gm.set_persistent(persistent)
    assert gm.persistent_active() == bool(persistent and name in PERSISTENT)
    n_pre = 560 if win else 12
    toks = rng.integers(0, cfg["vocab"], n_pre + 4)
    pre = gm.prefill(toks[:n_pre], want_logits=True)
    for t in toks[:n_pre - 1]:
        ref.forward_token(int(t), want_logits=False)
    _same(pre, ref.forward_token(int(toks[n_pre - 1])), "prefill")
    for i, t in enumerate(toks[n_pre:]):
        _same(gm.decode(int(t)), ref.forward_token(int(t)), f"decode {i}")
    gm.close()
    for m in mats:
        m.close()
