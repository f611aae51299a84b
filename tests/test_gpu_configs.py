"""Parity at the benchmark configurations' own shapes (configs 2-5 of BASELINE.json), through the C ABI,
against the oracle on the same seeded inputs.

- config 4: nf4g128 / nf3g128 / b6 GEMVs at 14336x4096 and 4096x14336, batch 1 and 4,
  weights from the product compiler (the bench's generator and seeds): per-(row, chunk)
  integer dots exact, exact-mode fp32 outputs bit-identical to the oracle's in-order
  fmaf epilogue (simd_lut.rs:4030-4059, 6334-6335), every token of a 4-token tile too.
- config 3: the SmolLM2-1.7B-shaped nf4g128 model (d 2048, 32 heads, ffn 8192, vocab
  49152) on the default persistent decode kernel, at 2 layers and at its full 24: a
  12-token prefill in 4-token weight passes, decode steps against OracleModel, and a
  device-side greedy run against the oracle's argmax.
- config 2: the SmolLM2-135M-shaped p55454 model at 2 layers and its full 30, at context
  512 (synthetic K/V, then a batched 64-token prefill), decode on the per-operation graph
  and on the mixed-plane persistent kernel.
- config 5: the Qwen3-30B-A3B shape at full width and two layers (hd 128, 32 q / 4 kv
  heads, QK-norm, 128 NF3 experts top 8, bf16 embedding, vocab 151936) at context 1100
  and at the bench's own 6600 (52 spans, 8 q heads per KV head), so decode runs the
  grouped-query attention kernel (span and merge workgroups in one launch).
- exact-order mode: configs 3 and 2 at two layers and full depth, every logit
  bit-identical to the x86 oracle's (north_star's 1e-4 relative, with no code flips).

Fast-mode bar: at two layers cosine > 0.9995 and max |diff| <= 2% of max |logit| on
every step, with no fallback (the fast path sums in tree order and uses the device expf,
so an int8 code can move by one where inv_rms / expf round differently: the reference's
own NEON and portable builds differ there too).  At the full 24 / 30 layers such
one-code flips compound, and the reference's two builds (x86 and aarch64 sum-of-squares
orders, real_llm.rs:903-962) themselves end about 1e-3 of cosine apart on these
random-init models; a full-depth step that misses the fixed bar (cosine > 0.9999) must
then stay within a bound set by that distance, computed in the test (_bar, _spread_ok).
The exact-order tests carry north_star's bar: bit-identical logits.
"""
import numpy as np
import pytest

import k2t
import oracle as O
from helpers import synthetic_kv
from model_oracle import Matrix, OracleModel

pytestmark = pytest.mark.gpu

SEED = 20261201  # bench.py's seed
THREADS = 16  # host threads for the oracle's integer-exact GEMVs (row ranges, split-independent)


def _t(a):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def _close(a, b, cos_min=0.9999):
    cos = float(np.dot(a, b) / (np.linalg.norm(a) * np.linalg.norm(b)))
    rel = float(np.abs(a - b).max() / np.abs(b).max())
    return rel <= 2e-2 and cos > cos_min, (rel, cos)


def _oracle_mats(host):
    return [Matrix(h.fmt, h.rows, h.cols, h.pair, h.tail, hp=h.hp, cb=h.cb, sgc=h.sgc) for h in host]


def _oracle_layers(cfg, conv):
    ones = np.ones(cfg["hidden"], np.float32)
    return [{"qkv": conv[4 * i], "o": conv[4 * i + 1], "gu": conv[4 * i + 2], "down": conv[4 * i + 3],
             "in_norm": ones, "post_norm": ones, "bias": None} for i in range(cfg["n_layers"])], ones


# ----------------------------------------------------------------------------- config 4
def _config4_acts(rng, cols, ntok):
    """~N(0, 1) with 0.1% outlier channels x30, int8 per token (the oracle's populate)."""
    qs, ss, ms = [], [], []
    for _ in range(ntok):
        x = rng.standard_normal(cols).astype(np.float32)
        x[rng.choice(cols, max(1, cols // 1000), replace=False)] *= 30.0
        q, s, m = O.populate_fwht(x)
        qs.append(q)
        ss.append(s)
        ms.append(m)
    return np.stack(qs), np.stack(ss), np.stack(ms)


@pytest.mark.parametrize("fmt", ["nf4", "nf3", "b6"])
@pytest.mark.parametrize("rows,cols", [(14336, 4096), (4096, 14336)])
def test_config4_gemv_full_shape(gpu_ctx, fmt, rows, cols):
    import torch
    print(f"config 4 {fmt} {rows}x{cols}", flush=True)
    W = k2t.synth_normal(SEED + rows * 3 + cols, rows * cols, 0.02).reshape(rows, cols)
    if fmt == "b6":
        pair, tail = k2t.compile_bipolar(W, 6)
        m = gpu_ctx.upload_nibble4(rows, cols, 2, pair, tail)

        def ref(q, s, sm, dots=False):
            return O.nibble4_gemv(pair, tail, rows, cols, 2, q, s, sm, want_dots=dots)
    else:
        bits = 3 if fmt == "nf3" else 4
        cb, _, pair, tail = k2t.compile_nf4(W, 2, bits=bits)
        m = gpu_ctx.upload_nf(rows, cols, bits, 2, cb, pair, tail)

        def ref(q, s, sm, dots=False):
            return O.nf_gemv(pair, tail, rows, cols, bits, 2, cb, q, s, want_dots=dots)
    del W
    rng = np.random.default_rng(SEED + cols)
    xq, xs, xsum = _config4_acts(rng, cols, 4)
    # batch 1: integer dots over the whole matrix, then the exact epilogue
    r1, dots = ref(xq[0], xs[0], xsum[0], dots=True)
    d = torch.zeros((rows, cols // 64), dtype=torch.int32, device="cuda")
    gpu_ctx.gemv_chunk_dots(m, _t(xq[0]), _t(xsum[0]), d)
    assert np.array_equal(d.cpu().numpy(), dots), "integer chunk dots differ"
    out = torch.full((4, rows), float("nan"), dtype=torch.float32, device="cuda")
    gpu_ctx.set_exact(True)
    try:
        gpu_ctx.gemv(m, _t(xq[:1]), _t(xs[:1]), _t(xsum[:1]), out, ntok=1, out_stride=rows)
        gpu_ctx.sync()
        assert np.array_equal(out[0].cpu().numpy().view(np.uint32), r1.view(np.uint32)), "batch-1 output"
        # batch 4: one weight pass for four tokens, each token bit-identical to its own GEMV
        out.fill_(float("nan"))
        gpu_ctx.gemv(m, _t(xq), _t(xs), _t(xsum), out, ntok=4, out_stride=rows)
        gpu_ctx.sync()
    finally:
        gpu_ctx.set_exact(False)
    got = out.cpu().numpy()
    for t in range(4):
        rt = r1 if t == 0 else ref(xq[t], xs[t], xsum[t])
        assert np.array_equal(got[t].view(np.uint32), rt.view(np.uint32)), f"batch-4 token {t}"
    # default fast epilogue on the tile: within 1e-5 * (1 + |y|)
    gpu_ctx.gemv(m, _t(xq), _t(xs), _t(xsum), out, ntok=4, out_stride=rows)
    gpu_ctx.sync()
    assert np.all(np.abs(out[0].cpu().numpy() - r1) <= 1e-5 * (1 + np.abs(r1)))
    m.close()


# ----------------------------------------------------------------------------- configs 3 and 2
def _cos_rel(a, b):
    return 1.0 - float(np.dot(a, b) / (np.linalg.norm(a) * np.linalg.norm(b))), \
        float(np.abs(a - b).max() / np.abs(b).max())


def _spread_ok(gpu, ora, ora_neon, what):
    """Full-depth bar: the GPU may differ from the oracle (x86 sum order) by at most 4x
    the distance between the reference's own two builds on the same inputs (x86 vs aarch64
    sum-of-squares order, real_llm.rs:903-962), plus 1e-4 of cosine; max |diff| at most
    2x theirs + 2%.  On random-init models an int8 code that flips in one layer is
    carried by every later layer, so this distance grows with depth (about 1e-3 of cosine
    at 24-30 layers)."""
    dg, rg = _cos_rel(gpu, ora)
    dr, rr = _cos_rel(ora_neon, ora)
    print(f"  {what}: gpu 1-cos {dg:.2e} rel {rg:.4f} | reference orders 1-cos {dr:.2e} rel {rr:.4f}", flush=True)
    return dg <= 4 * dr + 1e-4 and rg <= 2 * rr + 2e-2, (dg, rg, dr, rr)


def _oracles(cfg, host, max_seq, threads):
    conv = _oracle_mats(host)
    layers, ones = _oracle_layers(cfg, conv)
    return [OracleModel(dict(cfg, max_seq=max_seq), layers, conv[-1], ones, parity_threads=threads, rms_order=o)
            for o in ("x86", "neon")]


# Fast-mode bar at two layers: cosine > 0.9995 and max |diff| <= 2% of max |logit|, with
# no fallback.  The fast path sums squares, softmax terms and V rows in tree order and uses
# the device expf, so an int8 code can move by one against the x86 order; the exact-order
# mode (test_config3/2_exact_order below) is the check at north_star's 1e-4, bit for bit.
FAST_COS_2L = 0.9995


def _bar(gpu, ora, ora_neon, what, n_layers):
    """Two layers: the fixed fast-mode bar (FAST_COS_2L), no fallback.  Full depth: the
    fixed bar, or failing that the bar relative to the reference's own two builds
    (_spread_ok), since one-code flips compound over 24-30 layers."""
    if n_layers <= 2:
        return _close(gpu, ora, FAST_COS_2L)
    ok, info = _close(gpu, ora)
    return (True, info) if ok else _spread_ok(gpu, ora, ora_neon, what)


@pytest.mark.parametrize("n_layers", [2, 24])
def test_config3_1_7b_persistent_matches_oracle(gpu_ctx, n_layers):
    """The 1.7B nf4g128 shape (d 2048, 32 heads, ffn 8192, vocab 49152) on the default
    persistent kernel: its phase task layout over every CU, the 49152-row head and the
    cross-workgroup greedy pick.  A 12-token prefill in 4-token weight passes, 3 decode
    steps, then 12 device-side greedy steps in one generate() call, at 2 layers and at the
    full 24 (the bench model, same seeds).  Logits meet _bar; greedy tokens equal the
    oracle's argmax wherever its top-2 margin exceeds twice the largest GPU-oracle logit
    difference seen (a closer call is within rounding of a tie)."""
    print(f"config 3: 1.7B nf4g128 persistent decode vs oracle, {n_layers} layers", flush=True)
    cfg = dict(k2t.SMOLLM2_1_7B, n_layers=n_layers)
    model, mats, host = k2t.build_random_model(gpu_ctx, cfg, max_seq=64, fmt="nf4", seed=7, max_batch=16,
                                               keep_host=True)
    assert model.persistent_active(), "the 1.7B model should run the persistent kernel"
    ref, ref2 = _oracles(cfg, host, 64, THREADS)
    toks = np.random.default_rng(SEED).integers(0, cfg["vocab"], 13).astype(np.int32)
    pre = model.prefill(toks[:12], want_logits=True)  # 4-token weight passes

    def step(t, want=True):
        return ref.forward_token(t, want), ref2.forward_token(t, want)

    for t in toks[:11]:
        step(int(t), False)
    b, c = step(int(toks[11]))
    ok, info = _bar(pre, b, c, "prefill", n_layers)
    assert ok, f"prefill logits {info}"
    md = float(np.abs(pre - b).max())  # largest |GPU - oracle| logit difference seen
    tok = int(toks[12])
    checked = 0
    for i in range(3):
        assert model.persistent_active()
        a = model.decode(tok)
        b, c = step(tok)
        ok, info = _bar(a, b, c, f"decode {i}", n_layers)
        assert ok, f"decode step {i}: {info}"
        md = max(md, float(np.abs(a - b).max()))
        top2 = np.sort(b)[-2:]
        if top2[1] - top2[0] > 2 * md:
            assert int(np.argmax(a)) == int(np.argmax(b)), f"greedy token differs at step {i}"
            checked += 1
        tok = int(np.argmax(a))
    # the persistent kernel's own cross-workgroup greedy pick, several steps in one call:
    # each device pick against the argmax of the oracle's logits for the same input token
    # (twelve device steps: at 24 layers the fast path's largest logit difference, about
    # 0.16-0.17, leaves most steps' top-2 margins of this random model too close to call)
    got = list(model.generate(tok, 12))
    for g in got:
        b, _ = step(tok)
        top2 = np.sort(b)[-2:]
        if top2[1] - top2[0] > 2 * md:
            assert g == int(np.argmax(b)), f"device greedy token {g} vs oracle {int(np.argmax(b))}"
            checked += 1
        tok = g
    print(f"  greedy tokens checked: {checked} of 15 (margin > {2 * md:.4f})", flush=True)
    assert checked >= 3
    model.close()
    for m in mats:
        m.close()


@pytest.mark.parametrize("n_layers", [2, 30])
def test_config2_135m_p55454_ctx512_matches_oracle(gpu_ctx, n_layers):
    """135M p55454 at context 512 on both decode paths: the per-operation graph (mode 0)
    and the mixed-plane persistent kernel (mode 2).  Positions 0-447 hold the engine's
    seeded synthetic int8 K/V (replicated into the oracle's cache), positions 448-511 come
    from a batched 64-token prefill, then two decode steps attend 513-514 positions.  Two
    layers and all 30 (the bench model); logits meet _bar."""
    print(f"config 2: 135M p55454 ctx 512, per-op and persistent vs oracle, {n_layers} layers", flush=True)
    cfg = dict(k2t.SMOLLM2_135M, n_layers=n_layers)
    n_syn, n_pre = 448, 64
    models = []
    for mode in (0, 2):
        model, mats, host = k2t.build_random_model(gpu_ctx, cfg, max_seq=n_syn + n_pre + 8, fmt="n4", seed=7,
                                                   max_batch=64, keep_host=True)
        model.set_persistent(mode)
        assert model.persistent_active() == (mode == 2)
        models.append((model, mats))
    oras = _oracles(cfg, host, n_syn + n_pre + 8, 8)
    for r in oras:
        synthetic_kv(r, cfg["n_layers"], cfg["n_kv_heads"], cfg["head_dim"], n_syn, SEED)
    toks = np.random.default_rng(SEED + 1).integers(0, cfg["vocab"], n_pre + 2).astype(np.int32)
    for model, _ in models:
        model.kv_synthetic(n_syn, seed=SEED)
        model.prefill(toks[:n_pre], want_logits=False)
        assert model.position() == n_syn + n_pre
    for t in toks[:n_pre]:
        for r in oras:
            r.forward_token(int(t), want_logits=False)
    for i, t in enumerate(toks[n_pre:]):
        bs = [r.forward_token(int(t)) for r in oras]
        for mode, (model, _) in zip((0, 2), models):
            a = model.decode(int(t))
            ok, info = _bar(a, bs[0], bs[1], f"mode {mode} step {i}", n_layers)
            assert ok, f"mode {mode}, decode at context {n_syn + n_pre + i}: {info}"
    for model, mats in models:
        model.close()
        for m in mats:
            m.close()


# ----------------------------------------------------------------------------- exact order
def _same(a, b, what):
    a, b = np.asarray(a, np.float32), np.asarray(b, np.float32)
    ndiff = int(np.sum(a.view(np.uint32) != b.view(np.uint32)))
    rel = float(np.abs(a - b).max() / np.abs(b).max())
    print(f"  {what}: {ndiff} of {a.size} logits differ in any bit, max rel {rel:.2e}", flush=True)
    assert rel <= 1e-4, f"{what}: max rel {rel:.2e} above north_star's 1e-4"
    assert ndiff == 0, f"{what}: {ndiff} logits differ (max rel {rel:.2e})"


@pytest.mark.parametrize("n_layers", [2, 24])
def test_config3_exact_order(gpu_ctx, n_layers):
    """The 1.7B nf4g128 bench model (same seeds) in exact-order mode against the x86
    oracle, on both decode paths: the persistent kernel's exact-order variant (its real
    task layout over every CU, one attention task per head) and the per-operation graph.
    A 12-token batched prefill and 3 decode steps, every logit bit-identical (so within
    north_star's 1e-4 relative), at 2 layers and at the full 24: no int8 code flips
    anywhere in the stack."""
    print(f"config 3: 1.7B nf4g128 exact order vs x86 oracle, {n_layers} layers", flush=True)
    cfg = dict(k2t.SMOLLM2_1_7B, n_layers=n_layers)
    runs = []
    for pk in (1, 0):
        model, mats, host = k2t.build_random_model(gpu_ctx, cfg, max_seq=64, fmt="nf4", seed=7, max_batch=16,
                                                   keep_host=True)
        model.set_exact(True)
        model.set_persistent(pk)
        assert model.persistent_active() == bool(pk)
        runs.append((("persistent" if pk else "per-op"), model, mats))
    ref = _oracles(cfg, host, 64, THREADS)[0]
    toks = np.random.default_rng(SEED).integers(0, cfg["vocab"], 15).astype(np.int32)
    pres = [model.prefill(toks[:12], want_logits=True) for _, model, _ in runs]
    for t in toks[:11]:
        ref.forward_token(int(t), want_logits=False)
    want = ref.forward_token(int(toks[11]))
    for (name, _, _), pre in zip(runs, pres):
        _same(pre, want, f"{name} prefill")
    for i, t in enumerate(toks[12:]):
        want = ref.forward_token(int(t))
        for name, model, _ in runs:
            _same(model.decode(int(t)), want, f"{name} decode {i}")
    for _, model, mats in runs:
        model.close()
        for m in mats:
            m.close()


def test_config3_prefill_256_matrix_cores(gpu_ctx):
    """The bench's 256-token prefill at the 1.7B nf4g128 shape (2 layers): qkv with the
    q / k / v epilogue (two 16-token blocks per wave), gate_up with the SwiGLU epilogue
    (64-token workgroups), o and down at one block per wave, attention on the matrix cores.
    The last token's logits meet the two-layer fast bar against the oracle, and with the
    tiles copied by the GEMVs (mode 2: the separate q / k / v post and SwiGLU kernels) the
    logits are the same bit for bit."""
    print("config 3: 1.7B nf4g128 256-token matrix-core prefill vs oracle, 2 layers", flush=True)
    cfg = dict(k2t.SMOLLM2_1_7B, n_layers=2)
    n = 256
    model, mats, host = k2t.build_random_model(gpu_ctx, cfg, max_seq=n + 8, fmt="nf4", seed=7, max_batch=n,
                                               keep_host=True)
    try:
        toks = np.random.default_rng(SEED).integers(0, cfg["vocab"], n).astype(np.int32)
        pre = {}
        for mode in (1, 2):
            gpu_ctx.set_mfma(mode)
            model.reset()
            pre[mode] = model.prefill(toks, want_logits=True)
        assert np.array_equal(pre[1].view(np.uint32), pre[2].view(np.uint32)), "mode 1 / mode 2"
        ref = _oracles(cfg, host, n + 8, THREADS)[0]
        for t in toks[:-1]:
            ref.forward_token(int(t), want_logits=False)
        b = ref.forward_token(int(toks[-1]))
        ok, info = _close(pre[1], b, FAST_COS_2L)
        assert ok, f"prefill logits {info}"
    finally:
        gpu_ctx.set_mfma(1)
        model.close()
        for m in mats:
            m.close()


@pytest.mark.parametrize("tier,n_layers", [("p55454", 2), ("p55454", 30), ("b6", 2)])
def test_config2_exact_order(gpu_ctx, tier, n_layers):
    """The 135M bench model at context 512 (synthetic K/V 448 + a 64-token batched
    prefill) in exact-order mode, on the persistent kernel's exact-order variant (the
    mixed-plane kernel for p55454, the two-hi-plane kernel for all-b6) and on the
    per-operation graph: two decode steps, every logit bit-identical to the x86 oracle's;
    p55454 at 2 layers and at the full 30, b6 at 2."""
    print(f"config 2: 135M {tier} ctx 512 exact order vs x86 oracle, {n_layers} layers", flush=True)
    cfg = dict(k2t.SMOLLM2_135M, n_layers=n_layers)
    planes = k2t.P55454 if tier == "p55454" else {k: 6 for k in k2t.P55454}
    n_syn, n_pre = 448, 64
    toks = np.random.default_rng(SEED + 1).integers(0, cfg["vocab"], n_pre + 2).astype(np.int32)
    runs = []
    for pk in (1, 0):
        model, mats, host = k2t.build_random_model(gpu_ctx, cfg, max_seq=n_syn + n_pre + 8, fmt="n4", seed=7,
                                                   planes=planes, max_batch=64, keep_host=True)
        model.set_exact(True)
        model.set_persistent(pk)
        model.kv_synthetic(n_syn, seed=SEED)
        model.prefill(toks[:n_pre], want_logits=False)
        assert model.persistent_active() == bool(pk)
        runs.append((("persistent" if pk else "per-op"), model, mats))
    ref = _oracles(cfg, host, n_syn + n_pre + 8, 8)[0]
    synthetic_kv(ref, cfg["n_layers"], cfg["n_kv_heads"], cfg["head_dim"], n_syn, SEED)
    for t in toks[:n_pre]:
        ref.forward_token(int(t), want_logits=False)
    for i, t in enumerate(toks[n_pre:]):
        want = ref.forward_token(int(t))
        for name, model, _ in runs:
            _same(model.decode(int(t)), want, f"{name} decode {i} at context {n_syn + n_pre + i}")
    for _, model, mats in runs:
        model.close()
        for m in mats:
            m.close()


# ----------------------------------------------------------------------------- config 5
QWEN3_30B_A3B = dict(hidden=2048, n_heads=32, n_kv_heads=4, head_dim=128, intermediate=768, vocab=151936,
                     rms_eps=1e-6, rope_theta=1000000.0)


@pytest.mark.parametrize("n_ctx", [1100, 6600])
def test_config5_moe_full_width_matches_oracle(gpu_ctx, n_ctx):
    """Qwen3-30B-A3B shape at full width, two layers, context 1100 and the bench's 6600
    (above 1024: the grouped-query attention kernel, 128-position spans of each KV head
    scoring its 8 q heads -- 9 and 52 spans -- merged in the same launch), NF4g128 attention with
    QK-norm and q_dim 4096 != hidden, 128 NF3 g128 experts top-8 softmax + renorm from a
    .k2tm bank, bf16 untied embedding, NF4g128 head over 151936 rows."""
    from k2tb_writer import write_k2tm
    print(f"config 5: 30B-A3B shape, 2 layers, ctx {n_ctx} vs oracle", flush=True)
    n_layers, E, top_k, dff, pool_n = 2, 128, 8, 768, 16
    cfg = dict(QWEN3_30B_A3B, n_layers=n_layers, max_seq=n_ctx + 8)
    d, nq, nkv, hd, V = cfg["hidden"], cfg["n_heads"], cfg["n_kv_heads"], cfg["head_dim"], cfg["vocab"]
    # 16 distinct compiled experts, each id e uses pool[(e * 7 + layer) % 16]
    pool = []
    for j in range(pool_n):
        Wgu = k2t.synth_normal(SEED + 5000 + 2 * j, 2 * dff * d, 0.02).reshape(2 * dff, d)
        Wdn = k2t.synth_normal(SEED + 5001 + 2 * j, d * dff, 0.02).reshape(d, dff)
        cg, _, pg, tg = k2t.compile_nf4(Wgu, 2, bits=3)
        cd, _, pd, td = k2t.compile_nf4(Wdn, 2, bits=3)
        pool.append((dict(pair=pg, tail=tg, cb=cg, bits=3, sgc=2, rows=2 * dff, cols=d),
                     dict(pair=pd, tail=td, cb=cd, bits=3, sgc=2, rows=d, cols=dff)))
    experts = [[pool[(e * 7 + li) % pool_n] for e in range(E)] for li in range(n_layers)]
    bank = k2t.ExpertBank.upload(gpu_ctx, write_k2tm(experts, d, dff, 3, 2))
    rng = np.random.default_rng(SEED + 5)
    gm = k2t.Model(gpu_ctx, cfg, max_batch=1)
    mats, layers = [], []

    def nf4(rows, cols, seed):
        W = k2t.synth_normal(seed, rows * cols, 0.02).reshape(rows, cols)
        cb, _, pair, tail = k2t.compile_nf4(W, 2)
        mats.append(gpu_ctx.upload_nf(rows, cols, 4, 2, cb, pair, tail))
        return mats[-1], Matrix("nf4", rows, cols, pair, tail, cb=cb, sgc=2)

    for li in range(n_layers):
        (q, qh), (o, oh) = nf4((nq + 2 * nkv) * hd, d, SEED + 100 * li + 1), nf4(d, nq * hd, SEED + 100 * li + 2)
        in_n, post_n = (1 + 0.1 * rng.standard_normal((2, d))).astype(np.float32)
        qn, kn = (1 + 0.1 * rng.standard_normal((2, hd))).astype(np.float32)
        router = k2t.synth_normal(SEED + 100 * li + 3, E * d, 0.05).reshape(E, d)
        gm.set_layer(li, q, o, None, None, in_n, post_n)
        gm.set_qk_norm(li, qn, kn)
        gm.set_moe(li, bank, li, router, top_k, True, k2t.MOE_SOFTMAX)
        layers.append({"qkv": qh, "o": oh, "in_norm": in_n, "post_norm": post_n, "q_norm": qn, "k_norm": kn,
                       "bias": None, "moe": dict(router_w=router, router_b=None, top_k=top_k, norm_topk_prob=True,
                                                 scoring=0, experts=experts[li])})
    head, hh = nf4(V, d, SEED + 99991)
    emb = (k2t.synth_normal(SEED + 99992, V * d, 0.02).view(np.uint32) >> 16).astype(np.uint16)
    gm.set_embedding(k2t.EMBED_BF16, emb)
    fn = (1 + 0.1 * rng.standard_normal(d)).astype(np.float32)
    gm.set_head(head, fn)
    emb2 = emb.reshape(V, d)

    def embed(tok):
        return (emb2[tok].astype(np.uint32) << 16).view(np.float32)

    toks = np.random.default_rng(SEED + 6).integers(0, V, 3)
    # fast path: at 1100 the fixed bar; at 6600 the attention output is an average over
    # 6600 random V rows, near zero, and the grouped-query kernel's span-order sums move
    # single int8 codes of it against the oracle's sequential order (the kernel itself
    # is within 1e-4 of the oracle at this shape: test_attn_decode_grouped_queries_*), so
    # cosine > 0.9998 there; the exact-order run below then carries the tight bar
    cos_min = 0.9999 if n_ctx <= 1100 else 0.9998
    for exact in (False, True):
        gm.set_exact(exact)
        ref = OracleModel(cfg, layers, hh, fn, embed=embed, parity_threads=THREADS)
        gm.kv_synthetic(n_ctx, seed=SEED)
        synthetic_kv(ref, n_layers, nkv, hd, n_ctx, SEED)
        for i, t in enumerate(toks):
            a, b = gm.decode(int(t)), ref.forward_token(int(t))
            if exact:
                # exact-order mode, the MoE feed-forward included (x86 router dot, expf_rn
                # softmax, in-order GEMV epilogues): every logit equals the oracle's
                rel = float(np.abs(a - b).max() / np.abs(b).max())
                print(f"  exact order at context {n_ctx + i}: rel {rel:.2e}", flush=True)
                assert np.array_equal(a.view(np.uint32), b.view(np.uint32)), \
                    f"exact order, context {n_ctx + i}: rel {rel:.2e}, {int((a != b).sum())} logits differ"
            else:
                ok, info = _close(a, b, cos_min)
                assert ok, f"decode at context {n_ctx + i}: {info}"
    gm.close()
    for m in mats:
        m.close()
    bank.close()
