"""End-to-end decode parity: the GPU engine (C ABI k2t_model_*) against the oracle's
restatement of the decode megakernel (oracle/model_oracle.py) on small random-init
models, plus engine invariants (prefill == token-by-token, graph == eager, greedy).

Bar: logits of every step with cosine > 0.9999 against the oracle and max |diff| <=
2e-2 * max|logit|.  (The reference compares two paths of one model at cosine > 0.99995
-- batched prefill vs token-by-token, real_llm.rs:10466-10473 -- on a trained-like
model; these random-init toy models with random norms are more sensitive to a single
int8 rounding flip.)  Integer GEMV and
attention dots are exact (test_gpu_gemv.py), but inv_rms (tree vs sequential sum), expf
and the attention accumulation order differ in the last ulp and can move an int8 code by
one; the reference itself has two such orders (NEON vs portable, real_llm.rs:903-962).
"""
import numpy as np
import pytest

from helpers import synthetic_kv
from model_oracle import OracleModel, random_model

pytestmark = pytest.mark.gpu

TINY = dict(n_layers=2, hidden=256, n_heads=4, n_kv_heads=2, head_dim=64, intermediate=512, vocab=520,
            max_seq=40, rms_eps=1e-5, rope_theta=10000.0)
TINY128 = dict(n_layers=2, hidden=256, n_heads=2, n_kv_heads=1, head_dim=128, intermediate=384, vocab=300,
               max_seq=300, rms_eps=1e-5, rope_theta=100000.0)
P55454 = {"qkv": 5, "o": 5, "gu": 4, "down": 5, "head": 4}


def _upload(ctx, m):
    if m.fmt == "n4":
        return ctx.upload_nibble4(m.rows, m.cols, m.hp, m.pair, m.tail)
    return ctx.upload_nf(m.rows, m.cols, 4, m.sgc, m.cb, m.pair, m.tail)


def _gpu_model(ctx, cfg, layers, head, final_norm, max_batch=8):
    import k2t
    gm = k2t.Model(ctx, cfg, max_batch=max_batch)
    mats = []
    for i, L in enumerate(layers):
        q, o, gu, dn = (_upload(ctx, L[k]) for k in ("qkv", "o", "gu", "down"))
        mats += [q, o, gu, dn]
        gm.set_layer(i, q, o, gu, dn, L["in_norm"], L["post_norm"], L.get("bias"))
    hm = _upload(ctx, head)
    gm.set_head(hm, final_norm)
    return gm, mats + [hm]


def _close(a, b, cos_min=0.99995):
    cos = float(np.dot(a, b) / (np.linalg.norm(a) * np.linalg.norm(b)))
    rel = float(np.abs(a - b).max() / np.abs(b).max())
    return rel <= 2e-2 and cos > cos_min, (rel, cos)


@pytest.mark.parametrize("exact", [True, False])
@pytest.mark.parametrize("name,cfg,fmt,planes", [("nf4_hd64", TINY, "nf4", None),
                                                ("p55454_hd64", TINY, "n4", P55454),
                                                ("b6_hd128", TINY128, "n4", {k: 6 for k in P55454})])
def test_decode_matches_oracle(gpu_ctx, name, cfg, fmt, planes, exact):
    layers, head, fn = random_model(cfg, seed=len(name), fmt=fmt, planes=planes)
    ref = OracleModel(cfg, layers, head, fn)
    gm, _ = _gpu_model(gpu_ctx, cfg, layers, head, fn)
    gm.set_exact(exact)  # exact-order steps (bit-identical: test_gpu_exact.py), or the fast path
    # both modes run the persistent single-launch decode kernel: NF4; 4 or 5 bit planes
    # (p55454 mixes b5 and b4: the 256-thread variant that reads each matrix's plane
    # count); b6 (the 256-thread two-hi-plane variant)
    gm.set_persistent(2)
    assert gm.persistent_active()
    rng = np.random.default_rng(9)
    toks = rng.integers(0, cfg["vocab"], 8)
    for i, t in enumerate(toks):
        a = gm.decode(int(t))
        b = ref.forward_token(int(t))
        ok, info = _close(a, b, 0.9999)
        assert ok, f"{name} step {i}: max rel diff, cos = {info}"
    assert gm.position() == len(toks)


def test_long_context_splits(gpu_ctx):
    """hd 128 with > 256 positions: the attention is split over KV ranges and merged."""
    cfg = dict(TINY128, n_layers=1)
    layers, head, fn = random_model(cfg, seed=3, fmt="nf4")
    ref = OracleModel(cfg, layers, head, fn)
    gm, _ = _gpu_model(gpu_ctx, cfg, layers, head, fn, max_batch=64)
    rng = np.random.default_rng(4)
    toks = rng.integers(0, cfg["vocab"], 270)
    gm.prefill(toks[:-1], want_logits=False)
    for t in toks[:-1]:
        ref.forward_token(int(t))
    a = gm.decode(int(toks[-1]))
    b = ref.forward_token(int(toks[-1]))
    ok, info = _close(a, b)
    assert ok, info


@pytest.mark.parametrize("hd", [64, 128])
def test_gqa_long_context_xcd_order(gpu_ctx, hd):
    """GQA (8 q heads over 2 KV heads) with max_seq 2048: the cache is sized for the span
    path.  The batched prefill runs the per-head 256-position span kernels in their
    XCD-grouped order (the q heads of one KV head on one XCD) and the span merge; each
    decode step runs the grouped-query kernel (one workgroup per KV head and 128-position
    span scoring all 4 q heads of the group, merge workgroups in the same launch), at
    hd 64 and 128.  Decode logits vs the oracle."""
    print(f"gqa long context hd={hd}", flush=True)
    cfg = dict(n_layers=1, hidden=8 * hd, n_heads=8, n_kv_heads=2, head_dim=hd, intermediate=256, vocab=200,
               max_seq=2048, rms_eps=1e-5, rope_theta=10000.0)
    layers, head, fn = random_model(cfg, seed=11, fmt="nf4")
    ref = OracleModel(cfg, layers, head, fn)
    gm, _ = _gpu_model(gpu_ctx, cfg, layers, head, fn, max_batch=64)
    rng = np.random.default_rng(12)
    toks = rng.integers(0, cfg["vocab"], 300)
    gm.prefill(toks[:-2], want_logits=False)
    for t in toks[:-2]:
        ref.forward_token(int(t))
    for t in toks[-2:]:
        a, b = gm.decode(int(t)), ref.forward_token(int(t))
        ok, info = _close(a, b)
        assert ok, info


@pytest.mark.parametrize("hd", [64, 128])
def test_gqa_attention_past_64_spans(gpu_ctx, hd):
    """The grouped-query kernel's merge polls four spans per thread together (64 spans of
    128 positions); a context of 8400 positions has 66 spans, so the threads of the first
    two span subsets also take the one-span-at-a-time path.  K/V filled with the engine's
    seeded synthetic codes (the oracle gets the same), then decode steps vs the oracle."""
    print(f"gqa attention past 64 spans hd={hd}", flush=True)
    n_ctx = 8400
    cfg = dict(n_layers=1, hidden=8 * hd, n_heads=8, n_kv_heads=2, head_dim=hd, intermediate=256, vocab=200,
               max_seq=n_ctx + 8, rms_eps=1e-5, rope_theta=10000.0)
    layers, head, fn = random_model(cfg, seed=21, fmt="nf4")
    ref = OracleModel(cfg, layers, head, fn)
    gm, _ = _gpu_model(gpu_ctx, cfg, layers, head, fn)
    gm.kv_synthetic(n_ctx, seed=5)
    synthetic_kv(ref, 1, 2, hd, n_ctx, 5)
    for t in np.random.default_rng(22).integers(0, cfg["vocab"], 3):
        a, b = gm.decode(int(t)), ref.forward_token(int(t))
        ok, info = _close(a, b)
        assert ok, info



@pytest.mark.parametrize("hd,n_tok", [(64, 560), (128, 48)])
def test_sliding_window_ring_matches_oracle(gpu_ctx, hd, n_tok):
    """Sliding window 16 with 4 sinks (set_kv_sliding_window): attention over the sinks
    and the last 12 positions, K/V in a 524-slot ring; 560 tokens wrap the ring (hd 64),
    48 exercise the per-64-block window scores (hd 128).  Prefill and decode vs the oracle."""
    print(f"sliding window hd={hd} tokens={n_tok}", flush=True)
    cfg = dict(n_layers=1, hidden=2 * hd, n_heads=2, n_kv_heads=1, head_dim=hd, intermediate=128, vocab=160,
               max_seq=700, rms_eps=1e-5, rope_theta=10000.0)
    layers, head, fn = random_model(cfg, seed=21, fmt="nf4")
    ref = OracleModel(cfg, layers, head, fn, window=16, sinks=4)
    gm, _ = _gpu_model(gpu_ctx, cfg, layers, head, fn, max_batch=32)
    gm.set_kv_window(16, 4)
    assert gm.kv_window() == (16, 4) and not gm.persistent_active()
    toks = np.random.default_rng(22).integers(0, cfg["vocab"], n_tok)
    gm.prefill(toks[:-3], want_logits=False)
    for t in toks[:-3]:
        ref.forward_token(int(t))
    for t in toks[-3:]:
        a, b = gm.decode(int(t)), ref.forward_token(int(t))
        ok, info = _close(a, b)
        assert ok, info
    gm.set_kv_window(0, 0)
    assert gm.kv_window() == (0, 0) and gm.position() == 0


@pytest.mark.parametrize("n_tok", [300, 530])
def test_persistent_mixed_long_context_matches_oracle(gpu_ctx, n_tok):
    """p55454 on the 256-thread persistent kernel (mode 2) past 256 positions: each thread
    scores several positions, and the V slices beyond the first 128 positions (8 per
    position subset, prefetched) take the batched V path, one and several batches.
    Prefill (per-operation path), then decode steps on the persistent kernel vs the oracle."""
    print(f"persistent mixed long context tokens={n_tok}", flush=True)
    cfg = dict(TINY, max_seq=n_tok + 8)
    layers, head, fn = random_model(cfg, seed=31, fmt="n4", planes=P55454)
    ref = OracleModel(cfg, layers, head, fn)
    gm, _ = _gpu_model(gpu_ctx, cfg, layers, head, fn, max_batch=64)
    gm.set_persistent(2)
    assert gm.persistent_active()
    toks = np.random.default_rng(32).integers(0, cfg["vocab"], n_tok)
    gm.prefill(toks[:-3], want_logits=False)
    for t in toks[:-3]:
        ref.forward_token(int(t))
    for t in toks[-3:]:
        a, b = gm.decode(int(t)), ref.forward_token(int(t))
        ok, info = _close(a, b, 0.9999)
        assert ok, info


def test_prefill_equals_token_by_token_and_graph_equals_eager(gpu_ctx):
    """Batched prefill and token-by-token decode on the one-kernel-per-operation path run
    the same arithmetic (bit-exact); the persistent kernel sums attention and GEMV
    partials in its own fixed order (close, and graph replay == eager bit-exact)."""
    layers, head, fn = random_model(TINY, seed=5, fmt="nf4")
    gm, _ = _gpu_model(gpu_ctx, TINY, layers, head, fn, max_batch=4)
    toks = np.arange(11) * 37 % TINY["vocab"]
    pre = gm.prefill(toks)  # 3 batches of <= 4 tokens (4-token GEMV tiles)
    gm.set_persistent(False)
    gm.reset()
    gm.set_graph(False)
    for t in toks:
        eager = gm.decode(int(t))
    gm.reset()
    gm.set_graph(True)
    for t in toks:
        graph = gm.decode(int(t))
    assert np.array_equal(pre.view(np.uint32), eager.view(np.uint32))
    assert np.array_equal(graph.view(np.uint32), eager.view(np.uint32))
    gm.set_persistent(True)
    assert gm.persistent_active()
    gm.reset()
    gm.set_graph(False)
    for t in toks:
        pk_eager = gm.decode(int(t))
    gm.reset()
    gm.set_graph(True)
    for t in toks:
        pk_graph = gm.decode(int(t))
    assert np.array_equal(pk_graph.view(np.uint32), pk_eager.view(np.uint32))
    ok, info = _close(pk_eager, eager, 0.99999)
    assert ok, info


def test_persistent_decode_long_run_matches_per_op(gpu_ctx):
    """40 decode steps of a 3-layer b4 GQA model (hd 64) on the persistent kernel track the
    per-operation path step by step (same quantized inputs, different summation order)."""
    cfg = dict(TINY, n_layers=3, max_seq=48)
    layers, head, fn = random_model(cfg, seed=11, fmt="n4", planes={k: 4 for k in P55454})
    a, _ = _gpu_model(gpu_ctx, cfg, layers, head, fn)
    b, _ = _gpu_model(gpu_ctx, cfg, layers, head, fn)
    a.set_persistent(True)
    b.set_persistent(False)
    assert a.persistent_active() and not b.persistent_active()
    rng = np.random.default_rng(12)
    for i, t in enumerate(rng.integers(0, cfg["vocab"], 40)):
        x, y = a.decode(int(t)), b.decode(int(t))
        ok, info = _close(x, y, 0.9999)
        assert ok, (i, info)


def test_persistent_hands_over_to_per_op_past_1024(gpu_ctx):
    """Decode steps attending more than 1024 positions run the per-operation path even with
    the persistent kernel enabled (the captured graph is replaced when the context crosses
    1024); logits track a model on the per-operation path across the switch."""
    print("persistent -> per-op handover at 1024", flush=True)
    cfg = dict(TINY, max_seq=1040)
    layers, head, fn = random_model(cfg, seed=41, fmt="nf4")
    a, _ = _gpu_model(gpu_ctx, cfg, layers, head, fn, max_batch=64)
    b, _ = _gpu_model(gpu_ctx, cfg, layers, head, fn, max_batch=64)
    a.set_persistent(True)
    b.set_persistent(False)
    toks = np.random.default_rng(42).integers(0, cfg["vocab"], 1030)
    a.prefill(toks[:1020], want_logits=False)
    b.prefill(toks[:1020], want_logits=False)
    for i, t in enumerate(toks[1020:1028]):
        assert a.persistent_active() == (1020 + i + 1 <= 1024)
        x, y = a.decode(int(t)), b.decode(int(t))
        ok, info = _close(x, y, 0.9999)
        assert ok, (1020 + i, info)
    a.generate(int(toks[-1]), 2)
    assert a.position() == 1030
    a.reset()
    assert a.persistent_active()
    a.decode(int(toks[0]))  # back on the persistent kernel (the graph is captured again)
    assert a.position() == 1


@pytest.mark.parametrize("persistent", [False, True])
def test_greedy_generate_matches_oracle_argmax(gpu_ctx, persistent):
    layers, head, fn = random_model(TINY, seed=6, fmt="nf4")
    ref = OracleModel(TINY, layers, head, fn)
    gm, _ = _gpu_model(gpu_ctx, TINY, layers, head, fn)
    gm.set_persistent(persistent)
    out = gm.generate(17, 6)
    tok, seq = 17, []
    for _ in range(6):
        logits = ref.forward_token(tok)
        tok = int(np.argmax(logits))
        seq.append(tok)
    assert list(out) == seq


def test_model_argument_errors(gpu_ctx):
    import k2t
    with pytest.raises(k2t.K2TError):
        k2t.Model(gpu_ctx, dict(TINY, head_dim=96, hidden=384))
    gm = k2t.Model(gpu_ctx, TINY)
    with pytest.raises(k2t.K2TError):
        gm.decode(1)  # layers not set


def test_generate_hands_over_inside_one_call(gpu_ctx):
    """One generate() call that starts at position 1018 and runs 12 greedy steps crosses
    1024 attended positions inside its loop: the persistent kernel's graph is swapped for
    the per-operation one between two enqueued steps, and the next input token passes
    from the persistent kernel's own greedy pick to argmax_kernel.  The tokens equal those
    of the same model run on the per-operation path throughout."""
    print("generate across the 1024-position handover", flush=True)
    cfg = dict(TINY, max_seq=1040)
    layers, head, fn = random_model(cfg, seed=43, fmt="nf4")
    a, _ = _gpu_model(gpu_ctx, cfg, layers, head, fn, max_batch=64)
    b, _ = _gpu_model(gpu_ctx, cfg, layers, head, fn, max_batch=64)
    a.set_persistent(True)
    b.set_persistent(False)
    toks = np.random.default_rng(44).integers(0, cfg["vocab"], 1019)
    a.prefill(toks[:1018], want_logits=False)
    b.prefill(toks[:1018], want_logits=False)
    assert a.persistent_active()
    ga = list(a.generate(int(toks[1018]), 12))
    gb = list(b.generate(int(toks[1018]), 12))
    assert a.position() == b.position() == 1030
    assert not a.persistent_active()
    assert ga == gb, (ga, gb)


def test_persistent_kernel_with_large_max_seq(gpu_ctx):
    """The persistent kernel's LDS score buffer covers at most 1024 positions, so a model
    created with a long max_seq still runs it at short contexts (and matches the oracle)."""
    cfg = dict(TINY, max_seq=32768)
    layers, head, fn = random_model(cfg, seed=45, fmt="nf4")
    ref = OracleModel(cfg, layers, head, fn)
    gm, _ = _gpu_model(gpu_ctx, cfg, layers, head, fn)
    gm.set_persistent(True)
    assert gm.persistent_active()
    for t in (7, 123, 400):
        ok, info = _close(gm.decode(t), ref.forward_token(t), 0.9999)
        assert ok, info
