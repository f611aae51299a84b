"""Models loaded from .k2tb files (k2t_model_load_k2tb: load_bipolar + repack_sdot,
real_llm.rs:3902-4190, 3657-3702) decode like the same weights set up matrix by
matrix, and like the oracle; untied f32 / bf16 / NF4 embeddings (embed_token_into,
real_llm.rs:8063-8097) on the per-operation and the persistent decode paths.

Bar: the loaded model's logits equal the directly built model's bit for bit (same
bytes, same kernels); against the oracle the end-to-end bar of test_gpu_model.py
(cosine > 0.9999, max |diff| <= 2% of max |logit|).
"""
import numpy as np
import pytest

import k2t
import oracle as O
from k2tb_writer import bipolar_source, nf_source, write_k2tb
from model_oracle import Matrix, OracleModel

pytestmark = pytest.mark.gpu

CFG = dict(n_layers=2, hidden=256, n_heads=4, n_kv_heads=2, head_dim=64, intermediate=512, vocab=520,
           max_seq=24, rms_eps=1e-5, rope_theta=10000.0)


def _oracle_matrix(src, gu=False):
    """The repacked (GEMV-layout) form of a stored source matrix, built by the oracle."""
    r, c = src["rows"], src["cols"]
    if src["kind"] == "bipolar":
        pair, tail = O.nibble4_repack(src["inter"], src["scales"], r, c, src["planes"], gu)
        return Matrix("n4", r, c, pair, tail, hp=src["planes"] - 4)
    pair, tail = src["pair"], src["tail"]
    if gu:
        pairs = (r + 31) // 32
        blk = 2 * (pair.size // pairs)
        nci = r // 128
        b = pair.reshape(2 * nci, blk)
        pair = np.concatenate([b[i // 2 + (nci if i % 2 else 0)] for i in range(2 * nci)])
    return Matrix("nf4", r, c, pair, tail, cb=src["cb"], sgc=src["sgc"])


def _sources(seed, fmt, planes=None):
    rng = np.random.default_rng(seed)
    c = CFG
    d, nq, nkv, hd, inter, V = c["hidden"], c["n_heads"], c["n_kv_heads"], c["head_dim"], c["intermediate"], c["vocab"]
    planes = planes or {"qkv": 5, "o": 5, "gu": 4, "down": 5, "head": 4}

    def q(r, cc, name):
        W = (rng.standard_normal((r, cc)) * 0.02).astype(np.float32)
        return bipolar_source(W, planes[name]) if fmt == "n4" else nf_source(W, 4, 2)

    layers = []
    for _ in range(c["n_layers"]):
        layers.append({"qkv": q((nq + 2 * nkv) * hd, d, "qkv"), "o": q(d, nq * hd, "o"),
                       "gu": q(2 * inter, d, "gu"), "down": q(d, inter, "down"),
                       "in_norm": (1 + 0.1 * rng.standard_normal(d)).astype(np.float32),
                       "post_norm": (1 + 0.1 * rng.standard_normal(d)).astype(np.float32)})
    head = q(V, d, "head")
    fn = (1 + 0.1 * rng.standard_normal(d)).astype(np.float32)
    return rng, layers, head, fn


def _direct(ctx, layers, head, fn):
    gm = k2t.Model(ctx, CFG, max_batch=4)
    mats = []

    def up(m):
        if m.fmt == "n4":
            return ctx.upload_nibble4(m.rows, m.cols, m.hp, m.pair, m.tail)
        return ctx.upload_nf(m.rows, m.cols, 4, m.sgc, m.cb, m.pair, m.tail)

    for i, L in enumerate(layers):
        q, o, gu, dn = (up(L[k]) for k in ("qkv", "o", "gu", "down"))
        mats += [q, o, gu, dn]
        gm.set_layer(i, q, o, gu, dn, L["in_norm"], L["post_norm"])
    hm = up(head)
    gm.set_head(hm, fn)
    return gm, mats + [hm]


def _olayers(layers):
    return [{"qkv": _oracle_matrix(L["qkv"]), "o": _oracle_matrix(L["o"]), "gu": _oracle_matrix(L["gu"], True),
             "down": _oracle_matrix(L["down"]), "in_norm": L["in_norm"], "post_norm": L["post_norm"],
             "bias": None} for L in layers]


def _cos_ok(a, b):
    cos = float(np.dot(a, b) / (np.linalg.norm(a) * np.linalg.norm(b)))
    rel = float(np.abs(a - b).max() / np.abs(b).max())
    return cos > 0.9999 and rel <= 2e-2, (cos, rel)


@pytest.mark.parametrize("fmt,version", [("n4", 2), ("n4", 1), ("nf4", 3)])
def test_loaded_model_equals_direct_and_oracle(gpu_ctx, tmp_path, fmt, version):
    print(f"k2tb load: fmt {fmt} v{version}", flush=True)
    # K2TBIPOLAR1 holds one plane count for every matrix
    planes = {k: 4 for k in ("qkv", "o", "gu", "down", "head")} if version == 1 else None
    rng, layers, head, fn = _sources(5 + version, fmt, planes)
    path = tmp_path / "m.k2tb"
    write_k2tb(path, version, layers, fn, head)
    ol, oh = _olayers(layers), _oracle_matrix(head)
    ref = OracleModel(CFG, ol, oh, fn)
    direct, mats = _direct(gpu_ctx, ol, oh, fn)
    loaded = k2t.Model.load_k2tb(gpu_ctx, CFG, path, max_batch=4)
    assert loaded.persistent_active() == direct.persistent_active()
    toks = np.random.default_rng(3).integers(0, CFG["vocab"], 6)
    for i, t in enumerate(toks):
        a, b, r = loaded.decode(int(t)), direct.decode(int(t)), ref.forward_token(int(t))
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32)), f"step {i}: loaded != direct"
        ok, info = _cos_ok(a, r)
        assert ok, f"step {i}: vs oracle {info}"
    loaded.close()
    direct.close()
    for m in mats:
        m.close()


@pytest.mark.parametrize("kind", ["f32", "bf16", "nf4"])
@pytest.mark.parametrize("persistent", [False, True])
def test_untied_embeddings(gpu_ctx, tmp_path, kind, persistent):
    print(f"k2tb untied embedding: {kind} persistent={persistent}", flush=True)
    rng, layers, head, fn = _sources(21, "nf4")
    V, d = CFG["vocab"], CFG["hidden"]
    kw = {}
    if kind == "f32":
        rows = (rng.standard_normal((V, d)) * 0.5).astype(np.float32)
        kw["embed_f32"] = rows.ravel()
        emb = lambda t: rows[t]  # noqa: E731
    elif kind == "bf16":
        rows = ((rng.standard_normal((V, d)) * 0.5).astype(np.float32).view(np.uint32) >> 16).astype(np.uint16)
        kw["embed_bf16"] = rows.ravel()
        emb = lambda t: (rows[t].astype(np.uint32) << 16).view(np.float32)  # noqa: E731
    else:
        src = nf_source((rng.standard_normal((V, d)) * 0.02).astype(np.float32), 4, 2)
        kw["embed_nf4"] = src
        em = _oracle_matrix(src)
        emb = lambda t: O.ifwht64(em.row_rotated(t))  # noqa: E731
    path = tmp_path / "untied.k2tb"
    write_k2tb(path, 4, layers, fn, head, **kw)
    ref = OracleModel(CFG, _olayers(layers), _oracle_matrix(head), fn, embed=emb)
    gm = k2t.Model.load_k2tb(gpu_ctx, CFG, path, max_batch=4)
    gm.set_persistent(persistent)
    assert gm.persistent_active() == persistent
    for i, t in enumerate(np.random.default_rng(4).integers(0, V, 5)):
        a, r = gm.decode(int(t)), ref.forward_token(int(t))
        ok, info = _cos_ok(a, r)
        assert ok, f"{kind} step {i}: {info}"
    # a prompt through the batched path uses the same embedding rows
    gm.reset()
    ref2 = OracleModel(CFG, _olayers(layers), _oracle_matrix(head), fn, embed=emb)
    toks = [7, 300, 12]
    a = gm.prefill(np.array(toks, np.int32))
    for t in toks:
        r = ref2.forward_token(t)
    ok, info = _cos_ok(a, r)
    assert ok, f"{kind} prefill: {info}"
    gm.close()


def test_load_errors(gpu_ctx, tmp_path):
    rng, layers, head, fn = _sources(30, "nf4")
    path = tmp_path / "m.k2tb"
    write_k2tb(path, 3, layers, fn, head)
    with pytest.raises(k2t.K2TError) as ei:
        k2t.Model.load_k2tb(gpu_ctx, dict(CFG, n_layers=3), path)
    assert ei.value.code == -1 and "layer count" in str(ei.value)
    with pytest.raises(k2t.K2TError) as ei:
        k2t.Model.load_k2tb(gpu_ctx, dict(CFG, hidden=512, n_heads=8), path)
    assert ei.value.code == -1
    with pytest.raises(k2t.K2TError):
        k2t.Model.load_k2tb(gpu_ctx, CFG, tmp_path / "missing.k2tb")
