"""The .k2tb reader (k2t_k2tb_*, host code, no GPU): files written in save_bipolar's
format (real_llm.rs:3705-3895) from oracle-quantized matrices are read back and
repacked like load_bipolar + repack_sdot (real_llm.rs:3902-4190, 3657-3702).

Pins:
  - bit-plane bodies repack to exactly the oracle's from_bipolar_with_perm bytes
    (or_nibble4_repack), and, with the gate_up interleave, to the bytes the product
    compiler emits straight from the weights (k2t_compile_bipolar, a separate route);
  - NF gate_up block swap equals the oracle's row-permuted re-pack of the same indices;
  - every version's optional fields land where the format puts them;
  - truncation at any byte, a bad magic and unsupported tags fail with the documented
    error codes instead of reading past the file.
"""
import json
import os

import numpy as np
import pytest

import k2t
import oracle as O
from k2tb_writer import bipolar_source, nf_source, write_k2tb
from model_oracle import quantize_matrix

E_ARG, E_STATE = -1, -4


def _w(rng, r, c):
    return (rng.standard_normal((r, c)) * 0.02).astype(np.float32)


def _tiny(rng, fmt="bipolar", planes=(5, 5, 4, 5, 4), d=128, inter=256, nq=2, nkv=1, hd=64, V=200, L=2,
          bias=False):
    """Source matrices + weights of a tiny decoder (p55454-like planes or NF4)."""
    shapes = {"qkv": ((nq + 2 * nkv) * hd, d), "o": (d, nq * hd), "gu": (2 * inter, d), "down": (d, inter)}
    pl = dict(zip(("qkv", "o", "gu", "down", "head"), planes))
    Ws, layers = [], []
    for _ in range(L):
        Lw, Ls = {}, {}
        for k, (r, c) in shapes.items():
            W = _w(rng, r, c)
            Lw[k] = W
            Ls[k] = bipolar_source(W, pl[k]) if fmt == "bipolar" else nf_source(W, 4, 2)
        Ls["in_norm"] = (1 + 0.1 * rng.standard_normal(d)).astype(np.float32)
        Ls["post_norm"] = (1 + 0.1 * rng.standard_normal(d)).astype(np.float32)
        if bias:
            Ls["bias"] = (0.01 * rng.standard_normal(shapes["qkv"][0])).astype(np.float32)
        Ws.append(Lw)
        layers.append(Ls)
    Wh = _w(rng, V, d)
    head = bipolar_source(Wh, pl["head"]) if fmt == "bipolar" else nf_source(Wh, 4, 2)
    fn = (1 + 0.1 * rng.standard_normal(d)).astype(np.float32)
    return Ws, Wh, layers, head, fn


def test_bipolar_repack_matches_oracle_and_compiler(tmp_path):
    rng = np.random.default_rng(11)
    Ws, Wh, layers, head, fn = _tiny(rng)
    p = tmp_path / "m.k2tb"
    write_k2tb(p, 2, layers, fn, head, mode_words=(7, 5 | (2 << 8), 5, 4, 5, 4))
    with k2t.K2tb(p) as f:
        v, n, mw = f.header()
        assert (v, n) == (2, 2) and mw == [7, 5 | (2 << 8), 5, 4, 5, 4]
        for li, L in enumerate(layers):
            for wi, k in enumerate(("qkv", "o", "gu", "down")):
                s = L[k]
                gu = k == "gu"
                info, pair, tail = f.matrix(li, wi, interleave_gate_up=gu)
                assert (info.tag, info.fmt, info.rows, info.cols, info.planes_or_bits) == \
                       (0, 1, s["rows"], s["cols"], s["planes"])
                rp, rt = O.nibble4_repack(s["inter"], s["scales"], s["rows"], s["cols"], s["planes"], gu)
                assert np.array_equal(pair, rp) and np.array_equal(tail, rt), (li, k)
                # the product compiler's direct route from the weights gives the same bytes
                cp, ct = k2t.compile_bipolar(Ws[li][k], s["planes"], interleave_gate_up=gu, threads=2)
                assert np.array_equal(pair, cp) and np.array_equal(tail, ct), (li, k)
            assert np.array_equal(f.vector(li, 0), L["in_norm"])
            assert np.array_equal(f.vector(li, 1), L["post_norm"])
        info, pair, tail = f.matrix(-1, 4)
        rp, rt = O.nibble4_repack(head["inter"], head["scales"], head["rows"], head["cols"], head["planes"])
        assert np.array_equal(pair, rp) and np.array_equal(tail, rt)
        assert tail.size > 0  # V = 200 rows -> odd stripe count: the tail record path
        assert np.array_equal(f.vector(-1, 0), fn)
        assert f.vector(-1, 1).size == 0 and f.vector(-1, 2).size == 0


def test_nf_gate_up_interleave_matches_permuted_repack(tmp_path):
    rng = np.random.default_rng(12)
    Ws, Wh, layers, head, fn = _tiny(rng, fmt="nf", L=1)
    p = tmp_path / "nf.k2tb"
    write_k2tb(p, 3, layers, fn, head)
    with k2t.K2tb(p) as f:
        assert f.header()[0] == 3
        for wi, k in enumerate(("qkv", "o", "gu", "down")):
            gu = k == "gu"
            info, pair, tail = f.matrix(0, wi, interleave_gate_up=gu)
            want = quantize_matrix(Ws[0][k], "nf4", sgc=2, interleave_gate_up=gu)
            assert info.tag == 2 and info.fmt == 2 and info.planes_or_bits == 4 and info.sgc == 2
            assert np.array_equal(np.array(info.codebook[:], np.int8), want.cb)
            assert np.array_equal(pair, want.pair) and np.array_equal(tail, want.tail), k
        assert f.vector(0, 2).size == 0  # v3 stores an empty qkv_bias


def test_nf3_matrix_and_optional_fields(tmp_path):
    rng = np.random.default_rng(13)
    Ws, Wh, layers, head, fn = _tiny(rng, fmt="nf", L=1, bias=True)
    layers[0]["down"] = nf_source(Ws[0]["down"], 3, 2)
    d, V = 128, 200
    emb_bf16 = rng.integers(0, 1 << 16, V * d, dtype=np.uint16)
    p = tmp_path / "v6.k2tb"
    for L in layers:
        L["q_norm"], L["k_norm"] = None, None
    write_k2tb(p, 6, layers, fn, head, embed_bf16=emb_bf16, embed_nf4=nf_source(_w(rng, V, d), 4, 2))
    with k2t.K2tb(p) as f:
        assert f.header()[0] == 6
        info, pair, tail = f.matrix(0, 3)
        assert info.planes_or_bits == 3 and np.array_equal(pair, layers[0]["down"]["pair"])
        assert np.array_equal(f.vector(0, 2), layers[0]["bias"])
        assert f.vector(0, 3).size == 0 and f.vector(0, 4).size == 0
        assert np.array_equal(f.vector(-1, 2), emb_bf16)
        info, pair, tail = f.matrix(-1, 5)
        assert info.rows == V and info.cols == d and info.planes_or_bits == 4


def test_v1_untagged_bipolar(tmp_path):
    rng = np.random.default_rng(14)
    Ws, Wh, layers, head, fn = _tiny(rng, planes=(4, 4, 4, 4, 4), L=1)
    emb = (rng.standard_normal(200 * 128)).astype(np.float32)
    p = tmp_path / "v1.k2tb"
    write_k2tb(p, 1, layers, fn, head, mode_words=(0, 4, 0, 0, 0, 0), embed_f32=emb)
    with k2t.K2tb(p) as f:
        v, n, mw = f.header()
        assert v == 1 and mw[:2] == [0, 4]
        info, pair, tail = f.matrix(0, 0)
        s = layers[0]["qkv"]
        rp, rt = O.nibble4_repack(s["inter"], s["scales"], s["rows"], s["cols"], 4)
        assert np.array_equal(pair, rp)
        assert np.array_equal(f.vector(-1, 1), emb)


def test_truncation_and_bad_files_fail_cleanly(tmp_path):
    rng = np.random.default_rng(15)
    Ws, Wh, layers, head, fn = _tiny(rng, L=1, d=64, inter=128, nq=1, hd=64, V=48)
    p = tmp_path / "ok.k2tb"
    n = write_k2tb(p, 2, layers, fn, head)
    data = p.read_bytes()
    cuts = sorted(set([0, 5, 11, 12, 20, 60, 100, n // 3, n // 2, n - 9, n - 1]))
    for cut in cuts:
        q = tmp_path / f"cut{cut}.k2tb"
        q.write_bytes(data[:cut])
        with pytest.raises(k2t.K2TError) as ei:
            k2t.K2tb(q)
        assert ei.value.code == E_ARG, cut
    bad = tmp_path / "bad.k2tb"
    bad.write_bytes(b"NOTAK2TB" + data[8:])
    with pytest.raises(k2t.K2TError) as ei:
        k2t.K2tb(bad)
    assert ei.value.code == E_ARG and "magic" in str(ei.value)
    with pytest.raises(k2t.K2TError):
        k2t.K2tb(tmp_path / "missing.k2tb")
    # unsupported matrix kinds and the MoE core version
    for tag in (1, 3):
        L2 = [dict(layers[0], qkv={"kind": "raw_tag", "tag": tag})]
        q = tmp_path / f"tag{tag}.k2tb"
        write_k2tb(q, 2, L2, fn, head)
        with pytest.raises(k2t.K2TError) as ei:
            k2t.K2tb(q)
        assert ei.value.code == E_STATE
    q = tmp_path / "v5.k2tb"
    write_k2tb(q, 5, layers, fn, head)
    with pytest.raises(k2t.K2TError) as ei:
        k2t.K2tb(q)
    assert ei.value.code == E_STATE


def test_three_plane_bipolar_is_rejected_on_repack(tmp_path):
    rng = np.random.default_rng(16)
    Ws, Wh, layers, head, fn = _tiny(rng, L=1, d=64, inter=128, nq=1, hd=64, V=48)
    layers[0]["o"] = bipolar_source(Ws[0]["o"], 3)
    p = tmp_path / "p3.k2tb"
    write_k2tb(p, 2, layers, fn, head)
    with k2t.K2tb(p) as f:
        with pytest.raises(k2t.K2TError) as ei:
            f.matrix(0, 1)
        assert ei.value.code == E_STATE and "planes" in str(ei.value)
        with pytest.raises(k2t.K2TError):
            f.matrix(0, 7)


def test_load_llama_config(tmp_path):
    cfg = {"architectures": ["LlamaForCausalLM"], "hidden_size": 2048, "intermediate_size": 8192,
           "num_attention_heads": 32, "num_hidden_layers": 24, "num_key_value_heads": 32, "rms_norm_eps": 1e-05,
           "rope_theta": 130000, "vocab_size": 49152, "tie_word_embeddings": True, "head_dim": None}
    (tmp_path / "config.json").write_text(json.dumps(cfg))
    c = k2t.load_llama_config(tmp_path, 512)
    assert c["head_dim"] == 64 and c["hidden"] == 2048 and c["n_layers"] == 24 and c["max_seq"] == 512
    assert c["rope_theta"] == 130000.0 and c["vocab"] == 49152
    # defaults of from_config_json for missing keys (SmolLM2-135M shape)
    (tmp_path / "config.json").write_text("{}")
    c = k2t.load_llama_config(tmp_path, 64)
    assert (c["hidden"], c["intermediate"], c["n_layers"], c["n_heads"], c["n_kv_heads"], c["vocab"]) == \
           (576, 1536, 30, 9, 3, 49152)
    # NTK-alpha stretch: theta * alpha^(d/(d-2))
    (tmp_path / "config.json").write_text(json.dumps({"hidden_size": 128, "num_attention_heads": 2,
                                                      "rope_theta": 10000.0,
                                                      "rope_scaling": {"type": "dynamic", "alpha": 1000.0}}))
    c = k2t.load_llama_config(tmp_path, 64)
    assert abs(c["rope_theta"] - 10000.0 * 1000.0 ** (64 / 62)) < 1e-3 * c["rope_theta"]
    (tmp_path / "config.json").write_text(json.dumps({"num_experts": 128, "num_experts_per_tok": 8}))
    with pytest.raises(ValueError):
        k2t.load_llama_config(tmp_path, 64)
    assert os.path.exists(tmp_path / "config.json")
