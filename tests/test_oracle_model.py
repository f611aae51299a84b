"""Pins the oracle's decode-megakernel restatement (oracle/model_oracle.py) against a
plain float64 Llama forward pass on the same unquantized weights: the quantized,
Hadamard-rotated pipeline must track it closely (a wrong RoPE half, a missing residual,
a misplaced rotation index or a transposed head would not)."""
import numpy as np

import oracle as O
from model_oracle import OracleModel, quantize_matrix

CFG = dict(n_layers=2, hidden=128, n_heads=2, n_kv_heads=1, head_dim=64, intermediate=256, vocab=200,
           max_seq=16, rms_eps=1e-5, rope_theta=10000.0)


def _float_forward(cfg, W, tokens):
    d, nq, nkv, hd, inter = cfg["hidden"], cfg["n_heads"], cfg["n_kv_heads"], cfg["head_dim"], cfg["intermediate"]
    K = [[] for _ in W["layers"]]
    Vv = [[] for _ in W["layers"]]
    out = []
    for pos, tok in enumerate(tokens):
        h = W["head"][tok].astype(np.float64)
        half = hd // 2
        inv = 1.0 / cfg["rope_theta"] ** (np.arange(half) * 2 / hd)
        c, s = np.cos(pos * inv), np.sin(pos * inv)

        def rope(v):
            return np.concatenate([v[:half] * c - v[half:] * s, v[half:] * c + v[:half] * s])

        def norm(x, w):
            return x / np.sqrt(np.mean(x * x) + cfg["rms_eps"]) * w

        for li, L in enumerate(W["layers"]):
            qkv = L["qkv"] @ norm(h, L["in_norm"])
            q = [rope(qkv[i * hd:(i + 1) * hd]) for i in range(nq)]
            K[li].append([rope(qkv[(nq + j) * hd:(nq + j + 1) * hd]) for j in range(nkv)])
            Vv[li].append([qkv[(nq + nkv + j) * hd:(nq + nkv + j + 1) * hd] for j in range(nkv)])
            att = []
            for qh in range(nq):
                j = qh // (nq // nkv)
                ks = np.array([k[j] for k in K[li]])
                vs = np.array([v[j] for v in Vv[li]])
                sc = ks @ q[qh] / np.sqrt(hd)
                p = np.exp(sc - sc.max())
                att.append((p / p.sum()) @ vs)
            h = h + L["o"] @ np.concatenate(att)
            gu = L["gu"] @ norm(h, L["post_norm"])
            g, u = gu[:inter], gu[inter:]
            h = h + L["down"] @ (g / (1 + np.exp(-g)) * u)
        out.append(W["head"] @ norm(h, W["final_norm"]))
    return out


def test_oracle_model_tracks_float_llama():
    rng = np.random.default_rng(0)
    d, nq, nkv, hd, inter, V = 128, 2, 1, 64, 256, 200
    W = {"layers": [], "head": (rng.standard_normal((V, d)) * 0.5).astype(np.float32),
         "final_norm": np.ones(d, np.float32)}
    for _ in range(2):
        W["layers"].append({"qkv": (rng.standard_normal(((nq + 2 * nkv) * hd, d)) * 0.05).astype(np.float32),
                            "o": (rng.standard_normal((d, nq * hd)) * 0.05).astype(np.float32),
                            "gu": (rng.standard_normal((2 * inter, d)) * 0.05).astype(np.float32),
                            "down": (rng.standard_normal((d, inter)) * 0.05).astype(np.float32),
                            "in_norm": (1 + 0.1 * rng.standard_normal(d)).astype(np.float32),
                            "post_norm": (1 + 0.1 * rng.standard_normal(d)).astype(np.float32)})
    layers = [{"qkv": quantize_matrix(L["qkv"], "n4", planes=6), "o": quantize_matrix(L["o"], "n4", planes=6),
               "gu": quantize_matrix(L["gu"], "n4", planes=6, interleave_gate_up=True),
               "down": quantize_matrix(L["down"], "n4", planes=6), "in_norm": L["in_norm"],
               "post_norm": L["post_norm"], "bias": None} for L in W["layers"]]
    head = quantize_matrix(W["head"], "n4", planes=6)
    model = OracleModel(CFG, layers, head, W["final_norm"])
    toks = [3, 150, 7, 99, 42]
    ref = _float_forward(CFG, W, toks)
    for i, t in enumerate(toks):
        got = model.forward_token(t)
        cos = float(np.dot(got, ref[i]) / (np.linalg.norm(got) * np.linalg.norm(ref[i])))
        assert cos > 0.995, (i, cos)


def test_embedding_is_inverse_rotated_head_row():
    rng = np.random.default_rng(1)
    Wh = (rng.standard_normal((64, 128)) * 0.3).astype(np.float32)
    head = quantize_matrix(Wh, "nf4")
    for r in (0, 17, 63):
        e = O.ifwht64(head.row_rotated(r))
        cos = float(np.dot(e, Wh[r]) / (np.linalg.norm(e) * np.linalg.norm(Wh[r])))
        assert cos > 0.99


def test_sliding_window_slots_and_attention():
    """Window / sink ring (real_llm.rs:1116-1122, 1235-1257, 8596-8612): the attended
    positions are the sinks plus the last window - sinks positions; their ring slots are
    distinct and still hold those positions' data after the ring wraps.  The window
    attention with per-64-block scores equals the full-head form for hd 64 and stays
    within fp32 rounding of it for hd 128."""
    import oracle as O
    from model_oracle import OracleModel
    cfg = dict(n_layers=1, hidden=64, n_heads=1, n_kv_heads=1, head_dim=64, intermediate=64, vocab=8, max_seq=1200,
               rms_eps=1e-5, rope_theta=10000.0)
    om = OracleModel(cfg, [], None, None, window=16, sinks=4)
    assert (om.window, om.sinks, om.ring) == (16, 4, 12 + 512)
    owner = {}
    for pos in range(1100):  # wraps the 524-slot ring twice
        owner[om.slot_of_pos(pos)] = pos
        seq = pos + 1
        act = om.active_slots(seq)
        want = list(range(seq)) if seq <= 16 else list(range(4)) + list(range(seq - 12, seq))
        assert [owner[s] for s in act] == want
        assert len(set(act)) == len(act)
    # sinks capped at window / 2; a window without room for the slack disables the ring
    assert OracleModel(cfg, [], None, None, window=16, sinks=20).sinks == 8
    assert OracleModel(cfg, [], None, None, window=700, sinks=4).window == 0
    rng = np.random.default_rng(1)
    for hd in (64, 128):
        q = rng.standard_normal(hd).astype(np.float32)
        n = 37
        kq = rng.integers(-127, 128, (n, hd)).astype(np.int8)
        vq = rng.integers(-127, 128, (n, hd)).astype(np.int8)
        ks = rng.uniform(0.01, 0.03, n).astype(np.float32)
        vs = rng.uniform(0.01, 0.03, n).astype(np.float32)
        a = O.attn_q8_head(q, kq, ks, vq, vs, 0.125)
        b = O.attn_q8_head(q, kq, ks, vq, vs, 0.125, window=True)
        if hd == 64:
            assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
        else:
            assert np.allclose(a, b, rtol=1e-5, atol=1e-6)
