"""Sparse-MoE host pieces (no GPU): the .k2tm header / expert layout of the C ABI, and
the oracle's route_sorted.

Pins:
  - k2t_k2tm_expert_layout equals nf_expert_byte_layout's closed form for the
    30B-A3B expert (gate_up 1536x2048, down 2048x768, NF3 g128: 1,228,800 + 614,400 pair
    bytes, counted by hand from the record layout) and the test writer's layout;
  - header decoding round-trips the writer's page and rejects bad magic / sizes / bits;
  - route_sorted against brute force: top-k of distinct scores by argsort, softmax
    weights from the closed form, renormalized weights summing to 1, ties resolved to
    the lower expert id, output sorted by id, and the three scoring rules.
"""
import numpy as np
import pytest

import k2t
from k2tb_writer import K2TM_PAGE, expert_layout, random_moe_layer, write_k2tm
from model_oracle import SIGMOID, SOFTMAX, TOPK_SOFTMAX, route_sorted


def test_expert_layout_30b_shape():
    L = k2t.k2tm_expert_layout(2048, 768, 3, 2)
    # gate_up: 48 pairs x (16 scale groups x 64 B + 32 chunks x 2 x 384 B)
    assert L["gu_pair_bytes"] == 48 * (16 * 64 + 32 * 2 * 384) == 1228800
    # down: 64 pairs x (6 x 64 + 12 x 2 x 384)
    assert L["dn_pair_bytes"] == 64 * (6 * 64 + 12 * 2 * 384) == 614400
    assert L["gu_pair_off"] == 64 and L["gu_codebook_off"] == 0 and L["dn_codebook_off"] == 16
    assert L["dn_pair_off"] == 64 + 1228800
    assert L["aligned_expert_bytes"] == ((64 + 1228800 + 614400 + 16383) // 16384) * 16384
    for args in [(256, 128, 3, 2), (256, 128, 4, 2), (512, 192, 4, 1), (2048, 768, 4, 2)]:
        a, b = k2t.k2tm_expert_layout(*args), expert_layout(*args)
        assert (a["gu_pair_bytes"], a["dn_pair_off"], a["dn_pair_bytes"], a["aligned_expert_bytes"]) == \
               (b["gu_bytes"], b["dn_off"], b["dn_bytes"], b["aligned"])


def test_k2tm_header_roundtrip_and_errors():
    rng = np.random.default_rng(3)
    layers = [random_moe_layer(rng, 128, 64, 4, bits=3)[0] for _ in range(2)]
    blob = write_k2tm(layers, 128, 64, 3, 2)
    h = k2t.k2tm_read_header(blob[:K2TM_PAGE])
    assert (h["num_layers"], h["experts_per_layer"], h["d_model"], h["d_ff_expert"], h["bits"]) == (2, 4, 128, 64, 3)
    assert len(blob) == K2TM_PAGE + 2 * 4 * h["aligned_expert_bytes"]
    bad = bytearray(blob[:K2TM_PAGE])
    bad[0] = ord("X")
    with pytest.raises(k2t.K2TError):
        k2t.k2tm_read_header(bytes(bad))
    with pytest.raises(k2t.K2TError):
        k2t.k2tm_read_header(blob[:100])
    bad = bytearray(blob[:K2TM_PAGE])
    bad[16 + 5 * 8] ^= 0x40  # aligned_expert_bytes
    with pytest.raises(k2t.K2TError):
        k2t.k2tm_read_header(bytes(bad))
    bad = bytearray(blob[:K2TM_PAGE])
    bad[16 + 6 * 8] = 5  # NF5 experts
    with pytest.raises(k2t.K2TError) as ei:
        k2t.k2tm_read_header(bytes(bad))
    assert ei.value.code == -4


def test_route_sorted_against_brute_force():
    rng = np.random.default_rng(7)
    for E, k in [(16, 4), (128, 8), (60, 6)]:
        z = rng.standard_normal(E).astype(np.float32)
        r = route_sorted(z, k, True, SOFTMAX)
        top = sorted(np.argsort(-z.astype(np.float64))[:k].tolist())
        assert [e for e, _ in r] == top
        p = np.exp(z.astype(np.float64) - z.max())
        p /= p.sum()
        want = p[top] / p[top].sum()
        assert np.allclose([w for _, w in r], want, rtol=1e-5)
        assert abs(sum(w for _, w in r) - 1.0) < 1e-5
        # without renormalization: plain softmax probabilities
        r2 = route_sorted(z, k, False, SOFTMAX)
        assert np.allclose([w for _, w in r2], p[top], rtol=1e-5)
        # topk-softmax: softmax over the k largest logits
        r3 = route_sorted(z, k, True, TOPK_SOFTMAX)
        q = np.exp(z[top].astype(np.float64) - z[top].max())
        assert np.allclose([w for _, w in r3], q / q.sum(), rtol=1e-5)
        # sigmoid scores, renormalized
        r4 = route_sorted(z, k, True, SIGMOID)
        s = 1.0 / (1.0 + np.exp(-z[top].astype(np.float64)))
        assert np.allclose([w for _, w in r4], s / s.sum(), rtol=1e-5)


def test_route_sorted_ties_pick_lower_ids():
    z = np.array([1.0, 3.0, 3.0, 2.0, 3.0, 0.5], np.float32)
    r = route_sorted(z, 2, True, SOFTMAX)
    assert [e for e, _ in r] == [1, 2]
    assert abs(r[0][1] - 0.5) < 1e-7 and abs(r[1][1] - 0.5) < 1e-7
    r = route_sorted(z, 4, False, TOPK_SOFTMAX)
    assert [e for e, _ in r] == [1, 2, 3, 4]


@pytest.mark.parametrize("gated", [False, True])
def test_oracle_shared_expert_against_float_math(gated):
    """The oracle's shared expert (SharedMoeExpert::forward_single, NF backend) against the
    same computation in float64 on the dequantized weights (gate rows first, then up;
    SwiGLU; down; sigmoid gate scale): the int8 activations leave cosine > 0.999.  A
    swapped gate / up split or a missing scale fails this."""
    import oracle as O
    from model_oracle import quantize_matrix, shared_expert
    rng = np.random.default_rng(31 + gated)
    d, inter = 256, 192
    Wgu = (rng.standard_normal((2 * inter, d)) * 0.05).astype(np.float32)
    Wdn = (rng.standard_normal((d, inter)) * 0.05).astype(np.float32)
    gu, dn = quantize_matrix(Wgu, "nf4"), quantize_matrix(Wdn, "nf4")
    xn = rng.standard_normal(d).astype(np.float32)
    gate = (0.2 * rng.standard_normal(d)).astype(np.float32) if gated else None
    as_dict = lambda m: dict(pair=m.pair, tail=m.tail, cb=m.cb, bits=4, sgc=m.sgc, rows=m.rows, cols=m.cols)  # noqa
    aq, as_, _ = O.populate_fwht(xn)
    got = shared_expert(xn, aq, as_, dict(gate_up=as_dict(gu), down=as_dict(dn), gate_weight=gate))
    # float64 on the rotated-domain weights: W x = (W H^T)(H x) with H the signed FWHT
    deq = lambda m: np.stack([O.ifwht64(m.row_rotated(r)) for r in range(m.rows)]).astype(np.float64)  # noqa
    g = deq(gu) @ xn.astype(np.float64)
    sw = g[:inter] / (1 + np.exp(-g[:inter])) * g[inter:]
    want = deq(dn) @ sw
    if gated:
        want = want / (1 + np.exp(-float(np.dot(gate.astype(np.float64), xn))))
    cos = float(np.dot(got, want) / (np.linalg.norm(got) * np.linalg.norm(want)))
    assert cos > 0.999, cos
    assert abs(np.linalg.norm(got) / np.linalg.norm(want) - 1) < 0.02


def test_oracle_router_logits_sequential_float32():
    """The oracle's router logits follow dot_f32_moe on x86 (sparse_moe.rs:1644-1656):
    float32 products added in index order from 0.  Pinned against an explicit float32
    loop (the closed form of that order), and shown to differ from a float64 dot on some
    logit (so the order is observable and the test can fail)."""
    import oracle as O
    from model_oracle import moe_ffn
    rng = np.random.default_rng(5)
    d, E = 256, 16
    W = (rng.standard_normal((E, d)) * 0.05).astype(np.float32)
    h = rng.standard_normal(d).astype(np.float32)
    pn = (1 + 0.1 * rng.standard_normal(d)).astype(np.float32)
    xn = ((h * np.float32(O.inv_rms(h, 1e-6))) * pn).astype(np.float32)
    loop = np.zeros(E, np.float32)
    for e in range(E):
        a = np.float32(0.0)
        for i in range(d):
            a = np.float32(a + np.float32(W[e, i] * xn[i]))
        loop[e] = a
    via = np.cumsum((W * xn[None, :]).astype(np.float32), axis=1, dtype=np.float32)[:, -1]
    assert np.array_equal(loop.view(np.uint32), via.astype(np.float32).view(np.uint32))
    f64 = np.array([np.dot(W[e].astype(np.float64), xn.astype(np.float64)) for e in range(E)], np.float32)
    assert not np.array_equal(loop, f64)
    # moe_ffn routes on exactly these logits: its top-1 route is argmax of the loop's softmax
    lay, _ = random_moe_layer(rng, d, 64, E, bits=4)
    moe = dict(router_w=W, router_b=None, top_k=2, norm_topk_prob=True, scoring=SOFTMAX, experts=lay)
    _, routes = moe_ffn(h, pn, 1e-6, moe)
    assert set(e for e, _ in routes) == set(np.argsort(-loop, kind="stable")[:2].tolist())
