"""Sparse-MoE feed-forward on the GPU (k2t_moe_ffn, and MoE layers inside the decode
engine with per-head QK-norm and q_dim != hidden) against the oracle's restatement of
forward_layer_single (sparse_moe.rs:961-1084) / route_sorted (86-182).

Bar: the routed expert ids equal the oracle's (inputs are drawn so that no two of the
top-(k+1) router probabilities are within 1e-4 of each other: the router's fp32 dot
order, like the reference's NEON vs x86 orders, is not a bit-exact contract), the route
weights within 1e-5, and the layer output within the end-to-end bar (cosine > 0.99999,
max |diff| <= 1e-3 of max |hidden|).  Integer expert dots are exact (grouped NF GEMV),
but an int8 code of x_norm or of the SwiGLU output can move by one where inv_rms / expf
round differently.
"""
import numpy as np
import pytest
import torch

import k2t
from k2tb_writer import K2TM_PAGE, random_moe_layer, write_k2tm
from model_oracle import Matrix, OracleModel, moe_ffn, quantize_matrix

pytestmark = pytest.mark.gpu


def _moe_dict(experts, router, top_k, norm, scoring, bias=None):
    return dict(router_w=router, router_b=bias, top_k=top_k, norm_topk_prob=norm, scoring=scoring,
                experts=experts)


def _well_separated(hidden, post_norm, eps, router, k, bias=None):
    from model_oracle import rms_norm
    z = router.astype(np.float64) @ rms_norm(hidden, post_norm, eps).astype(np.float64)
    if bias is not None:
        z = z + bias
    s = np.sort(z)[::-1][:k + 1]
    return np.min(np.abs(np.diff(s))) > 1e-3


# d <= 2048 routes inside the gate_up launch (two waves per router row); d = 3072 takes the
# separate route kernel; the biased case covers the bias added after the two halves.
@pytest.mark.parametrize("bits,E,k,scoring,norm,d,biased", [(3, 16, 4, 0, True, 256, False),
                                                           (4, 16, 4, 0, False, 256, False),
                                                           (3, 64, 8, 1, True, 256, False),
                                                           (3, 32, 6, 2, True, 256, False),
                                                           (3, 48, 4, 2, True, 256, True),
                                                           (3, 16, 4, 0, True, 3072, True)])
def test_moe_ffn_matches_oracle(gpu_ctx, bits, E, k, scoring, norm, d, biased):
    print(f"moe_ffn bits={bits} E={E} k={k} scoring={scoring} d={d} biased={biased}", flush=True)
    dff = 128
    rng = np.random.default_rng(100 + E + bits + d)
    layers = [random_moe_layer(rng, d, dff, E, bits=bits) for _ in range(2)]
    bias = (0.3 * rng.standard_normal(E)).astype(np.float32) if biased else None
    blob = write_k2tm([l[0] for l in layers], d, dff, bits, 2)
    bank = k2t.ExpertBank.upload(gpu_ctx, blob)
    assert bank.info()["experts_per_layer"] == E
    post_norm = (1 + 0.1 * rng.standard_normal(d)).astype(np.float32)
    ids = torch.zeros(k, dtype=torch.int32, device="cuda")
    wts = torch.zeros(k, dtype=torch.float32, device="cuda")
    dbias = torch.from_numpy(bias).cuda() if biased else None
    checked = 0
    for trial in range(12):
        hidden = rng.standard_normal(d).astype(np.float32)
        layer = trial % 2
        experts, router = layers[layer]
        if not _well_separated(hidden, post_norm, 1e-6, router, k, bias):
            continue
        want, routes = moe_ffn(hidden, post_norm, 1e-6, _moe_dict(experts, router, k, norm, scoring, bias))
        dh = torch.from_numpy(hidden).cuda()
        gpu_ctx.moe_ffn(bank, layer, torch.from_numpy(router).cuda(), dh, torch.from_numpy(post_norm).cuda(), 1e-6,
                        k, norm, scoring, router_bias=dbias, route_ids=ids, route_weights=wts)
        gpu_ctx.sync()
        got_ids = ids.cpu().numpy().tolist()
        assert got_ids == [e for e, _ in routes], f"trial {trial}: routes {got_ids} vs {routes}"
        assert np.allclose(wts.cpu().numpy(), [w for _, w in routes], rtol=1e-5, atol=1e-7)
        got = dh.cpu().numpy()
        delta_w, delta_g = want - hidden, got - hidden
        cos = float(np.dot(delta_w, delta_g) / (np.linalg.norm(delta_w) * np.linalg.norm(delta_g)))
        assert cos > 0.9999, f"trial {trial}: moe output cos {cos}"
        assert np.abs(got - want).max() <= 1e-3 * np.abs(want).max()
        checked += 1
    assert checked >= 6
    bank.close()


@pytest.mark.parametrize("scoring", [0, 1, 2])
def test_moe_route_ties_pick_lowest_id(gpu_ctx, scoring):
    """Equal router logits (duplicated router rows give bit-identical dots) rank by the
    lower expert id, as route_sorted's strict comparisons do (sparse_moe.rs:86-182): rows
    2 and 9 are equal and largest, rows 5, 6 and 12 equal and next, so top-3 = {2, 9, 5}."""
    print(f"moe route ties scoring={scoring}", flush=True)
    d, dff, E, k = 256, 128, 16, 3
    rng = np.random.default_rng(55)
    layers = [random_moe_layer(rng, d, dff, E, bits=3)]
    experts, router = layers[0]
    router = (0.01 * router).astype(np.float32)
    hidden = rng.standard_normal(d).astype(np.float32)
    post_norm = np.ones(d, np.float32)
    xn = hidden / np.sqrt(np.mean(hidden.astype(np.float64) ** 2) + 1e-6)
    top = (4.0 * xn / np.dot(xn, xn)).astype(np.float32)
    router[2] = router[9] = top
    router[5] = router[6] = router[12] = 0.5 * top
    blob = write_k2tm([experts], d, dff, 3, 2)
    bank = k2t.ExpertBank.upload(gpu_ctx, blob)
    ids = torch.zeros(k, dtype=torch.int32, device="cuda")
    wts = torch.zeros(k, dtype=torch.float32, device="cuda")
    _, routes = moe_ffn(hidden, post_norm, 1e-6, _moe_dict(experts, router, k, True, scoring))
    assert [e for e, _ in routes] == [2, 5, 9]
    gpu_ctx.moe_ffn(bank, 0, torch.from_numpy(router).cuda(), torch.from_numpy(hidden).cuda(),
                    torch.from_numpy(post_norm).cuda(), 1e-6, k, True, scoring, route_ids=ids, route_weights=wts)
    gpu_ctx.sync()
    assert ids.cpu().numpy().tolist() == [2, 5, 9]
    w = wts.cpu().numpy()
    assert w[0] == w[2] and np.allclose(w, [x for _, x in routes], rtol=1e-5, atol=1e-7)
    bank.close()


def test_moe_wrapped_bank_lane_order(gpu_ctx):
    """A wrapped NF3 bank streams the .k2tm layout as it lies; k2t_experts_nf3_lane_order
    rearranges it in place and the MoE output stays bit-identical, as for an uploaded
    bank (converted at upload).  Header page and codebooks are untouched."""
    print("moe wrapped bank lane order", flush=True)
    d, dff, E, k = 256, 128, 16, 4
    rng = np.random.default_rng(404)
    layers = [random_moe_layer(rng, d, dff, E, bits=3) for _ in range(2)]
    blob = write_k2tm([l[0] for l in layers], d, dff, 3, 2)
    host = np.frombuffer(blob, np.uint8)
    dev = torch.from_numpy(host.copy()).cuda()
    wrapped = k2t.ExpertBank.wrap(gpu_ctx, dev, host.size, host[:16384])
    uploaded = k2t.ExpertBank.upload(gpu_ctx, blob)
    post_norm = (1 + 0.1 * rng.standard_normal(d)).astype(np.float32)
    router = torch.from_numpy(layers[1][1]).cuda()
    pn = torch.from_numpy(post_norm).cuda()
    hidden = rng.standard_normal(d).astype(np.float32)

    def run(bank):
        h = torch.from_numpy(hidden).cuda()
        gpu_ctx.moe_ffn(bank, 1, router, h, pn, 1e-6, k, True, 0)
        gpu_ctx.sync()
        return h.cpu().numpy()

    a = run(wrapped)
    wrapped.nf3_lane_order()
    got = dev.cpu().numpy()
    mark = np.frombuffer(b"K2T-NF3-LANE-V1\0", np.uint8)
    assert np.array_equal(got[:16384 - 16], host[:16384 - 16]) and np.array_equal(got[16384 - 16:16384], mark)
    assert not host[16384 - 16:16384].any()
    assert not np.array_equal(got[16384:], host[16384:])
    assert np.array_equal(np.sort(got[16384:]), np.sort(host[16384:]))
    b, c = run(wrapped), run(uploaded)
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
    assert np.array_equal(a.view(np.uint32), c.view(np.uint32))
    # a second wrap of the converted bytes reads them in lane order; converting is a no-op
    wrapped.close()
    again = k2t.ExpertBank.wrap(gpu_ctx, dev, host.size, host[:16384])
    again.nf3_lane_order()
    assert np.array_equal(dev.cpu().numpy(), got)
    assert np.array_equal(run(again).view(np.uint32), a.view(np.uint32))
    again.close()
    uploaded.close()


def test_moe_ffn_argument_errors(gpu_ctx):
    rng = np.random.default_rng(5)
    experts, router = random_moe_layer(rng, 128, 64, 4, bits=3)
    bank = k2t.ExpertBank.upload(gpu_ctx, write_k2tm([experts], 128, 64, 3, 2))
    h = torch.zeros(128, device="cuda")
    r = torch.from_numpy(router).cuda()
    with pytest.raises(k2t.K2TError):
        gpu_ctx.moe_ffn(bank, 1, r, h, h, 1e-6, 2)  # shard layer out of range
    with pytest.raises(k2t.K2TError):
        gpu_ctx.moe_ffn(bank, 0, r, h, h, 1e-6, 5)  # top_k > experts
    with pytest.raises(k2t.K2TError):
        gpu_ctx.moe_ffn(bank, 0, r, h, h, 1e-6, 2, scoring=7)
    blob = bytearray(write_k2tm([experts], 128, 64, 3, 2))
    with pytest.raises(k2t.K2TError):
        k2t.ExpertBank.upload(gpu_ctx, bytes(blob[:-100]))  # truncated shard
    bank.close()


CFG = dict(n_layers=2, hidden=256, n_heads=4, n_kv_heads=2, head_dim=128, intermediate=64, vocab=300,
           max_seq=32, rms_eps=1e-6, rope_theta=1000000.0)


def _attn_layer(rng, cfg):
    d, nq, nkv, hd = cfg["hidden"], cfg["n_heads"], cfg["n_kv_heads"], cfg["head_dim"]
    w = lambda r, c: (rng.standard_normal((r, c)) * 0.02).astype(np.float32)  # noqa: E731
    return {"qkv": quantize_matrix(w((nq + 2 * nkv) * hd, d), "nf4"), "o": quantize_matrix(w(d, nq * hd), "nf4"),
            "in_norm": (1 + 0.1 * rng.standard_normal(d)).astype(np.float32),
            "post_norm": (1 + 0.1 * rng.standard_normal(d)).astype(np.float32),
            "q_norm": (1 + 0.1 * rng.standard_normal(hd)).astype(np.float32),
            "k_norm": (1 + 0.1 * rng.standard_normal(hd)).astype(np.float32), "bias": None}


@pytest.mark.parametrize("graph", [True, False])
def test_moe_model_decode_matches_oracle(gpu_ctx, graph):
    """Qwen3-MoE-shaped toy: q_dim (512) != hidden (256), hd 128, QK-norm, every layer
    sparse (16 NF3 experts, top 4, softmax + renorm), NF4 attention, tied NF4 head.
    Decode vs the oracle, prefill vs the oracle, and prefill == token-by-token decode."""
    print(f"moe model decode graph={graph}", flush=True)
    cfg = CFG
    rng = np.random.default_rng(77)
    d, E, k, dff = cfg["hidden"], 16, 4, 128
    moe_layers = [random_moe_layer(rng, d, dff, E, bits=3) for _ in range(cfg["n_layers"])]
    blob = write_k2tm([m[0] for m in moe_layers], d, dff, 3, 2)
    bank = k2t.ExpertBank.upload(gpu_ctx, blob)
    layers = []
    for li in range(cfg["n_layers"]):
        L = _attn_layer(rng, cfg)
        L["moe"] = _moe_dict(moe_layers[li][0], moe_layers[li][1], k, True, 0)
        layers.append(L)
    head = quantize_matrix((rng.standard_normal((cfg["vocab"], d)) * 0.02).astype(np.float32), "nf4")
    fn = (1 + 0.1 * rng.standard_normal(d)).astype(np.float32)
    ref = OracleModel(cfg, layers, head, fn)
    gm = k2t.Model(gpu_ctx, cfg, max_batch=4)
    gm.set_graph(graph)
    mats = []
    up = lambda m: gpu_ctx.upload_nf(m.rows, m.cols, 4, m.sgc, m.cb, m.pair, m.tail)  # noqa: E731
    for li, L in enumerate(layers):
        q, o = up(L["qkv"]), up(L["o"])
        mats += [q, o]
        gm.set_layer(li, q, o, None, None, L["in_norm"], L["post_norm"])
        gm.set_qk_norm(li, L["q_norm"], L["k_norm"])
        gm.set_moe(li, bank, li, moe_layers[li][1], k, True, 0)
    hm = up(head)
    gm.set_head(hm, fn)
    assert not gm.persistent_active()
    toks = np.random.default_rng(8).integers(0, cfg["vocab"], 6)
    for i, t in enumerate(toks):
        a, b = gm.decode(int(t)), ref.forward_token(int(t))
        cos = float(np.dot(a, b) / (np.linalg.norm(a) * np.linalg.norm(b)))
        rel = float(np.abs(a - b).max() / np.abs(b).max())
        assert cos > 0.9999 and rel <= 2e-2, f"step {i}: cos {cos} rel {rel}"
    # prompt path: MoE runs per token inside a batch
    gm.reset()
    ref2 = OracleModel(cfg, layers, head, fn)
    a = gm.prefill(np.array([3, 250, 17], np.int32))
    for t in (3, 250, 17):
        b = ref2.forward_token(t)
    cos = float(np.dot(a, b) / (np.linalg.norm(a) * np.linalg.norm(b)))
    assert cos > 0.9999, f"prefill cos {cos}"
    # token by token: the qkv / gate_up activations are built inside the GEMVs (one token);
    # the batch builds them with rmsnorm_act.  Same codes, so the logits are bit-identical.
    gm.reset()
    for t in (3, 250, 17):
        c = gm.decode(t)
    assert np.array_equal(a.view(np.uint32), c.view(np.uint32))
    # exact-order mode (the MoE in the x86 reference's order too): decode equals the oracle
    # bit for bit
    gm.set_exact(True)
    gm.reset()
    ref3 = OracleModel(cfg, layers, head, fn)
    for i, t in enumerate(toks):
        a, b = gm.decode(int(t)), ref3.forward_token(int(t))
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32)), \
            f"exact step {i}: rel {float(np.abs(a - b).max() / np.abs(b).max()):.2e}"
    gm.set_exact(False)
    gm.close()
    for m in mats + [hm]:
        m.close()
    bank.close()


def test_moe_model_shared_expert_matches_oracle(gpu_ctx):
    """Qwen2-MoE-style layers with a shared expert (SharedMoeExpert, NF backend,
    sparse_moe.rs:209-312): layer 0 with a sigmoid gate row, layer 1 without, inter 192 in
    [gate; up] row order.  Decode in exact-order mode bit-identical to the oracle and on the
    fast path within its bar, a 3-token prefill vs the oracle; removing the shared expert
    changes the logits."""
    print("moe model with a shared expert", flush=True)
    cfg = CFG
    rng = np.random.default_rng(91)
    d, E, k, dff, inter_s = cfg["hidden"], 16, 4, 128, 192
    moe_layers = [random_moe_layer(rng, d, dff, E, bits=3) for _ in range(cfg["n_layers"])]
    bank = k2t.ExpertBank.upload(gpu_ctx, write_k2tm([m[0] for m in moe_layers], d, dff, 3, 2))
    w = lambda r, c: (rng.standard_normal((r, c)) * 0.02).astype(np.float32)  # noqa: E731
    layers, shared = [], []
    for li in range(cfg["n_layers"]):
        L = _attn_layer(rng, cfg)
        sgu, sdn = quantize_matrix(w(2 * inter_s, d), "nf4"), quantize_matrix(w(d, inter_s), "nf4")
        gate = (0.05 * rng.standard_normal(d)).astype(np.float32) if li == 0 else None
        L["moe"] = _moe_dict(moe_layers[li][0], moe_layers[li][1], k, True, 0)
        as_dict = lambda m: dict(pair=m.pair, tail=m.tail, cb=m.cb, bits=4, sgc=m.sgc, rows=m.rows,  # noqa: E731
                                 cols=m.cols)
        L["moe"]["shared"] = dict(gate_up=as_dict(sgu), down=as_dict(sdn), gate_weight=gate)
        layers.append(L)
        shared.append((sgu, sdn, gate))
    head = quantize_matrix((rng.standard_normal((cfg["vocab"], d)) * 0.02).astype(np.float32), "nf4")
    fn = (1 + 0.1 * rng.standard_normal(d)).astype(np.float32)
    ref = OracleModel(cfg, layers, head, fn)
    gm = k2t.Model(gpu_ctx, cfg, max_batch=4)
    mats = []
    up = lambda m: gpu_ctx.upload_nf(m.rows, m.cols, 4, m.sgc, m.cb, m.pair, m.tail)  # noqa: E731
    for li, L in enumerate(layers):
        q, o = up(L["qkv"]), up(L["o"])
        sgu, sdn = up(shared[li][0]), up(shared[li][1])
        mats += [q, o, sgu, sdn]
        gm.set_layer(li, q, o, None, None, L["in_norm"], L["post_norm"])
        gm.set_qk_norm(li, L["q_norm"], L["k_norm"])
        gm.set_moe(li, bank, li, moe_layers[li][1], k, True, 0)
        gm.set_moe_shared(li, sgu, sdn, shared[li][2])
    hm = up(head)
    gm.set_head(hm, fn)
    toks = np.random.default_rng(9).integers(0, cfg["vocab"], 5)
    # exact-order steps (x86 sum-of-squares order, expf_rn, sequential attention sums, the
    # MoE's sequential router dot, shared-expert gate and in-order GEMV epilogues) equal the
    # oracle bit for bit at every step; the fast path moves single int8 codes (1 - cos up to
    # about 1.4e-4 here, 4e-5 with no shared expert), so its bar is cosine > 0.9998
    last = None
    for exact in (True, False):
        gm.set_exact(exact)
        gm.reset()
        ref = OracleModel(cfg, layers, head, fn)
        for i, t in enumerate(toks):
            a, b = gm.decode(int(t)), ref.forward_token(int(t))
            cos = float(np.dot(a, b) / (np.linalg.norm(a) * np.linalg.norm(b)))
            rel = float(np.abs(a - b).max() / np.abs(b).max())
            if exact:
                assert np.array_equal(a.view(np.uint32), b.view(np.uint32)), f"exact step {i}: cos {cos} rel {rel}"
            else:
                assert cos > 0.9998 and rel <= 2e-2, f"step {i}: cos {cos} rel {rel}"
            last = a
    gm.reset()
    ref2 = OracleModel(cfg, layers, head, fn)
    a = gm.prefill(np.array([3, 250, 17], np.int32))
    for t in (3, 250, 17):
        b = ref2.forward_token(t)
    cos = float(np.dot(a, b) / (np.linalg.norm(a) * np.linalg.norm(b)))
    assert cos > 0.9999, f"prefill cos {cos}"
    # without the shared experts the same prompt gives other logits
    for li in range(cfg["n_layers"]):
        gm.set_moe_shared(li, None, None)
    gm.reset()
    c = gm.prefill(np.array([3, 250, 17], np.int32))
    assert np.abs(c - a).max() > 1e-3 * np.abs(a).max()
    assert last is not None
    gm.close()
    for m in mats + [hm]:
        m.close()
    bank.close()


def test_kv_synthetic_sets_position(gpu_ctx):
    cfg = dict(CFG, n_layers=1)
    rng = np.random.default_rng(3)
    L = _attn_layer(rng, cfg)
    layers, head = [L], quantize_matrix((rng.standard_normal((cfg["vocab"], cfg["hidden"])) * 0.02)
                                        .astype(np.float32), "nf4")
    experts, router = random_moe_layer(rng, cfg["hidden"], 64, 8, bits=3)
    bank = k2t.ExpertBank.upload(gpu_ctx, write_k2tm([experts], cfg["hidden"], 64, 3, 2))
    gm = k2t.Model(gpu_ctx, cfg, max_batch=2)
    up = lambda m: gpu_ctx.upload_nf(m.rows, m.cols, 4, m.sgc, m.cb, m.pair, m.tail)  # noqa: E731
    q, o, hm = up(L["qkv"]), up(L["o"]), up(head)
    gm.set_layer(0, q, o, None, None, L["in_norm"], L["post_norm"])
    gm.set_moe(0, bank, 0, router, 2)
    gm.set_head(hm, np.ones(cfg["hidden"], np.float32))
    gm.kv_synthetic(20, seed=1)
    assert gm.position() == 20
    logits = gm.decode(5)
    assert np.isfinite(logits).all() and gm.position() == 21
    with pytest.raises(k2t.K2TError):
        gm.kv_synthetic(cfg["max_seq"])
    gm.close()
    for m in (q, o, hm):
        m.close()
    bank.close()
