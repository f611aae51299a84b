"""KV-cache store and decode attention as standalone ops (k2t_kv_store, k2t_attn_decode;
the engine runs the same device code) against the oracle, for the int8 and the NF4
Hadamard caches, with and without the sliding-window ring; plus NF4-KV models end to end.

Bars: the store is integer / byte work and BF16 scales: bit-exact.  Attention fp32
outputs within 1e-4 relative of max |out| (flash-decoding splits and the merge change the
summation order of the reference's single pass; exp is `expf` on both sides)."""
import numpy as np
import pytest
import torch

import k2t
import oracle as O
from model_oracle import OracleModel, random_model

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("bits", [8, 4])
@pytest.mark.parametrize("hd", [64, 128])
def test_kv_store_bit_exact(gpu_ctx, bits, hd):
    print(f"kv_store bits={bits} hd={hd}", flush=True)
    rng = np.random.default_rng(hd + bits)
    n = 37
    heads = (rng.standard_normal((n, hd)) * rng.uniform(0.01, 4.0, (n, 1))).astype(np.float32)
    heads[5] = 0.0
    heads[9, :3] *= 50.0  # outliers
    dh = torch.from_numpy(heads).cuda()
    if bits == 8:
        q = torch.zeros((n, hd), dtype=torch.int8, device="cuda")
        s = torch.zeros(n, dtype=torch.float32, device="cuda")
    else:
        q = torch.zeros((n, hd // 2), dtype=torch.uint8, device="cuda")
        s = torch.zeros((n, hd // 64), dtype=torch.int16, device="cuda")
    gpu_ctx.kv_store(bits, dh, n, hd, q, s)
    gpu_ctx.sync()
    gq, gs = q.cpu().numpy(), s.cpu().numpy()
    for t in range(n):
        if bits == 8:
            rq, rs = O.kv_quant_head(heads[t])
            assert np.array_equal(gq[t], rq) and np.float32(gs[t]).view(np.uint32) == np.float32(rs).view(np.uint32), t
        else:
            rq, rs = O.kv_quant_head_q4(heads[t])
            assert np.array_equal(gq[t], rq) and np.array_equal(gs[t].view(np.uint16), rs), t


def _cache(rng, bits, n_kv, cap, hd, fill):
    """A cache of n_kv x cap slots with `fill` random heads stored by the oracle."""
    if bits == 8:
        kq = np.zeros((n_kv, cap, hd), np.int8)
        ks = np.zeros((n_kv, cap), np.float32)
    else:
        kq = np.full((n_kv, cap, hd // 2), 0x88, np.uint8)
        ks = np.zeros((n_kv, cap, hd // 64), np.uint16)
    vq, vs = kq.copy(), ks.copy()
    for h in range(n_kv):
        for t in range(fill):
            k, v = rng.standard_normal(hd).astype(np.float32), rng.standard_normal(hd).astype(np.float32)
            f = O.kv_quant_head if bits == 8 else O.kv_quant_head_q4
            kq[h, t], ks[h, t] = f(k)
            vq[h, t], vs[h, t] = f(v)
    return kq, ks, vq, vs


# (seq above 1024: 256-position spans and the merge kernel, whose loads go out in one round
# up to 32 spans and in batches above (8300 positions = 33 spans); up to 1024 the
# whole-context kernel)
@pytest.mark.parametrize("bits,hd,seq,window,sinks", [(8, 64, 300, 0, 0), (8, 128, 70, 0, 0), (4, 64, 300, 0, 0),
                                                      (4, 128, 70, 0, 0), (8, 128, 90, 24, 4), (4, 64, 90, 24, 4),
                                                      (8, 128, 1300, 0, 0), (8, 64, 1100, 0, 0), (4, 64, 1100, 0, 0),
                                                      (8, 128, 8300, 0, 0), (4, 64, 8300, 0, 0)])
def test_attn_decode_matches_oracle(gpu_ctx, bits, hd, seq, window, sinks):
    print(f"attn_decode bits={bits} hd={hd} seq={seq} window={window}", flush=True)
    rng = np.random.default_rng(seq + hd + bits)
    nq, nkv = 4, 2
    cap = seq if window == 0 else 40  # ring = cap - sinks slots
    kq, ks, vq, vs = _cache(rng, bits, nkv, cap, hd, min(seq, cap))
    q = rng.standard_normal((nq, hd)).astype(np.float32)
    scale = 1.0 / np.sqrt(hd)
    out = torch.zeros((nq, hd), dtype=torch.float32, device="cuda")
    dev = lambda a: torch.from_numpy(np.ascontiguousarray(a)).cuda()  # noqa: E731
    gpu_ctx.attn_decode(bits, dev(q), nq, nkv, hd, dev(kq), dev(ks.view(np.int16) if bits == 4 else ks), dev(vq),
                        dev(vs.view(np.int16) if bits == 4 else vs), cap, seq, scale, out, window, sinks)
    got = out.cpu().numpy()
    ring = cap - sinks
    if window and seq > window:
        pos = list(range(sinks)) + list(range(seq - (window - sinks), seq))
    else:
        pos = list(range(seq))
    slots = [p if (not window or p < sinks) else sinks + (p - sinks) % ring for p in pos]
    for h in range(nq):
        kv = h // (nq // nkv)
        if bits == 8:
            want = O.attn_q8_head(q[h], kq[kv, slots], ks[kv, slots], vq[kv, slots], vs[kv, slots], scale,
                                  window=bool(window))
        else:
            want = O.attn_q4_head(q[h], kq[kv, slots], ks[kv, slots], vq[kv, slots], vs[kv, slots], scale)
        assert np.abs(got[h] - want).max() <= 1e-4 * np.abs(want).max(), (h, np.abs(got[h] - want).max())


# Grouped queries at long context: k2t_attn_decode runs the model's grouped-query kernel
# (span workgroups per (KV head, 128 positions) scoring all G q heads of the group, merge
# workgroups polling the span words in the same launch).  The config-5 shape (32 q / 4 KV
# heads, hd 128: G = 8) at the bench's context 6600 (52 spans), G = 4 at 2000 and G = 8 at
# hd 64; two calls per case (the words' epoch advances between launches).
@pytest.mark.parametrize("nq,nkv,hd,seq", [(32, 4, 128, 6600), (16, 4, 64, 2000), (32, 4, 64, 3000)])
def test_attn_decode_grouped_queries_matches_oracle(gpu_ctx, nq, nkv, hd, seq):
    print(f"attn_decode grouped queries nq={nq} nkv={nkv} hd={hd} seq={seq}", flush=True)
    rng = np.random.default_rng(seq + nq)
    kq, ks, vq, vs = _cache(rng, 8, nkv, seq, hd, seq)
    dev = lambda a: torch.from_numpy(np.ascontiguousarray(a)).cuda()  # noqa: E731
    dk, dks, dv, dvs = dev(kq), dev(ks), dev(vq), dev(vs)
    scale = 1.0 / np.sqrt(hd)
    for call in range(2):
        q = rng.standard_normal((nq, hd)).astype(np.float32)
        out = torch.full((nq, hd), float("nan"), dtype=torch.float32, device="cuda")
        gpu_ctx.attn_decode(8, dev(q), nq, nkv, hd, dk, dks, dv, dvs, seq, seq - call, scale, out)
        gpu_ctx.sync()
        got = out.cpu().numpy()
        n = seq - call
        for h in range(nq):
            kv = h // (nq // nkv)
            want = O.attn_q8_head(q[h], kq[kv, :n], ks[kv, :n], vq[kv, :n], vs[kv, :n], scale)
            err = np.abs(got[h] - want).max()
            assert err <= 1e-4 * np.abs(want).max(), (call, h, err, np.abs(want).max())


@pytest.mark.parametrize("window", [0, 16])
def test_nf4_kv_model_matches_oracle(gpu_ctx, window):
    """set_kv_bits(4): the engine stores and reads the NF4 Hadamard KV cache; decode vs the
    oracle's NF4 cache (with the sliding-window ring when window > 0)."""
    print(f"nf4 kv model window={window}", flush=True)
    cfg = dict(n_layers=2, hidden=256, n_heads=4, n_kv_heads=2, head_dim=64, intermediate=256, vocab=300,
               max_seq=600, rms_eps=1e-5, rope_theta=10000.0)
    layers, head, fn = random_model(cfg, seed=31, fmt="nf4")
    ref = OracleModel(cfg, layers, head, fn, window=window, sinks=4, kv_bits=4)
    gm = k2t.Model(gpu_ctx, cfg, max_batch=16)
    mats = []
    up = lambda m: gpu_ctx.upload_nf(m.rows, m.cols, 4, m.sgc, m.cb, m.pair, m.tail)  # noqa: E731
    for i, L in enumerate(layers):
        qm, om, gu, dn = (up(L[k]) for k in ("qkv", "o", "gu", "down"))
        mats += [qm, om, gu, dn]
        gm.set_layer(i, qm, om, gu, dn, L["in_norm"], L["post_norm"])
    hm = up(head)
    gm.set_head(hm, fn)
    gm.set_kv_bits(4)
    if window:
        gm.set_kv_window(window, 4)
    assert gm.kv_bits() == 4 and not gm.persistent_active()  # the window keeps the bit width
    assert gm.kv_window() == ((window, 4) if window else (0, 0))
    toks = np.random.default_rng(32).integers(0, cfg["vocab"], 40)
    gm.prefill(toks[:-3], want_logits=False)
    for t in toks[:-3]:
        ref.forward_token(int(t))
    for t in toks[-3:]:
        a, b = gm.decode(int(t)), ref.forward_token(int(t))
        cos = float(np.dot(a, b) / (np.linalg.norm(a) * np.linalg.norm(b)))
        rel = float(np.abs(a - b).max() / np.abs(b).max())
        assert cos > 0.9999 and rel <= 2e-2, (cos, rel)
    gm.close()
    for m in mats + [hm]:
        m.close()


def _tiny_nf4_model(gpu_ctx, cfg, seed, max_batch):
    layers, head, fn = random_model(cfg, seed=seed, fmt="nf4")
    gm = k2t.Model(gpu_ctx, cfg, max_batch=max_batch)
    mats = []
    up = lambda m: gpu_ctx.upload_nf(m.rows, m.cols, 4, m.sgc, m.cb, m.pair, m.tail)  # noqa: E731
    for i, L in enumerate(layers):
        qm, om, gu, dn = (up(L[k]) for k in ("qkv", "o", "gu", "down"))
        mats += [qm, om, gu, dn]
        gm.set_layer(i, qm, om, gu, dn, L["in_norm"], L["post_norm"])
    hm = up(head)
    gm.set_head(hm, fn)
    return gm, mats + [hm]


def _mk_bf16(n, seed, scale):
    """The reference test's weight generator (real_llm.rs:10500-10511): SplitMix64 of
    i + seed * 0x9E3779B97F4A7C15, top 24 bits -> u in [0, 1), (2u - 1) * scale, BF16."""
    M = (1 << 64) - 1
    i = np.arange(n, dtype=np.uint64)
    z = (i + np.uint64((seed * 0x9E3779B97F4A7C15) & M)) & np.uint64(M)
    z = ((z ^ (z >> np.uint64(30))) * np.uint64(0xBF58476D1CE4E5B9)) & np.uint64(M)
    z = ((z ^ (z >> np.uint64(27))) * np.uint64(0x94D049BB133111EB)) & np.uint64(M)
    z = z ^ (z >> np.uint64(31))
    u = (z >> np.uint64(40)).astype(np.float32) / np.float32(1 << 24)
    v = ((np.float32(2.0) * u - np.float32(1.0)) * np.float32(scale)).astype(np.float32)
    b = v.view(np.uint32)
    b16 = ((b + np.uint32(0x7FFF) + ((b >> np.uint32(16)) & np.uint32(1))) >> np.uint32(16)).astype(np.uint16)
    return b16


def test_reference_kv_invariants(gpu_ctx):
    """The reference's own KV test (real_llm.rs:10480-10625) on the GPU engine, with its
    model: vocab 192, hidden 256, 2 layers, 2 heads / 1 KV head of 128, ffn 512, weights
    from its generator (uniform, BF16; untied BF16 embedding and lm_head), compiled here
    with the NF4 g128 RTN compiler (the reference uses GPTQ).  Its bars: Q4-KV vs Q8-KV
    prefill logits cosine > 0.998; with Q4 KV and a 16-token window with 4 sinks, a
    640-token batched prefill (past the 528-slot ring) equals token-by-token decode at
    cosine > 0.9999."""
    print("reference kv invariants", flush=True)
    V, h, inter, nl, kvd = 192, 256, 512, 2, 128
    cfg = dict(n_layers=nl, hidden=h, n_heads=2, n_kv_heads=1, head_dim=128, intermediate=inter, vocab=V,
               max_seq=1024, rms_eps=1e-5, rope_theta=100000.0)
    f32 = lambda b16: (b16.astype(np.uint32) << 16).view(np.float32)  # noqa: E731
    gm = k2t.Model(gpu_ctx, cfg, max_batch=64)
    mats = []

    def nf4(W, gu=False):
        cb, _, pair, tail = k2t.compile_nf4(np.ascontiguousarray(W, np.float32), 2, interleave_gate_up=gu)
        m = gpu_ctx.upload_nf(W.shape[0], W.shape[1], 4, 2, cb, pair, tail)
        mats.append(m)
        return m

    for l in range(nl):
        q = f32(_mk_bf16(h * h, 13 + l, 0.08)).reshape(h, h)
        k = f32(_mk_bf16(kvd * h, 17 + l, 0.08)).reshape(kvd, h)
        v = f32(_mk_bf16(kvd * h, 19 + l, 0.08)).reshape(kvd, h)
        o = f32(_mk_bf16(h * h, 41 + l, 0.08)).reshape(h, h)
        g = f32(_mk_bf16(inter * h, 43 + l, 0.08)).reshape(inter, h)
        u = f32(_mk_bf16(inter * h, 47 + l, 0.08)).reshape(inter, h)
        d = f32(_mk_bf16(h * inter, 53 + l, 0.055)).reshape(h, inter)
        gm.set_layer(l, nf4(np.concatenate([q, k, v])), nf4(o), nf4(np.concatenate([g, u]), gu=True), nf4(d),
                     f32(_mk_bf16(h, 7 + l, 1.0)), f32(_mk_bf16(h, 11 + l, 1.0)))
    gm.set_embedding(k2t.EMBED_BF16, _mk_bf16(V * h, 31, 0.4))
    gm.set_head(nf4(f32(_mk_bf16(V * h, 61, 0.3)).reshape(V, h)), f32(_mk_bf16(h, 59, 1.0)))
    cos = lambda a, b: float(np.dot(a.astype(np.float64), b) / (np.linalg.norm(a) * np.linalg.norm(b)))  # noqa: E731
    prompt = np.array([(i * 11 + 3) % V for i in range(24)], np.int32)
    gm.set_kv_bits(8)
    l8 = gm.prefill(prompt)
    gm.set_kv_bits(4)
    l4 = gm.prefill(prompt)
    assert cos(l8, l4) > 0.998, cos(l8, l4)
    long_seq = np.array([(i * 13 + 5) % V for i in range(640)], np.int32)
    gm.set_kv_window(16, 4)
    lb = gm.prefill(long_seq)
    gm.set_kv_window(16, 4)  # resets the position
    for t in long_seq:
        ls = gm.decode(int(t))
    assert cos(lb, ls) > 0.9999, cos(lb, ls)
    gm.close()
    for m in mats:
        m.close()


@pytest.mark.parametrize("hd", [64, 128])
def test_reference_q8_kv_attention_accuracy(gpu_ctx, hd):
    """test_hadamard_q8_kv_cache_attention_accuracy (real_llm.rs:10190-10284) with its own
    inputs: 6 q heads over 2 KV heads, K/V/q from f(i, m) = ((i*m % 101)/101 - 0.5)*1.6 with
    columns 7 and hd/2 + 7 scaled x12, 37 cached positions; the GPU's Hadamard int8 store
    + decode attention against fp32 attention on the unquantized K/V at cosine > 0.9998
    (the reference's bar) for pos 0, 7, 15, 36."""
    heads, kvh, n_max = 6, 2, 37
    kv_dim = kvh * hd
    scale = 1.0 / np.sqrt(np.float32(hd))

    def f(i, m):
        i = np.asarray(i, np.int64)
        base = ((i * m % 101).astype(np.float32) / np.float32(101.0) - np.float32(0.5)) * np.float32(1.6)
        col = i % hd
        return np.where((col == 7) | (col == hd // 2 + 7), base * np.float32(12.0), base).astype(np.float32)

    k_all = f(np.arange(n_max * kv_dim), 19).reshape(n_max, kvh, hd)
    v_all = f(np.arange(n_max * kv_dim), 29).reshape(n_max, kvh, hd)
    # cache layout [kv head][slot]: store each head's 37 rows
    dev = lambda a: torch.from_numpy(np.ascontiguousarray(a)).cuda()  # noqa: E731
    kq = torch.zeros((kvh, n_max, hd), dtype=torch.int8, device="cuda")
    vq = torch.zeros((kvh, n_max, hd), dtype=torch.int8, device="cuda")
    ks = torch.zeros((kvh, n_max), dtype=torch.float32, device="cuda")
    vs = torch.zeros((kvh, n_max), dtype=torch.float32, device="cuda")
    for h in range(kvh):
        gpu_ctx.kv_store(8, dev(k_all[:, h]), n_max, hd, kq[h], ks[h])
        gpu_ctx.kv_store(8, dev(v_all[:, h]), n_max, hd, vq[h], vs[h])
    out = torch.zeros((heads, hd), dtype=torch.float32, device="cuda")
    for pos in (0, 7, 15, 36):
        q = f(np.arange(heads * hd) + pos * 13, 37).reshape(heads, hd)
        gpu_ctx.attn_decode(8, dev(q), heads, kvh, hd, kq, ks, vq, vs, n_max, pos + 1, float(scale), out)
        got = out.cpu().numpy().astype(np.float64).ravel()
        want = np.zeros((heads, hd))
        for h in range(heads):
            g = h // (heads // kvh)
            K, V = k_all[:pos + 1, g].astype(np.float64), v_all[:pos + 1, g].astype(np.float64)
            z = K @ q[h].astype(np.float64) * float(scale)
            p = np.exp(z - z.max())
            want[h] = (p / p.sum()) @ V
        cos = float(np.dot(got, want.ravel()) / (np.linalg.norm(got) * np.linalg.norm(want)))
        assert cos > 0.99980, (hd, pos, cos)
