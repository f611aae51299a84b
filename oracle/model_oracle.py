"""CPU restatement of the decode megakernel (forward_token_sdot_megakernel,
real_llm.rs:6794-7403) built from the C oracle's primitives.

TEST INFRASTRUCTURE ONLY (imported by tests/ and the smoke check, never by the
product).  Per layer, in the reference's order:
  1. inv_rms + RMSNorm*w + FWHT + int8 (6929-6950), qkv GEMV (6957-6977), bias, RoPE on q
     and k heads, Hadamard int8 store of k and v (6990-7021);
  2. q8 attention per query head (causal_gqa_group_q8, 8471-8594) -> ifwht -> FWHT with
     chunk index qh*cph+sub -> int8 (7060-7084);
  3. o_proj GEMV, hidden += proj (7163-7189);
  4. post-attention norm -> interleaved gate_up GEMV -> SwiGLU -> FWHT (chunk ic) -> int8
     (7207-7296);
  5. down GEMV, hidden += (7308-7333);
then final norm -> lm_head GEMV (7338-7391).  The embedding is the tied quantized
head's row, dequantized and inverse-rotated (embed_token_into, 8063-8097), unless an
untied embedding function is given (f32 / bf16 rows, NF4 matrix: 8073-8090).
"""
import numpy as np

import oracle as O


_POOLS = {}


def _pool(n):
    """A persistent host thread pool per width (the C calls release the GIL)."""
    if n not in _POOLS:
        import concurrent.futures as cf
        _POOLS[n] = cf.ThreadPoolExecutor(max_workers=n)
    return _POOLS[n]


class Matrix:
    """A quantized matrix in the reference's stream layout."""

    def __init__(self, fmt, rows, cols, pair, tail, hp=0, cb=None, sgc=2):
        self.fmt, self.rows, self.cols, self.pair, self.tail = fmt, rows, cols, pair, tail
        self.hp, self.cb, self.sgc = hp, cb, sgc

    def gemv(self, xq, xs, xsum, threads=1):
        """Integer-exact path (simd_lut.rs:3766-4091 / 6074-6364).  With threads > 1 the
        stripe range is split over host threads; each output row is computed by exactly
        one call, so the result does not depend on the split."""
        def run(s0, s1):
            if self.fmt == "n4":
                return O.nibble4_gemv(self.pair, self.tail, self.rows, self.cols, self.hp, xq, xs, xsum, s0=s0,
                                      s1=s1)
            return O.nf_gemv(self.pair, self.tail, self.rows, self.cols, 4, self.sgc, self.cb, xq, xs, s0=s0, s1=s1)

        stripes = (self.rows + 15) // 16
        if threads <= 1 or stripes < 4:
            return run(0, stripes)
        out = np.zeros(self.rows, np.float32)
        per = max(2, ((stripes + threads - 1) // threads + 1) & ~1)

        def work(s0, s1):
            out[s0 * 16:min(s1 * 16, self.rows)] = run(s0, s1)[s0 * 16:min(s1 * 16, self.rows)]

        list(_pool(threads).map(lambda a: work(a, min(stripes, a + per)), range(0, stripes, per)))
        return out

    def gemv_portable(self, xq, xs, threads=1):
        """Portable path (simd_lut.rs:3558-3581 / 5719-5748), stripe ranges over host threads
        like the reference's pool (real_llm.rs:829-836)."""
        import threading
        stripes = (self.rows + 15) // 16
        out = np.zeros(self.rows, np.float32)
        per = max(2, ((stripes + threads - 1) // threads + 1) & ~1)

        def work(s0, s1):
            if self.fmt == "n4":
                o = O.nibble4_gemv_portable(self.pair, self.tail, self.rows, self.cols, self.hp, xq, xs, s0, s1)
            else:
                o = O.nf_gemv_portable(self.pair, self.tail, self.rows, self.cols, 4, self.sgc, self.cb, xq, xs,
                                       s0, s1)
            out[s0 * 16:min(s1 * 16, self.rows)] = o[s0 * 16:min(s1 * 16, self.rows)]

        ths = [threading.Thread(target=work, args=(a, min(stripes, a + per))) for a in range(0, stripes, per)]
        for t in ths:
            t.start()
        for t in ths:
            t.join()
        return out

    def row_rotated(self, r):
        if self.fmt == "n4":
            return O.nibble4_dequant_row(self.pair, self.tail, self.rows, self.cols, self.hp, r)
        return O.nf_dequant_row(self.pair, self.tail, self.rows, self.cols, 4, self.sgc, self.cb, r)


def quantize_matrix(W, fmt, planes=4, sgc=2, interleave_gate_up=False):
    """Oracle quantizers: Hadamard RTN bit planes (compiler.rs:992-1107 + repack) or NF4."""
    rows, cols = W.shape
    if fmt == "n4":
        u, sc = O.bipolar_rtn(W, planes)
        pair, tail = O.nibble4_repack(O.pack_interleaved(u, planes), sc, rows, cols, planes, interleave_gate_up)
        return Matrix("n4", rows, cols, pair, tail, hp=planes - 4)
    cb, mu = O.nf_fit_codebook(W, 4, sgc)
    idx, sc = O.nf_rtn(W, 4, sgc, cb, mu)
    if interleave_gate_up:
        inter = rows // 2
        perm = [(b // 2) * 64 + o + (inter if b % 2 else 0) for b in range(rows // 64) for o in range(64)]
        nsg = (cols // 64 + sgc - 1) // sgc
        s3 = np.stack([sc.reshape(-1, nsg, 16)[r // 16, :, r % 16] for r in range(rows)])[perm]
        idx = idx[perm]
        sc = np.stack([s3[s * 16:(s + 1) * 16].T for s in range(rows // 16)]).ravel()
    pair, tail = O.nf_from_indices(idx, sc, rows, cols, 4, sgc)
    return Matrix("nf4", rows, cols, pair, tail, cb=cb, sgc=sgc)


class OracleModel:
    """`gemv_threads` > 0 switches every projection to the threaded portable path (the
    timed CPU baseline); 0 keeps the NEON-semantics integer path (the parity oracle)."""

    def __init__(self, cfg, layers, head, final_norm, gemv_threads=0, embed=None, window=0, sinks=0, kv_bits=8,
                 parity_threads=1, rms_order="x86"):
        self.gemv_threads = gemv_threads
        # sum-of-squares order of the hidden-state norms: "x86" or "neon", the reference's
        # two builds (real_llm.rs:903-962); everything else is the same arithmetic
        self.rms_order = rms_order
        self.parity_threads = parity_threads  # host threads for the integer-exact GEMVs
        self.embed_fn = embed  # untied embedding: token -> f32[hidden] (embed_token_into)
        self.cfg = cfg
        self.layers = layers  # dicts: qkv, o, gu, down (Matrix), in_norm, post_norm, bias
        self.head = head
        self.final_norm = final_norm
        L, nkv, hd, cap = cfg["n_layers"], cfg["n_kv_heads"], cfg["head_dim"], cfg["max_seq"]
        # QuantizedKvCache::new_with_opts (real_llm.rs:1235-1257): sliding-window ring
        self.window = self.sinks = self.ring = 0
        if window >= 8 and window + 512 < cap:
            self.window, self.sinks = window, min(sinks, window // 2)
            self.ring = (window - self.sinks) + 512
            cap = self.sinks + self.ring
        self.kv_bits = kv_bits
        if kv_bits == 4:  # NF4 nibbles + BF16 block scales (QuantizedKvCache bits 4)
            self.k4 = np.full((L, nkv, cap, hd // 2), 0x88, np.uint8)
            self.v4 = np.full((L, nkv, cap, hd // 2), 0x88, np.uint8)
            self.ks16 = np.zeros((L, nkv, cap, hd // 64), np.uint16)
            self.vs16 = np.zeros((L, nkv, cap, hd // 64), np.uint16)
        self.kq = np.zeros((L, nkv, cap, hd), np.int8)
        self.vq = np.zeros((L, nkv, cap, hd), np.int8)
        self.ks = np.zeros((L, nkv, cap), np.float32)
        self.vs = np.zeros((L, nkv, cap), np.float32)
        self.pos = 0

    def seed_kv(self, n_pos, seed=0):
        """Fills cache positions 0 .. n_pos-1 with seeded random int8 K/V and scales and
        sets the position, so that a timed step attends n_pos + 1 positions without a
        prefill (the values only matter for timing)."""
        rng = np.random.default_rng(seed)
        L, nkv = self.kq.shape[0], self.kq.shape[1]
        hd = self.kq.shape[3]
        self.kq[:, :, :n_pos] = rng.integers(-127, 128, (L, nkv, n_pos, hd), dtype=np.int8)
        self.vq[:, :, :n_pos] = rng.integers(-127, 128, (L, nkv, n_pos, hd), dtype=np.int8)
        self.ks[:, :, :n_pos] = rng.uniform(0.005, 0.05, (L, nkv, n_pos)).astype(np.float32)
        self.vs[:, :, :n_pos] = rng.uniform(0.005, 0.05, (L, nkv, n_pos)).astype(np.float32)
        self.pos = n_pos

    def _gemv(self, m, xq, xs, xsum):
        if self.gemv_threads:
            return m.gemv_portable(xq, xs, self.gemv_threads)
        return m.gemv(xq, xs, xsum, self.parity_threads)

    def slot_of_pos(self, pos):
        """real_llm.rs:1116-1122"""
        if self.ring == 0 or pos < self.sinks:
            return pos
        return self.sinks + (pos - self.sinks) % self.ring

    def active_slots(self, seq):
        """active_kv_len / active_kv_pos (real_llm.rs:8596-8612) mapped to cache slots."""
        if self.window > 0 and seq > self.window:
            pos = list(range(self.sinks)) + list(range(seq - (self.window - self.sinks), seq))
        else:
            pos = list(range(seq))
        return [self.slot_of_pos(p) for p in pos]

    def embed(self, token):
        if self.embed_fn is not None:
            return self.embed_fn(token)
        return O.ifwht64(self.head.row_rotated(token))

    def forward_token(self, token, want_logits=True):
        """One decode step; want_logits=False stops after the last layer (a prefill
        token whose logits nobody reads; the KV cache and position advance the same)."""
        c = self.cfg
        d, nq, nkv, hd, inter, eps = c["hidden"], c["n_heads"], c["n_kv_heads"], c["head_dim"], c["intermediate"], \
            c["rms_eps"]
        pos = self.pos
        rope = O.rope_row(hd, float(np.float32(c["rope_theta"])), pos)
        scale = np.float32(1.0) / np.sqrt(np.float32(hd))
        hidden = self.embed(token).astype(np.float32)
        self.last_routes = []
        for li, L in enumerate(self.layers):
            xq, xs, xsum = O.populate_fwht(hidden, L["in_norm"], O.inv_rms(hidden, eps, self.rms_order))
            qkv = self._gemv(L["qkv"], xq, xs, xsum).reshape(-1, hd)
            if L.get("bias") is not None:
                qkv = (qkv + L["bias"].reshape(-1, hd)).astype(np.float32)
            # per-head q / k RMSNorm before RoPE (apply_qk_norm_rope, 8139-8178); hd is a
            # power of two, so sum*(1/hd) equals the mean or_inv_rms forms
            for h in range(nq + nkv):
                wn = L.get("q_norm") if h < nq else L.get("k_norm")
                if wn is not None:
                    qkv[h] = ((qkv[h] * np.float32(O.inv_rms(qkv[h], eps))) * wn).astype(np.float32)
            for h in range(nq + nkv):
                qkv[h] = O.rope_apply(qkv[h], rope)
            sl = self.slot_of_pos(pos)
            for kvh in range(nkv):
                if self.kv_bits == 4:
                    self.k4[li, kvh, sl], self.ks16[li, kvh, sl] = O.kv_quant_head_q4(qkv[nq + kvh])
                    self.v4[li, kvh, sl], self.vs16[li, kvh, sl] = O.kv_quant_head_q4(qkv[nq + nkv + kvh])
                else:
                    self.kq[li, kvh, sl], self.ks[li, kvh, sl] = O.kv_quant_head(qkv[nq + kvh])
                    self.vq[li, kvh, sl], self.vs[li, kvh, sl] = O.kv_quant_head(qkv[nq + nkv + kvh])
            group = nq // nkv
            outs = []
            act = self.active_slots(pos + 1)
            for qh in range(nq):
                kvh = qh // group
                if self.kv_bits == 4:
                    outs.append(O.attn_q4_head(qkv[qh], self.k4[li, kvh, act], self.ks16[li, kvh, act],
                                               self.v4[li, kvh, act], self.vs16[li, kvh, act], scale))
                elif self.window:
                    outs.append(O.attn_q8_head(qkv[qh], self.kq[li, kvh, act], self.ks[li, kvh, act],
                                               self.vq[li, kvh, act], self.vs[li, kvh, act], scale, window=True))
                else:
                    outs.append(O.attn_q8_head(qkv[qh], self.kq[li, kvh, :pos + 1], self.ks[li, kvh, :pos + 1],
                                               self.vq[li, kvh, :pos + 1], self.vs[li, kvh, :pos + 1], scale))
            aq, as_, asum = O.populate_fwht(np.concatenate(outs))
            hidden = (hidden + self._gemv(L["o"], aq, as_, asum)).astype(np.float32)
            if L.get("moe") is not None:
                hidden, routes = moe_ffn(hidden, L["post_norm"], eps, L["moe"])
                self.last_routes.append(routes)
                continue
            xq, xs, xsum = O.populate_fwht(hidden, L["post_norm"], O.inv_rms(hidden, eps, self.rms_order))
            gu = self._gemv(L["gu"], xq, xs, xsum).reshape(-1, 128)
            sw = np.concatenate([O.swiglu(gu[ic, :64], gu[ic, 64:]) for ic in range(inter // 64)])
            iq, is_, isum = O.populate_fwht(sw)
            hidden = (hidden + self._gemv(L["down"], iq, is_, isum)).astype(np.float32)
        self.pos += 1
        if not want_logits:
            return None
        xq, xs, xsum = O.populate_fwht(hidden, self.final_norm, O.inv_rms(hidden, eps, self.rms_order))
        return self._gemv(self.head, xq, xs, xsum)


# ------------------------------------------------------------------ sparse MoE
SOFTMAX, TOPK_SOFTMAX, SIGMOID = 0, 1, 2


def route_sorted(logits, top_k, norm_topk_prob, scoring):
    """DenseMoeRouter::route_sorted after the logits (sparse_moe.rs:86-182) in float32, the
    x86 build's order: scoring with the platform expf (O.expf) and sequential sums,
    select_topk_by_score (strict '>' insertion, 185-206), renormalization in selection
    order, then sort by ascending expert id."""
    z = np.asarray(logits, np.float32).copy()
    E = z.size
    k = min(top_k, E)
    f32 = np.float32
    if scoring == SOFTMAX:
        m = z.max()
        s = f32(0.0)
        for e in range(E):
            z[e] = O.expf(f32(z[e] - m))[0]
            s = f32(s + z[e])
        inv = f32(1.0) / s if s > 0 else f32(1.0) / f32(E)
        z = (z * inv).astype(np.float32)
    elif scoring == SIGMOID:
        z = (f32(1.0) / (f32(1.0) + O.expf(-z))).astype(np.float32)
    out = []
    for e in range(E):
        v = z[e]
        if len(out) < k:
            pos = len(out)
            while pos > 0 and v > out[pos - 1][1]:
                pos -= 1
            out.insert(pos, (e, v))
        elif v > out[k - 1][1]:
            pos = k - 1
            while pos > 0 and v > out[pos - 1][1]:
                pos -= 1
            out.insert(pos, (e, v))
            out.pop()
    if scoring == TOPK_SOFTMAX:
        mz = max(w for _, w in out)
        ws = [O.expf(f32(w - mz))[0] for _, w in out]
        s = f32(0.0)
        for w in ws:
            s = f32(s + w)
        inv = f32(1.0) / s if s > 0 else f32(1.0) / f32(k)
        out = [(e, f32(w * inv)) for (e, _), w in zip(out, ws)]
    elif norm_topk_prob:
        s = f32(0.0)
        for _, w in out:
            s = f32(s + w)
        if s > 0:
            inv = f32(1.0) / s
            out = [(e, f32(w * inv)) for e, w in out]
    return sorted(out, key=lambda t: t[0])


def rms_norm(x, w, eps):
    """rms_norm (real_llm.rs:9858-9898): (x * inv_rms) * w."""
    return ((np.asarray(x, np.float32) * np.float32(O.inv_rms(x, eps))) * np.asarray(w, np.float32)).astype(np.float32)


def shared_expert(xn, aq, as_, sh):
    """SharedMoeExpert::forward_single, NF backend (sparse_moe.rs:252-312): gate_up GEMV on
    the layer's int8 activation, rows [gate; up]; SwiGLU; fwht64_signed_inplace over the
    whole inter vector then populate (= populate_fwht); down GEMV; times the gate scale
    1 / (1 + exp(-gate . x_norm)) (241-250; dot_f32_moe, sequential on x86) when it
    differs from 1 by more than f32::EPSILON.  sh: dict(gate_up, down: Matrix-like NF dicts
    with pair/tail/cb/bits/sgc/rows/cols, gate_weight [d] or None)."""
    gu, dn = sh["gate_up"], sh["down"]
    g = O.nf_gemv(gu["pair"], gu["tail"], gu["rows"], gu["cols"], gu["bits"], gu["sgc"], gu["cb"], aq, as_)
    inter = gu["rows"] // 2
    sw = O.swiglu(g[:inter], g[inter:])
    mq, ms, _ = O.populate_fwht(sw)
    out = O.nf_gemv(dn["pair"], dn["tail"], dn["rows"], dn["cols"], dn["bits"], dn["sgc"], dn["cb"], mq, ms)
    gw = sh.get("gate_weight")
    if gw is not None:
        z = np.float32(0.0)
        for a, b in zip(np.asarray(gw, np.float32), np.asarray(xn, np.float32)):
            z = np.float32(z + np.float32(a * b))
        scale = np.float32(1.0) / (np.float32(1.0) + O.expf(-z)[0])
        if abs(float(scale) - 1.0) > float(np.finfo(np.float32).eps):
            out = (out * scale).astype(np.float32)
    return out


def moe_ffn(hidden, post_norm, eps, moe):
    """forward_layer_single (sparse_moe.rs:961-1084) + the residual add (real_llm.rs:6711-6714).
    moe: dict(router_w [E][d] f32, router_b [E] or None, top_k, norm_topk_prob, scoring,
    experts: list of (gu Matrix-like dict, dn dict) with pair/cb/bits/sgc/rows/cols;
    optional shared: see shared_expert).  Returns (new hidden, routes)."""
    xn = rms_norm(hidden, post_norm, eps)
    W = np.asarray(moe["router_w"], np.float32)
    # dot_f32_moe on x86 (sparse_moe.rs:1644-1656): f32 products added in index order
    # (np.cumsum accumulates sequentially in float32)
    logits = np.cumsum((W * xn[None, :]).astype(np.float32), axis=1, dtype=np.float32)[:, -1].astype(np.float32)
    if moe.get("router_b") is not None:
        logits = (logits + moe["router_b"]).astype(np.float32)
    routes = route_sorted(logits, moe["top_k"], moe["norm_topk_prob"], moe["scoring"])
    aq, as_, _ = O.populate_fwht(xn)
    out = np.zeros(hidden.size, np.float32)
    sh = moe.get("shared")
    if sh is not None:
        out = shared_expert(xn, aq, as_, sh)
    for e, w in routes:
        gu, dn = moe["experts"][e]
        g = O.nf_gemv(gu["pair"], np.zeros(0, np.uint8), gu["rows"], gu["cols"], gu["bits"], gu["sgc"], gu["cb"],
                      aq, as_)
        dff = gu["rows"] // 2
        sw = O.swiglu(g[:dff], g[dff:])
        mq, ms, _ = O.populate_fwht(sw)
        y = O.nf_gemv(dn["pair"], np.zeros(0, np.uint8), dn["rows"], dn["cols"], dn["bits"], dn["sgc"], dn["cb"],
                      mq, ms)
        out = (out + (np.float32(w) * y).astype(np.float32)).astype(np.float32)
    return (hidden + out).astype(np.float32), routes


def random_model(cfg, seed, fmt="nf4", planes=None):
    """Random-init weights ~N(0, 0.02), norms 1 + 0.1*N(0,1); quantized by the oracle.
    `planes` maps projection -> bit planes for fmt "n4" (p55454 = qkv5/o5/gu4/down5/head4)."""
    rng = np.random.default_rng(seed)
    d, nq, nkv, hd, inter, V = cfg["hidden"], cfg["n_heads"], cfg["n_kv_heads"], cfg["head_dim"], \
        cfg["intermediate"], cfg["vocab"]
    planes = planes or {"qkv": 4, "o": 4, "gu": 4, "down": 4, "head": 4}

    def q(W, name, gu=False):
        if fmt == "n4":
            return quantize_matrix(W, "n4", planes=planes[name], interleave_gate_up=gu)
        return quantize_matrix(W, "nf4", sgc=2, interleave_gate_up=gu)

    def w(r, c_):
        return (rng.standard_normal((r, c_)) * 0.02).astype(np.float32)

    layers = []
    for _ in range(cfg["n_layers"]):
        layers.append({
            "qkv": q(w((nq + 2 * nkv) * hd, d), "qkv"),
            "o": q(w(d, nq * hd), "o"),
            "gu": q(w(2 * inter, d), "gu", gu=True),
            "down": q(w(d, inter), "down"),
            "in_norm": (1.0 + 0.1 * rng.standard_normal(d)).astype(np.float32),
            "post_norm": (1.0 + 0.1 * rng.standard_normal(d)).astype(np.float32),
            "bias": None,
        })
    head = q(w(V, d), "head")
    final_norm = (1.0 + 0.1 * rng.standard_normal(d)).astype(np.float32)
    return layers, head, final_norm
