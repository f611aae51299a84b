"""Writes .k2tb files in the byte format of RealLlamaEngine::save_bipolar
(real_llm.rs:3705-3895) from oracle-quantized matrices, so the loader can be tested
without the reference binary.

TEST INFRASTRUCTURE ONLY.  Matrices are dicts:
  {"kind": "bipolar", "rows", "cols", "planes", "inter": bytes [stripes][cols/8][planes][16],
   "scales": uint16 [stripes][nc][16]}             (FusedBipolarLutMatrix, tag 0)
  {"kind": "nf", "rows", "cols", "bits", "sgc", "cb": int8[16], "pair", "tail"}
                                                    (NfSdotMatrix, tag 2)
  {"kind": "raw_tag", "tag": t}                     (a bare tag, for error tests)
Gate_up matrices are stored un-interleaved, as save_bipolar requires.
"""
import struct

import numpy as np

import oracle as O

MAGIC = {1: b"K2TBIPOLAR1\n", 2: b"K2TKRONOS2\n", 3: b"K2TKRONOS3\n", 4: b"K2TKRONOS4\n",
         5: b"K2TKRONOS5\n", 6: b"K2TKRONOS6\n"}


def _u64(v):
    return struct.pack("<Q", int(v))


def _f32s(v):
    a = np.ascontiguousarray(v if v is not None else [], np.float32)
    return _u64(a.size) + a.tobytes()


def _matrix(m, version):
    out = b""
    if m["kind"] == "raw_tag":
        return _u64(m["tag"])
    if m["kind"] == "bipolar":
        if version >= 2:
            out += _u64(0)
        inter = np.ascontiguousarray(m["inter"], np.uint8)
        sc = np.ascontiguousarray(m["scales"], np.uint16)
        out += _u64(m["rows"]) + _u64(m["cols"]) + _u64(m["planes"])
        out += _u64(inter.size) + inter.tobytes() + _u64(sc.size) + sc.tobytes()
        return out
    assert version >= 2, "NF matrices need K2TKRONOS2 or later"
    cb = np.ascontiguousarray(m["cb"], np.int8)
    pair = np.ascontiguousarray(m["pair"], np.uint8)
    tail = np.ascontiguousarray(m["tail"], np.uint8)
    out += _u64(2) + _u64(m["rows"]) + _u64(m["cols"]) + _u64(m["bits"]) + _u64(m["sgc"])
    out += cb.tobytes() + _u64(pair.size) + pair.tobytes() + _u64(tail.size) + tail.tobytes()
    return out


def write_k2tb(path, version, layers, final_norm, head, mode_words=(5, 4, 2, 0, 0, 0), embed_f32=None,
               embed_bf16=None, embed_nf4=None):
    """layers: dicts with qkv, o, gu, down (matrix dicts), in_norm, post_norm and optional
    bias, q_norm, k_norm."""
    b = bytearray(MAGIC[version])
    for w in mode_words:
        b += _u64(w)
    b += _u64(len(layers))
    for L in layers:
        b += _f32s(L["in_norm"]) + _f32s(L["post_norm"])
        if version >= 3:
            b += _f32s(L.get("bias"))
        if version >= 6:
            b += _f32s(L.get("q_norm")) + _f32s(L.get("k_norm"))
        for k in ("qkv", "o", "gu", "down"):
            b += _matrix(L[k], version)
    b += _f32s(final_norm)
    b += _matrix(head, version)
    b += _f32s(embed_f32)
    if version >= 3:
        e = np.ascontiguousarray(embed_bf16 if embed_bf16 is not None else [], np.uint16)
        b += _u64(e.size) + e.tobytes()
    if version >= 4:
        if embed_nf4 is None:
            b += _u64(0)
        else:
            b += _u64(1) + _matrix(embed_nf4, version)
    with open(path, "wb") as f:
        f.write(bytes(b))
    return len(b)


def bipolar_source(W, planes):
    """Oracle RTN of W into the stored FusedBipolar form (u codes packed, scales)."""
    u, sc = O.bipolar_rtn(W, planes)
    rows, cols = W.shape
    return {"kind": "bipolar", "rows": rows, "cols": cols, "planes": planes,
            "inter": O.pack_interleaved(u, planes), "scales": sc}


def nf_source(W, bits=4, sgc=2):
    """Oracle NF fit + RTN of W into the stored (un-interleaved) NfSdotMatrix streams."""
    rows, cols = W.shape
    cb, mu = O.nf_fit_codebook(W, bits, sgc)
    idx, sc = O.nf_rtn(W, bits, sgc, cb, mu)
    pair, tail = O.nf_from_indices(idx, sc, rows, cols, bits, sgc)
    return {"kind": "nf", "rows": rows, "cols": cols, "bits": bits, "sgc": sgc, "cb": cb, "pair": pair, "tail": tail}


# ------------------------------------------------------------------ .k2tm shards
K2TM_PAGE = 16384
K2TM_MAGIC = b"K2TM800B_V1\0"


def _align(v, a):
    return (v + a - 1) // a * a


def expert_layout(d_model, d_ff, bits, sgc):
    """nf_expert_byte_layout (moe_800b.rs:1332-1375)."""
    chunk_b = 384 if bits == 3 else 512
    sgc = max(sgc, 1)
    gu_chunks, dn_chunks = d_model // 64, d_ff // 64
    gu_pair = (2 * d_ff // 32) * (-(-gu_chunks // sgc) * 64 + gu_chunks * 2 * chunk_b)
    dn_pair = (d_model // 32) * (-(-dn_chunks // sgc) * 64 + dn_chunks * 2 * chunk_b)
    dn_off = _align(64 + gu_pair, 64)
    return dict(gu_cb=0, dn_cb=16, gu_off=64, gu_bytes=gu_pair, dn_off=dn_off, dn_bytes=dn_pair,
                aligned=_align(dn_off + dn_pair, K2TM_PAGE))


def write_k2tm(experts, d_model, d_ff, bits, sgc):
    """K2tmShardHeader page + pack_nf_expert_record per expert (moe_800b.rs:792-854,
    1377-1404).  experts[layer][e] = (gu nf_source dict, dn nf_source dict).  Returns bytes."""
    L = expert_layout(d_model, d_ff, bits, sgc)
    n_layers, E = len(experts), len(experts[0])
    buf = bytearray(K2TM_PAGE + n_layers * E * L["aligned"])
    buf[0:12] = K2TM_MAGIC
    for i, w in enumerate((n_layers, E, d_model, d_ff, sgc, L["aligned"], bits)):
        buf[16 + 8 * i:24 + 8 * i] = struct.pack("<Q", w)
    for li, layer in enumerate(experts):
        for e, (gu, dn) in enumerate(layer):
            assert gu["tail"].size == 0 and dn["tail"].size == 0
            assert gu["pair"].size == L["gu_bytes"] and dn["pair"].size == L["dn_bytes"]
            base = K2TM_PAGE + (li * E + e) * L["aligned"]
            buf[base + L["gu_cb"]:base + L["gu_cb"] + 16] = np.asarray(gu["cb"], np.int8).tobytes()
            buf[base + L["dn_cb"]:base + L["dn_cb"] + 16] = np.asarray(dn["cb"], np.int8).tobytes()
            buf[base + L["gu_off"]:base + L["gu_off"] + L["gu_bytes"]] = gu["pair"].tobytes()
            buf[base + L["dn_off"]:base + L["dn_off"] + L["dn_bytes"]] = dn["pair"].tobytes()
    return bytes(buf)


def random_moe_layer(rng, d_model, d_ff, E, bits=3, sgc=2):
    """One layer's experts: gate_up = [gate; up] rows (2*d_ff x d_model) and down
    (d_model x d_ff), ~N(0, 0.02), NF-quantized by the oracle; plus an fp32 router."""
    experts = []
    for _ in range(E):
        Wgu = (rng.standard_normal((2 * d_ff, d_model)) * 0.02).astype(np.float32)
        Wdn = (rng.standard_normal((d_model, d_ff)) * 0.02).astype(np.float32)
        experts.append((nf_source(Wgu, bits, sgc), nf_source(Wdn, bits, sgc)))
    router = (rng.standard_normal((E, d_model)) * 0.05).astype(np.float32)
    return experts, router
