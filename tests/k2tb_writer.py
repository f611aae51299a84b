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
