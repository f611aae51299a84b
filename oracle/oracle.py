"""ctypes view of the CPU oracle (oracle/k2t_oracle.c).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and the
cpu_baseline leg of bench.py, never by the product library.  Each wrapper
names the reference file:line restated by the C function it calls.
"""
import ctypes as C
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "libk2t_oracle.so")
_lib = None

F32P = np.ctypeslib.ndpointer(np.float32, flags="C_CONTIGUOUS")
I8P = np.ctypeslib.ndpointer(np.int8, flags="C_CONTIGUOUS")
U8P = np.ctypeslib.ndpointer(np.uint8, flags="C_CONTIGUOUS")
U16P = np.ctypeslib.ndpointer(np.uint16, flags="C_CONTIGUOUS")
I32P = np.ctypeslib.ndpointer(np.int32, flags="C_CONTIGUOUS")
SZ = C.c_size_t
VP = C.c_void_p


def build():
    """Compile the oracle with its Makefile (gcc, -ffp-contract=off)."""
    subprocess.run(["make", "-s", "-C", _HERE, "libk2t_oracle.so"], check=True)


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        L = C.CDLL(_LIB_PATH)
        sig = {
            "or_sign_bits": (C.c_uint64, [C.c_uint64]),
            "or_fwht64_block": (None, [F32P, C.c_uint64]),
            "or_ifwht64_block": (None, [F32P, C.c_uint64]),
            "or_fwht64": (None, [F32P, SZ]),
            "or_ifwht64": (None, [F32P, SZ]),
            "or_f32_to_bf16": (C.c_uint16, [C.c_float]),
            "or_populate_fwht": (None, [F32P, VP, C.c_float, SZ, I8P, F32P, I32P]),
            "or_populate_plain": (None, [F32P, SZ, I8P, F32P, I32P]),
            "or_inv_rms": (C.c_float, [F32P, SZ, C.c_float]),
            "or_inv_rms_neon": (C.c_float, [F32P, SZ, C.c_float]),
            "or_bipolar_rtn": (None, [F32P, SZ, SZ, C.c_int, U8P, U16P]),
            "or_pack_interleaved": (None, [U8P, SZ, SZ, C.c_int, U8P]),
            "or_nibble4_repack": (None, [U8P, U16P, SZ, SZ, C.c_int, C.c_int, U8P, U8P]),
            "or_nibble4_dequant_row": (None, [U8P, U8P, SZ, SZ, C.c_int, SZ, F32P]),
            "or_nibble4_row_codes": (None, [U8P, U8P, SZ, SZ, C.c_int, SZ, U8P]),
            "or_nibble4_gemv": (None, [U8P, U8P, SZ, SZ, C.c_int, I8P, F32P, I32P, SZ, SZ, F32P, VP]),
            "or_nibble4_gemv_portable": (None, [U8P, U8P, SZ, SZ, C.c_int, I8P, F32P, SZ, SZ, F32P]),
            "or_nf_fit_codebook": (C.c_float, [F32P, SZ, SZ, C.c_int, SZ, I8P]),
            "or_nf_rtn": (None, [F32P, SZ, SZ, C.c_int, SZ, I8P, C.c_float, U8P, U16P]),
            "or_nf_from_indices": (None, [U8P, U16P, SZ, SZ, C.c_int, SZ, U8P, U8P]),
            "or_nf_row_indices": (None, [U8P, U8P, SZ, SZ, C.c_int, SZ, SZ, U8P]),
            "or_nf_dequant_row": (None, [U8P, U8P, SZ, SZ, C.c_int, SZ, I8P, SZ, F32P]),
            "or_nf_gemv": (None, [U8P, U8P, SZ, SZ, C.c_int, SZ, I8P, I8P, F32P, SZ, SZ, F32P, VP]),
            "or_nf_gemv_portable": (None, [U8P, U8P, SZ, SZ, C.c_int, SZ, I8P, I8P, F32P, SZ, SZ, F32P]),
            "or_nf_pair_total": (SZ, [SZ, C.c_int, SZ]),
            "or_nf_tail_total": (SZ, [SZ, C.c_int, SZ]),
            "or_kv_quant_head": (None, [F32P, SZ, I8P, F32P]),
            "or_attn_q8_head": (None, [F32P, I8P, F32P, I8P, F32P, SZ, SZ, C.c_float, F32P, F32P]),
            "or_attn_q8_head_window": (None, [F32P, I8P, F32P, I8P, F32P, SZ, SZ, C.c_float, F32P, F32P]),
            "or_nf4_nearest_idx": (C.c_int, [C.c_float]),
            "or_kv_quant_head_q4": (None, [F32P, SZ, U8P, U16P]),
            "or_attn_q4_head": (None, [F32P, U8P, U16P, U8P, U16P, SZ, SZ, C.c_float, F32P, F32P]),
            "or_rope_row": (None, [SZ, C.c_double, SZ, F32P]),
            "or_rope_apply": (None, [F32P, SZ, F32P]),
            "or_swiglu": (None, [F32P, F32P, F32P, SZ]),
            "or_expf_mismatches": (C.c_uint64, [VP, C.c_uint64, C.c_uint64, C.c_int, C.POINTER(C.c_uint32)]),
            "or_expf_array": (None, [F32P, F32P, SZ]),
        }
        for name, (res, args) in sig.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def _ptr(a):
    return None if a is None else a.ctypes.data_as(VP)


def _f32(a):
    return np.ascontiguousarray(a, dtype=np.float32)


# --------------------------------------------------------------------------- FWHT
def sign_bits(block):
    """hadamard.rs:29-44."""
    return int(lib().or_sign_bits(block))


def fwht64(x):
    """hadamard.rs:48-99 (blocks indexed 0..n/64)."""
    y = _f32(x).copy()
    lib().or_fwht64(y, y.size)
    return y


def ifwht64(x):
    """hadamard.rs:176-228."""
    y = _f32(x).copy()
    lib().or_ifwht64(y, y.size)
    return y


def fwht64_block(x64, block_idx):
    y = _f32(x64).copy()
    lib().or_fwht64_block(y, block_idx)
    return y


def ifwht64_block(x64, block_idx):
    y = _f32(x64).copy()
    lib().or_ifwht64_block(y, block_idx)
    return y


def f32_to_bf16(v):
    return int(lib().or_f32_to_bf16(float(v)))


# --------------------------------------------------------------------------- activations
def populate_fwht(x, w=None, inv_rms=1.0):
    """simd_lut.rs:2954-3196: (optional RMSNorm scale) + FWHT-64 + int8 per 64-chunk."""
    x = _f32(x)
    K = x.size
    q = np.zeros(K, np.int8)
    s = np.zeros(K // 64, np.float32)
    sm = np.zeros(K // 64, np.int32)
    wv = None if w is None else _f32(w)
    lib().or_populate_fwht(x, _ptr(wv), float(inv_rms), K, q, s, sm)
    return q, s, sm


def populate_plain(x):
    """simd_lut.rs:3235-3255."""
    x = _f32(x)
    K = x.size
    q = np.zeros(K, np.int8)
    s = np.zeros(K // 64, np.float32)
    sm = np.zeros(K // 64, np.int32)
    lib().or_populate_plain(x, K, q, s, sm)
    return q, s, sm


def inv_rms(x, eps, order="x86"):
    """real_llm.rs:903-926 (x86: four scalar accumulators) or, with order="neon",
    929-962 (aarch64: 4x4 fused-multiply-add accumulators)."""
    x = _f32(x)
    fn = lib().or_inv_rms_neon if order == "neon" else lib().or_inv_rms
    return float(fn(x, x.size, float(eps)))


# --------------------------------------------------------------------------- bit-plane
def bipolar_rtn(W, planes):
    """compiler.rs:992-1107 (RTN, no Hessian) -> (u codes [rows, cols], bf16 scales)."""
    W = _f32(W)
    rows, cols = W.shape
    stripes = (rows + 15) // 16
    u = np.zeros((rows, cols), np.uint8)
    sc = np.zeros(stripes * (cols // 64) * 16, np.uint16)
    lib().or_bipolar_rtn(W, rows, cols, planes, u, sc)
    return u, sc


def pack_interleaved(u, planes):
    """simd_lut.rs:1771-1795."""
    u = np.ascontiguousarray(u, np.uint8)
    rows, cols = u.shape
    stripes = (rows + 15) // 16
    out = np.zeros(stripes * (cols // 8) * planes * 16, np.uint8)
    lib().or_pack_interleaved(u, rows, cols, planes, out)
    return out


def nibble4_sizes(rows, cols, hp):
    stripes = (rows + 15) // 16
    nc = cols // 64
    return (stripes // 2) * nc * (1024 + 256 * hp + 64), (stripes & 1) * nc * (512 + 128 * hp + 32)


def nibble4_repack(inter, scales, rows, cols, planes, interleave_gate_up=False):
    """simd_lut.rs:3297-3400 from_bipolar_with_perm -> (pair_stream, tail_stream)."""
    pl, tl = nibble4_sizes(rows, cols, planes - 4)
    pair = np.zeros(max(pl, 1), np.uint8)
    tail = np.zeros(max(tl, 1), np.uint8)
    lib().or_nibble4_repack(np.ascontiguousarray(inter, np.uint8), np.ascontiguousarray(scales, np.uint16),
                            rows, cols, planes, int(interleave_gate_up), pair, tail)
    return pair[:pl], tail[:tl]


def _nz(a):
    return a if a.size else np.zeros(1, a.dtype)


def nibble4_dequant_row(pair, tail, rows, cols, hp, r):
    out = np.zeros(cols, np.float32)
    lib().or_nibble4_dequant_row(_nz(pair), _nz(tail), rows, cols, hp, r, out)
    return out


def nibble4_row_codes(pair, tail, rows, cols, hp, r):
    out = np.zeros(cols, np.uint8)
    lib().or_nibble4_row_codes(_nz(pair), _nz(tail), rows, cols, hp, r, out)
    return out


def nibble4_gemv(pair, tail, rows, cols, hp, xq, xs, xsum, want_dots=False, s0=0, s1=None):
    """simd_lut.rs:3766-4091 semantics (integer dots + in-order fmaf epilogue)."""
    stripes = (rows + 15) // 16
    s1 = stripes if s1 is None else s1
    out = np.zeros(rows, np.float32)
    dots = np.zeros((rows, cols // 64), np.int32) if want_dots else None
    lib().or_nibble4_gemv(_nz(pair), _nz(tail), rows, cols, hp, np.ascontiguousarray(xq, np.int8), _f32(xs),
                          np.ascontiguousarray(xsum, np.int32), s0, s1, out, _ptr(dots))
    return (out, dots) if want_dots else out


def nibble4_gemv_portable(pair, tail, rows, cols, hp, xq, xs, s0=0, s1=None):
    """simd_lut.rs:3558-3581: dequantize + fp32 dot (portable baseline)."""
    stripes = (rows + 15) // 16
    s1 = stripes if s1 is None else s1
    out = np.zeros(rows, np.float32)
    lib().or_nibble4_gemv_portable(_nz(pair), _nz(tail), rows, cols, hp, np.ascontiguousarray(xq, np.int8),
                                   _f32(xs), s0, s1, out)
    return out


# --------------------------------------------------------------------------- NF
def nf_fit_codebook(W, bits, sgc):
    """compiler.rs:1404-1526 -> (codebook i8[16], mu_top)."""
    W = _f32(W)
    cb = np.zeros(16, np.int8)
    mu = lib().or_nf_fit_codebook(W, W.shape[0], W.shape[1], bits, sgc, cb)
    return cb, float(mu)


def nf_rtn(W, bits, sgc, cb, mu_top):
    """compiler.rs:1628-1866 (no Hessian) -> (indices [rows, cols], bf16 scales)."""
    W = _f32(W)
    rows, cols = W.shape
    nsg = (cols // 64 + sgc - 1) // sgc
    idx = np.zeros((rows, cols), np.uint8)
    sc = np.zeros(((rows + 15) // 16) * nsg * 16, np.uint16)
    lib().or_nf_rtn(W, rows, cols, bits, sgc, np.ascontiguousarray(cb, np.int8), float(mu_top), idx, sc)
    return idx, sc


def nf_sizes(rows, cols, bits, sgc):
    stripes = (rows + 15) // 16
    L = lib()
    return (stripes // 2) * L.or_nf_pair_total(cols, bits, sgc), (stripes & 1) * L.or_nf_tail_total(cols, bits, sgc)


def nf_from_indices(idx, scales, rows, cols, bits, sgc):
    """simd_lut.rs:4850-5023."""
    pl, tl = nf_sizes(rows, cols, bits, sgc)
    pair = np.zeros(max(pl, 1), np.uint8)
    tail = np.zeros(max(tl, 1), np.uint8)
    lib().or_nf_from_indices(np.ascontiguousarray(idx, np.uint8), np.ascontiguousarray(scales, np.uint16),
                             rows, cols, bits, sgc, pair, tail)
    return pair[:pl], tail[:tl]


def nf_row_indices(pair, tail, rows, cols, bits, sgc, r):
    out = np.zeros(cols, np.uint8)
    lib().or_nf_row_indices(_nz(pair), _nz(tail), rows, cols, bits, sgc, r, out)
    return out


def nf_dequant_row(pair, tail, rows, cols, bits, sgc, cb, r):
    out = np.zeros(cols, np.float32)
    lib().or_nf_dequant_row(_nz(pair), _nz(tail), rows, cols, bits, sgc, np.ascontiguousarray(cb, np.int8), r, out)
    return out


def nf_gemv(pair, tail, rows, cols, bits, sgc, cb, xq, xs, want_dots=False, s0=0, s1=None):
    """simd_lut.rs:6074-6364 semantics."""
    stripes = (rows + 15) // 16
    s1 = stripes if s1 is None else s1
    out = np.zeros(rows, np.float32)
    dots = np.zeros((rows, cols // 64), np.int32) if want_dots else None
    lib().or_nf_gemv(_nz(pair), _nz(tail), rows, cols, bits, sgc, np.ascontiguousarray(cb, np.int8),
                     np.ascontiguousarray(xq, np.int8), _f32(xs), s0, s1, out, _ptr(dots))
    return (out, dots) if want_dots else out


def nf_gemv_portable(pair, tail, rows, cols, bits, sgc, cb, xq, xs, s0=0, s1=None):
    """simd_lut.rs:5719-5748."""
    stripes = (rows + 15) // 16
    s1 = stripes if s1 is None else s1
    out = np.zeros(rows, np.float32)
    lib().or_nf_gemv_portable(_nz(pair), _nz(tail), rows, cols, bits, sgc, np.ascontiguousarray(cb, np.int8),
                              np.ascontiguousarray(xq, np.int8), _f32(xs), s0, s1, out)
    return out


# --------------------------------------------------------------------------- KV / attention / glue
def kv_quant_head(src):
    """real_llm.rs:8282-8365."""
    src = _f32(src)
    q = np.zeros(src.size, np.int8)
    s = np.zeros(1, np.float32)
    lib().or_kv_quant_head(src, src.size, q, s)
    return q, float(s[0])


def attn_q8_head(q_head, k_q8, ks, v_q8, vs, attn_scale, window=False):
    """real_llm.rs:8471-8594 (portable branches); window=True: the sliding-window path
    (8794-8937) over rows already gathered in active_kv_pos order."""
    q_head = _f32(q_head)
    hd = q_head.size
    seq = len(ks)
    out = np.zeros(hd, np.float32)
    sc = np.zeros(max(seq, 1), np.float32)
    fn = lib().or_attn_q8_head_window if window else lib().or_attn_q8_head
    fn(q_head, np.ascontiguousarray(k_q8, np.int8).reshape(-1), _f32(ks),
                          np.ascontiguousarray(v_q8, np.int8).reshape(-1), _f32(vs), seq, hd,
                          float(attn_scale), out, sc)
    return out


def nf4_nearest_idx(y):
    return int(lib().or_nf4_nearest_idx(float(y)))


def kv_quant_head_q4(src):
    """store_hadamard_q4_head_raw (real_llm.rs:8646-8700): (nibbles [hd/2], bf16 scales [hd/64])."""
    src = _f32(src)
    hd = src.size
    q4 = np.zeros(hd // 2, np.uint8)
    s16 = np.zeros(hd // 64, np.uint16)
    lib().or_kv_quant_head_q4(src, hd, q4, s16)
    return q4, s16


def attn_q4_head(q_head, k4, ks16, v4, vs16, attn_scale):
    """NF4-KV attention (real_llm.rs:8827-8849, 8881-8906) over rows in attended order."""
    q_head = _f32(q_head)
    hd = q_head.size
    seq = len(k4)
    out = np.zeros(hd, np.float32)
    sc = np.zeros(max(seq, 1), np.float32)
    lib().or_attn_q4_head(q_head, np.ascontiguousarray(k4, np.uint8).reshape(-1),
                          np.ascontiguousarray(ks16, np.uint16).reshape(-1), np.ascontiguousarray(v4, np.uint8).reshape(-1),
                          np.ascontiguousarray(vs16, np.uint16).reshape(-1), seq, hd, float(attn_scale), out, sc)
    return out


def rope_row(hd, theta, pos):
    row = np.zeros(hd, np.float32)
    lib().or_rope_row(hd, float(theta), pos, row)
    return row


def rope_apply(head, row):
    h = _f32(head).copy()
    lib().or_rope_apply(h, h.size, _f32(row))
    return h


def expf(x):
    """The platform libm's expf elementwise (glibc on the x86 host: the reference's x86
    `f32::exp`, real_llm.rs:9595 / 9803, sparse_moe.rs:131, 155)."""
    x = np.ascontiguousarray(x, np.float32).reshape(-1)
    y = np.empty_like(x)
    lib().or_expf_array(x, y, x.size)
    return y


def swiglu(g, u):
    g = _f32(g)
    out = np.zeros_like(g)
    lib().or_swiglu(g, _f32(u), out, g.size)
    return out
