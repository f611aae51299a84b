"""Python binding of the C ABI in include/k2t_hip.h (libk2t_hip.so, built in-tree).

This is the host-side mirror used by tests and bench.py: a thin ctypes layer with
the same entry points, argument meaning and error behaviour as the C ABI (each
negative status raises K2TError carrying k2t_last_error()).  Device buffers are
torch tensors on the ROCm device -- torch is only plumbing for memory and
streams here; every kernel that runs is in libk2t_hip.so.

Loading fails loudly when the shared library is missing: there is no CPU
fallback in the product path.
"""
import atexit
import ctypes as C
import os

_HERE = os.path.dirname(os.path.abspath(__file__))
# K2T_LIB_PATH selects another build of the library (a measurement build, for example)
LIB_PATH = os.environ.get("K2T_LIB_PATH") or os.path.join(_HERE, "libk2t_hip.so")
_lib = None
_shutting_down = False


def _mark_shutdown():
    global _shutting_down
    _shutting_down = True


atexit.register(_mark_shutdown)

VP = C.c_void_p
I32 = C.c_int32
SZ = C.c_size_t


class K2TError(RuntimeError):
    def __init__(self, code, msg):
        super().__init__(f"k2t error {code}: {msg}")
        self.code = code


# Every exported symbol of include/k2t_hip.h with (restype, argtypes).
SIGNATURES = {
    "k2t_version": (C.c_char_p, []),
    "k2t_last_error": (C.c_char_p, []),
    "k2t_device_count": (I32, []),
    "k2t_ctx_create": (I32, [I32, C.POINTER(VP)]),
    "k2t_ctx_destroy": (None, [VP]),
    "k2t_ctx_set_stream": (I32, [VP, VP]),
    "k2t_ctx_sync": (I32, [VP]),
    "k2t_ctx_set_splitk": (I32, [VP, I32]),
    "k2t_ctx_set_exact": (I32, [VP, I32]),
    "k2t_ctx_set_mfma": (I32, [VP, I32]),
    "k2t_malloc": (I32, [VP, SZ, C.POINTER(VP)]),
    "k2t_free": (I32, [VP, VP]),
    "k2t_memcpy_h2d": (I32, [VP, VP, VP, SZ]),
    "k2t_memcpy_d2h": (I32, [VP, VP, VP, SZ]),
    "k2t_mat_upload_nibble4": (I32, [VP, I32, I32, I32, VP, SZ, VP, SZ, C.POINTER(VP)]),
    "k2t_mat_upload_nf": (I32, [VP, I32, I32, I32, I32, VP, VP, SZ, VP, SZ, C.POINTER(VP)]),
    "k2t_mat_wrap_nibble4": (I32, [VP, I32, I32, I32, VP, SZ, VP, SZ, C.POINTER(VP)]),
    "k2t_mat_wrap_nf": (I32, [VP, I32, I32, I32, I32, VP, VP, SZ, VP, SZ, C.POINTER(VP)]),
    "k2t_mat_nf3_lane_order": (I32, [VP]),
    "k2t_mat_destroy": (None, [VP]),
    "k2t_mat_info": (I32, [VP, C.POINTER(I32), C.POINTER(I32), C.POINTER(I32), C.POINTER(C.c_uint64)]),
    "k2t_act_quant": (I32, [VP, VP, VP, VP, I32, I32, VP, VP, VP]),
    "k2t_act_quant_rmsnorm": (I32, [VP, VP, VP, C.c_float, I32, I32, VP, VP, VP]),
    "k2t_gemv": (I32, [VP, VP, VP, VP, VP, I32, I32, I32, VP, SZ]),
    "k2t_gemv_chunk_dots": (I32, [VP, VP, VP, VP, VP]),
    "k2t_stream_sizes": (I32, [I32, I32, I32, I32, I32, C.POINTER(SZ), C.POINTER(SZ)]),
    "k2t_compile_bipolar": (I32, [VP, I32, I32, I32, I32, I32, VP, SZ, VP, SZ]),
    "k2t_compile_nf": (I32, [VP, I32, I32, I32, I32, I32, I32, VP, VP, VP, SZ, VP, SZ]),
    "k2t_synth_normal": (I32, [C.c_uint64, C.c_float, VP, SZ, I32]),
    "k2t_model_create": (I32, [VP, VP, I32, C.POINTER(VP)]),
    "k2t_model_destroy": (None, [VP]),
    "k2t_model_set_layer": (I32, [VP, I32, VP, VP, VP, VP, VP, VP, VP]),
    "k2t_model_set_head": (I32, [VP, VP, VP]),
    "k2t_model_set_graph": (I32, [VP, I32]),
    "k2t_model_set_exact": (I32, [VP, I32]),
    "k2t_model_set_persistent": (I32, [VP, I32]),
    "k2t_model_stream": (I32, [VP, C.POINTER(VP)]),
    "k2t_model_persistent_active": (I32, [VP, C.POINTER(I32)]),
    "k2t_model_reset": (I32, [VP]),
    "k2t_model_position": (I32, [VP, C.POINTER(I32)]),
    "k2t_model_decode": (I32, [VP, I32, VP]),
    "k2t_model_prefill": (I32, [VP, VP, I32, VP]),
    "k2t_model_generate": (I32, [VP, I32, I32, VP]),
    "k2t_model_logits": (I32, [VP, C.POINTER(VP)]),
    "k2t_model_sync": (I32, [VP]),
    "k2t_model_set_embedding": (I32, [VP, I32, VP, VP]),
    "k2t_k2tb_open": (I32, [C.c_char_p, C.POINTER(VP)]),
    "k2t_k2tb_close": (None, [VP]),
    "k2t_k2tb_header": (I32, [VP, C.POINTER(I32), C.POINTER(I32), VP]),
    "k2t_k2tb_matrix": (I32, [VP, I32, I32, I32, VP, VP, SZ, VP, SZ]),
    "k2t_k2tb_vector": (I32, [VP, I32, I32, C.POINTER(SZ), VP, SZ]),
    "k2t_model_load_k2tb": (I32, [VP, VP, C.c_char_p, I32, C.POINTER(VP)]),
    "k2t_k2tm_read_header": (I32, [VP, SZ, VP]),
    "k2t_k2tm_expert_layout": (I32, [C.c_int64, C.c_int64, I32, I32, VP]),
    "k2t_experts_upload": (I32, [VP, VP, SZ, C.POINTER(VP)]),
    "k2t_experts_wrap": (I32, [VP, VP, SZ, VP, C.POINTER(VP)]),
    "k2t_experts_nf3_lane_order": (I32, [VP]),
    "k2t_experts_destroy": (None, [VP]),
    "k2t_experts_info": (I32, [VP, VP]),
    "k2t_moe_ffn": (I32, [VP, VP, I32, VP, VP, I32, I32, I32, VP, VP, C.c_float, VP, VP]),
    "k2t_model_set_qk_norm": (I32, [VP, I32, VP, VP]),
    "k2t_model_set_moe": (I32, [VP, I32, VP, I32, VP, VP, I32, I32, I32]),
    "k2t_model_set_moe_shared": (I32, [VP, I32, VP, VP, VP]),
    "k2t_model_kv_synthetic": (I32, [VP, I32, C.c_uint64]),
    "k2t_model_set_kv_window": (I32, [VP, I32, I32]),
    "k2t_model_kv_window": (I32, [VP, C.POINTER(I32), C.POINTER(I32)]),
    "k2t_model_set_kv_bits": (I32, [VP, I32]),
    "k2t_model_kv_bits": (I32, [VP, C.POINTER(I32)]),
    "k2t_kv_store": (I32, [VP, I32, VP, I32, I32, VP, VP]),
    "k2t_attn_decode": (I32, [VP, I32, VP, I32, I32, I32, VP, VP, VP, VP, I32, I32, I32, I32, C.c_float, VP]),
    "k2t_stream_read_probe": (I32, [VP, VP, SZ, VP]),
    "k2t_expf_host": (C.c_float, [C.c_float]),
    "k2t_expf_device": (I32, [VP, VP, VP, SZ]),
    "k2t_attn_decode_noalloc": (I32, [VP, I32, VP, I32, I32, I32, VP, VP, VP, VP, I32, I32, I32, I32, C.c_float,
                                      VP]),
}

MOE_SOFTMAX, MOE_TOPK_SOFTMAX, MOE_SIGMOID = 0, 1, 2

EMBED_TIED, EMBED_F32, EMBED_BF16, EMBED_NF4 = 0, 1, 2, 3


class ModelConfig(C.Structure):
    """k2t_model_config (LlamaConfig subset)."""
    _fields_ = [("n_layers", I32), ("hidden", I32), ("n_heads", I32), ("n_kv_heads", I32), ("head_dim", I32),
                ("intermediate", I32), ("vocab", I32), ("max_seq", I32), ("rms_eps", C.c_float),
                ("rope_theta", C.c_float)]


class K2tmHeader(C.Structure):
    """k2t_k2tm_header (K2tmShardHeader)."""
    _fields_ = [(n, C.c_int64) for n in ("num_layers", "experts_per_layer", "d_model", "d_ff_expert",
                                         "scale_group_chunks", "aligned_expert_bytes", "bits")]


class K2tmLayout(C.Structure):
    """k2t_k2tm_layout (NfExpertByteLayout offsets)."""
    _fields_ = [(n, C.c_int64) for n in ("gu_codebook_off", "dn_codebook_off", "gu_pair_off", "gu_pair_bytes",
                                         "dn_pair_off", "dn_pair_bytes", "aligned_expert_bytes")]


def k2tm_read_header(page):
    import numpy as np
    b = np.frombuffer(page, np.uint8) if isinstance(page, (bytes, bytearray)) else np.ascontiguousarray(page, np.uint8)
    h = K2tmHeader()
    check(lib().k2t_k2tm_read_header(b.ctypes.data_as(VP), b.size, C.byref(h)))
    return {n: getattr(h, n) for n, _ in K2tmHeader._fields_}


def k2tm_expert_layout(d_model, d_ff, bits, sgc):
    out = K2tmLayout()
    check(lib().k2t_k2tm_expert_layout(d_model, d_ff, bits, sgc, C.byref(out)))
    return {n: getattr(out, n) for n, _ in K2tmLayout._fields_}


class K2tbMatrixInfo(C.Structure):
    """k2t_k2tb_matrix_info."""
    _fields_ = [("tag", I32), ("fmt", I32), ("rows", I32), ("cols", I32), ("planes_or_bits", I32), ("sgc", I32),
                ("codebook", C.c_int8 * 16), ("pair_len", SZ), ("tail_len", SZ)]


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"{LIB_PATH} is not built; run __graft_entry__.build() (no CPU fallback exists)")
        L = C.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def check(rc):
    if rc != 0:
        raise K2TError(rc, lib().k2t_last_error().decode())
    return rc


def _p(t):
    """Device pointer of a torch tensor (or None / int passthrough)."""
    if t is None:
        return None
    if isinstance(t, int):
        return t
    return t.data_ptr()


def _host(a):
    import numpy as np
    a = np.ascontiguousarray(a)
    return a.ctypes.data_as(VP) if a.size else None, a


class Ctx:
    """k2t_ctx: one per device stream."""

    def __init__(self, device=0, stream=None):
        h = VP()
        check(lib().k2t_ctx_create(device, C.byref(h)))
        self.h = h
        self.device = device
        if stream is not None:
            self.set_stream(stream)

    def set_stream(self, stream):
        check(lib().k2t_ctx_set_stream(self.h, VP(stream.cuda_stream if hasattr(stream, "cuda_stream") else stream)))

    def set_splitk(self, n):
        check(lib().k2t_ctx_set_splitk(self.h, int(n)))

    def set_exact(self, on):
        check(lib().k2t_ctx_set_exact(self.h, int(bool(on))))

    def set_mfma(self, mode):
        """0 off, 1 on (default), 2 on with the GEMV copying the activation tiles itself."""
        check(lib().k2t_ctx_set_mfma(self.h, int(mode)))

    def sync(self):
        check(lib().k2t_ctx_sync(self.h))

    def close(self):
        if self.h and not _shutting_down:
            lib().k2t_ctx_destroy(self.h)
        self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    # -- matrices
    def upload_nibble4(self, rows, cols, hi_planes, pair, tail):
        pp, pa = _host(pair)
        tp, ta = _host(tail)
        h = VP()
        check(lib().k2t_mat_upload_nibble4(self.h, rows, cols, hi_planes, pp, pa.nbytes, tp, ta.nbytes, C.byref(h)))
        return Mat(self, h, rows, cols)

    def upload_nf(self, rows, cols, bits, sgc, codebook, pair, tail):
        cp, ca = _host(codebook)
        pp, pa = _host(pair)
        tp, ta = _host(tail)
        h = VP()
        check(lib().k2t_mat_upload_nf(self.h, rows, cols, bits, sgc, cp, pp, pa.nbytes, tp, ta.nbytes, C.byref(h)))
        return Mat(self, h, rows, cols)

    def wrap_nibble4(self, rows, cols, hi_planes, d_pair, pair_len, d_tail, tail_len):
        h = VP()
        check(lib().k2t_mat_wrap_nibble4(self.h, rows, cols, hi_planes, _p(d_pair), pair_len, _p(d_tail),
                                         tail_len, C.byref(h)))
        return Mat(self, h, rows, cols, keep=(d_pair, d_tail))

    def wrap_nf(self, rows, cols, bits, sgc, codebook, d_pair, pair_len, d_tail, tail_len):
        cp, ca = _host(codebook)
        h = VP()
        check(lib().k2t_mat_wrap_nf(self.h, rows, cols, bits, sgc, cp, _p(d_pair), pair_len, _p(d_tail),
                                    tail_len, C.byref(h)))
        return Mat(self, h, rows, cols, keep=(d_pair, d_tail))

    # -- activations
    def act_quant(self, x, q, scales, sums, K, ntok, norm_w=None, inv_rms=None):
        check(lib().k2t_act_quant(self.h, _p(x), _p(norm_w), _p(inv_rms), K, ntok, _p(q), _p(scales), _p(sums)))

    def act_quant_rmsnorm(self, x, norm_w, eps, q, scales, sums, K, ntok):
        check(lib().k2t_act_quant_rmsnorm(self.h, _p(x), _p(norm_w), float(eps), K, ntok, _p(q), _p(scales),
                                          _p(sums)))

    # -- GEMV
    def gemv(self, m, xq, xs, xsum, out, ntok=1, s0=0, s1=-1, out_stride=0):
        check(lib().k2t_gemv(self.h, m.h, _p(xq), _p(xs), _p(xsum), ntok, s0, s1, _p(out), out_stride))

    def kv_store(self, bits, heads, n, head_dim, q, scales):
        """k2t_kv_store: n post-RoPE heads -> Hadamard int8 / NF4 KV slots 0..n-1."""
        check(lib().k2t_kv_store(self.h, bits, _p(heads), n, head_dim, _p(q), _p(scales)))

    def attn_decode(self, bits, q, n_heads, n_kv_heads, head_dim, kq, ks, vq, vs, cap, seq, attn_scale, out,
                    window=0, sink_tokens=0):
        """k2t_attn_decode: one token's attention over a KV cache in k2t_kv_store's layout."""
        check(lib().k2t_attn_decode(self.h, bits, _p(q), n_heads, n_kv_heads, head_dim, _p(kq), _p(ks), _p(vq),
                                    _p(vs), cap, seq, window, sink_tokens, float(attn_scale), _p(out)))

    def stream_read_probe(self, src, nbytes, sink):
        """k2t_stream_read_probe: one streaming read of nbytes of a device buffer (HBM
        read-ceiling measurement)."""
        check(lib().k2t_stream_read_probe(self.h, _p(src), nbytes, _p(sink)))

    def attn_decode_noalloc(self, bits, q, n_heads, n_kv_heads, head_dim, kq, ks, vq, vs, cap, seq, attn_scale,
                            out, window=0, sink_tokens=0):
        """k2t_attn_decode_noalloc: attn_decode with the library's fixed device scratch
        (allocates nothing; asynchronous on the context's stream)."""
        check(lib().k2t_attn_decode_noalloc(self.h, bits, _p(q), n_heads, n_kv_heads, head_dim, _p(kq), _p(ks),
                                            _p(vq), _p(vs), cap, seq, window, sink_tokens, float(attn_scale),
                                            _p(out)))

    def moe_ffn(self, bank, shard_layer, router_w, hidden, post_norm, eps, top_k, norm_topk_prob=True,
                scoring=0, router_bias=None, route_ids=None, route_weights=None):
        """k2t_moe_ffn: hidden (device f32 [d]) += the MoE feed-forward of one token."""
        check(lib().k2t_moe_ffn(self.h, bank.h, shard_layer, _p(router_w), _p(router_bias), top_k,
                                int(bool(norm_topk_prob)), scoring, _p(hidden), _p(post_norm), float(eps),
                                _p(route_ids), _p(route_weights)))

    def gemv_chunk_dots(self, m, xq, xsum, dots):
        check(lib().k2t_gemv_chunk_dots(self.h, m.h, _p(xq), _p(xsum), _p(dots)))


class ExpertBank:
    """k2t_experts: a .k2tm shard in HBM (uploaded from host bytes, or wrapping device memory)."""

    def __init__(self, ctx, h, keep=None):
        self.ctx, self.h, self._keep = ctx, h, keep

    @classmethod
    def upload(cls, ctx, k2tm_bytes):
        import numpy as np
        b = np.frombuffer(k2tm_bytes, np.uint8) if isinstance(k2tm_bytes, (bytes, bytearray)) else \
            np.ascontiguousarray(k2tm_bytes, np.uint8)
        h = VP()
        check(lib().k2t_experts_upload(ctx.h, b.ctypes.data_as(VP), b.size, C.byref(h)))
        return cls(ctx, h)

    @classmethod
    def wrap(cls, ctx, d_tensor, nbytes, header_page):
        import numpy as np
        hp = np.ascontiguousarray(np.frombuffer(header_page, np.uint8) if isinstance(header_page, (bytes, bytearray))
                                  else header_page, np.uint8)
        h = VP()
        check(lib().k2t_experts_wrap(ctx.h, _p(d_tensor), nbytes, hp.ctypes.data_as(VP), C.byref(h)))
        return cls(ctx, h, keep=d_tensor)

    def nf3_lane_order(self):
        """k2t_experts_nf3_lane_order: NF3 experts rearranged in place into the GEMV's lane order
        (a wrapped bank's borrowed bytes included)."""
        check(lib().k2t_experts_nf3_lane_order(self.h))

    def info(self):
        h = K2tmHeader()
        check(lib().k2t_experts_info(self.h, C.byref(h)))
        return {n: getattr(h, n) for n, _ in K2tmHeader._fields_}

    def close(self):
        if self.h and not _shutting_down:
            lib().k2t_experts_destroy(self.h)
        self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class Mat:
    def __init__(self, ctx, h, rows, cols, keep=None):
        self.ctx = ctx
        self.h = h
        self.rows = rows
        self.cols = cols
        self._keep = keep

    def nf3_lane_order(self):
        """k2t_mat_nf3_lane_order: an NF3 matrix's streams rearranged in place into lane order."""
        check(lib().k2t_mat_nf3_lane_order(self.h))

    def info(self):
        r, c, s, b = I32(), I32(), I32(), C.c_uint64()
        check(lib().k2t_mat_info(self.h, C.byref(r), C.byref(c), C.byref(s), C.byref(b)))
        return r.value, c.value, s.value, b.value

    def close(self):
        if self.h and not _shutting_down:
            lib().k2t_mat_destroy(self.h)
        self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


# ---------------------------------------------------------------------------- offline compiler
def stream_sizes(fmt, rows, cols, planes_or_bits, sgc=1):
    pl, tl = SZ(), SZ()
    check(lib().k2t_stream_sizes(fmt, rows, cols, planes_or_bits, sgc, C.byref(pl), C.byref(tl)))
    return pl.value, tl.value


def compile_bipolar(W, planes, interleave_gate_up=False, threads=0):
    """Host RTN bit-plane compile -> (pair, tail) numpy uint8 streams."""
    import numpy as np
    W = np.ascontiguousarray(W, np.float32)
    rows, cols = W.shape
    pl, tl = stream_sizes(1, rows, cols, planes)
    pair = np.empty(pl, np.uint8)
    tail = np.empty(tl, np.uint8)
    check(lib().k2t_compile_bipolar(W.ctypes.data_as(VP), rows, cols, planes, int(interleave_gate_up), threads,
                                    pair.ctypes.data_as(VP) if pl else None, pl,
                                    tail.ctypes.data_as(VP) if tl else None, tl))
    return pair, tail


def compile_nf4(W, sgc=2, interleave_gate_up=False, threads=0, bits=4):
    """Host RTN NF4 (bits=4) / NF3 (bits=3) compile -> (codebook int8[16], mu_top, pair, tail)."""
    import numpy as np
    W = np.ascontiguousarray(W, np.float32)
    rows, cols = W.shape
    pl, tl = stream_sizes(2, rows, cols, bits, sgc)
    pair = np.empty(pl, np.uint8)
    tail = np.empty(tl, np.uint8)
    cb = np.zeros(16, np.int8)
    mu = C.c_float()
    check(lib().k2t_compile_nf(W.ctypes.data_as(VP), rows, cols, bits, sgc, int(interleave_gate_up), threads,
                               cb.ctypes.data_as(VP), C.byref(mu), pair.ctypes.data_as(VP) if pl else None, pl,
                               tail.ctypes.data_as(VP) if tl else None, tl))
    return cb, mu.value, pair, tail


def synth_normal(seed, n, std=1.0, threads=0):
    import numpy as np
    out = np.empty(n, np.float32)
    check(lib().k2t_synth_normal(seed, std, out.ctypes.data_as(VP) if n else None, n, threads))
    return out


class Model:
    """k2t_model: device-resident decoder (forward_token / forward_prompt / greedy loop)."""

    def __init__(self, ctx, cfg: dict, max_batch=4):
        import numpy as np  # noqa: F401
        self.ctx = ctx
        self.cfg = dict(cfg)
        c = ModelConfig(**{k: cfg[k] for k, _ in ModelConfig._fields_})
        h = VP()
        check(lib().k2t_model_create(ctx.h, C.byref(c), max_batch, C.byref(h)))
        self.h = h
        self._keep = []

    def set_layer(self, layer, qkv, o, gate_up, down, in_norm, post_norm, qkv_bias=None):
        import numpy as np
        inn = np.ascontiguousarray(in_norm, np.float32)
        pn = np.ascontiguousarray(post_norm, np.float32)
        b = None if qkv_bias is None else np.ascontiguousarray(qkv_bias, np.float32)
        check(lib().k2t_model_set_layer(self.h, layer, qkv.h, o.h, None if gate_up is None else gate_up.h,
                                        None if down is None else down.h, inn.ctypes.data_as(VP),
                                        pn.ctypes.data_as(VP), None if b is None else b.ctypes.data_as(VP)))
        self._keep.append((qkv, o, gate_up, down))

    def set_head(self, head, final_norm):
        import numpy as np
        fn = np.ascontiguousarray(final_norm, np.float32)
        check(lib().k2t_model_set_head(self.h, head.h, fn.ctypes.data_as(VP)))
        self._keep.append(head)

    def set_qk_norm(self, layer, q_norm=None, k_norm=None):
        import numpy as np
        qn = None if q_norm is None else np.ascontiguousarray(q_norm, np.float32)
        kn = None if k_norm is None else np.ascontiguousarray(k_norm, np.float32)
        check(lib().k2t_model_set_qk_norm(self.h, layer, None if qn is None else qn.ctypes.data_as(VP),
                                          None if kn is None else kn.ctypes.data_as(VP)))

    def set_moe(self, layer, bank, shard_layer, router_w, top_k, norm_topk_prob=True, scoring=0,
                router_bias=None):
        import numpy as np
        rw = np.ascontiguousarray(router_w, np.float32)
        rb = None if router_bias is None else np.ascontiguousarray(router_bias, np.float32)
        check(lib().k2t_model_set_moe(self.h, layer, bank.h, shard_layer, rw.ctypes.data_as(VP),
                                      None if rb is None else rb.ctypes.data_as(VP), top_k,
                                      int(bool(norm_topk_prob)), scoring))
        self._keep.append(bank)

    def set_moe_shared(self, layer, gate_up, down, gate_weight=None):
        """k2t_model_set_moe_shared: the layer's shared expert (NF gate_up in [gate; up]
        row order, NF down, optional sigmoid gate row); gate_up None removes it."""
        import numpy as np
        gw = None if gate_weight is None else np.ascontiguousarray(gate_weight, np.float32)
        check(lib().k2t_model_set_moe_shared(self.h, layer, None if gate_up is None else gate_up.h,
                                             None if down is None else down.h,
                                             None if gw is None else gw.ctypes.data_as(VP)))
        if gate_up is not None:
            self._keep += [gate_up, down]

    def set_kv_window(self, window, sink_tokens=4):
        """k2t_model_set_kv_window (set_kv_sliding_window); window 0 restores the full cache."""
        check(lib().k2t_model_set_kv_window(self.h, int(window), int(sink_tokens)))

    def set_kv_bits(self, bits):
        check(lib().k2t_model_set_kv_bits(self.h, int(bits)))

    def kv_bits(self):
        b = I32()
        check(lib().k2t_model_kv_bits(self.h, C.byref(b)))
        return b.value

    def kv_window(self):
        w, s = I32(), I32()
        check(lib().k2t_model_kv_window(self.h, C.byref(w), C.byref(s)))
        return w.value, s.value

    def kv_synthetic(self, n_pos, seed=0):
        check(lib().k2t_model_kv_synthetic(self.h, int(n_pos), int(seed)))

    def set_embedding(self, kind, rows=None, nf4=None):
        """k2t_model_set_embedding: EMBED_TIED, EMBED_F32 / EMBED_BF16 (host rows
        [vocab][hidden], float32 / uint16) or EMBED_NF4 (a Mat of the same context)."""
        import numpy as np
        r = None
        if kind == EMBED_F32:
            r = np.ascontiguousarray(rows, np.float32)
        elif kind == EMBED_BF16:
            r = np.ascontiguousarray(rows, np.uint16)
        check(lib().k2t_model_set_embedding(self.h, int(kind), None if r is None else r.ctypes.data_as(VP),
                                            None if nf4 is None else nf4.h))
        if nf4 is not None:
            self._keep.append(nf4)

    @classmethod
    def load_k2tb(cls, ctx, cfg: dict, path, max_batch=4):
        """k2t_model_load_k2tb: a compiled .k2tb model (load_bipolar + repack_sdot)
        for the config `cfg` (see load_llama_config), uploaded to the context's device."""
        self = cls.__new__(cls)
        self.ctx = ctx
        self.cfg = dict(cfg)
        c = ModelConfig(**{k: cfg[k] for k, _ in ModelConfig._fields_})
        h = VP()
        check(lib().k2t_model_load_k2tb(ctx.h, C.byref(c), os.fsencode(path), max_batch, C.byref(h)))
        self.h = h
        self._keep = []
        return self

    def set_graph(self, on):
        check(lib().k2t_model_set_graph(self.h, int(bool(on))))

    def set_exact(self, on):
        check(lib().k2t_model_set_exact(self.h, int(bool(on))))

    def stream(self):
        """The hipStream_t (int) the model's steps run on."""
        s = VP()
        check(lib().k2t_model_stream(self.h, C.byref(s)))
        return s.value or 0

    def set_persistent(self, on):
        """True / 1: the persistent decode kernel where supported; 2: also for mixed 4/5-plane
        bit-plane models; False / 0: one kernel per operation."""
        check(lib().k2t_model_set_persistent(self.h, 2 if on == 2 else int(bool(on))))

    def persistent_active(self):
        v = I32()
        check(lib().k2t_model_persistent_active(self.h, C.byref(v)))
        return bool(v.value)

    def reset(self):
        check(lib().k2t_model_reset(self.h))

    def position(self):
        p = I32()
        check(lib().k2t_model_position(self.h, C.byref(p)))
        return p.value

    def decode(self, token, want_logits=True):
        import numpy as np
        out = np.empty(self.cfg["vocab"], np.float32) if want_logits else None
        check(lib().k2t_model_decode(self.h, int(token), None if out is None else out.ctypes.data_as(VP)))
        return out

    def prefill(self, tokens, want_logits=True):
        import numpy as np
        t = np.ascontiguousarray(tokens, np.int32)
        out = np.empty(self.cfg["vocab"], np.float32) if want_logits else None
        check(lib().k2t_model_prefill(self.h, t.ctypes.data_as(VP), t.size,
                                      None if out is None else out.ctypes.data_as(VP)))
        return out

    def generate(self, first_token, n_steps, want_tokens=True):
        import numpy as np
        out = np.empty(max(n_steps, 1), np.int32) if want_tokens else None
        check(lib().k2t_model_generate(self.h, int(first_token), int(n_steps),
                                       None if out is None else out.ctypes.data_as(VP)))
        return None if out is None else out[:n_steps]

    def sync(self):
        check(lib().k2t_model_sync(self.h))

    def close(self):
        if self.h and not _shutting_down:
            lib().k2t_model_destroy(self.h)
        self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


# ---------------------------------------------------------------------------- .k2tb files
class K2tb:
    """A memory-mapped .k2tb file (k2t_k2tb_*): header, vectors and matrices repacked
    into the GEMV layouts on the host.  Needs no GPU."""

    def __init__(self, path):
        h = VP()
        check(lib().k2t_k2tb_open(os.fsencode(path), C.byref(h)))
        self.h = h

    def header(self):
        import numpy as np
        v, n = I32(), I32()
        mw = np.zeros(6, np.uint64)
        check(lib().k2t_k2tb_header(self.h, C.byref(v), C.byref(n), mw.ctypes.data_as(VP)))
        return v.value, n.value, [int(x) for x in mw]

    def matrix(self, layer, which, interleave_gate_up=False):
        """(info, pair bytes, tail bytes); layer -1 with which 4 = lm_head, 5 = NF4 embedding."""
        import numpy as np
        info = K2tbMatrixInfo()
        check(lib().k2t_k2tb_matrix(self.h, layer, which, int(interleave_gate_up), C.byref(info), None, 0, None, 0))
        pair = np.empty(info.pair_len, np.uint8)
        tail = np.empty(max(info.tail_len, 1), np.uint8)
        check(lib().k2t_k2tb_matrix(self.h, layer, which, int(interleave_gate_up), C.byref(info),
                                    pair.ctypes.data_as(VP), pair.size, tail.ctypes.data_as(VP), tail.size))
        return info, pair, tail[:info.tail_len]

    def vector(self, layer, which):
        import numpy as np
        n = SZ()
        check(lib().k2t_k2tb_vector(self.h, layer, which, C.byref(n), None, 0))
        dt = np.uint16 if (layer < 0 and which == 2) else np.float32
        out = np.empty(max(n.value, 1), dt)
        check(lib().k2t_k2tb_vector(self.h, layer, which, C.byref(n), out.ctypes.data_as(VP), out.size))
        return out[:n.value]

    def close(self):
        if self.h and not _shutting_down:
            lib().k2t_k2tb_close(self.h)
        self.h = None

    def __enter__(self):
        return self

    def __exit__(self, *a):
        self.close()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def load_llama_config(model_dir, max_seq):
    """The k2t_model_config fields of LlamaConfig::from_config_json (real_llm.rs:125-410)
    read from `model_dir`/config.json, with the reference's defaults for missing keys.
    rope_theta is the effective base (NTK-alpha stretch, real_llm.rs:415-422).  Raises
    ValueError for shapes this path does not run (MoE, per-layer sliding masks)."""
    import json
    with open(os.path.join(model_dir, "config.json")) as f:
        j = json.load(f)

    def opt_pos(k):  # parse_opt_usize: null or 0 -> None
        v = j.get(k)
        return int(v) if v else None

    hidden = int(j.get("hidden_size", 576))
    n_heads = int(j.get("num_attention_heads", 9))
    head_dim = opt_pos("head_dim") or hidden // n_heads
    theta = float(j.get("rope_theta", 100000.0))
    rs = j.get("rope_scaling")
    if isinstance(rs, dict):
        alpha = float(rs.get("alpha", 0.0) or 0.0)
        kind = rs.get("type", rs.get("rope_type"))
        if kind == "dynamic" and alpha > 1.0:
            d = float(head_dim)
            # effective_rope_theta: f32 theta widened, alpha stored as f32
            a32 = float(C.c_float(alpha).value)
            theta = float(C.c_float(theta).value) * a32 ** (d / (d - 2.0))
    n_experts = opt_pos("num_experts") or opt_pos("num_local_experts") or 0
    if n_experts > 1:
        raise ValueError("sparse-MoE configs are not supported by this loader")
    inter = int(j.get("intermediate_size", 1536))
    return dict(n_layers=int(j.get("num_hidden_layers", 30)), hidden=hidden, n_heads=n_heads,
                n_kv_heads=int(j.get("num_key_value_heads", 3)), head_dim=head_dim, intermediate=inter,
                vocab=int(j.get("vocab_size", 49152)), max_seq=int(max_seq),
                rms_eps=float(j.get("rms_norm_eps", 1e-5)), rope_theta=theta,
                tie_word_embeddings=bool(j.get("tie_word_embeddings", True)))


# ---------------------------------------------------------------------------- synthetic models
SMOLLM2_135M = dict(n_layers=30, hidden=576, n_heads=9, n_kv_heads=3, head_dim=64, intermediate=1536, vocab=49152,
                    rms_eps=1e-5, rope_theta=100000.0)
SMOLLM2_1_7B = dict(n_layers=24, hidden=2048, n_heads=32, n_kv_heads=32, head_dim=64, intermediate=8192,
                    vocab=49152, rms_eps=1e-5, rope_theta=130000.0)
# parse_mode "p55454" (chat.rs:278-281): qkv 5, o 5, gate_up 4, down 5, head 4 planes
P55454 = {"qkv": 5, "o": 5, "gu": 4, "down": 5, "head": 4}


class HostMatrix:
    """Compiled streams of one matrix kept on the host (for CPU baselines)."""

    def __init__(self, fmt, rows, cols, pair, tail, hp=0, cb=None, sgc=2):
        self.fmt, self.rows, self.cols, self.pair, self.tail, self.hp, self.cb, self.sgc = \
            fmt, rows, cols, pair, tail, hp, cb, sgc


def build_random_model(ctx, cfg, max_seq, fmt="nf4", planes=None, seed=1, max_batch=4, keep_host=False,
                       threads=0, log=None):
    """Random-init weights ~N(0, 0.02) (norms 1.0) compiled with the host RTN compiler
    (Hadamard + NF4 g128, or bit planes per projection) and uploaded: the synthetic
    stand-in for a .k2tb model.  Returns (Model, [k2t Mat], [HostMatrix] or None)."""
    import numpy as np
    full = dict(cfg, max_seq=max_seq)
    model = Model(ctx, full, max_batch=max_batch)
    d, nq, nkv, hd, inter, V = cfg["hidden"], cfg["n_heads"], cfg["n_kv_heads"], cfg["head_dim"], \
        cfg["intermediate"], cfg["vocab"]
    planes = planes or P55454
    mats, host = [], [] if keep_host else None
    counter = [seed * 1000003]

    def make(rows, cols, name, gu=False):
        counter[0] += 1
        W = synth_normal(counter[0], rows * cols, 0.02, threads).reshape(rows, cols)
        if fmt == "nf4":
            cb, mu, pair, tail = compile_nf4(W, 2, gu, threads)
            m = ctx.upload_nf(rows, cols, 4, 2, cb, pair, tail)
            hm = HostMatrix("nf4", rows, cols, pair, tail, cb=cb, sgc=2)
        else:
            p = planes[name]
            pair, tail = compile_bipolar(W, p, gu, threads)
            m = ctx.upload_nibble4(rows, cols, p - 4, pair, tail)
            hm = HostMatrix("n4", rows, cols, pair, tail, hp=p - 4)
        mats.append(m)
        if host is not None:
            host.append(hm)
        return m

    ones = np.ones(d, np.float32)
    for layer in range(cfg["n_layers"]):
        q = make((nq + 2 * nkv) * hd, d, "qkv")
        o = make(d, nq * hd, "o")
        gu = make(2 * inter, d, "gu", gu=True)
        dn = make(d, inter, "down")
        model.set_layer(layer, q, o, gu, dn, ones, ones)
        if log:
            log(f"layer {layer} compiled")
    head = make(V, d, "head")
    model.set_head(head, ones)
    return model, mats, host
