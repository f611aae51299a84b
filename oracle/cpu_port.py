"""ctypes view of the timed CPU baseline (oracle/k2t_cpu_port.c).

TEST INFRASTRUCTURE ONLY: used by bench.py's cpu_baseline leg and by tests/, never by the
product library.  CpuPortModel runs the reference's portable x86 decode step
(forward_token_sdot_megakernel's order, real_llm.rs:6794-7403, portable GEMV leaves
simd_lut.rs:3558-3581 / 5719-5748) from a C loop over a pool of host threads, built with
-O3 -march=native on the machine that runs it."""
import ctypes as C
import os
import subprocess
import tempfile

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_libs = {}


def build(out_dir=None):
    """Compiles libk2t_cpu_port.so for this host into out_dir (default: a private temp
    directory) and returns its path."""
    out_dir = out_dir or tempfile.mkdtemp(prefix="k2t_cpu_port_")
    subprocess.run(["make", "-s", "-C", _HERE, "port", f"PORT_DIR={out_dir}"], check=True)
    return os.path.join(out_dir, "libk2t_cpu_port.so")


def lib(path=None):
    path = path or build()
    if path not in _libs:
        L = C.CDLL(path)
        VP, SZ, I = C.c_void_p, C.c_size_t, C.c_int
        sig = {"cp_model_create": (VP, [I, I, I, I, I, I, I, I, C.c_float, C.c_double, I]),
               "cp_model_set_matrix": (None, [VP, I, I, I, I, I, SZ, SZ, VP, VP, VP]),
               "cp_model_set_norms": (None, [VP, I, VP, VP]),
               "cp_model_seed_kv": (None, [VP, I, C.c_uint64]),
               "cp_model_decode": (None, [VP, I, VP]),
               "cp_model_destroy": (None, [VP])}
        for name, (res, args) in sig.items():
            fn = getattr(L, name)
            fn.restype, fn.argtypes = res, args
        _libs[path] = L
    return _libs[path]


class CpuPortModel:
    """A dense decoder on the C port: `mats` are objects with fmt ("n4" / "nf4"), rows,
    cols, pair, tail, hp, cb, sgc (4 per layer: qkv, o, interleaved gate_up, down; then the
    tied head); norms default to ones."""

    def __init__(self, cfg, mats, threads, max_seq, lib_path=None, norms=None, final_norm=None):
        self.L = lib(lib_path)
        self.cfg = cfg
        self.keep = []
        self.h = self.L.cp_model_create(cfg["n_layers"], cfg["hidden"], cfg["n_heads"], cfg["n_kv_heads"],
                                        cfg["head_dim"], cfg["intermediate"], cfg["vocab"], max_seq,
                                        cfg["rms_eps"], float(np.float32(cfg["rope_theta"])), threads)
        for i, m in enumerate(mats):
            pair = np.ascontiguousarray(m.pair, np.uint8)
            tail = np.ascontiguousarray(m.tail if m.tail is not None and m.tail.size else np.zeros(16, np.uint8),
                                        np.uint8)
            cb = None if m.fmt == "n4" else np.ascontiguousarray(m.cb, np.int8)
            self.keep += [pair, tail, cb]
            self.L.cp_model_set_matrix(self.h, i, 0 if m.fmt == "n4" else 1, m.hp if m.fmt == "n4" else 0,
                                       0 if m.fmt == "n4" else 4, m.sgc, m.rows, m.cols, pair.ctypes.data,
                                       tail.ctypes.data, None if cb is None else cb.ctypes.data)
        ones = np.ones(cfg["hidden"], np.float32)
        self.keep.append(ones)
        for layer in range(cfg["n_layers"]):
            a, b = norms[layer] if norms else (ones, ones)
            a, b = np.ascontiguousarray(a, np.float32), np.ascontiguousarray(b, np.float32)
            self.keep += [a, b]
            self.L.cp_model_set_norms(self.h, layer, a.ctypes.data, b.ctypes.data)
        fn = np.ascontiguousarray(final_norm if final_norm is not None else ones, np.float32)
        self.keep.append(fn)
        self.L.cp_model_set_norms(self.h, -1, fn.ctypes.data, None)

    def seed_kv(self, n_pos, seed=1):
        self.L.cp_model_seed_kv(self.h, n_pos, seed)

    def decode(self, token, want_logits=True):
        out = np.empty(self.cfg["vocab"], np.float32) if want_logits else None
        self.L.cp_model_decode(self.h, int(token), None if out is None else out.ctypes.data)
        return out

    def close(self):
        if self.h:
            self.L.cp_model_destroy(self.h)
        self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
