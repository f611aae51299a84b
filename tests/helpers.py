"""Shared input generators for the parity tests (seeded, numpy)."""
import numpy as np

import oracle as O


def normal(rng, shape, std=1.0):
    return (rng.standard_normal(shape) * std).astype(np.float32)


def activation(rng, K, outlier_frac=0.0, outlier_scale=20.0, n_outliers=0, zero_chunk=None):
    x = normal(rng, K)
    n = max(n_outliers, int(round(outlier_frac * K)))
    if n:
        idx = rng.choice(K, size=n, replace=False)
        x[idx] *= outlier_scale
    if zero_chunk is not None and zero_chunk < K // 64:
        x[zero_chunk * 64:(zero_chunk + 1) * 64] = 0.0
    return x


def random_bf16_scales(rng, n, lo=1e-4, hi=5e-3):
    v = rng.uniform(lo, hi, n).astype(np.float32)
    return (v.view(np.uint32) >> 16).astype(np.uint16)


def random_nibble4_streams(rng, rows, cols, hp):
    """A valid Nibble4 pair/tail stream: random code bytes, finite BF16 scales."""
    pl, tl = O.nibble4_sizes(rows, cols, hp)
    nc = cols // 64
    pair = rng.integers(0, 256, pl, dtype=np.uint8)
    tail = rng.integers(0, 256, tl, dtype=np.uint8)
    prec, trec = 1024 + 256 * hp + 64, 512 + 128 * hp + 32
    if pl:
        p2 = pair.reshape(-1, prec)
        p2[:, 1024 + 256 * hp:] = random_bf16_scales(rng, p2.shape[0] * 32).view(np.uint8).reshape(-1, 64)
    if tl:
        t2 = tail.reshape(nc, trec)
        t2[:, 512 + 128 * hp:] = random_bf16_scales(rng, nc * 16).view(np.uint8).reshape(-1, 32)
    return pair, tail


def quantized_nibble4(rng, rows, cols, planes, std=0.02, interleave=False):
    """W ~ N(0, std) -> Hadamard RTN bit planes -> FusedBipolar -> Nibble4 (oracle)."""
    W = normal(rng, (rows, cols), std)
    u, sc = O.bipolar_rtn(W, planes)
    inter = O.pack_interleaved(u, planes)
    pair, tail = O.nibble4_repack(inter, sc, rows, cols, planes, interleave)
    return W, u, sc, pair, tail


def random_nf_streams(rng, rows, cols, sgc, bits=4):
    idx = rng.integers(0, 1 << bits, (rows, cols), dtype=np.uint8)
    nsg = (cols // 64 + sgc - 1) // sgc
    sc = random_bf16_scales(rng, ((rows + 15) // 16) * nsg * 16)
    pair, tail = O.nf_from_indices(idx, sc, rows, cols, bits, sgc)
    return idx, sc, pair, tail


def quantized_nf4(rng, rows, cols, sgc=2, std=0.02):
    W = normal(rng, (rows, cols), std)
    cb, mu = O.nf_fit_codebook(W, 4, sgc)
    idx, sc = O.nf_rtn(W, 4, sgc, cb, mu)
    pair, tail = O.nf_from_indices(idx, sc, rows, cols, 4, sgc)
    return W, cb, idx, sc, pair, tail


def acts(rng, K, ntok, **kw):
    """ntok activation rows quantized by the oracle populate_fwht."""
    qs, ss, ms = [], [], []
    for _ in range(ntok):
        q, s, m = O.populate_fwht(activation(rng, K, **kw))
        qs.append(q)
        ss.append(s)
        ms.append(m)
    return np.stack(qs), np.stack(ss), np.stack(ms)


def mix64(z):
    z = np.uint64(z)
    with np.errstate(over="ignore"):
        z = (z ^ (z >> np.uint64(30))) * np.uint64(0xBF58476D1CE4E5B9)
        z = (z ^ (z >> np.uint64(27))) * np.uint64(0x94D049BB133111EB)
    return z ^ (z >> np.uint64(31))


def synthetic_kv(ref, n_layers, nkv, hd, n_pos, seed):
    """The engine's kv_synthetic fill (seeded int8 codes, scales in [0.005, 0.05]) written
    into the oracle's cache: slot (layer*nkv + kvh, pos), hash base
    seed*golden + slot_lin*FNV, codes (h & 0xFF) - 128 and ((h >> 8) & 0xFF) - 128 with
    -128 clamped to -127."""
    with np.errstate(over="ignore"):
        lin = np.arange(n_layers * nkv * n_pos, dtype=np.uint64)
        base = np.uint64(seed) * np.uint64(0x9E3779B97F4A7C15) + lin * np.uint64(0x100000001B3)
        h = mix64(base[:, None] + np.arange(hd, dtype=np.uint64)[None, :])
        hs = mix64(base ^ np.uint64(0xD1B54A32D192ED03))
    k = (h & np.uint64(0xFF)).astype(np.int32) - 128
    v = ((h >> np.uint64(8)) & np.uint64(0xFF)).astype(np.int32) - 128
    k[k == -128] = -127
    v[v == -128] = -127
    f = np.float32
    a = f(0.005) + (f(0.045) * (hs & np.uint64(0xFFFF)).astype(np.float32)) / f(65535.0)
    b = f(0.005) + (f(0.045) * ((hs >> np.uint64(16)) & np.uint64(0xFFFF)).astype(np.float32)) / f(65535.0)
    shape = (n_layers, nkv, n_pos)
    ref.kq[:, :, :n_pos] = k.astype(np.int8).reshape(*shape, hd)
    ref.vq[:, :, :n_pos] = v.astype(np.int8).reshape(*shape, hd)
    ref.ks[:, :, :n_pos] = a.astype(np.float32).reshape(shape)
    ref.vs[:, :, :n_pos] = b.astype(np.float32).reshape(shape)
    ref.pos = n_pos
