"""k2t_attn_decode_noalloc (the allocation-free variant of k2t_attn_decode, whose span
partials live in the library's fixed device array) against k2t_attn_decode on the same
inputs: bit-identical outputs on two calls in a row, the second with a smaller input
(the array keeps the first call's contents), and a clear error past its size limit."""
import numpy as np
import pytest
import torch

import k2t

pytestmark = pytest.mark.gpu


def _case(rng, bits, nq, nkv, hd, seq):
    cap = seq + 3
    if bits == 8:
        kq = rng.integers(-127, 128, (nkv, cap, hd), dtype=np.int8)
        vq = rng.integers(-127, 128, (nkv, cap, hd), dtype=np.int8)
        ks = rng.uniform(0.005, 0.05, (nkv, cap)).astype(np.float32)
        vs = rng.uniform(0.005, 0.05, (nkv, cap)).astype(np.float32)
    else:
        kq = rng.integers(0, 256, (nkv, cap, hd // 2), dtype=np.uint8)
        vq = rng.integers(0, 256, (nkv, cap, hd // 2), dtype=np.uint8)
        ks = (rng.uniform(0.005, 0.05, (nkv, cap, hd // 64)).astype(np.float32).view(np.uint32) >> 16) \
            .astype(np.uint16).view(np.int16)
        vs = (rng.uniform(0.005, 0.05, (nkv, cap, hd // 64)).astype(np.float32).view(np.uint32) >> 16) \
            .astype(np.uint16).view(np.int16)
    q = rng.standard_normal((nq, hd)).astype(np.float32)
    dev = lambda a: torch.from_numpy(np.ascontiguousarray(a)).cuda()  # noqa: E731
    return dev(q), dev(kq), dev(ks), dev(vq), dev(vs), cap


@pytest.mark.parametrize("first,second", [((8, 32, 4, 128, 3000, 0, 0), (8, 8, 2, 64, 700, 0, 0)),
                                          ((4, 16, 2, 64, 1300, 0, 0), (4, 4, 1, 128, 90, 24, 4))])
def test_attn_decode_noalloc_matches(gpu_ctx, first, second):
    print(f"attn_decode_noalloc {first} then {second}", flush=True)
    rng = np.random.default_rng(first[4])
    for bits, nq, nkv, hd, seq, window, sinks in (first, second):
        q, kq, ks, vq, vs, cap = _case(rng, bits, nq, nkv, hd, seq)
        if window:
            cap = window + 16
        scale = 1.0 / np.sqrt(hd)
        want = torch.full((nq, hd), float("nan"), dtype=torch.float32, device="cuda")
        got = torch.full((nq, hd), float("nan"), dtype=torch.float32, device="cuda")
        gpu_ctx.attn_decode(bits, q, nq, nkv, hd, kq, ks, vq, vs, cap, seq, scale, want, window, sinks)
        gpu_ctx.attn_decode_noalloc(bits, q, nq, nkv, hd, kq, ks, vq, vs, cap, seq, scale, got, window, sinks)
        gpu_ctx.sync()
        w, g = want.cpu().numpy(), got.cpu().numpy()
        assert np.isfinite(w).all()
        assert np.array_equal(g.view(np.uint32), w.view(np.uint32)), (bits, nq, hd, seq)


def test_attn_decode_noalloc_size_limit(gpu_ctx):
    """64 heads x 157 spans (40000 positions) x 130 floats exceeds the fixed array: the
    call is refused before anything runs."""
    t = torch.zeros(64 * 128, dtype=torch.float32, device="cuda")
    k8 = torch.zeros(16, dtype=torch.int8, device="cuda")
    with pytest.raises(k2t.K2TError, match="exceeds its fixed scratch"):
        gpu_ctx.attn_decode_noalloc(8, t, 64, 8, 128, k8, t, k8, t, 40000, 40000, 0.1, t)
