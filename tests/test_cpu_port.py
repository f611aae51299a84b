"""The timed CPU baseline (oracle/k2t_cpu_port.c: the portable decode step driven from C
over a thread pool, built -O3 -march=native) computes what the oracle's Python-driven
portable path computes (OracleModel with gemv_threads > 0): bit-identical logits on a
small nf4 model and a small p55454 model, at 1 and 3 threads (-ffp-contract=off and no
fast-math, so the optimization level changes no rounding)."""
import numpy as np
import pytest

from cpu_port import CpuPortModel
from model_oracle import OracleModel, random_model

TINY = dict(n_layers=2, hidden=256, n_heads=4, n_kv_heads=2, head_dim=64, intermediate=512, vocab=520,
            max_seq=40, rms_eps=1e-5, rope_theta=10000.0)
P55454 = {"qkv": 5, "o": 5, "gu": 4, "down": 5, "head": 4}


@pytest.mark.parametrize("threads", [1, 3])
@pytest.mark.parametrize("fmt,planes", [("nf4", None), ("n4", P55454)])
def test_cpu_port_matches_oracle_portable_path(fmt, planes, threads):
    layers, head, fn = random_model(TINY, seed=5, fmt=fmt, planes=planes)
    ref = OracleModel(TINY, layers, head, fn, gemv_threads=2)
    mats = [L[k] for L in layers for k in ("qkv", "o", "gu", "down")] + [head]
    port = CpuPortModel(TINY, mats, threads, TINY["max_seq"], norms=[(L["in_norm"], L["post_norm"]) for L in layers],
                        final_norm=fn)
    for t in (3, 17, 400, 5, 9):
        a, b = port.decode(t), ref.forward_token(t)
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32)), t
    port.close()
