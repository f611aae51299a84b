"""GPU path (C ABI -> HIP) against the committed golden fixtures: activation quant,
per-(row, chunk) integer dots and the exact-mode fp32 GEMV output, all bit-exact."""
import numpy as np
import pytest

from test_golden import NAMES, load

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("name", NAMES)
def test_gpu_matches_fixture(gpu_ctx, name):
    import torch
    g = load(name)
    rows, cols, p = int(g["rows"]), int(g["cols"]), int(g["p"])
    print(f"golden {name}", flush=True)
    if str(g["fmt"]) == "n4":
        m = gpu_ctx.upload_nibble4(rows, cols, p - 4, g["pair"], g["tail"])
    else:
        m = gpu_ctx.upload_nf(rows, cols, 4, p, g["cb"], g["pair"], g["tail"])
    x = torch.from_numpy(g["x"]).cuda()
    q = torch.empty(cols, dtype=torch.int8, device="cuda")
    s = torch.empty(cols // 64, dtype=torch.float32, device="cuda")
    sm = torch.empty(cols // 64, dtype=torch.int32, device="cuda")
    gpu_ctx.act_quant(x, q, s, sm, cols, 1)
    out = torch.full((rows,), float("nan"), device="cuda")
    dots = torch.zeros((rows, cols // 64), dtype=torch.int32, device="cuda")
    gpu_ctx.set_exact(True)
    try:
        gpu_ctx.gemv(m, q, s, sm, out)
        gpu_ctx.gemv_chunk_dots(m, q, sm, dots)
        gpu_ctx.sync()
    finally:
        gpu_ctx.set_exact(False)
    assert np.array_equal(q.cpu().numpy(), g["q"])
    assert np.array_equal(s.cpu().numpy().view(np.uint32), g["s"].view(np.uint32))
    assert np.array_equal(sm.cpu().numpy(), g["sm"])
    assert np.array_equal(dots.cpu().numpy(), g["dots"])
    assert np.array_equal(out.cpu().numpy().view(np.uint32), g["out"].view(np.uint32))
    m.close()
