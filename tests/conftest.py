import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for p in (ROOT, os.path.join(ROOT, "oracle"), os.path.join(ROOT, "kronos-2t_amd"), os.path.join(ROOT, "tests")):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and the built libk2t_hip.so")


@pytest.fixture(scope="session")
def gpu_ctx():
    import torch
    import k2t
    if not torch.cuda.is_available():
        pytest.fail("GPU test selected but no GPU is visible")
    ctx = k2t.Ctx(0)
    yield ctx
    ctx.close()
