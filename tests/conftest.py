import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")


def gpu_available() -> bool:
    try:
        import torch
        return torch.cuda.is_available()
    except Exception:
        return False


@pytest.fixture(params=["exact", "folded"])
def gemm_mode(request):
    """Runs a Q4_0 GEMM test under the default arithmetic (exact nibbles,
    fp32 block scale) and again with the opt-in folded-scale kernels;
    restores the previous mode afterwards."""
    import hypno_amd as hk
    prev = hk.set_gemm_numerics(hk.GEMM_FOLDED if request.param == "folded" else hk.GEMM_AUTO)
    yield request.param
    hk.set_gemm_numerics(prev)


@pytest.fixture(scope="session")
def orc():
    from oracle import oracle
    oracle.lib()
    return oracle
