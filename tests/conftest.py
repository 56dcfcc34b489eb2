import pathlib
import sys

import pytest

ROOT = pathlib.Path(__file__).resolve().parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) and the built libunholy_amd.so")


@pytest.fixture(params=["exact", "scaled"])
def gemm_arith(request):
    """The prefill GEMM's arithmetic for one test: exact bf16 dequantization (the default, the parity arithmetic) or
    the block-scaled MFMA (a speed mode; its tests hold it to the looser bars written in each test)."""
    from unholy_amd import call
    prev = call("uh_mx_gemm_set_exact", 1 if request.param == "exact" else 0)
    yield request.param
    call("uh_mx_gemm_set_exact", prev)
